"""GPU parity of the fused Clifford packs against the oracle, through the
drop-in modules: old pack (K=3 special + generic K), CIGN switch pack (all
interaction x weighting modes, with and without tanh) and the CIGN generic-K
pack, forward and backward (extension objects and autograd). fp32 tolerance
1e-4 rel / 1e-5 abs."""
import numpy as np
import pytest
import torch

from oracle import cign_oracle as O
from tests.conftest import assert_close, colsum_atol

pytestmark = pytest.mark.gpu
T32 = dict(rtol=1e-4, atol=1e-5)


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def _n(t):
    return t.detach().double().cpu().numpy()


def _inputs(rng, n, D, K):
    H, C = rng.standard_normal((n, D)), rng.standard_normal((n, D))
    props = [rng.standard_normal((n, 2 * D)) for _ in range(K)]
    alpha = rng.random((n, K))
    return H.astype(np.float32), C.astype(np.float32), [p.astype(np.float32) for p in props], alpha.astype(np.float32)


def _check_grads(grads, expected, name):
    gH, gC, gP, gA = grads
    eH, eC, eP, eA = expected
    assert_close(_n(gH), eH, name=f"{name} gH", **T32)
    assert_close(_n(gC), eC, name=f"{name} gC", **T32)
    for k, (g, e) in enumerate(zip(gP, eP)):
        assert_close(_n(g), e, name=f"{name} gP{k}", **T32)
    assert_close(_n(gA), eA, name=f"{name} gA", **T32)


@pytest.mark.parametrize("module,tanh", [("fused_clifford_cign_pack", False), ("fused_clifford_switch_pack", True)])
@pytest.mark.parametrize("interaction", ["old", "new"])
@pytest.mark.parametrize("weighting", ["old", "new"])
@pytest.mark.parametrize("n,D", [(600, 256), (130, 6)])
def test_switch_pack_all_modes(module, tanh, interaction, weighting, n, D):
    import importlib

    mod = importlib.import_module(f"cign_amd.{module}")
    print(f"{module} {interaction}/{weighting} n={n} D={D}", flush=True)
    rng = np.random.default_rng(n + D + len(interaction) + 3 * len(weighting))
    H, C, props, alpha = _inputs(rng, n, D, 3)
    icode = 0 if interaction == "old" else (2 if tanh else 1)
    wcode = 0 if weighting == "old" else 1
    Ht, Ct, Pt = _t(H).requires_grad_(), _t(C).requires_grad_(), [_t(p).requires_grad_() for p in props]
    At = _t(alpha).requires_grad_()
    out = mod.fused_clifford_switch_pack(Ht, Ct, Pt, At, interaction, weighting)
    eout = O.clifford_pack_forward(H, C, props, alpha, icode, wcode)
    assert out.shape == eout.shape
    assert_close(_n(out), eout, name="out", **T32)
    G = rng.standard_normal(eout.shape).astype(np.float32)
    (out * _t(G)).sum().backward()
    expected = O.clifford_pack_backward(G, H, C, props, alpha, icode, wcode)
    _check_grads((Ht.grad, Ct.grad, [p.grad for p in Pt], At.grad), expected, f"{interaction}/{weighting}")


@pytest.mark.parametrize("n,D,K", [(500, 256, 3), (300, 32, 2), (200, 12, 5), (90, 3, 1)])
def test_old_pack_special_and_generic(n, D, K):
    from cign_amd.fused_clifford_pack import ensure_fused_clifford_pack_loaded, fused_clifford_pack

    print(f"old pack n={n} D={D} K={K}", flush=True)
    rng = np.random.default_rng(n * K + D)
    H, C, props, alpha = _inputs(rng, n, D, K)
    Ht, Ct, Pt = _t(H).requires_grad_(), _t(C).requires_grad_(), [_t(p).requires_grad_() for p in props]
    At = _t(alpha[:, :, None]).requires_grad_()  # [N,K,1] is accepted and squeezed
    out = fused_clifford_pack(Ht, Ct, Pt, At)
    eout = O.clifford_pack_forward(H, C, props, alpha, 0, 0)
    assert_close(_n(out), eout, name="out", **T32)
    G = rng.standard_normal(eout.shape).astype(np.float32)
    (out * _t(G)).sum().backward()
    eH, eC, eP, eA = O.clifford_pack_backward(G, H, C, props, alpha, 0, 0)
    _check_grads((Ht.grad, Ct.grad, [p.grad for p in Pt], At.grad[:, :, 0]), (eH, eC, eP, eA), "old")
    # the extension object of the matching kind
    ext = ensure_fused_clifford_pack_loaded(hop_count=K)
    if K == 3:
        o = ext.forward(_t(H), _t(C), *[_t(p) for p in props], _t(alpha))
        grads = ext.backward(_t(G), _t(H), _t(C), *[_t(p) for p in props], _t(alpha))
        assert len(grads) == 6
    else:
        (o,) = ext.forward(_t(H), _t(C), _t(np.stack(props, 1)), _t(alpha))
        grads = ext.backward(_t(G), _t(H), _t(C), _t(np.stack(props, 1)), _t(alpha))
        assert grads[2].shape == (n, K, 2 * D)
    assert_close(_n(o), eout, name="ext out", **T32)


@pytest.mark.parametrize("n,D,K", [(400, 256, 3), (150, 20, 4), (60, 7, 2)])
def test_cign_generic_pack(n, D, K):
    from cign_amd.fused_clifford_cign_generic import fused_clifford_pack

    rng = np.random.default_rng(n + 5 * D + K)
    H, C, props, alpha = _inputs(rng, n, D, K)
    Ht, Ct, Pt = _t(H).requires_grad_(), _t(C).requires_grad_(), [_t(p).requires_grad_() for p in props]
    At = _t(alpha).requires_grad_()
    out = fused_clifford_pack(Ht, Ct, Pt, At)
    eout = O.clifford_pack_forward(H, C, props, alpha, 1, 0)
    assert_close(_n(out), eout, name="out", **T32)
    G = rng.standard_normal(eout.shape).astype(np.float32)
    (out * _t(G)).sum().backward()
    _check_grads((Ht.grad, Ct.grad, [p.grad for p in Pt], At.grad),
                 O.clifford_pack_backward(G, H, C, props, alpha, 1, 0), "cign generic")


def test_pack_argument_errors_and_alpha_default():
    from cign_amd.fused_clifford_cign_pack import ensure_fused_clifford_switch_pack_loaded, fused_clifford_switch_pack
    from cign_amd.fused_clifford_pack import fused_clifford_pack

    rng = np.random.default_rng(1)
    H, C, props, alpha = _inputs(rng, 50, 8, 3)
    Ht, Ct, Pt = _t(H), _t(C), [_t(p) for p in props]
    with pytest.raises(ValueError, match="exactly 3 hops"):
        fused_clifford_switch_pack(Ht, Ct, Pt[:2], None, "old", "old")
    with pytest.raises(ValueError, match="interaction_mode must be old/new"):
        fused_clifford_switch_pack(Ht, Ct, Pt, None, "mixed", "old")
    with pytest.raises(ValueError, match="Expected alpha"):
        fused_clifford_pack(Ht, Ct, Pt, _t(alpha[:, :2]))
    with pytest.raises(ValueError, match="propagated cannot be empty"):
        fused_clifford_pack(Ht, Ct, [], None)
    with pytest.raises(RuntimeError, match=r"alpha must be \[N,3\]"):
        ensure_fused_clifford_switch_pack_loaded().forward(Ht, Ct, *Pt, _t(alpha[:, :2]), 0, 0)
    with pytest.raises(RuntimeError, match="interaction_mode must be 0"):
        ensure_fused_clifford_switch_pack_loaded().forward(Ht, Ct, *Pt, _t(alpha), 3, 0)
    # alpha=None means all-ones weights
    out = fused_clifford_pack(Ht, Ct, Pt, None)
    assert_close(_n(out), O.clifford_pack_forward(H, C, props, np.ones((50, 3)), 0, 0), name="alpha ones", **T32)


@pytest.mark.parametrize("n,D,K,interaction,weighting,score", [
    (600, 256, 3, 1, 0, 1), (600, 256, 3, 2, 1, 1), (601, 256, 3, 0, 0, 0), (300, 64, 2, 1, 1, 0),
    (200, 48, 4, 2, 0, 1), (150, 32, 5, 1, 0, 1), (90, 6, 3, 0, 1, 1), (40, 256, 1, 1, 0, 0),
    (300, 768, 3, 1, 0, 1), (200, 384, 4, 2, 1, 0), (4096, 256, 3, 1, 0, 1)])
def test_gated_pack_matches_oracle(n, D, K, interaction, weighting, score):
    """The node-mode gate fused into the pack (cign_pack_gate_fwd/bwd) against
    the oracle's gate followed by its pack: G_raw, and grad H / C (the pack's
    and the gate's terms summed), grad P_k, grad gate weight and bias."""
    from cign_amd.hop_gate import PackGateFunction

    print(f"gated pack n={n} D={D} K={K} interaction={interaction} weighting={weighting} score={score}", flush=True)
    rng = np.random.default_rng(n + D + K)
    H, C, props, _ = _inputs(rng, n, D, K)
    C[:, 0] = H[:, 0]  # ties of |H - C|: sign(0) = 0 in the gradient
    W = (0.2 * rng.standard_normal((K, 2 * D))).astype(np.float32)
    b = rng.standard_normal(K).astype(np.float32)
    alpha = O.hop_gate_forward(H, C, W, b, score)
    out = O.clifford_pack_forward(H, C, props, alpha, interaction, weighting)
    g = rng.standard_normal(out.shape).astype(np.float32)
    pH, pC, pP, pA = O.clifford_pack_backward(g, H, C, props, alpha, interaction, weighting)
    gH, gC, gW, gb = O.hop_gate_backward(pA, H, C, W, b, score)

    Ht, Ct, Wt, bt = (_t(a).requires_grad_() for a in (H, C, W, b))
    Pt = [_t(p).requires_grad_() for p in props]
    got = PackGateFunction.apply(interaction, weighting, score, Ht, Ct, Wt, bt, *Pt)
    assert_close(_n(got), out, name="G_raw", **T32)
    (got * _t(g)).sum().backward()
    assert_close(_n(Ht.grad), pH + gH, name="grad H", **T32)
    assert_close(_n(Ct.grad), pC + gC, name="grad C", **T32)
    for k in range(K):
        assert_close(_n(Pt[k].grad), pP[k], name=f"grad P{k}", **T32)
    # Parameter gradients sum over n rows: bound from their terms' magnitudes.
    a = O.hop_gate_forward(H, C, W, b, score)
    gl_abs = np.abs(a * (pA - (a * pA).sum(axis=1, keepdims=True)))
    s_abs = np.abs(O.hop_gate_score(H, C, score))
    assert_close(_n(Wt.grad), gW, name="grad gate weight", rtol=1e-4, atol=colsum_atol(gl_abs.T @ s_abs, n))
    assert_close(_n(bt.grad), gb, name="grad gate bias", rtol=1e-4, atol=colsum_atol(gl_abs.sum(0), n))


def test_gated_pack_equals_gate_then_pack():
    """The fused path and the two-call path (node_hop_gate, then the pack) of
    the block agree, value and gradients, within fp32 rounding."""
    from cign_amd import _pack
    from cign_amd.hop_gate import gated_clifford_pack, node_hop_gate

    rng = np.random.default_rng(7)
    n, D, K = 500, 256, 3
    H, C, props, _ = _inputs(rng, n, D, K)
    lin = torch.nn.Linear(2 * D, K).cuda()
    g = _t(rng.standard_normal((n, 2 * K * D)))
    res = []
    for fused in (True, False):
        Ht, Ct = _t(H).requires_grad_(), _t(C).requires_grad_()
        Pt = [_t(p).requires_grad_() for p in props]
        lin.zero_grad()
        if fused:
            out = gated_clifford_pack(Ht, Ct, Pt, lin, "new", 1, 0)
        else:
            out = _pack.clifford_pack_any(Ht, Ct, Pt, node_hop_gate(Ht, Ct, lin, "new"), 1, 0)
        (out * g).sum().backward()
        res.append([out.detach(), Ht.grad, Ct.grad, *[p.grad for p in Pt], lin.weight.grad.clone(),
                    lin.bias.grad.clone()])
    for i, (a, e) in enumerate(zip(*res)):
        assert_close(_n(a), _n(e), name=f"output {i}", rtol=1e-4, atol=1e-4)
