"""The fused pack projection (cign_pack_proj_fwd / _bwd through
cign_amd.pack_proj): the Clifford pack (weighting old) built inside the proj
MFMA kernels, G never stored, against the float64 torch restatement of the
same lines (oracle/block_oracle._pack and _linear: model_cign.py:803-846,
:927-933, the gates of :721-749): output and every input and parameter
gradient, eval mode. fp32: |a - e64| <= 1e-5 + 1e-4 |e64| + 4 |e32 - e64|
with e32 the same restatement run in float32 (the error of an fp32 sum of
the same terms in another order); bf16 autocast: 2e-2 relative plus one
bf16 ulp of the tensor's scale (conftest.bf16_flip_atol), the restatement
rounding where autocast does. With dropout, the fused kernels against the
unfused pair (gated pack + linear_gamma_residual) on the same seed: the same
mask bit for bit and values within fp32 reordering. Shapes: D = 64 and 256
(the production width), K = 1..4 hops, n with a partial last row tile, all
interaction and gate modes."""
import numpy as np
import pytest
import torch

from tests.conftest import assert_close, assert_close_fp32_derived, bf16_flip_atol

pytestmark = pytest.mark.gpu


def _inputs(n, D, K, seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)
    return dict(h=r(n, D), Hn=r(n, D), Cn=r(n, D), props=[r(n, 2 * D) for _ in range(K)], gw=r(K, 2 * D) * 0.1,
                gb=r(K) * 0.1, logits=r(K), Wp=r(D, 2 * K * D) * (0.5 / np.sqrt(2 * K * D)), bp=r(D) * 0.1,
                gamma=r(D) * 0.5, G=r(n, D))


def _ref(t, gate, score, interaction, amp):
    """Oracle tail: h + gamma * proj(pack(...)) (eval mode)."""
    import torch.nn.functional as F

    from oracle import block_oracle as B

    Hn, Cn = t["Hn"], t["Cn"]
    if gate == "none":
        alpha = None
    elif gate == "global":
        alpha = torch.softmax(t["logits"], 0).view(1, -1, 1)
    else:
        s = torch.cat([Hn, Cn], -1) if score == "old" else torch.cat([Hn + Cn, torch.abs(Hn - Cn)], -1)
        alpha = torch.softmax(F.linear(s, t["gw"], t["gb"]), -1).unsqueeze(-1)
    G = B._pack(Hn, Cn, t["props"], alpha, interaction, 0)
    return t["h"] + t["gamma"] * B._linear(G, t["Wp"], t["bp"], amp)


LEAVES = ["h", "Hn", "Cn", "gw", "gb", "logits", "Wp", "bp", "gamma"]
PROPS = ("P0", "P1", "P2", "P3")


def _run_gpu(t, gate, score, interaction, amp, p=0.0, seed=11, fused=True):
    from cign_amd.pack_proj import pack_proj_gamma_residual

    dev = torch.device("cuda")
    d = {k: (v.to(dev).requires_grad_() if k != "props" and k != "G" else v) for k, v in t.items()}
    props = [x.to(dev).requires_grad_() for x in t["props"]]
    K, D = t["gw"].shape[0], t["Wp"].shape[0]
    gate_lin = torch.nn.Linear(2 * D, K).to(dev)
    proj = torch.nn.Linear(2 * K * D, D).to(dev)
    with torch.no_grad():
        gate_lin.weight.copy_(d["gw"])
        gate_lin.bias.copy_(d["gb"])
        proj.weight.copy_(d["Wp"])
        proj.bias.copy_(d["bp"])
    if fused:
        out = pack_proj_gamma_residual(d["h"], d["Hn"], d["Cn"], props, gate, gate_lin, d["logits"], score,
                                       interaction, proj, d["gamma"], p, amp, seed=seed)
    else:
        from cign_amd import _pack
        from cign_amd.hop_gate import gated_clifford_pack
        from cign_amd.linear import linear_gamma_residual

        if gate == "node":
            G = gated_clifford_pack(d["Hn"], d["Cn"], props, gate_lin, score, interaction, 0)
        else:
            alpha = None if gate == "none" else torch.softmax(d["logits"], 0).view(1, -1, 1).expand(
                d["Hn"].size(0), -1, -1)
            G = _pack.clifford_pack_any(d["Hn"], d["Cn"], props, alpha, interaction, 0)
        out = linear_gamma_residual(d["h"], G, proj, d["gamma"], p, amp, seed=seed)
    (out * t["G"].to(dev)).sum().backward()
    grads = {k: d[k].grad for k in ("h", "Hn", "Cn", "gamma")}
    grads["Wp"], grads["bp"] = proj.weight.grad, proj.bias.grad
    grads["gw"], grads["gb"] = gate_lin.weight.grad, gate_lin.bias.grad
    grads["logits"] = d["logits"].grad
    grads["props"] = [x.grad for x in props]
    return out, grads


def _ref_grads(t, gate, score, interaction, amp, dt):
    tt = {k: ([x.to(dt).requires_grad_() for x in v] if k == "props" else v.to(dt).requires_grad_())
          for k, v in t.items() if k != "G"}
    out = _ref(tt, gate, score, interaction, amp)
    (out * t["G"].to(dt)).sum().backward()
    g = {k: tt[k].grad for k in LEAVES}
    g["props"] = [x.grad for x in tt["props"]]
    return out, g


CASES = [
    # (n, D, K, interaction, gate, score)
    (300, 64, 3, 1, "node", "new"),
    (300, 64, 2, 0, "node", "old"),
    (130, 64, 1, 2, "global", "new"),
    (300, 64, 4, 1, "none", "new"),
    (257, 128, 3, 2, "node", "new"),
    (300, 256, 3, 1, "node", "new"),
    (200, 256, 3, 0, "global", "old"),
    (1, 256, 2, 2, "none", "new"),
]


@pytest.mark.parametrize("amp", [False, True])
@pytest.mark.parametrize("n,D,K,interaction,gate,score", CASES)
def test_pack_proj_matches_oracle(n, D, K, interaction, gate, score, amp):
    print(f"pack_proj n={n} D={D} K={K} interaction={interaction} gate={gate} score={score} amp={amp}", flush=True)
    t = _inputs(n, D, K, seed=D + K + n)
    out, grads = _run_gpu(t, gate, score, interaction, amp)
    torch.cuda.synchronize()
    e64, g64 = _ref_grads(t, gate, score, interaction, amp, torch.float64)
    e32, g32 = _ref_grads(t, gate, score, interaction, amp, torch.float32)
    np_ = lambda x: x.detach().double().cpu().numpy()

    def check(name, a, x64, x32):
        if amp:
            assert_close(np_(a), np_(x64), rtol=2e-2, atol=1e-5 + bf16_flip_atol(np_(x64)), name=name)
        else:
            # node tensors (first axis n) take the per-row spread term
            per_row = a.dim() >= 1 and a.shape[0] == n and name.split()[-1] in ("out", "h", "Hn", "Cn") + PROPS
            assert_close_fp32_derived(np_(a), np_(x64), np_(x32), name=name, per_row=per_row)

    check("out", out, e64, e32)
    for k in LEAVES:
        if gate != "node" and k in ("gw", "gb"):
            continue
        if gate != "global" and k == "logits":
            continue
        check(f"grad {k}", grads[k], g64[k], g32[k])
    for i, (a, x64, x32) in enumerate(zip(grads["props"], g64["props"], g32["props"])):
        check(f"grad P{i}", a, x64, x32)


@pytest.mark.parametrize("D,amp", [(64, False), (256, False), (256, True)])
def test_pack_proj_dropout_matches_unfused(D, amp):
    """Training mode: the fused kernels draw the unfused pair's dropout mask
    (same seed, same splitmix64 index) and agree in value."""
    check_dropout_against_unfused(300, D, 0.28, amp)


def check_dropout_against_unfused(n, D, p, amp, K=3):
    t = _inputs(n, D, K, seed=5)
    out_f, g_f = _run_gpu(t, "node", "new", 1, amp, p=p, seed=123, fused=True)
    out_u, g_u = _run_gpu(t, "node", "new", 1, amp, p=p, seed=123, fused=False)
    torch.cuda.synchronize()
    # dropped outputs equal h exactly in both
    dropped_f = out_f == t["h"].cuda()
    dropped_u = out_u == t["h"].cuda()
    assert torch.equal(dropped_f, dropped_u)
    assert abs(dropped_f.float().mean().item() - p) < 0.08
    rtol, atol = (2 ** -7, 1e-5) if amp else (1e-4, 1e-5)
    np_ = lambda x: x.detach().double().cpu().numpy()
    assert_close(np_(out_f), np_(out_u), rtol=rtol, atol=atol + (bf16_flip_atol(np_(out_u)) if amp else 0.0),
                 name="out")
    for k in ("Hn", "Cn", "Wp", "gamma", "gw"):
        scale = float(g_u[k].abs().max())
        assert_close(np_(g_f[k]), np_(g_u[k]), rtol=2e-2 if amp else 1e-3, atol=(2e-2 if amp else 1e-4) * scale,
                     name=f"grad {k}")


def test_pack_proj_rejects_bad_shapes():
    import ctypes

    from cign_amd import _lib

    lib = _lib.load_library()
    x = torch.zeros(64, 96, device="cuda")
    arr = _lib.ptr_array([x.data_ptr()])
    args = [_lib.stream_ptr(), 64, 48, 1, 1, 0, x.data_ptr(), x.data_ptr(), ctypes.addressof(arr), 96, x.data_ptr(), 0,
            x.data_ptr(), None, x.data_ptr(), x.data_ptr(), 0.0, 0, x.data_ptr(), x.data_ptr(), x.data_ptr(), None, 0]
    with pytest.raises(RuntimeError, match="D=48"):
        lib.call("cign_pack_proj_fwd", *args)
    args[2], args[3] = 64, 5
    with pytest.raises(RuntimeError, match="K=5"):
        lib.call("cign_pack_proj_fwd", *args)
    assert lib.cign_pack_proj_bwd_workspace_bytes(100, 48, 3) == 0
    assert lib.cign_pack_proj_fwd_workspace_bytes(256, 3, 0) == 0
    assert lib.cign_pack_proj_fwd_workspace_bytes(256, 3, 1) == 2 * 256 * 6 * 256
