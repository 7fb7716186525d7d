"""GPU parity of the GAT side ops and the block ops against the oracle,
through the drop-in modules (extension objects and autograd wrappers), which
call the C-ABI. Tolerances fp32 1e-4 rel / 1e-5 abs (LayerNorm rows of D<=256
summed in fp32: 1e-4 rel / 1e-4 abs); dropout masks bit-exact."""
import numpy as np
import pytest
import torch

from oracle import cign_oracle as O
from tests.conftest import assert_close, colsum_atol

pytestmark = pytest.mark.gpu
T32 = dict(rtol=1e-4, atol=1e-5)
TLN = dict(rtol=1e-4, atol=1e-4)


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def _n(t):
    return t.detach().double().cpu().numpy()


# ---------------------------------------------------------------------------
# attention logits
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n,H,C", [(500, 4, 16), (300, 6, 256), (257, 3, 5), (64, 1, 1), (40, 2, 1024), (7, 8, 12)])
def test_attention_logits_matches_oracle(n, H, C):
    from cign_amd.fused_gat_sideops import ensure_fused_gat_sideops_loaded

    print(f"attention logits n={n} H={H} C={C}", flush=True)
    rng = np.random.default_rng(n + H + C)
    x, a_s, a_d = rng.standard_normal((n, H, C)), rng.standard_normal((1, H, C)), rng.standard_normal((1, H, C))
    gs, gd = rng.standard_normal((n, H)), rng.standard_normal((n, H))
    ext = ensure_fused_gat_sideops_loaded()
    xs, ass, ads = _t(x), _t(a_s), _t(a_d)
    s, d = ext.attention_forward(xs, ass, ads)
    es, ed = O.attention_logits_forward(x.astype(np.float32), a_s.astype(np.float32), a_d.astype(np.float32))
    assert_close(_n(s), es, name="alpha_src", **T32)
    assert_close(_n(d), ed, name="alpha_dst", **T32)
    gx, g_s, g_d = ext.attention_backward(_t(gs), _t(gd), xs, ass, ads)
    egx, egs, egd = O.attention_logits_backward(gs.astype(np.float32), gd.astype(np.float32), x.astype(np.float32),
                                                a_s.astype(np.float32), a_d.astype(np.float32))
    assert g_s.shape == (1, H, C)
    assert_close(_n(gx), egx, name="grad_x", **T32)
    # sum over n rows: fp32 accumulation error grows like sqrt(n) * |terms|
    assert_close(_n(g_s), egs, name="grad_att_src", rtol=1e-4, atol=1e-4)
    assert_close(_n(g_d), egd, name="grad_att_dst", rtol=1e-4, atol=1e-4)


def test_attention_autograd_and_errors():
    from cign_amd.fused_gat_sideops import fused_attention_logits

    rng = np.random.default_rng(5)
    n, H, C = 300, 4, 16
    x = _t(rng.standard_normal((n, H, C))).requires_grad_()
    a_s = _t(rng.standard_normal((1, H, C))).requires_grad_()
    a_d = _t(rng.standard_normal((1, H, C))).requires_grad_()
    s, d = fused_attention_logits(x, a_s, a_d)
    w1, w2 = rng.standard_normal((n, H)), rng.standard_normal((n, H))
    (s * _t(w1) + d * _t(w2)).sum().backward()
    egx, egs, egd = O.attention_logits_backward(w1, w2, _n(x), _n(a_s), _n(a_d))
    assert_close(_n(x.grad), egx, name="x.grad", **T32)
    assert_close(_n(a_s.grad), egs, name="att_src.grad", rtol=1e-4, atol=1e-4)
    assert_close(_n(a_d.grad), egd, name="att_dst.grad", rtol=1e-4, atol=1e-4)
    with pytest.raises(TypeError):
        fused_attention_logits(x.detach().double(), a_s, a_d)
    from cign_amd.fused_gat_sideops import ensure_fused_gat_sideops_loaded

    with pytest.raises(RuntimeError, match=r"att_src must be \[1,H,C\]"):
        ensure_fused_gat_sideops_loaded().attention_forward(x.detach(), a_s.detach()[0], a_d.detach())
    with pytest.raises(RuntimeError, match="too wide"):
        z = torch.zeros(2, 1, 1028, device="cuda")
        ensure_fused_gat_sideops_loaded().attention_forward(z, z[:1], z[:1])


# ---------------------------------------------------------------------------
# head mean + bias + SiLU
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n,H,C", [(500, 4, 16), (300, 6, 256), (101, 3, 7), (1, 1, 1), (33, 2, 1030)])
def test_head_silu_matches_oracle(n, H, C):
    from cign_amd.fused_gat_sideops import ensure_fused_gat_sideops_loaded

    print(f"head silu n={n} H={H} C={C}", flush=True)
    rng = np.random.default_rng(n * 7 + C)
    out, b, gy = rng.standard_normal((n, H, C)), rng.standard_normal(C), rng.standard_normal((n, C))
    ext = ensure_fused_gat_sideops_loaded()
    y, pre = ext.head_silu_forward(_t(out), _t(b))
    ey, epre = O.head_silu_forward(out.astype(np.float32), b.astype(np.float32))
    assert_close(_n(pre), epre, name="pre", **T32)
    assert_close(_n(y), ey, name="y", **T32)
    g_out, g_b = ext.head_silu_backward(_t(gy), pre, H)
    ego, egb = O.head_silu_backward(gy.astype(np.float32), _n(pre), H)
    assert_close(_n(g_out), ego, name="grad_out", **T32)
    assert_close(_n(g_b), egb, name="grad_bias", rtol=1e-4, atol=1e-4)


def test_head_silu_autograd_matches_collapsed_gat_epilogue():
    """fused_head_mean_bias_silu(out, bias) == SiLU(mean_h out + bias), with
    gradients, through the autograd wrapper."""
    from cign_amd.fused_gat_sideops import fused_head_mean_bias_silu

    rng = np.random.default_rng(9)
    n, H, C = 200, 4, 16
    out = _t(rng.standard_normal((n, H, C))).requires_grad_()
    b = _t(rng.standard_normal(C)).requires_grad_()
    y = fused_head_mean_bias_silu(out, b)
    w = rng.standard_normal((n, C))
    (y * _t(w)).sum().backward()
    ey, epre = O.head_silu_forward(_n(out), _n(b))
    assert_close(_n(y), ey, name="y", **T32)
    ego, egb = O.head_silu_backward(w, epre, H)
    assert_close(_n(out.grad), ego, name="out.grad", **T32)
    assert_close(_n(b.grad), egb, name="bias.grad", rtol=1e-4, atol=1e-4)
    with pytest.raises(ValueError, match="bias"):
        fused_head_mean_bias_silu(out, None)


# ---------------------------------------------------------------------------
# block ops
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n,D,p", [(1000, 256, 0.0), (1000, 256, 0.3), (777, 64, 0.5), (300, 100, 0.1), (65, 7, 0.2),
                                   (10, 1, 0.0), (513, 255, 0.4), (4096, 256, 0.3), (20000, 64, 0.0)])
def test_dropout_layernorm_matches_oracle(n, D, p):
    from cign_amd.fused_block_ops import ensure_fused_block_ops_loaded

    print(f"dropout LN n={n} D={D} p={p}", flush=True)
    rng = np.random.default_rng(n + D)
    x, w, b, gy = (rng.standard_normal((n, D)), rng.standard_normal(D), rng.standard_normal(D),
                   rng.standard_normal((n, D)))
    seed = 0x1234_5678_9ABC
    ext = ensure_fused_block_ops_loaded()
    y, mean, rstd, mask = ext.dropout_layernorm_forward(_t(x), _t(w), _t(b), p, 1e-5, seed)
    keep = O.block_dropout_keep(seed, n * D, p).reshape(n, D)
    assert np.array_equal(mask.cpu().numpy() != 0, keep), "dropout mask must be bit-exact"
    x32, w32, b32 = (a.astype(np.float32) for a in (x, w, b))
    ey, emu, ers = O.dropout_layernorm_forward(x32, w32, b32, np.float32(p), 1e-5, keep)
    assert_close(_n(y), ey, name="y", **TLN)
    assert_close(_n(mean), emu, name="mean", **TLN)
    assert_close(_n(rstd), ers, name="rstd", rtol=1e-4, atol=1e-4)
    dx, dw, db = ext.dropout_layernorm_backward(_t(gy), _t(x), _t(w), mean, rstd, mask, p)
    edx, edw, edb = O.dropout_layernorm_backward(gy.astype(np.float32), x32, w32, np.float32(p), 1e-5, keep)
    assert_close(_n(dx), edx, name="dx", **TLN)
    xhat = (np.where(keep, x32 / (1.0 - p) if p > 0 else x32, 0.0) - emu[:, None]) * ers[:, None]
    assert_close(_n(dw), edw, name="dw", rtol=1e-4, atol=colsum_atol(np.abs(gy * xhat).sum(0), n))
    assert_close(_n(db), edb, name="db", rtol=1e-4, atol=colsum_atol(np.abs(gy).sum(0), n))


@pytest.mark.parametrize("n,D", [(1000, 256), (300, 100), (50, 3), (4096, 256), (20000, 64)])
def test_add_layernorm_matches_oracle(n, D):
    from cign_amd.fused_block_ops import ensure_fused_block_ops_loaded

    rng = np.random.default_rng(n * 3 + D)
    a, b0, w, b, gy = (rng.standard_normal((n, D)), rng.standard_normal((n, D)), rng.standard_normal(D),
                       rng.standard_normal(D), rng.standard_normal((n, D)))
    ext = ensure_fused_block_ops_loaded()
    y, mean, rstd = ext.add_layernorm_forward(_t(a), _t(b0), _t(w), _t(b), 1e-5)
    f = [v.astype(np.float32) for v in (a, b0, w, b)]
    ey, emu, ers = O.add_layernorm_forward(*f, 1e-5)
    assert_close(_n(y), ey, name="y", **TLN)
    dz, dw, db = ext.add_layernorm_backward(_t(gy), _t(a), _t(b0), _t(w), mean, rstd)
    edz, edw, edb = O.add_layernorm_backward(gy.astype(np.float32), f[0], f[1], f[2], 1e-5)
    assert_close(_n(dz), edz, name="dz", **TLN)
    xhat = (f[0] + f[1] - emu[:, None]) * ers[:, None]
    assert_close(_n(dw), edw, name="dw", rtol=1e-4, atol=colsum_atol(np.abs(gy * xhat).sum(0), n))
    assert_close(_n(db), edb, name="db", rtol=1e-4, atol=colsum_atol(np.abs(gy).sum(0), n))


@pytest.mark.parametrize("n,D,p", [(1000, 256, 0.5), (400, 64, 0.0), (77, 9, 0.25), (20000, 256, 0.3)])
def test_gamma_residual_matches_oracle(n, D, p):
    from cign_amd.fused_block_ops import ensure_fused_block_ops_loaded

    rng = np.random.default_rng(n + 11 * D)
    h, g, gamma, gy = (rng.standard_normal((n, D)), rng.standard_normal((n, D)), rng.standard_normal(D),
                       rng.standard_normal((n, D)))
    seed = 987654321
    ext = ensure_fused_block_ops_loaded()
    y, mask = ext.dropout_gamma_residual_forward(_t(h), _t(g), _t(gamma), p, seed)
    keep = O.block_dropout_keep(seed, n * D, p).reshape(n, D)
    assert np.array_equal(mask.cpu().numpy() != 0, keep)
    f = [v.astype(np.float32) for v in (h, g, gamma)]
    assert_close(_n(y), O.gamma_residual_forward(f[0], f[1], f[2], np.float32(p), keep), name="y", **T32)
    gg, ggamma = ext.dropout_gamma_residual_backward(_t(gy), _t(g), _t(gamma), mask, p)
    _, egg, eggamma = O.gamma_residual_backward(gy.astype(np.float32), f[1], f[2], np.float32(p), keep)
    assert_close(_n(gg), egg, name="grad_g", **T32)
    m = np.where(keep, 1.0 / (1.0 - p) if p > 0 else 1.0, 0.0)
    assert_close(_n(ggamma), eggamma, name="grad_gamma", rtol=1e-4, atol=colsum_atol(np.abs(gy * f[1] * m).sum(0), n))


def test_block_ops_autograd_seed_stream_and_errors():
    """Public wrappers: the per-call seed follows fused_block_ops.py:46-50
    (counter advances only when p > 0), masks follow that seed, and
    gradients flow to every input."""
    import cign_amd.fused_block_ops as B

    rng = np.random.default_rng(3)
    n, D = 200, 32
    x = _t(rng.standard_normal((n, D))).requires_grad_()
    w = _t(rng.standard_normal(D)).requires_grad_()
    b = _t(rng.standard_normal(D)).requires_grad_()
    torch.manual_seed(4242)
    B._CALL_COUNTER = __import__("itertools").count()
    y0 = B.fused_dropout_layernorm(x, w, b, 0.0, 1e-5)  # p = 0: seed 0, counter unchanged
    y1 = B.fused_dropout_layernorm(x, w, b, 0.5, 1e-5)  # call 1, tag 1
    seed1 = O.block_ops_seed(4242, 1, 1, 0.5)
    keep = O.block_dropout_keep(seed1, n * D, 0.5).reshape(n, D)
    ey, _, _ = O.dropout_layernorm_forward(_n(x), _n(w), _n(b), np.float32(0.5), 1e-5, keep)
    assert_close(_n(y1), ey, name="y1", **TLN)
    h = _t(rng.standard_normal((n, D))).requires_grad_()
    gam = _t(rng.standard_normal(D)).requires_grad_()
    y2 = B.fused_dropout_gamma_residual(h, y1, gam, 0.25)  # call 2, tag 2
    keep2 = O.block_dropout_keep(O.block_ops_seed(4242, 2, 2, 0.25), n * D, 0.25).reshape(n, D)
    assert_close(_n(y2), O.gamma_residual_forward(_n(h), _n(y1), _n(gam), np.float32(0.25), keep2), name="y2",
                 **T32)
    a2 = _t(rng.standard_normal((n, D))).requires_grad_()
    y3 = B.fused_add_layernorm(y2, a2, w, b, 1e-5)
    (y0.sum() + y3.square().sum()).backward()
    for t in (x, w, b, h, gam, a2):
        assert t.grad is not None and torch.isfinite(t.grad).all()
    with pytest.raises(ValueError, match="1<=D<=256"):
        B.fused_dropout_layernorm(torch.zeros(4, 257, device="cuda"), torch.zeros(257, device="cuda"),
                                  torch.zeros(257, device="cuda"), 0.0, 1e-5)
    with pytest.raises(TypeError):
        B.fused_add_layernorm(torch.zeros(4, 8), torch.zeros(4, 8), torch.zeros(8), torch.zeros(8), 1e-5)
    with pytest.raises(RuntimeError, match=r"dropout_p must be in \[0,1\)"):
        B.ensure_fused_block_ops_loaded().dropout_layernorm_forward(x.detach(), w.detach(), b.detach(), 1.0, 1e-5, 1)


def test_block_ops_empty_rows_give_zero_parameter_grads():
    from cign_amd.fused_block_ops import ensure_fused_block_ops_loaded

    ext = ensure_fused_block_ops_loaded()
    D = 16
    x = torch.zeros(0, D, device="cuda")
    w = torch.ones(D, device="cuda")
    y, mean, rstd, mask = ext.dropout_layernorm_forward(x, w, w, 0.2, 1e-5, 1)
    dx, dw, db = ext.dropout_layernorm_backward(x, x, w, mean, rstd, mask, 0.2)
    assert dx.shape == (0, D) and torch.equal(dw, torch.zeros_like(dw)) and torch.equal(db, torch.zeros_like(db))


# ---------------------------------------------------------------------------
# hop gate
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n,D,K,mode", [(1000, 256, 3, 1), (1000, 256, 3, 0), (1003, 256, 3, 1), (501, 64, 4, 0),
                                        (300, 32, 5, 1), (77, 7, 16, 1), (50, 300, 1, 0), (10, 4, 2, 1),
                                        (4096, 256, 3, 1), (20000, 64, 3, 0)])
def test_hop_gate_matches_oracle(n, D, K, mode):
    from cign_amd.hop_gate import HopGateFunction

    print(f"hop gate n={n} D={D} K={K} mode={mode}", flush=True)
    rng = np.random.default_rng(n + D + K)
    H, C = rng.standard_normal((n, D)).astype(np.float32), rng.standard_normal((n, D)).astype(np.float32)
    C[:, 0] = H[:, 0]  # ties of |H - C|: sign(0) = 0 in the gradient
    W, b = (0.2 * rng.standard_normal((K, 2 * D))).astype(np.float32), rng.standard_normal(K).astype(np.float32)
    g = rng.standard_normal((n, K)).astype(np.float32)
    Ht, Ct, Wt, bt = (_t(a).requires_grad_() for a in (H, C, W, b))
    a = HopGateFunction.apply(Ht, Ct, Wt, bt, mode)
    assert_close(_n(a), O.hop_gate_forward(H, C, W, b, mode), name="alpha", **T32)
    (a * _t(g)).sum().backward()
    gH, gC, gW, gb = O.hop_gate_backward(g, H, C, W, b, mode)
    assert_close(_n(Ht.grad), gH, name="grad H", **T32)
    assert_close(_n(Ct.grad), gC, name="grad C", **T32)
    gl_abs, s_abs = _gate_terms(g, H, C, W, b, mode)
    assert_close(_n(Wt.grad), gW, name="grad weight", rtol=1e-4, atol=colsum_atol(gl_abs.T @ s_abs, n))
    assert_close(_n(bt.grad), gb, name="grad bias", rtol=1e-4, atol=colsum_atol(gl_abs.sum(0), n))


def _gate_terms(g_alpha, H, C, W, b, mode):
    """|d loss / d logits| and |score| of the hop gate: the magnitudes of the
    per-row terms of its weight and bias gradients (for their error bound)."""
    a = O.hop_gate_forward(H, C, W, b, mode)
    g = np.asarray(g_alpha, np.float64)
    return np.abs(a * (g - (a * g).sum(axis=1, keepdims=True))), np.abs(O.hop_gate_score(H, C, mode))


@pytest.mark.parametrize("n,D", [(1000, 256), (333, 100), (50, 6), (4096, 256), (20000, 64)])
def test_add_layernorm_cat_matches_oracle(n, D):
    """(LN(a + b), [b | LN(a + b)]) and the backward given both outputs'
    gradients (cign_add_ln_cat_fwd/bwd) against the oracle's add+LayerNorm:
    grad a = the LN backward of grad_y + grad_cat[:, D:], grad b = grad a +
    grad_cat[:, :D]; weight and bias gradients from the summed grad_y."""
    from cign_amd.fused_block_ops import fused_add_layernorm_cat

    print(f"add+ln+cat n={n} D={D}", flush=True)
    rng = np.random.default_rng(n + D)
    a, b = rng.standard_normal((n, D)).astype(np.float32), rng.standard_normal((n, D)).astype(np.float32)
    w, bias = (1 + 0.3 * rng.standard_normal(D)).astype(np.float32), rng.standard_normal(D).astype(np.float32)
    gy, gcat = rng.standard_normal((n, D)).astype(np.float32), rng.standard_normal((n, 2 * D)).astype(np.float32)
    at, bt, wt, bst = (_t(x).requires_grad_() for x in (a, b, w, bias))
    y, cat = fused_add_layernorm_cat(at, bt, wt, bst, 1e-5)
    ey = O.add_layernorm_forward(a, b, w, bias, 1e-5)[0]
    assert_close(_n(y), ey, name="y", **T32)
    assert_close(_n(cat[:, D:]), ey, name="cat right", **T32)
    assert np.array_equal(_n(cat[:, :D]), b.astype(np.float64))
    ((y * _t(gy)).sum() + (cat * _t(gcat)).sum()).backward()
    dz, gw, gb = O.add_layernorm_backward(gy + gcat[:, D:], a, b, w, 1e-5)
    assert_close(_n(at.grad), dz, name="grad a", **T32)
    assert_close(_n(bt.grad), dz + gcat[:, :D], name="grad b", **T32)
    _, mu, rs = O.add_layernorm_forward(a, b, w, bias, 1e-5)
    xhat = (a.astype(np.float64) + b - mu[:, None]) * rs[:, None]
    gsum = gy.astype(np.float64) + gcat[:, D:]
    assert_close(_n(wt.grad), gw, name="grad weight", rtol=1e-4, atol=colsum_atol(np.abs(gsum * xhat).sum(0), n))
    assert_close(_n(bst.grad), gb, name="grad bias", rtol=1e-4, atol=colsum_atol(np.abs(gsum).sum(0), n))
