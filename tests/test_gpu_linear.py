"""GPU parity of the MFMA projections (cign_linear_*: plain, fused GAT
attention logits, fused dropout-gamma-residual) and their backward against
the float64 oracle, through the drop-in Python API (cign_amd.linear) and the
C-ABI. Tolerances: fp32 math 1e-4 rel / 1e-5 abs; bf16 autocast math 2e-2
rel / 2e-2 abs against the float64 oracle. Under autocast the backward reads
bf16 operands and returns bf16 grad_x, grad_W and grad_b, as the bf16
Linear's backward does: they are bf16 values, and within one bf16 rounding
of the float64 oracle with the same rounding points (O.linear_backward(amp=
True), conftest.assert_bf16_sum_close). Dropout masks are bit-exact against
the splitmix64 oracle."""
import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import cign_oracle as O
from tests.conftest import assert_bf16_sum_close, assert_close, colsum_atol

pytestmark = pytest.mark.gpu
F32 = dict(rtol=1e-4, atol=1e-5)
BF16 = dict(rtol=2e-2, atol=2e-2)


def _t(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dtype).cuda()


def _np(t):
    return t.detach().double().cpu().numpy()


@pytest.mark.parametrize("M,N,K", [(1000, 64, 300), (777, 256, 1536), (130, 1536, 256), (5, 48, 20), (300, 50, 8),
                                   (129, 3, 37), (64, 17, 5), (0, 16, 16), (2000, 5, 768), (333, 16, 70),
                                   (5000, 5, 128)])
@pytest.mark.parametrize("amp", [False, True])
def test_linear_forward_backward(M, N, K, amp):
    from cign_amd.linear import mfma_linear

    print(f"linear M={M} N={N} K={K} amp={amp}", flush=True)
    rng = np.random.default_rng(M + N + K)
    lin = nn.Linear(K, N).cuda()
    with torch.no_grad():
        lin.weight.copy_(_t(rng.standard_normal((N, K)) / np.sqrt(K)))
        lin.bias.copy_(_t(rng.standard_normal(N) * 0.1))
    x = _t(rng.standard_normal((M, K))).requires_grad_(True)
    y = mfma_linear(lin, x, amp)
    gy = (rng.standard_normal((M, N)) / np.sqrt(max(M, 1))).astype(np.float32)  # a mean-loss scale
    y.backward(_t(gy))
    tol = BF16 if amp else F32
    ref = O.linear_forward(_np(x), _np(lin.weight), _np(lin.bias), amp=amp)
    assert y.dtype == torch.float32
    # amp: both sides round the same operands and the output to bf16, so they
    # differ by at most one bf16 ulp (2^-7 relative) where fp32 and fp64 sums
    # round differently.
    assert_close(_np(y), ref, name="y", **(dict(rtol=2.0 ** -7, atol=1e-6) if amp else tol))
    gx, gw, gb = O.linear_backward(gy, _np(x), _np(lin.weight))
    assert_close(_np(x.grad), gx, name="grad_x", **tol)
    # grad_W and grad_b sum over the M rows: fp32 within the float32
    # summation bound of their terms (the split-M chunks summed in order)
    assert_close(_np(lin.weight.grad), gw, name="grad_w", **_m_tol(tol, np.abs(gy).T @ np.abs(_np(x)), M))
    assert_close(_np(lin.bias.grad), gb, name="grad_b", **_m_tol(tol, np.abs(gy).sum(0), M))
    if amp:
        # autocast backward: bf16 operands, fp32 accumulation, bf16 results
        _check_amp_backward(gy, _np(x), _np(lin.weight), _np(x.grad), _np(lin.weight.grad), _np(lin.bias.grad))


def _m_tol(tol, abs_terms, M):
    """tol for a sum over M rows: fp32 gets colsum_atol of its terms' sum of
    magnitudes (at least the flat 1e-5); bf16 keeps its bar."""
    if tol is BF16:
        return tol
    return dict(rtol=tol["rtol"], atol=np.maximum(tol["atol"], colsum_atol(abs_terms, M)))


def _check_amp_backward(gy, x, w, gx, gw, gb):
    """The bf16-autocast backward against O.linear_backward(amp=True): each
    gradient a float32 sum of products of bf16 operands rounded once to bf16
    (conftest.assert_bf16_sum_close)."""
    gyr, xr, wr = O.bf16_round(gy), O.bf16_round(x), O.bf16_round(w)
    ex, ew, eb = O.linear_backward(gy, x, w, amp=True)
    M, N = gy.shape
    assert_bf16_sum_close(gx, ex, np.abs(gyr) @ np.abs(wr), N, "grad_x (amp)")
    assert_bf16_sum_close(gw, ew, np.abs(gyr).T @ np.abs(xr), M, "grad_w (amp)")
    if gb is not None:
        assert_bf16_sum_close(gb, eb, np.abs(gyr).sum(0), M, "grad_b (amp)")


def test_linear_bf16_input():
    from cign_amd.linear import mfma_linear

    rng = np.random.default_rng(3)
    lin = nn.Linear(64, 96, bias=False).cuda()
    x = _t(rng.standard_normal((500, 64)), torch.bfloat16)
    y = mfma_linear(lin, x, True)
    assert_close(_np(y), O.linear_forward(_np(x), _np(lin.weight), None, amp=True), name="y", **BF16)
    with pytest.raises(RuntimeError, match="bfloat16 inputs need math=1"):
        mfma_linear(lin, x, False)


@pytest.mark.parametrize("H,C,K,amp", [(4, 16, 300, False), (4, 16, 256, True), (6, 32, 128, False),
                                       (2, 64, 64, False), (1, 128, 96, True), (6, 256, 256, False), (3, 20, 40, False)])
def test_linear_attention_logits(H, C, K, amp, M=777):
    from cign_amd.linear import linear_attention_logits

    print(f"lin+logits M={M} H={H} C={C} K={K} amp={amp}", flush=True)
    rng = np.random.default_rng(H * C + K)
    W = _t(rng.standard_normal((H * C, K)) / np.sqrt(K)).requires_grad_(True)
    s = _t(rng.standard_normal((1, H, C)) * 0.3).requires_grad_(True)
    d = _t(rng.standard_normal((1, H, C)) * 0.3).requires_grad_(True)
    x = _t(rng.standard_normal((M, K))).requires_grad_(True)
    xp, a_src, a_dst = linear_attention_logits(x, W, s, d, H, amp)
    sc = 1.0 / np.sqrt(M)  # gradient probes at a mean-loss scale
    g_xp = (rng.standard_normal((M, H, C)) * sc).astype(np.float32)
    g_s = (rng.standard_normal((M, H)) * sc).astype(np.float32)
    g_d = (rng.standard_normal((M, H)) * sc).astype(np.float32)
    torch.autograd.backward([xp, a_src, a_dst], [_t(g_xp), _t(g_s), _t(g_d)])
    tol = BF16 if amp else F32
    xp_ref = O.linear_forward(_np(x), _np(W), None, amp=amp).reshape(M, H, C)
    assert_close(_np(xp), xp_ref, name="x_proj", **tol)
    as_ref, ad_ref = O.attention_logits_forward(_np(xp), _np(s)[0], _np(d)[0])
    assert_close(_np(a_src), as_ref, name="alpha_src", **F32)  # from the kernel's own x_proj
    assert_close(_np(a_dst), ad_ref, name="alpha_dst", **F32)
    gx_log, gs_ref, gd_ref = O.attention_logits_backward(g_s, g_d, _np(xp), _np(s)[0], _np(d)[0])
    g_tot = (g_xp + gx_log).reshape(M, H * C)
    gx, gw, _ = O.linear_backward(g_tot, _np(x), _np(W))
    assert_close(_np(x.grad), gx, name="grad_x", **tol)
    assert_close(_np(W.grad), gw, name="grad_w", **_m_tol(tol, np.abs(g_tot).T @ np.abs(_np(x)), M))
    if amp:  # the bf16 Linear's backward outputs
        assert np.array_equal(O.bf16_round(_np(x.grad)), _np(x.grad))
        assert np.array_equal(O.bf16_round(_np(W.grad)), _np(W.grad))
    xp_abs = np.abs(_np(xp))
    assert_close(_np(s.grad).reshape(H, C), gs_ref.reshape(H, C), name="grad_att_src",
                 **_m_tol(F32, (np.abs(g_s)[:, :, None] * xp_abs).sum(0), M))
    assert_close(_np(d.grad).reshape(H, C), gd_ref.reshape(H, C), name="grad_att_dst",
                 **_m_tol(F32, (np.abs(g_d)[:, :, None] * xp_abs).sum(0), M))


@pytest.mark.parametrize("M,N,K,p,amp", [(900, 256, 1536, 0.0, False), (900, 256, 1536, 0.3, False),
                                         (500, 64, 128, 0.5, True), (33, 20, 12, 0.1, False)])
def test_linear_gamma_residual(M, N, K, p, amp):
    from cign_amd.linear import linear_gamma_residual

    print(f"proj+gamma M={M} N={N} K={K} p={p} amp={amp}", flush=True)
    rng = np.random.default_rng(M + K)
    lin = nn.Linear(K, N).cuda()
    with torch.no_grad():
        lin.weight.copy_(_t(rng.standard_normal((N, K)) / np.sqrt(K)))
        lin.bias.copy_(_t(rng.standard_normal(N) * 0.1))
    h = _t(rng.standard_normal((M, N))).requires_grad_(True)
    x = _t(rng.standard_normal((M, K))).requires_grad_(True)
    gamma = _t(rng.uniform(0.2, 0.8, N)).requires_grad_(True)
    seed = 987654321
    out = linear_gamma_residual(h, x, lin, gamma, p, amp, seed=seed)
    gy = (rng.standard_normal((M, N)) / np.sqrt(M)).astype(np.float32)  # a mean-loss scale
    out.backward(_t(gy))
    keep = O.block_dropout_keep(seed, M * N, p).reshape(M, N)
    g_ref = O.linear_forward(_np(x), _np(lin.weight), _np(lin.bias), amp=amp)
    tol = BF16 if amp else F32
    assert_close(_np(out), O.gamma_residual_forward(_np(h), g_ref, _np(gamma), p, keep), name="out", **tol)
    _, gg, ggamma = O.gamma_residual_backward(gy, g_ref, _np(gamma), p, keep)
    gx, gw, gb = O.linear_backward(gg, _np(x), _np(lin.weight))
    assert_close(_np(h.grad), gy, name="grad_h", rtol=0, atol=0)
    assert_close(_np(x.grad), gx, name="grad_x", **tol)
    assert_close(_np(lin.weight.grad), gw, name="grad_w", **_m_tol(tol, np.abs(gg).T @ np.abs(_np(x)), M))
    assert_close(_np(lin.bias.grad), gb, name="grad_b", **_m_tol(tol, np.abs(gg).sum(0), M))
    assert_close(_np(gamma.grad), ggamma, name="grad_gamma", **_m_tol(tol, (np.abs(gy) * np.abs(g_ref)).sum(0) /
                                                                          (1.0 - p), M))
    if amp:  # the bf16 Linear's backward outputs
        for name, t in (("grad_x", x.grad), ("grad_w", lin.weight.grad), ("grad_b", lin.bias.grad)):
            assert np.array_equal(O.bf16_round(_np(t)), _np(t)), name


def test_linear_gamma_mask_bits():
    """The fused epilogue's mask is the block-op splitmix64 stream, bit for bit."""
    from cign_amd import _lib

    lib = _lib.load_library()
    rng = np.random.default_rng(9)
    M, N, K, p, seed = 300, 64, 32, 0.37, 424242
    x, w, h = _t(rng.standard_normal((M, K))), _t(rng.standard_normal((N, K))), _t(rng.standard_normal((M, N)))
    gamma = _t(np.ones(N))
    g = torch.empty(M, N, device="cuda")
    y = torch.empty(M, N, device="cuda")
    mask = torch.empty(M, N, dtype=torch.uint8, device="cuda")
    lib.call("cign_linear_gamma_fwd", _lib.stream_ptr(), M, N, K, 0, 0, x.data_ptr(), w.data_ptr(), None,
             h.data_ptr(), gamma.data_ptr(), p, seed, g.data_ptr(), y.data_ptr(), mask.data_ptr())
    torch.cuda.synchronize()
    keep = O.block_dropout_keep(seed, M * N, p).reshape(M, N)
    assert np.array_equal(mask.cpu().numpy().astype(bool), keep)


def test_linear_argument_errors():
    from cign_amd import _lib

    lib = _lib.load_library()
    x = torch.zeros(4, 6, device="cuda")
    w = torch.zeros(8, 6, device="cuda")
    y = torch.empty(4, 8, device="cuda")
    with pytest.raises(RuntimeError, match="math must be"):
        lib.call("cign_linear_fwd", _lib.stream_ptr(), 4, 8, 6, 0, 5, x.data_ptr(), w.data_ptr(), None, y.data_ptr())
    with pytest.raises(RuntimeError, match="channels=20"):
        a = torch.empty(4, 2, device="cuda")
        lib.call("cign_linear_logits_fwd", _lib.stream_ptr(), 4, 2, 20, 8, 0, 0, x.data_ptr(), w.data_ptr(),
                 w.data_ptr(), w.data_ptr(), y.data_ptr(), a.data_ptr(), a.data_ptr())


@pytest.mark.parametrize("M,N,K,xdt,ybf16,bias", [
    (24492, 1536, 256, torch.float32, True, False),   # the production block's GAT lin
    (1000, 1536, 256, torch.bfloat16, True, True),
    (777, 200, 192, torch.float32, True, True),       # N % 64 != 0: a partial last column tile
    (500, 96, 64, torch.bfloat16, True, False),
    (333, 100, 128, torch.float32, True, True),       # N % 8 != 0: guarded bf16 stores
    (130, 1536, 256, torch.float32, False, True),     # fp32 y
    (257, 72, 128, torch.float32, False, False),
])
def test_linear_bf16_x_resident_matches_tiled(M, N, K, xdt, ybf16, bias, monkeypatch):
    """The x-resident bf16 kernel (K <= 256, a multiple of 64) runs every
    output through the same MFMA sequence as the 128 x BN tiled kernel:
    its bytes equal the tiled kernel's (CIGN_GEMM_XRES=0), for bf16 and fp32
    y, partial tiles and rows, with and without a bias. Both are pinned to
    the oracle by test_linear_forward_backward."""
    from cign_amd import _lib

    print(f"x-resident M={M} N={N} K={K} x={xdt} ybf16={ybf16} bias={bias}", flush=True)
    lib = _lib.load_library()
    rng = np.random.default_rng(M + N + K)
    x = _t(rng.standard_normal((M, K)), xdt)
    w = _t(rng.standard_normal((N, K)) / np.sqrt(K))
    b = _t(rng.standard_normal(N) * 0.1) if bias else None
    outs = []
    for mode in ("0", "1"):
        monkeypatch.setenv("CIGN_GEMM_XRES", mode)
        y = torch.full((M, N), float("nan"), dtype=torch.bfloat16 if ybf16 else torch.float32, device="cuda")
        if ybf16:
            lib.call("cign_linear_fwd_bf16y", _lib.stream_ptr(), M, N, K, _lib.dtype_code(x), x.data_ptr(),
                     w.data_ptr(), _lib.ptr(b), y.data_ptr())
        else:
            lib.call("cign_linear_fwd", _lib.stream_ptr(), M, N, K, _lib.dtype_code(x), 1, x.data_ptr(), w.data_ptr(),
                     _lib.ptr(b), y.data_ptr())
        torch.cuda.synchronize()
        outs.append(y)
    it = torch.int16 if ybf16 else torch.int32
    assert not torch.isnan(outs[1].float()).any(), "x-resident kernel left outputs unwritten"
    assert torch.equal(outs[0].view(it), outs[1].view(it))
    if M <= 1000:  # and the oracle, with autocast's rounding points
        ref = O.linear_forward(_np(x), _np(w), None if b is None else _np(b), amp=True)
        assert_close(_np(outs[1]), ref, name="y", rtol=2.0 ** -7, atol=1e-6)
