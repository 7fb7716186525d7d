"""Fused block ops on gfx950: a drop-in for the reference module
fused_block_ops.py, with the same public names, seeds, masks and errors.

The three fused ops are:
- dropout + LayerNorm;
- add + LayerNorm;
- dropout-gamma-residual.

Each has a backward, for rows of 1 <= D <= 256 in float32. The extension object has
the reference binding's six entry points (fused_block_ops.py:15 inline
binding; fused_block_ops_ext/fused_block_ops.cpp:39-98), over the C-ABI
entry points cign_dropout_ln_*, cign_add_ln_* and cign_gamma_residual_*.
Dropout keep bits are splitmix64(seed ^ (idx * 0xD2B74407B1CE6E93)) >> 11 as a
53-bit uniform, keep = u >= p, idx = n*D + c. The reference's per-call seed
(_next_seed, fused_block_ops.py:46-50) is kept bit for bit.
"""
from __future__ import annotations

import itertools

import torch

from . import _lib
from ._lib import check, check_input

_EXT = None
_EXT_ERROR = None
_CALL_COUNTER = itertools.count()


def _extension_name() -> str:
    return "cign_amd_fused_block_ops_hip"


def _check_2d(x, name):
    """check_2d of the binding: [N,D] float32 with 1<=D<=256."""
    check_input(x, name)
    check(x.dim() == 2, f"{name} must be [N,D]")
    check(1 <= x.size(1) <= 256, f"{name} requires 1<=D<=256")
    return int(x.size(1))


def _check_param(x, name, D):
    check_input(x, name)
    check(x.dim() == 1 and x.numel() == D, f"{name} must have D elements")


def _check_mask(m, shape):
    check(isinstance(m, torch.Tensor) and m.is_cuda, "mask must be CUDA")
    check(m.is_contiguous(), "mask must be contiguous")
    check(m.dtype == torch.uint8, "mask must be uint8")
    check(m.shape == shape, "mask shape mismatch")


class _BlockOpsExt:
    """Extension object with the reference binding's six entry points."""

    @staticmethod
    def dropout_layernorm_forward(x, w, b, p, eps, seed):
        D = _check_2d(x, "x")
        _check_param(w, "weight", D)
        _check_param(b, "bias", D)
        check(0.0 <= p < 1.0, "dropout_p must be in [0,1)")
        lib = _lib.load_library()
        N = x.size(0)
        y = torch.empty_like(x)
        mean = torch.empty((N,), dtype=torch.float32, device=x.device)
        rstd = torch.empty_like(mean)
        mask = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
        lib.call("cign_dropout_ln_fwd", _lib.stream_ptr(x.device), N, D, x.data_ptr(), w.data_ptr(), b.data_ptr(),
                 float(p), float(eps), int(seed) & ((1 << 64) - 1), y.data_ptr(), mean.data_ptr(), rstd.data_ptr(),
                 mask.data_ptr())
        return [y, mean, rstd, mask]

    @staticmethod
    def dropout_layernorm_backward(gy, x, w, mean, rstd, mask, p):
        D = _check_2d(x, "x")
        check(_check_2d(gy, "grad_y") == D, "grad_y D mismatch")
        _check_param(w, "weight", D)
        check_input(mean, "mean")
        check_input(rstd, "rstd")
        _check_mask(mask, x.shape)
        check(gy.shape == x.shape, "grad_y/x shape mismatch")
        check(mean.dim() == 1 and mean.size(0) == x.size(0), "mean must be [N]")
        check(rstd.shape == mean.shape, "rstd must be [N]")
        lib = _lib.load_library()
        N = x.size(0)
        dx = torch.empty_like(x)
        gw = torch.empty((D,), dtype=torch.float32, device=x.device)
        gb = torch.empty_like(gw)
        ws_bytes = int(lib.cign_colsum_workspace_bytes(N, D, 2))
        ws = _lib.workspace(ws_bytes, x.device)
        lib.call("cign_dropout_ln_bwd", _lib.stream_ptr(x.device), N, D, gy.data_ptr(), x.data_ptr(), w.data_ptr(),
                 mean.data_ptr(), rstd.data_ptr(), mask.data_ptr(), float(p), dx.data_ptr(), gw.data_ptr(),
                 gb.data_ptr(), ws.data_ptr(), ws_bytes)
        return [dx, gw, gb]

    @staticmethod
    def add_layernorm_forward(a, b, w, bias, eps):
        D = _check_2d(a, "a")
        check(_check_2d(b, "b") == D, "b D mismatch")
        _check_param(w, "weight", D)
        _check_param(bias, "bias", D)
        check(a.shape == b.shape, "a/b shape mismatch")
        lib = _lib.load_library()
        N = a.size(0)
        y = torch.empty_like(a)
        mean = torch.empty((N,), dtype=torch.float32, device=a.device)
        rstd = torch.empty_like(mean)
        lib.call("cign_add_ln_fwd", _lib.stream_ptr(a.device), N, D, a.data_ptr(), b.data_ptr(), w.data_ptr(),
                 bias.data_ptr(), float(eps), y.data_ptr(), mean.data_ptr(), rstd.data_ptr())
        return [y, mean, rstd]

    @staticmethod
    def add_layernorm_backward(gy, a, b, w, mean, rstd):
        D = _check_2d(a, "a")
        check(_check_2d(b, "b") == D and _check_2d(gy, "grad_y") == D, "D mismatch")
        _check_param(w, "weight", D)
        check_input(mean, "mean")
        check_input(rstd, "rstd")
        check(a.shape == b.shape and a.shape == gy.shape, "shape mismatch")
        check(mean.dim() == 1 and mean.size(0) == a.size(0), "mean must be [N]")
        check(rstd.shape == mean.shape, "rstd must be [N]")
        lib = _lib.load_library()
        N = a.size(0)
        dz = torch.empty_like(a)
        gw = torch.empty((D,), dtype=torch.float32, device=a.device)
        gb = torch.empty_like(gw)
        ws_bytes = int(lib.cign_colsum_workspace_bytes(N, D, 2))
        ws = _lib.workspace(ws_bytes, a.device)
        lib.call("cign_add_ln_bwd", _lib.stream_ptr(a.device), N, D, gy.data_ptr(), a.data_ptr(), b.data_ptr(),
                 w.data_ptr(), mean.data_ptr(), rstd.data_ptr(), dz.data_ptr(), gw.data_ptr(), gb.data_ptr(),
                 ws.data_ptr(), ws_bytes)
        return [dz, gw, gb]

    @staticmethod
    def dropout_gamma_residual_forward(h, g, gamma, p, seed):
        D = _check_2d(h, "h")
        check(_check_2d(g, "g") == D, "g D mismatch")
        _check_param(gamma, "gamma", D)
        check(h.shape == g.shape, "h/g shape mismatch")
        check(0.0 <= p < 1.0, "dropout_p must be in [0,1)")
        lib = _lib.load_library()
        N = h.size(0)
        y = torch.empty_like(h)
        mask = torch.empty(h.shape, dtype=torch.uint8, device=h.device)
        lib.call("cign_gamma_residual_fwd", _lib.stream_ptr(h.device), N, D, h.data_ptr(), g.data_ptr(),
                 gamma.data_ptr(), float(p), int(seed) & ((1 << 64) - 1), y.data_ptr(), mask.data_ptr())
        return [y, mask]

    @staticmethod
    def dropout_gamma_residual_backward(gy, g, gamma, mask, p):
        D = _check_2d(g, "g")
        check(_check_2d(gy, "grad_y") == D, "grad_y D mismatch")
        _check_param(gamma, "gamma", D)
        _check_mask(mask, g.shape)
        check(gy.shape == g.shape, "shape mismatch")
        lib = _lib.load_library()
        N = g.size(0)
        gg = torch.empty_like(g)
        ggamma = torch.empty((D,), dtype=torch.float32, device=g.device)
        ws_bytes = int(lib.cign_colsum_workspace_bytes(N, D, 1))
        ws = _lib.workspace(ws_bytes, g.device)
        lib.call("cign_gamma_residual_bwd", _lib.stream_ptr(g.device), N, D, gy.data_ptr(), g.data_ptr(),
                 gamma.data_ptr(), mask.data_ptr(), float(p), gg.data_ptr(), ggamma.data_ptr(), ws.data_ptr(),
                 ws_bytes)
        return [gg, ggamma]


def ensure_fused_block_ops_loaded(verbose: bool = False):
    """Loads libcign_amd once (fused_block_ops.py:35-45 semantics)."""
    global _EXT, _EXT_ERROR
    if _EXT is not None:
        return _EXT
    if _EXT_ERROR is not None:
        raise RuntimeError("fused block-op extension previously failed to load") from _EXT_ERROR
    if not torch.cuda.is_available():
        raise RuntimeError("fused block ops require a HIP GPU")
    try:
        _lib.load_library()
        _EXT = _BlockOpsExt()
        return _EXT
    except Exception as exc:
        _EXT_ERROR = exc
        raise


def _next_seed(tag: int, dropout_p: float) -> int:
    """Per-call dropout seed, fused_block_ops.py:46-50: 0 when p <= 0 (the
    call counter does not advance), else (initial_seed + golden * call +
    0xD2B74407B1CE6E93 * tag) mod 2^63 with call = 1, 2, ..."""
    if float(dropout_p) <= 0.0:
        return 0
    base = int(torch.initial_seed()) & ((1 << 63) - 1)
    call = next(_CALL_COUNTER) + 1
    return (base + 0x9E3779B97F4A7C15 * call + 0xD2B74407B1CE6E93 * int(tag)) & ((1 << 63) - 1)


class _DropoutLayerNormFn(torch.autograd.Function):
    """fused_block_ops.py:52-70."""

    @staticmethod
    def forward(ctx, x, weight, bias, dropout_p, eps, seed):
        ext = ensure_fused_block_ops_loaded(False)
        y, mean, rstd, mask = ext.dropout_layernorm_forward(x.contiguous(), weight.contiguous(), bias.contiguous(),
                                                            float(dropout_p), float(eps), int(seed))
        ctx.save_for_backward(x, weight, mean, rstd, mask)
        ctx.dropout_p = float(dropout_p)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        ext = ensure_fused_block_ops_loaded(False)
        x, weight, mean, rstd, mask = ctx.saved_tensors
        gx, gw, gb = ext.dropout_layernorm_backward(grad_y.to(dtype=torch.float32).contiguous(), x.contiguous(),
                                                    weight.contiguous(), mean, rstd, mask, ctx.dropout_p)
        return gx, gw, gb, None, None, None


class _AddLayerNormFn(torch.autograd.Function):
    """fused_block_ops.py:72-88."""

    @staticmethod
    def forward(ctx, a, b, weight, bias, eps):
        ext = ensure_fused_block_ops_loaded(False)
        y, mean, rstd = ext.add_layernorm_forward(a.contiguous(), b.contiguous(), weight.contiguous(),
                                                  bias.contiguous(), float(eps))
        ctx.save_for_backward(a, b, weight, mean, rstd)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        ext = ensure_fused_block_ops_loaded(False)
        a, b, weight, mean, rstd = ctx.saved_tensors
        gz, gw, gb = ext.add_layernorm_backward(grad_y.to(dtype=torch.float32).contiguous(), a.contiguous(),
                                                b.contiguous(), weight.contiguous(), mean, rstd)
        return gz, gz, gw, gb, None


class _AddLayerNormCatFn(torch.autograd.Function):
    """y = LayerNorm(a + b) and cat = [b | y] from one kernel
    (cign_add_ln_cat_fwd): the block's C_norm and HC_norm (model_cign.py:
    781-792). The backward takes both outputs' gradients in one kernel
    (cign_add_ln_cat_bwd), so neither the concatenation's gradient slices nor
    the sums of y's two uses and of b's two uses pass through separate
    additions."""

    @staticmethod
    def forward(ctx, a, b, weight, bias, eps):
        for t, n in ((a, "a"), (b, "b"), (weight, "weight"), (bias, "bias")):
            check_input(t, n)
        N, D = a.shape
        lib = _lib.load_library()
        y = torch.empty_like(a)
        cat = torch.empty((N, 2 * D), dtype=torch.float32, device=a.device)
        mean = torch.empty((N,), dtype=torch.float32, device=a.device)
        rstd = torch.empty_like(mean)
        lib.call("cign_add_ln_cat_fwd", _lib.stream_ptr(a.device), N, D, a.data_ptr(), b.data_ptr(),
                 weight.data_ptr(), bias.data_ptr(), float(eps), y.data_ptr(), cat.data_ptr(), mean.data_ptr(),
                 rstd.data_ptr())
        ctx.save_for_backward(a, b, weight, mean, rstd)
        return y, cat

    @staticmethod
    def backward(ctx, grad_y, grad_cat):
        a, b, weight, mean, rstd = ctx.saved_tensors
        N, D = a.shape
        lib = _lib.load_library()
        gy = grad_y.to(dtype=torch.float32).contiguous()
        gc = grad_cat.to(dtype=torch.float32).contiguous()
        ga, gbb = torch.empty_like(a), torch.empty_like(b)
        gw = torch.empty((D,), dtype=torch.float32, device=a.device)
        gbias = torch.empty_like(gw)
        ws_bytes = int(lib.cign_colsum_workspace_bytes(N, D, 2))
        ws = _lib.workspace(ws_bytes, a.device)
        lib.call("cign_add_ln_cat_bwd", _lib.stream_ptr(a.device), N, D, gy.data_ptr(), gc.data_ptr(), a.data_ptr(),
                 b.data_ptr(), weight.data_ptr(), mean.data_ptr(), rstd.data_ptr(), ga.data_ptr(), gbb.data_ptr(),
                 gw.data_ptr(), gbias.data_ptr(), ws.data_ptr(), ws_bytes)
        return ga, gbb, gw, gbias, None


class _DropoutGammaResidualFn(torch.autograd.Function):
    """fused_block_ops.py:90-106."""

    @staticmethod
    def forward(ctx, h, g, gamma, dropout_p, seed):
        ext = ensure_fused_block_ops_loaded(False)
        y, mask = ext.dropout_gamma_residual_forward(h.contiguous(), g.contiguous(), gamma.contiguous(),
                                                     float(dropout_p), int(seed))
        ctx.save_for_backward(g, gamma, mask)
        ctx.dropout_p = float(dropout_p)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        ext = ensure_fused_block_ops_loaded(False)
        g, gamma, mask = ctx.saved_tensors
        grad_y = grad_y.to(dtype=torch.float32).contiguous()
        gg, ggamma = ext.dropout_gamma_residual_backward(grad_y, g.contiguous(), gamma.contiguous(), mask,
                                                         ctx.dropout_p)
        return grad_y, gg, ggamma, None, None


def _check_py_2d(x, name):
    """fused_block_ops.py:108-111."""
    if x.device.type != "cuda" or x.dtype != torch.float32:
        raise TypeError(f"{name} must be CUDA float32")
    if x.dim() != 2 or not (1 <= x.size(1) <= 256):
        raise ValueError(f"{name} must be [N,D] with 1<=D<=256, got {tuple(x.shape)}")
    return int(x.size(1))


def fused_dropout_layernorm(x, weight, bias, dropout_p, eps):
    """LayerNorm(dropout(x)) (fused_block_ops.py:113-116)."""
    D = _check_py_2d(x, "x")
    if weight.numel() != D or bias.numel() != D:
        raise ValueError("LayerNorm weight/bias must match hidden dimension")
    return _DropoutLayerNormFn.apply(x, weight, bias, float(dropout_p), float(eps), _next_seed(1, dropout_p))


def fused_add_layernorm(a, b, weight, bias, eps):
    """LayerNorm(a + b) (fused_block_ops.py:118-121)."""
    D = _check_py_2d(a, "a")
    _check_py_2d(b, "b")
    if a.shape != b.shape or weight.numel() != D or bias.numel() != D:
        raise ValueError("Add+LayerNorm shapes do not match")
    return _AddLayerNormFn.apply(a, b, weight, bias, float(eps))


def fused_add_layernorm_cat(a, b, weight, bias, eps):
    """(LayerNorm(a + b), [b | LayerNorm(a + b)]): the add-LayerNorm and the
    concatenation of GraphCliffordBlock.forward (model_cign.py:781-792) in
    one kernel each way. Inputs become float32 contiguous tensors."""
    D = _check_py_2d(a, "a")
    _check_py_2d(b, "b")
    if a.shape != b.shape or weight.numel() != D or bias.numel() != D:
        raise ValueError("Add+LayerNorm shapes do not match")
    f = lambda t: t.to(dtype=torch.float32).contiguous()
    return _AddLayerNormCatFn.apply(f(a), f(b), f(weight), f(bias), float(eps))


def fused_dropout_gamma_residual(h, g, gamma, dropout_p):
    """h + gamma * dropout(g) (fused_block_ops.py:123-128)."""
    D = _check_py_2d(h, "h")
    _check_py_2d(g, "g")
    if h.shape != g.shape:
        raise ValueError("h and g must have the same shape")
    if gamma.dim() != 1 or gamma.numel() != D:
        raise ValueError(f"vector gamma must have shape [{D}]")
    return _DropoutGammaResidualFn.apply(h, g, gamma, float(dropout_p), _next_seed(2, dropout_p))
