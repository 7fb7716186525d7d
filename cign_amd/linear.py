"""Dense projections of the Clifford block on gfx950 MFMA (rows a10 and a15 of
the hot path), with the elementwise work that follows them fused into the
GEMM epilogue. Drop-in for the reference's ``_local_amp_linear``
(generic_engine/model_cign.py:86-103) and for the two compositions that
follow its calls in the block:

* ``mfma_linear(linear, x, amp, amp_dtype)``: ``y = x W^T + b`` returned as
  float32. With ``amp`` (the reference's local bf16 autocast) x, W and b are
  rounded to bf16 in registers, the products run on bf16 MFMA with fp32
  accumulation and the output is rounded to bf16 (autocast's output dtype)
  before it is returned as float32; without it the GEMM is exact fp32 MFMA.
* ``linear_attention_logits(x, weight, att_src, att_dst, heads, amp)``: the
  GAT ``lin`` projection (no bias) and the attention logits
  alpha_src[n,h] = <x_proj[n,h,:], att_src[h,:]>, alpha_dst likewise
  (model_cign.py:546-553 followed by fused_gat_sideops.py:94-97), in one
  kernel when the channel count is 16, 32, 64 or 128.
* ``linear_gamma_residual(h, x, linear, gamma, dropout_p, amp)``:
  ``h + gamma * dropout(x W^T + b)`` (model_cign.py:927-933 with
  fused_block_ops.fused_dropout_gamma_residual), the dropout mask drawn with
  the reference's block-op seed stream.

Backward (all three): grad_x = grad_y W on the forward's MFMA kernel against
a transposed W, grad_W = grad_y^T x on a split-M MFMA kernel, grad_b =
sum_n grad_y; with ``amp`` every product reads
bf16-rounded operands with fp32 accumulation and grad_x, grad_W and grad_b
are rounded to bf16 (grad_b the sum of the bf16-rounded grad_y), as the bf16
Linear's backward under autocast returns them; grad_W and grad_b are
deterministic (chunk partials summed in order). The
logits and gamma-residual parts run on their existing kernels
(cign_attn_logits_bwd, cign_gamma_residual_bwd).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib


def _math_code(amp: bool, amp_dtype) -> int:
    if not amp:
        return 0
    if amp_dtype != torch.bfloat16:
        raise ValueError(f"MFMA linear supports bf16 autocast only, got {amp_dtype}")
    return 1


def _prep_x(x: torch.Tensor) -> torch.Tensor:
    if not x.is_cuda:
        raise RuntimeError("MFMA linear requires a HIP tensor")
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"MFMA linear input must be float32 or bfloat16, got {x.dtype}")
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    return x


def _linear_bwd(grad_y: torch.Tensor, x2: torch.Tensor, weight: torch.Tensor, has_bias: bool, math: int,
                need_x: bool, need_w: bool):
    """(grad_x, grad_w, grad_b) of y = x W^T + b for x2 [M, K] float32."""
    lib = _lib.load_library()
    M, K = x2.shape
    N = weight.size(0)
    dev = x2.device
    gy = grad_y.reshape(M, N).to(torch.float32).contiguous()
    xf = x2 if x2.dtype == torch.float32 else x2.float()
    grad_x = torch.empty((M, K), dtype=torch.float32, device=dev) if need_x else None
    grad_w = torch.empty((N, K), dtype=torch.float32, device=dev)
    grad_b = torch.empty((N,), dtype=torch.float32, device=dev) if has_bias else None
    ws_bytes = int(lib.cign_linear_bwd_workspace_bytes(M, N, K, 1 if has_bias else 0))
    ws = _lib.workspace(ws_bytes, dev)
    lib.call("cign_linear_bwd", _lib.stream_ptr(dev), M, N, K, math, gy.data_ptr(), xf.data_ptr(),
             weight.data_ptr(), _lib.ptr(grad_x), grad_w.data_ptr(), _lib.ptr(grad_b), ws.data_ptr(), ws_bytes)
    return grad_x, (grad_w if need_w else None), grad_b


class _LinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, math):
        lib = _lib.load_library()
        shape = x.shape
        x2 = _prep_x(x.reshape(-1, shape[-1]))
        w = weight.detach().float().contiguous()
        M, K = x2.shape
        N = w.size(0)
        y = torch.empty((M, N), dtype=torch.float32, device=x.device)
        lib.call("cign_linear_fwd", _lib.stream_ptr(x.device), M, N, K, _lib.dtype_code(x2), math, x2.data_ptr(),
                 w.data_ptr(), _lib.ptr(None if bias is None else bias.detach().float().contiguous()), y.data_ptr())
        ctx.save_for_backward(x2, w)
        ctx.has_bias = bias is not None
        ctx.math = math
        ctx.in_shape = shape
        ctx.x_dtype = x.dtype
        return y.reshape(*shape[:-1], N)

    @staticmethod
    def backward(ctx, grad_y):
        x2, w = ctx.saved_tensors
        gx, gw, gb = _linear_bwd(grad_y, x2, w, ctx.has_bias, ctx.math, ctx.needs_input_grad[0],
                                 ctx.needs_input_grad[1])
        if gx is not None:
            gx = gx.reshape(ctx.in_shape).to(ctx.x_dtype)
        return gx, gw, gb, None


def mfma_linear(linear: nn.Linear, x: torch.Tensor, enabled: bool = False,
                amp_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """_local_amp_linear (model_cign.py:86-103) on MFMA: float32 result."""
    return _LinearFn.apply(x, linear.weight, linear.bias, _math_code(bool(enabled), amp_dtype))


class _LinearLogitsFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, att_src, att_dst, heads, math):
        lib = _lib.load_library()
        x2 = _prep_x(x)
        w = weight.detach().float().contiguous()
        M, K = x2.shape
        H = int(heads)
        C = w.size(0) // H
        dev = x.device
        xp = torch.empty((M, H, C), dtype=torch.float32, device=dev)
        a_src = torch.empty((M, H), dtype=torch.float32, device=dev)
        a_dst = torch.empty((M, H), dtype=torch.float32, device=dev)
        s, d = att_src.detach().float().contiguous(), att_dst.detach().float().contiguous()
        lib.call("cign_linear_logits_fwd", _lib.stream_ptr(dev), M, H, C, K, _lib.dtype_code(x2), math,
                 x2.data_ptr(), w.data_ptr(), s.data_ptr(), d.data_ptr(), xp.data_ptr(), a_src.data_ptr(),
                 a_dst.data_ptr())
        ctx.save_for_backward(x2, w, xp, s, d)
        ctx.math = math
        ctx.x_dtype = x.dtype
        return xp, a_src, a_dst

    @staticmethod
    def backward(ctx, grad_xp, grad_src, grad_dst):
        x2, w, xp, s, d = ctx.saved_tensors
        lib = _lib.load_library()
        M, H, C = xp.shape
        dev = xp.device
        grad_src = torch.zeros((M, H), device=dev) if grad_src is None else grad_src.float().contiguous()
        grad_dst = torch.zeros((M, H), device=dev) if grad_dst is None else grad_dst.float().contiguous()
        gx_log = torch.empty_like(xp)
        g_s = torch.empty_like(s)
        g_d = torch.empty_like(d)
        ws_bytes = int(lib.cign_colsum_workspace_bytes(M, H * C, 2))
        ws = _lib.workspace(ws_bytes, dev)
        lib.call("cign_attn_logits_bwd", _lib.stream_ptr(dev), M, H, C, grad_src.data_ptr(), grad_dst.data_ptr(),
                 xp.data_ptr(), s.data_ptr(), d.data_ptr(), gx_log.data_ptr(), g_s.data_ptr(), g_d.data_ptr(),
                 ws.data_ptr(), ws_bytes)
        g_total = gx_log if grad_xp is None else gx_log.add_(grad_xp.float())
        gx, gw, _ = _linear_bwd(g_total, x2, w, False, ctx.math, ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        if gx is not None:
            gx = gx.to(ctx.x_dtype)
        return gx, gw, g_s, g_d, None, None


def linear_attention_logits(x: torch.Tensor, weight: torch.Tensor, att_src: torch.Tensor, att_dst: torch.Tensor,
                            heads: int, enabled: bool = False, amp_dtype: torch.dtype = torch.bfloat16):
    """x_proj = lin(x).view(-1, H, C) and its attention logits (alpha_src,
    alpha_dst) (model_cign.py:546-553, fused_gat_sideops.py:94-97). Channels
    16/32/64/128 run as one fused MFMA kernel; other widths as the MFMA
    projection followed by the logits kernel."""
    if x.dim() != 2:
        raise ValueError(f"expected [N, in] node features, got {tuple(x.shape)}")
    H = int(heads)
    C = weight.size(0) // H
    math = _math_code(bool(enabled), amp_dtype)
    if C in (16, 32, 64, 128):
        return _LinearLogitsFn.apply(x, weight, att_src, att_dst, H, math)
    from .fused_gat_sideops import fused_attention_logits

    xp = _LinearFn.apply(x, weight, None, math).view(-1, H, C)
    a_src, a_dst = fused_attention_logits(xp, att_src, att_dst)
    return xp, a_src, a_dst


class _LinearGammaFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, h, x, weight, bias, gamma, dropout_p, seed, math):
        lib = _lib.load_library()
        x2 = _prep_x(x)
        w = weight.detach().float().contiguous()
        M, K = x2.shape
        N = w.size(0)
        dev = x.device
        hh = h.detach().float().contiguous()
        gm = gamma.detach().float().contiguous()
        g_lin = torch.empty((M, N), dtype=torch.float32, device=dev)
        out = torch.empty((M, N), dtype=torch.float32, device=dev)
        mask = torch.empty((M, N), dtype=torch.uint8, device=dev)
        lib.call("cign_linear_gamma_fwd", _lib.stream_ptr(dev), M, N, K, _lib.dtype_code(x2), math, x2.data_ptr(),
                 w.data_ptr(), _lib.ptr(None if bias is None else bias.detach().float().contiguous()),
                 hh.data_ptr(), gm.data_ptr(), float(dropout_p), int(seed) & ((1 << 64) - 1), g_lin.data_ptr(),
                 out.data_ptr(), mask.data_ptr())
        ctx.save_for_backward(x2, w, g_lin, gm, mask)
        ctx.has_bias = bias is not None
        ctx.p = float(dropout_p)
        ctx.math = math
        ctx.x_dtype = x.dtype
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x2, w, g_lin, gm, mask = ctx.saved_tensors
        lib = _lib.load_library()
        M, N = g_lin.shape
        dev = g_lin.device
        go = grad_out.float().contiguous()
        grad_g = torch.empty_like(g_lin)
        grad_gamma = torch.empty((N,), dtype=torch.float32, device=dev)
        ws_bytes = int(lib.cign_colsum_workspace_bytes(M, N, 1))
        ws = _lib.workspace(ws_bytes, dev)
        lib.call("cign_gamma_residual_bwd", _lib.stream_ptr(dev), M, N, go.data_ptr(), g_lin.data_ptr(),
                 gm.data_ptr(), mask.data_ptr(), ctx.p, grad_g.data_ptr(), grad_gamma.data_ptr(), ws.data_ptr(),
                 ws_bytes)
        gx, gw, gb = _linear_bwd(grad_g, x2, w, ctx.has_bias, ctx.math, ctx.needs_input_grad[1],
                                 ctx.needs_input_grad[2])
        if gx is not None:
            gx = gx.to(ctx.x_dtype)
        return go, gx, gw, gb, grad_gamma, None, None, None


def linear_gamma_residual(h: torch.Tensor, x: torch.Tensor, linear: nn.Linear, gamma: torch.Tensor,
                          dropout_p: float, enabled: bool = False, amp_dtype: torch.dtype = torch.bfloat16,
                          seed: int | None = None) -> torch.Tensor:
    """h + gamma * dropout(linear(x)) (model_cign.py:927-933): the projection,
    its bias, the dropout and the gamma residual in one MFMA kernel. The seed
    follows the reference's block-op stream (fused_block_ops.py:46-50) unless
    given."""
    if seed is None:
        from .fused_block_ops import _next_seed

        seed = _next_seed(2, dropout_p)
    if h.shape[-1] != linear.out_features or gamma.numel() != linear.out_features:
        raise ValueError("h, gamma and the projection output must share the last dimension")
    return _LinearGammaFn.apply(h, x, linear.weight, linear.bias, gamma, float(dropout_p), int(seed),
                                _math_code(bool(enabled), amp_dtype))
