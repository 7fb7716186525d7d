"""Fused GAT side ops on gfx950: a drop-in for the reference module
fused_gat_sideops.py, with the same public names, arguments and errors.

``ensure_fused_gat_sideops_loaded()`` returns an extension object with the
reference binding's four entry points (fused_gat_sideops_ext/
fused_gat_sideops.cpp:45-95). Each one calls the C-ABI of libcign_amd:
- ``attention_forward`` / ``attention_backward`` call cign_attn_logits_fwd / _bwd;
- ``head_silu_forward`` / ``head_silu_backward`` call cign_head_silu_fwd / _bwd.
All tensors are float32, like the reference.
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import check, check_input

_EXT = None
_EXT_ERROR = None


def _extension_name() -> str:
    return "cign_amd_fused_gat_sideops_hip"


def _validate_attention(x, att_src, att_dst):
    """fused_gat_sideops.cpp:31-43."""
    check_input(x, "x")
    check_input(att_src, "att_src")
    check_input(att_dst, "att_dst")
    check(x.dim() == 3, "x must be [N,H,C]")
    check(att_src.dim() == 3 and att_src.size(0) == 1, "att_src must be [1,H,C]")
    check(att_dst.shape == att_src.shape, "att_dst must match att_src")
    check(att_src.size(1) == x.size(1) and att_src.size(2) == x.size(2), "attention shapes do not match x")


class _SideOpsExt:
    """Extension object with the reference binding's entry points."""

    @staticmethod
    def attention_forward(x, att_src, att_dst):
        _validate_attention(x, att_src, att_dst)
        lib = _lib.load_library()
        N, H, C = x.shape
        a_src = torch.empty((N, H), dtype=torch.float32, device=x.device)
        a_dst = torch.empty((N, H), dtype=torch.float32, device=x.device)
        lib.call("cign_attn_logits_fwd", _lib.stream_ptr(x.device), N, H, C, x.data_ptr(), att_src.data_ptr(),
                 att_dst.data_ptr(), a_src.data_ptr(), a_dst.data_ptr())
        return [a_src, a_dst]

    @staticmethod
    def attention_backward(grad_src, grad_dst, x, att_src, att_dst):
        _validate_attention(x, att_src, att_dst)
        check_input(grad_src, "grad_src")
        check_input(grad_dst, "grad_dst")
        check(grad_src.dim() == 2 and grad_src.size(0) == x.size(0) and grad_src.size(1) == x.size(1),
              "grad_src must be [N,H]")
        check(grad_dst.shape == grad_src.shape, "grad_dst must match grad_src")
        lib = _lib.load_library()
        N, H, C = x.shape
        gx = torch.empty_like(x)
        g_src = torch.empty_like(att_src)
        g_dst = torch.empty_like(att_dst)
        ws_bytes = int(lib.cign_colsum_workspace_bytes(N, H * C, 2))
        ws = _lib.workspace(ws_bytes, x.device)
        lib.call("cign_attn_logits_bwd", _lib.stream_ptr(x.device), N, H, C, grad_src.data_ptr(),
                 grad_dst.data_ptr(), x.data_ptr(), att_src.data_ptr(), att_dst.data_ptr(), gx.data_ptr(),
                 g_src.data_ptr(), g_dst.data_ptr(), ws.data_ptr(), ws_bytes)
        return [gx, g_src, g_dst]

    @staticmethod
    def head_silu_forward(out, bias):
        """fused_gat_sideops.cpp:68-76."""
        check_input(out, "out")
        check_input(bias, "bias")
        check(out.dim() == 3, "out must be [N,H,C]")
        check(bias.dim() == 1 and bias.size(0) == out.size(2), "bias must be [C]")
        lib = _lib.load_library()
        N, H, C = out.shape
        y = torch.empty((N, C), dtype=torch.float32, device=out.device)
        pre = torch.empty_like(y)
        lib.call("cign_head_silu_fwd", _lib.stream_ptr(out.device), N, H, C, out.data_ptr(), bias.data_ptr(),
                 y.data_ptr(), pre.data_ptr())
        return [y, pre]

    @staticmethod
    def head_silu_backward(grad_y, pre, heads):
        """fused_gat_sideops.cpp:78-88."""
        check_input(grad_y, "grad_y")
        check_input(pre, "pre")
        check(grad_y.dim() == 2, "grad_y must be [N,C]")
        check(pre.shape == grad_y.shape, "pre must match grad_y")
        check(int(heads) > 0, "heads must be positive")
        lib = _lib.load_library()
        N, C = grad_y.shape
        H = int(heads)
        g_out = torch.empty((N, H, C), dtype=torch.float32, device=grad_y.device)
        g_bias = torch.empty((C,), dtype=torch.float32, device=grad_y.device)
        ws_bytes = int(lib.cign_colsum_workspace_bytes(N, C, 1))
        ws = _lib.workspace(ws_bytes, grad_y.device)
        lib.call("cign_head_silu_bwd", _lib.stream_ptr(grad_y.device), N, H, C, grad_y.data_ptr(), pre.data_ptr(),
                 g_out.data_ptr(), g_bias.data_ptr(), ws.data_ptr(), ws_bytes)
        return [g_out, g_bias]


def ensure_fused_gat_sideops_loaded(verbose: bool = False):
    """Loads libcign_amd once (fused_gat_sideops.py:17-47 semantics: a
    missing device raises RuntimeError; a failed load is cached and re-raised)."""
    global _EXT, _EXT_ERROR
    if _EXT is not None:
        return _EXT
    if _EXT_ERROR is not None:
        raise RuntimeError("fused GAT side-op extension previously failed to load") from _EXT_ERROR
    if not torch.cuda.is_available():
        raise RuntimeError("fused GAT side ops require a HIP GPU")
    try:
        _lib.load_library()
        _EXT = _SideOpsExt()
        return _EXT
    except Exception as exc:
        _EXT_ERROR = exc
        raise


class _AttentionLogitsFn(torch.autograd.Function):
    """fused_gat_sideops.py:50-70."""

    @staticmethod
    def forward(ctx, x, att_src, att_dst):
        ext = ensure_fused_gat_sideops_loaded(False)
        x = x.contiguous()
        att_src = att_src.contiguous()
        att_dst = att_dst.contiguous()
        alpha_src, alpha_dst = ext.attention_forward(x, att_src, att_dst)
        ctx.save_for_backward(x, att_src, att_dst)
        return alpha_src, alpha_dst

    @staticmethod
    def backward(ctx, grad_src, grad_dst):
        ext = ensure_fused_gat_sideops_loaded(False)
        x, att_src, att_dst = ctx.saved_tensors
        if grad_src is None:
            grad_src = torch.zeros(x.shape[:2], dtype=x.dtype, device=x.device)
        if grad_dst is None:
            grad_dst = torch.zeros(x.shape[:2], dtype=x.dtype, device=x.device)
        grad_x, grad_att_src, grad_att_dst = ext.attention_backward(
            grad_src.contiguous(), grad_dst.contiguous(), x, att_src, att_dst)
        return grad_x, grad_att_src, grad_att_dst


class _HeadMeanBiasSiLUFn(torch.autograd.Function):
    """fused_gat_sideops.py:73-91."""

    @staticmethod
    def forward(ctx, out, bias):
        ext = ensure_fused_gat_sideops_loaded(False)
        y, pre = ext.head_silu_forward(out.contiguous(), bias.contiguous())
        ctx.save_for_backward(pre)
        ctx.heads = int(out.size(1))
        return y

    @staticmethod
    def backward(ctx, grad_y):
        ext = ensure_fused_gat_sideops_loaded(False)
        (pre,) = ctx.saved_tensors
        grad_out, grad_bias = ext.head_silu_backward(grad_y.contiguous(), pre, ctx.heads)
        return grad_out, grad_bias


def fused_attention_logits(x: torch.Tensor, att_src: torch.Tensor, att_dst: torch.Tensor):
    """(alpha_src, alpha_dst) = (<x, att_src>, <x, att_dst>) over channels
    (fused_gat_sideops.py:94-97)."""
    if x.dtype != torch.float32 or x.device.type != "cuda":
        raise TypeError("fused attention logits require CUDA float32 tensors")
    return _AttentionLogitsFn.apply(x, att_src, att_dst)


def fused_head_mean_bias_silu(out: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """SiLU(mean_h out + bias) (fused_gat_sideops.py:100-105)."""
    if bias is None:
        raise ValueError("fused head reduction requires GAT bias=True")
    if out.dtype != torch.float32 or out.device.type != "cuda":
        raise TypeError("fused head reduction requires CUDA float32 tensors")
    return _HeadMeanBiasSiLUFn.apply(out, bias)
