"""The context GAT's projection, attention logits and collapsed GAT under
selective bf16 AMP as one autograd function, with x_proj held in bf16.

In the reference the GAT ``lin`` runs under a local bf16 autocast and
returns float32 (``_local_amp_linear``, generic_engine/model_cign.py:86-103),
so x_proj = lin(x).float() holds bf16 values; the attention logits
(fused_gat_sideops.py:94-97) and the collapsed GAT (collapsed_gat.py:164-225)
then read it as float32 (model_cign.py:546-566). Here the projection writes
those values as bf16 (half the bytes) and every consumer reads them as bf16
with float32 math, so the forward computes exactly what the float32 x_proj
gives. The backward keeps the reference's rounding points: the collapsed
GAT's gradient of x_proj is float32, the logits' term is added to it in
float32 (what autograd's sum of the two consumers' gradients does), and the
projection's backward rounds that sum to bf16 like autocast's backward. It
is one function because autograd would round each consumer's gradient to
the dtype of a bf16 x_proj before summing them.
"""
from __future__ import annotations

import torch

from . import _lib
from .collapsed_gat import _check, bf16_f32_supported, ensure_collapsed_gat_loaded, next_seed
from .linear import _linear_bwd, _prep_x
from .schedule import gat_schedule

_MATH_BF16 = 1
_FUSED_LOGITS_C = (16, 32, 64, 128)


def supported(heads: int, channels: int, amp_dtype) -> bool:
    """Whether the bf16-held x_proj path covers this GAT (bf16 autocast, a
    feature-layout shape of the library)."""
    return amp_dtype == torch.bfloat16 and bf16_f32_supported(heads, channels)


class _AmpLinGatFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, att_src, att_dst, bias, rowptr, col, colptr, row, perm, negative_slope, attn_drop,
                seed, heads):
        lib = _lib.load_library()
        x2 = _prep_x(x)
        w = weight.detach().float().contiguous()
        M, K = x2.shape
        H = int(heads)
        C = w.size(0) // H
        dev = x2.device
        st = _lib.stream_ptr(dev)
        xp = torch.empty((M, H, C), dtype=torch.bfloat16, device=dev)
        a_src = torch.empty((M, H), dtype=torch.float32, device=dev)
        a_dst = torch.empty((M, H), dtype=torch.float32, device=dev)
        s = att_src.detach().float().contiguous()
        d = att_dst.detach().float().contiguous()
        if C in _FUSED_LOGITS_C:
            lib.call("cign_linear_logits_fwd_bf16y", st, M, H, C, K, _lib.dtype_code(x2), x2.data_ptr(),
                     w.data_ptr(), s.data_ptr(), d.data_ptr(), xp.data_ptr(), a_src.data_ptr(), a_dst.data_ptr())
        else:
            lib.call("cign_linear_fwd_bf16y", st, M, H * C, K, _lib.dtype_code(x2), x2.data_ptr(), w.data_ptr(),
                     None, xp.data_ptr())
            lib.call("cign_attn_logits_fwd_bf16", st, M, H, C, xp.data_ptr(), s.data_ptr(), d.data_ptr(),
                     a_src.data_ptr(), a_dst.data_ptr())
        rowptr, col, colptr, row, perm = (t.contiguous() for t in (rowptr, col, colptr, row, perm))
        bias_c = bias.detach().float().contiguous()
        # the backward's schedules, built now so the backward never synchronises
        gat_schedule(rowptr, 1, 2, H, C)
        gat_schedule(colptr, 1, 2, H, C)
        ext = ensure_collapsed_gat_loaded(False)
        (y, pre, edge_max, edge_sum, edge_mask), agg = ext.forward_agg(
            a_dst, a_src, rowptr, col, float(negative_slope), xp, bias_c, float(attn_drop), int(seed), True,
            f32_out=True)
        ctx.save_for_backward(x2, w, s, d, xp, a_src, a_dst, col, row, perm, edge_max, edge_sum, edge_mask, pre,
                              agg)
        ctx.graph = (rowptr, colptr)
        ctx.negative_slope = float(negative_slope)
        ctx.attn_drop = float(attn_drop)
        ctx.x_dtype = x.dtype
        ctx.in_shape = x.shape
        return y

    @staticmethod
    def backward(ctx, grad_y):
        (x2, w, s, d, xp, a_src, a_dst, col, row, perm, edge_max, edge_sum, edge_mask, pre,
         agg) = ctx.saved_tensors
        rowptr, colptr = ctx.graph
        lib = _lib.load_library()
        ext = ensure_collapsed_gat_loaded(False)
        M, H, C = xp.shape
        dev = xp.device
        grad_feat, g_attn_row, g_attn_col, g_bias = ext.backward(
            ctx.negative_slope, ctx.attn_drop, rowptr, col, colptr, row, perm, edge_max, edge_sum, edge_mask, xp,
            a_dst, a_src, pre, grad_y.float().contiguous(), agg, f32_out=True)
        # d alpha_src = the GAT's attn_col gradient, d alpha_dst its attn_row
        # gradient; grad_feat += the logits' term, in place.
        g_s = torch.empty_like(s)
        g_d = torch.empty_like(d)
        ws_bytes = int(lib.cign_colsum_workspace_bytes(M, H * C, 2))
        ws = _lib.workspace(ws_bytes, dev)
        lib.call("cign_attn_logits_bwd_bf16", _lib.stream_ptr(dev), M, H, C, g_attn_col.data_ptr(),
                 g_attn_row.data_ptr(), xp.data_ptr(), s.data_ptr(), d.data_ptr(), grad_feat.data_ptr(),
                 grad_feat.data_ptr(), g_s.data_ptr(), g_d.data_ptr(), ws.data_ptr(), ws_bytes)
        gx, gw, _ = _linear_bwd(grad_feat, x2, w, False, _MATH_BF16, ctx.needs_input_grad[0],
                                ctx.needs_input_grad[1])
        if gx is not None:
            gx = gx.reshape(ctx.in_shape).to(ctx.x_dtype)
        return (gx, gw, g_s, g_d, g_bias) + (None,) * 9


def amp_lin_gat(x: torch.Tensor, weight: torch.Tensor, att_src: torch.Tensor, att_dst: torch.Tensor,
                bias: torch.Tensor, csr, csc, perm: torch.Tensor, negative_slope: float, attn_drop: float,
                heads: int) -> torch.Tensor:
    """SiLU(mean_h GAT_h(x_proj) + bias) with x_proj = bf16-autocast lin(x)
    and its attention logits (model_cign.py:546-566 under selective AMP).
    Dropout seeds as collapsed_gat_mean_bias_silu: one per call."""
    _check(bias is not None, "collapsed GAT currently requires bias=True")
    _check(x.dim() == 2, f"FusedGAT expects a 2-D node feature tensor, got {tuple(x.shape)}")
    (rowptr, col), (row, colptr) = csr, csc
    return _AmpLinGatFn.apply(x, weight, att_src, att_dst, bias, rowptr, col, colptr, row, perm,
                              float(negative_slope), float(attn_drop), next_seed(attn_drop), int(heads))
