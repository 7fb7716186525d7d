"""The context GAT's projection, attention logits and collapsed GAT as one
autograd function (CompatibleCollapsedFusedGATConv.forward,
generic_engine/model_cign.py:546-566).

The reference runs three functions: ``_local_amp_linear`` (the ``lin``,
model_cign.py:86-103), the attention logits (fused_gat_sideops.py:94-97) and
the collapsed GAT (collapsed_gat.py:164-225). x_proj feeds both the logits
and the GAT, so autograd sums their two gradients of it in a pass of its own
before the projection's backward; here the logits' backward adds the GAT's
gradient as it writes its own (cign_attn_logits_bwd_acc), which is that sum.

Under selective bf16 AMP the ``lin`` returns ``.float()`` of a bf16 result,
so x_proj holds bf16 values. Where the library runs the GAT on bf16 features
with fp32 outputs and gradients (its feature-layout shapes, dtype 2) the
projection stores those values as bf16 and every consumer reads them so
with fp32 math: the forward computes what the fp32 x_proj gives, in half the
bytes, and the backward rounds where the reference does (the two gradients
summed in fp32, then rounded to bf16 for the projection's backward, as
autocast's backward does; the logits' backward stores the sum so rounded,
and cign_linear_bwd_bf16gy reads it in half the bytes and returns grad_x and
grad_W rounded to bf16, the bf16 Linear's backward outputs). That needs one
function: autograd would round each consumer's gradient to the dtype of a
bf16 x_proj before summing.
"""
from __future__ import annotations

import torch

from . import _lib
from .collapsed_gat import _check, bf16_f32_supported, ensure_collapsed_gat_loaded, next_seed
from .linear import _linear_bwd, _math_code, _prep_x
from .schedule import gat_schedule

_FUSED_LOGITS_C = (16, 32, 64, 128)
# Largest average degree at which bf16 x_proj is gathered again in the
# backward instead of saving per-row aggregates, and the narrowest rows
# (H*C values) for which it is: a gather of 64-value rows is a chain of
# short dependent loads (the c2 lin, 4 x 16: the rows pass took 14.0 us
# gathering against 5.2 us reading aggregates).
_GATHER_MAX_DEGREE = 12
_GATHER_MIN_WIDTH = 512
# cign_linear_bwd runs outputs up to this many on VALU kernels
_SMALL_N = 16
_NARROW_N = 64  # cign_lin_logits_wgrad's widest projection


def holds_bf16(heads: int, channels: int, math: int) -> bool:
    """Whether x_proj is held in bf16: bf16 autocast (math 1) on a shape the
    library runs with bf16 features and fp32 outputs."""
    return math == 1 and bf16_f32_supported(heads, channels)


class _LinGatFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, att_src, att_dst, bias, rowptr, col, colptr, row, perm, negative_slope, attn_drop,
                seed, heads, math):
        lib = _lib.load_library()
        x2 = _prep_x(x)
        w = weight.detach().float().contiguous()
        M, K = x2.shape
        H = int(heads)
        C = w.size(0) // H
        dev = x2.device
        st = _lib.stream_ptr(dev)
        hold = holds_bf16(H, C, math)
        xp = torch.empty((M, H, C), dtype=torch.bfloat16 if hold else torch.float32, device=dev)
        a_src = torch.empty((M, H), dtype=torch.float32, device=dev)
        a_dst = torch.empty((M, H), dtype=torch.float32, device=dev)
        s = att_src.detach().float().contiguous()
        d = att_dst.detach().float().contiguous()
        xd = _lib.dtype_code(x2)
        if C in _FUSED_LOGITS_C:
            if hold:
                lib.call("cign_linear_logits_fwd_bf16y", st, M, H, C, K, xd, x2.data_ptr(), w.data_ptr(),
                         s.data_ptr(), d.data_ptr(), xp.data_ptr(), a_src.data_ptr(), a_dst.data_ptr())
            else:
                lib.call("cign_linear_logits_fwd", st, M, H, C, K, xd, math, x2.data_ptr(), w.data_ptr(),
                         s.data_ptr(), d.data_ptr(), xp.data_ptr(), a_src.data_ptr(), a_dst.data_ptr())
        else:
            if hold:
                lib.call("cign_linear_fwd_bf16y", st, M, H * C, K, xd, x2.data_ptr(), w.data_ptr(), None,
                         xp.data_ptr())
                lib.call("cign_attn_logits_fwd_bf16", st, M, H, C, xp.data_ptr(), s.data_ptr(), d.data_ptr(),
                         a_src.data_ptr(), a_dst.data_ptr())
            else:
                lib.call("cign_linear_fwd", st, M, H * C, K, xd, math, x2.data_ptr(), w.data_ptr(), None,
                         xp.data_ptr())
                lib.call("cign_attn_logits_fwd", st, M, H, C, xp.data_ptr(), s.data_ptr(), d.data_ptr(),
                         a_src.data_ptr(), a_dst.data_ptr())
        rowptr, col, colptr, row, perm = (t.contiguous() for t in (rowptr, col, colptr, row, perm))
        bias_c = bias.detach().float().contiguous()
        # the backward's schedules, built now so the backward never synchronises
        code = 2 if hold else 0
        gat_schedule(rowptr, 1, code, H, C)
        gat_schedule(colptr, 1, code, H, C)
        ext = ensure_collapsed_gat_loaded(False)
        # The per-row aggregates (4n(2HC + H) bytes written here and read back
        # by the backward) against the backward's second gather of x_proj (E
        # rows): with bf16 rows on a sparse graph the gather is cheaper, its
        # rows largely cache hits (production block, average degree 8.6:
        # forward + backward 336 -> 292 us; fp32 rows: 434 against 463 us).
        want_agg = not (hold and H * C >= _GATHER_MIN_WIDTH and col.numel() <= _GATHER_MAX_DEGREE * M)
        (y, pre, edge_max, edge_sum, edge_mask), agg = ext.forward_agg(
            a_dst, a_src, rowptr, col, float(negative_slope), xp, bias_c, float(attn_drop), int(seed), want_agg,
            f32_out=hold)
        ctx.save_for_backward(x2, w, s, d, xp, a_src, a_dst, col, row, perm, edge_max, edge_sum, edge_mask, pre,
                              agg)
        ctx.graph = (rowptr, colptr)
        ctx.negative_slope = float(negative_slope)
        ctx.attn_drop = float(attn_drop)
        ctx.hold = hold
        ctx.math = int(math)
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
            a_dst, a_src, pre, grad_y.float().contiguous(), agg, f32_out=ctx.hold)
        # d alpha_src is the GAT's attn_col gradient, d alpha_dst its attn_row
        # gradient; the logits' term is added to grad_feat in place.
        g_s = torch.empty_like(s)
        g_d = torch.empty_like(d)
        st = _lib.stream_ptr(dev)
        K = x2.size(1)
        if (not ctx.needs_input_grad[0] and _SMALL_N < H * C <= _NARROW_N and C % 4 == 0 and K % 4 == 0
                and x2.dtype == torch.float32 and x2.is_contiguous() and x2.data_ptr() % 16 == 0):
            # input features that are data (config c2): the logits' backward
            # fused into the weight gradient, gy never stored
            gw = torch.empty((H * C, K), dtype=torch.float32, device=dev)
            ws_bytes = int(lib.cign_lin_logits_wgrad_workspace_bytes(M, H * C, K))
            ws = _lib.workspace(ws_bytes, dev)
            lib.call("cign_lin_logits_wgrad", st, M, H, C, K, 1 if ctx.hold else 0, ctx.math, grad_feat.data_ptr(),
                     g_attn_col.data_ptr(), g_attn_row.data_ptr(), xp.data_ptr(), s.data_ptr(), d.data_ptr(),
                     x2.data_ptr(), gw.data_ptr(), g_s.data_ptr(), g_d.data_ptr(), ws.data_ptr(), ws_bytes)
            return (None, gw if ctx.needs_input_grad[1] else None, g_s, g_d, g_bias) + (None,) * 10
        # With x_proj held in bf16 the sum is written rounded to bf16, the
        # values the projection's bf16-math backward reads of it.
        gy16 = ctx.hold and C % 8 == 0 and H * C > _SMALL_N
        gy = torch.empty((M, H, C), dtype=torch.bfloat16, device=dev) if gy16 else grad_feat
        ws_bytes = int(lib.cign_colsum_workspace_bytes(M, H * C, 2))
        ws = _lib.workspace(ws_bytes, dev)
        lib.call("cign_attn_logits_bwd_acc", st, M, H, C, 1 if ctx.hold else 0, 1 if gy16 else 0,
                 g_attn_col.data_ptr(), g_attn_row.data_ptr(), xp.data_ptr(), s.data_ptr(), d.data_ptr(),
                 grad_feat.data_ptr(), gy.data_ptr(), g_s.data_ptr(), g_d.data_ptr(), ws.data_ptr(), ws_bytes)
        if gy16:
            K = x2.size(1)
            xf = x2 if x2.dtype == torch.float32 else x2.float()
            gx = torch.empty((M, K), dtype=torch.float32, device=dev) if ctx.needs_input_grad[0] else None
            gw = torch.empty((H * C, K), dtype=torch.float32, device=dev)
            lws_bytes = int(lib.cign_linear_bwd_workspace_bytes(M, H * C, K, 0))
            lws = _lib.workspace(lws_bytes, dev)
            lib.call("cign_linear_bwd_bf16gy", st, M, H * C, K, gy.data_ptr(), xf.data_ptr(), w.data_ptr(),
                     _lib.ptr(gx), gw.data_ptr(), lws.data_ptr(), lws_bytes)
            gw = gw if ctx.needs_input_grad[1] else None
        else:
            gx, gw, _ = _linear_bwd(grad_feat, x2, w, False, ctx.math, ctx.needs_input_grad[0],
                                    ctx.needs_input_grad[1])
        if gx is not None:
            gx = gx.reshape(ctx.in_shape).to(ctx.x_dtype)
        return (gx, gw, g_s, g_d, g_bias) + (None,) * 10


def lin_gat(x: torch.Tensor, weight: torch.Tensor, att_src: torch.Tensor, att_dst: torch.Tensor,
            bias: torch.Tensor, csr, csc, perm: torch.Tensor, negative_slope: float, attn_drop: float, heads: int,
            amp: bool = False, amp_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """SiLU(mean_h GAT_h(x_proj) + bias) with x_proj = lin(x) (bf16 autocast
    with ``amp``) and its attention logits (model_cign.py:546-566). Dropout
    seeds as collapsed_gat_mean_bias_silu: one per call."""
    _check(bias is not None, "collapsed GAT currently requires bias=True")
    _check(x.dim() == 2, f"FusedGAT expects a 2-D node feature tensor, got {tuple(x.shape)}")
    math = _math_code(bool(amp), amp_dtype)
    (rowptr, col), (row, colptr) = csr, csc
    return _LinGatFn.apply(x, weight, att_src, att_dst, bias, rowptr, col, colptr, row, perm, float(negative_slope),
                           float(attn_drop), next_seed(attn_drop), int(heads), math)
