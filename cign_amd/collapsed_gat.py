"""Collapsed-head GAT on gfx950 (drop-in for the reference module
collapsed_gat.py: same public names, argument meaning, seeds and errors).

``ensure_collapsed_gat_loaded()`` returns an extension object whose
``forward`` / ``backward`` have the reference extension's signatures
(collapsed_gat_ext/collapsed_gat.cpp:45-102) and call the C-ABI entry points
cign_gat_fwd / cign_gat_bwd. Unlike the reference binding, which only accepts
H=6, C=256 (collapsed_gat.cpp:67-68), every shape of the wrapper's advertised
range (1<=H<=32, 1<=C<=256) runs on the HIP kernels; in_feat may be float32
(the reference dtype) or bfloat16 (storage only).
"""
from __future__ import annotations

import itertools

import torch

from . import _lib
from .schedule import gat_schedule

_EXT = None
_EXT_ERROR = None
_CALL_COUNTER = itertools.count()


def _extension_name() -> str:
    return "cign_amd_collapsed_gat_hip"


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _check_dev(t: torch.Tensor, name: str, dtypes) -> None:
    _check(t.is_cuda, f"{name} must be CUDA")
    _check(t.is_contiguous(), f"{name} must be contiguous")
    _check(t.dtype in dtypes, f"{name} must be {' or '.join(str(d).replace('torch.', '') for d in dtypes)}")


_F32 = (torch.float32,)
_FEAT = (torch.float32, torch.bfloat16)
_I32 = (torch.int32,)

# Library dtype of bf16 features with float32 outputs and gradients.
GAT_BF16_F32 = 2


def _gat_code(in_feat: torch.Tensor, f32_out: bool) -> int:
    if not f32_out:
        return _lib.dtype_code(in_feat)
    _check(in_feat.dtype == torch.bfloat16, "f32_out takes bfloat16 in_feat")
    return GAT_BF16_F32


def bf16_f32_supported(heads: int, channels: int) -> bool:
    """Whether the library runs bf16 features with float32 outputs for this
    shape (its feature-layout kernels)."""
    lib = _lib.load_library(require_gpu=False)
    return int(lib.cign_gat_row_agg_floats(GAT_BF16_F32, 1, int(heads), int(channels))) > 0


class _CollapsedGATExt:
    """Extension object with the reference binding's two entry points."""

    @staticmethod
    def forward(attn_row, attn_col, row_ptr, col_ind, negative_slope, in_feat, bias, attn_drop, seed):
        return _CollapsedGATExt.forward_agg(attn_row, attn_col, row_ptr, col_ind, negative_slope, in_feat, bias,
                                            attn_drop, seed, False)[0]

    @staticmethod
    def forward_agg(attn_row, attn_col, row_ptr, col_ind, negative_slope, in_feat, bias, attn_drop, seed,
                    want_agg, f32_out=False):
        """forward() plus, with ``want_agg`` on shapes that support it, the
        per-row aggregate buffer that lets backward() skip its second gather
        of in_feat (None otherwise). ``f32_out`` with bfloat16 in_feat: the
        output is float32 (library dtype 2; feature-layout shapes only), the
        results of float32 in_feat holding the same values."""
        for t, n in ((attn_row, "attn_row"), (attn_col, "attn_col"), (bias, "bias")):
            _check_dev(t, n, _F32)
        _check_dev(row_ptr, "row_ptr", _I32)
        _check_dev(col_ind, "col_ind", _I32)
        _check_dev(in_feat, "in_feat", _FEAT)
        _check(attn_row.dim() == 2, "attn_row must be [N,H]")
        _check(attn_col.shape == attn_row.shape, "attn_col must match attn_row")
        _check(in_feat.dim() == 3, "in_feat must be [N,H,C]")
        _check(in_feat.size(0) == attn_row.size(0) and in_feat.size(1) == attn_row.size(1), "in_feat N/H mismatch")
        _check(bias.dim() == 1 and bias.size(0) == in_feat.size(2), "bias must be [C]")
        _check(1 <= in_feat.size(1) <= 32 and 1 <= in_feat.size(2) <= 256, "collapsed GAT requires 1<=H<=32, 1<=C<=256")
        _check(0.0 <= attn_drop < 1.0, "attn_drop must be in [0,1)")
        _check(row_ptr.numel() == in_feat.size(0) + 1, "row_ptr must have N+1 entries")
        lib = _lib.load_library()
        n, H, C = (int(v) for v in in_feat.shape)
        nnz = int(col_ind.numel())
        dev = in_feat.device
        if in_feat.data_ptr() % 16:
            in_feat = in_feat.clone()
        code = _gat_code(in_feat, f32_out)
        sched = gat_schedule(row_ptr, 0, code, H, C)
        out = torch.empty((n, C), dtype=torch.float32 if code == 2 else in_feat.dtype, device=dev)
        pre = torch.empty((n, C), dtype=torch.float32, device=dev)
        edge_max = torch.empty((n, H), dtype=torch.float32, device=dev)
        edge_sum = torch.empty((n, H), dtype=torch.float32, device=dev)
        edge_mask = torch.empty((nnz, H), dtype=torch.uint8, device=dev)
        ws_bytes = int(lib.cign_gat_fwd_workspace_bytes(sched.n_seg, H, C))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        agg = None
        if want_agg:
            agg_floats = int(lib.cign_gat_row_agg_floats(code, n, H, C))
            if agg_floats > 0:
                agg = torch.empty(agg_floats, dtype=torch.float32, device=dev)
        lib.call("cign_gat_fwd", _lib.stream_ptr(dev), code, n, nnz, H, C, attn_row.data_ptr(),
                 attn_col.data_ptr(), col_ind.data_ptr(), *sched.args(),
                 sched.counters.data_ptr(), float(negative_slope), in_feat.data_ptr(), bias.data_ptr(),
                 float(attn_drop), int(seed) & ((1 << 64) - 1), out.data_ptr(), pre.data_ptr(), edge_max.data_ptr(),
                 edge_sum.data_ptr(), edge_mask.data_ptr(), ws.data_ptr(), ws_bytes, _lib.ptr(agg))
        return [out, pre, edge_max, edge_sum, edge_mask], agg

    @staticmethod
    def backward(negative_slope, attn_drop, row_ptr, col_ind, col_ptr, row_ind, permute, edge_max, edge_sum,
                 edge_mask, in_feat, attn_row, attn_col, pre, grad_y, row_agg=None, f32_out=False):
        """``row_agg``: the buffer forward_agg() returned for the same inputs,
        or None (the rows pass then gathers in_feat per edge). ``f32_out``
        as in forward_agg: grad_y and grad_feat are float32."""
        for t, n in ((row_ptr, "row_ptr"), (col_ind, "col_ind"), (col_ptr, "col_ptr"), (row_ind, "row_ind"),
                     (permute, "permute")):
            _check_dev(t, n, _I32)
        for t, n in ((edge_max, "edge_max"), (edge_sum, "edge_sum"), (attn_row, "attn_row"),
                     (attn_col, "attn_col"), (pre, "pre")):
            _check_dev(t, n, _F32)
        _check_dev(edge_mask, "edge_mask", (torch.uint8,))
        _check_dev(in_feat, "in_feat", _FEAT)
        code = _gat_code(in_feat, f32_out)
        _check_dev(grad_y, "grad_y", (torch.float32,) if code == 2 else (in_feat.dtype,))
        _check(in_feat.dim() == 3 and 1 <= in_feat.size(1) <= 32 and 1 <= in_feat.size(2) <= 256,
               "collapsed GAT requires in_feat [N,H,C] with 1<=H<=32, 1<=C<=256")
        _check(pre.shape == grad_y.shape, "pre and grad_y must match")
        lib = _lib.load_library()
        n, H, C = (int(v) for v in in_feat.shape)
        nnz = int(col_ind.numel())
        dev = in_feat.device
        rs = gat_schedule(row_ptr, 1, code, H, C)
        cs = gat_schedule(col_ptr, 1, code, H, C)
        row_blocks = rs.n_seg + (rs.n_light + 3) // 4
        ws_bytes = int(lib.cign_gat_bwd_workspace_bytes(n, nnz, H, C, row_blocks, rs.n_seg, cs.n_seg))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        grad_feat = torch.empty_like(in_feat, dtype=torch.float32 if code == 2 else in_feat.dtype)
        grad_attn_row = torch.empty_like(attn_row)
        grad_attn_col = torch.empty_like(attn_col)
        grad_bias = torch.empty((C,), dtype=torch.float32, device=dev)
        lib.call("cign_gat_bwd", _lib.stream_ptr(dev), code, n, nnz, H, C, float(negative_slope),
                 float(attn_drop), col_ind.data_ptr(), row_ind.data_ptr(),
                 permute.data_ptr(), edge_max.data_ptr(), edge_sum.data_ptr(), edge_mask.data_ptr(),
                 in_feat.data_ptr(), attn_row.data_ptr(), attn_col.data_ptr(), pre.data_ptr(), grad_y.data_ptr(),
                 *rs.args(), rs.counters.data_ptr(), *cs.args(), cs.counters.data_ptr(), ws.data_ptr(), ws_bytes,
                 grad_feat.data_ptr(), grad_attn_row.data_ptr(), grad_attn_col.data_ptr(), grad_bias.data_ptr(),
                 _lib.ptr(row_agg))
        return [grad_feat, grad_attn_row, grad_attn_col, grad_bias]


def ensure_collapsed_gat_loaded(verbose: bool = False):
    """Loads the HIP library once (collapsed_gat.py:19-54): a missing GPU raises
    RuntimeError; the first load failure is cached and re-raised."""
    global _EXT, _EXT_ERROR
    if _EXT is not None:
        return _EXT
    if _EXT_ERROR is not None:
        raise RuntimeError("collapsed GAT HIP library previously failed to load") from _EXT_ERROR
    if not torch.cuda.is_available():
        raise RuntimeError("collapsed GAT requires a HIP GPU")
    try:
        _lib.load_library()
        _EXT = _CollapsedGATExt()
        if verbose:
            print(f"[cign_amd] {_extension_name()} loaded from {_lib.LIB_PATH}")
        return _EXT
    except Exception as exc:
        _EXT_ERROR = exc
        raise


class _CollapsedGATFn(torch.autograd.Function):
    """collapsed_gat.py:57-161 (same saved tensors, same 12-slot backward)."""

    @staticmethod
    def forward(ctx, attn_row, attn_col, rowptr, col, colptr, row, perm, negative_slope, in_feat, bias, attn_drop,
                seed):
        ext = ensure_collapsed_gat_loaded(False)
        attn_row = attn_row.contiguous()
        attn_col = attn_col.contiguous()
        rowptr = rowptr.contiguous()
        col = col.contiguous()
        colptr = colptr.contiguous()
        row = row.contiguous()
        perm = perm.contiguous()
        in_feat = in_feat.contiguous()
        bias = bias.contiguous()
        # Schedules are keyed on the graph tensors the caller holds; build the
        # backward's schedules now so the backward never synchronises.
        code = _lib.dtype_code(in_feat)
        H, C = int(in_feat.size(1)), int(in_feat.size(2))
        gat_schedule(rowptr, 1, code, H, C)
        gat_schedule(colptr, 1, code, H, C)
        (y, pre, edge_max, edge_sum, edge_mask), agg = ext.forward_agg(
            attn_row, attn_col, rowptr, col, float(negative_slope), in_feat, bias, float(attn_drop), int(seed), True)
        # agg (per-row aggregates, or None) spares the backward a second
        # gather of in_feat; it is saved beside the reference's tensors.
        ctx.save_for_backward(rowptr, col, colptr, row, perm, edge_max, edge_sum, edge_mask, in_feat, attn_row,
                              attn_col, pre, agg)
        ctx.graph = (rowptr, colptr)  # keeps the schedule cache keys alive and identical
        ctx.negative_slope = float(negative_slope)
        ctx.attn_drop = float(attn_drop)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        ext = ensure_collapsed_gat_loaded(False)
        (_rowptr, col, _colptr, row, perm, edge_max, edge_sum, edge_mask, in_feat, attn_row, attn_col,
         pre, agg) = ctx.saved_tensors
        rowptr, colptr = ctx.graph
        grad_feat, grad_attn_row, grad_attn_col, grad_bias = ext.backward(
            float(ctx.negative_slope), float(ctx.attn_drop), rowptr, col, colptr, row, perm, edge_max, edge_sum,
            edge_mask, in_feat, attn_row, attn_col, pre, grad_y.to(dtype=in_feat.dtype).contiguous(), agg)
        return (grad_attn_row, grad_attn_col, None, None, None, None, None, None, grad_feat, grad_bias, None, None)


def collapsed_gat_mean_bias_silu(attn_row: torch.Tensor, attn_col: torch.Tensor, csr, csc, perm: torch.Tensor,
                                 negative_slope: float, in_feat: torch.Tensor, bias: torch.Tensor,
                                 attn_drop: float) -> torch.Tensor:
    """SiLU(mean_h GAT_h(in_feat) + bias) for concat=False, 1<=H<=32, 1<=C<=256
    (collapsed_gat.py:164-225). attn_row = destination logits, attn_col =
    source logits; csr = (rowptr, col), csc = (row, colptr); perm maps CSC
    positions to CSR edge ids. Dropout seeds follow the reference exactly:
    torch.initial_seed() plus a per-process call counter that only advances
    when attn_drop > 0."""
    if in_feat.dtype not in (torch.float32, torch.bfloat16) or in_feat.device.type != "cuda":
        raise TypeError("collapsed GAT requires GPU float32 (or bfloat16) in_feat")
    if bias is None:
        raise ValueError("collapsed GAT currently requires bias=True")
    if in_feat.dim() != 3:
        raise ValueError(f"in_feat must be [N,H,C], got {tuple(in_feat.shape)}")
    C = int(in_feat.size(2))
    H = int(in_feat.size(1))
    if not (1 <= C <= 256):
        raise ValueError(f"collapsed GAT requires 1<=C<=256; got C={C}")
    if not (1 <= H <= 32):
        raise ValueError(f"collapsed GAT requires 1<=H<=32; got H={H}")
    (rowptr, col), (row, colptr) = csr, csc
    return _CollapsedGATFn.apply(attn_row, attn_col, rowptr, col, colptr, row, perm, float(negative_slope), in_feat,
                                 bias, float(attn_drop), next_seed(attn_drop))


def next_seed(attn_drop: float) -> int:
    """Dropout seed of the next collapsed-GAT call (collapsed_gat.py:204-211):
    torch.initial_seed() plus a per-process call counter that only advances
    when attn_drop > 0; 0 without dropout."""
    base_seed = int(torch.initial_seed()) & ((1 << 63) - 1)
    call_id = next(_CALL_COUNTER) if float(attn_drop) > 0.0 else -1
    return 0 if call_id < 0 else (base_seed + 0x9E3779B97F4A7C15 * (call_id + 1)) & ((1 << 63) - 1)
