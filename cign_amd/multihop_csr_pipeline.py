"""Multihop CSR SpMM pipeline on gfx950 (drop-in for the reference module
multihop_csr_pipeline.py, same public names and behaviour).

``MultiHopCsrPlan`` mirrors the reference's native plan class
(multihop_csr_ext/multihop_csr_pipeline.h:8-37): it owns int32 copies of
CSR(P) and CSR(P^T), their row schedules (built once, like the reference's
``prepare``) and the SpMM partial-sum scratch; ``forward3`` / ``backward3``
enqueue the three chained HIP SpMMs of cign_spmm_fwd3 / cign_spmm_bwd3 on the
current stream with no host synchronisation. ``algorithm`` (1, 2, 3) is kept
for API compatibility; the HIP schedule does not depend on it.

Dense operands may be float32 (the reference's only dtype) or bfloat16
(storage only; accumulation is float32).
"""
from __future__ import annotations

from typing import Dict, Tuple

import torch

from . import _lib
from .graph import _hip_parts
from .schedule import build_row_schedule

_EXT = None
_EXT_ERROR = None


class _MultihopExt:
    """Stand-in for the reference's compiled extension module."""

    MultiHopCsrPlan = None  # set below


def ensure_multihop_csr_loaded():
    """Loads libcign_amd (multihop_csr_pipeline.py:15-35). Raises
    RuntimeError without a HIP device or without the built library."""
    global _EXT, _EXT_ERROR
    if _EXT is not None:
        return _EXT
    if _EXT_ERROR is not None:
        raise RuntimeError("Multihop CSR HIP library previously failed to load") from _EXT_ERROR
    if not torch.cuda.is_available():
        raise RuntimeError("MultiHopCSR requires a HIP GPU.")
    try:
        _lib.load_library()
    except Exception as exc:
        _EXT_ERROR = exc
        raise
    _EXT = _MultihopExt
    return _EXT


def _csr_parts_int32(csr: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """int32 crow / col and float32 values, cloned (multihop_csr_pipeline.py:38-48)."""
    if csr.layout != torch.sparse_csr:
        raise TypeError(f"Expected sparse CSR tensor, got {csr.layout}.")
    if csr.device.type != "cuda":
        raise RuntimeError("CSR tensors must already be on the GPU.")
    if csr.dtype != torch.float32:
        raise TypeError(f"MultiHop CSR requires float32 sparse values, got {csr.dtype}.")
    crow = csr.crow_indices().to(dtype=torch.int32).clone().contiguous()
    col = csr.col_indices().to(dtype=torch.int32).clone().contiguous()
    val = csr.values().to(dtype=torch.float32).clone().contiguous()
    return crow, col, val


class MultiHopCsrPlan:
    """Native 3-hop plan (multihop_csr_ext/multihop_csr_pipeline_cuda.cu:113-369)."""

    def __init__(self, p_crow, p_col, p_values, pt_crow, pt_col, pt_values, rows, dense_cols, algorithm):
        rows, dense_cols, algorithm = int(rows), int(dense_cols), int(algorithm)
        if algorithm not in (1, 2, 3):
            raise RuntimeError(f"MultiHopCsrPlan algorithm must be 1, 2, or 3; got {algorithm}")
        if rows <= 0 or dense_cols <= 0:
            raise RuntimeError("rows and dense_cols must be positive.")
        if not p_values.is_cuda:
            raise RuntimeError("CSR tensors must be CUDA.")
        dev = p_values.device
        for name, t in (("p_crow", p_crow), ("p_col", p_col), ("p_values", p_values), ("pt_crow", pt_crow),
                        ("pt_col", pt_col), ("pt_values", pt_values)):
            if not t.is_cuda:
                raise RuntimeError(f"{name} must be CUDA.")
            if t.device != dev:
                raise RuntimeError(f"{name} is on wrong CUDA device.")
            if not t.is_contiguous():
                raise RuntimeError(f"{name} must be contiguous.")
        if not all(t.dtype == torch.int32 for t in (p_crow, p_col, pt_crow, pt_col)):
            raise RuntimeError("MultiHopCsrPlan requires int32 CSR indices.")
        if p_values.dtype != torch.float32 or pt_values.dtype != torch.float32:
            raise RuntimeError("MultiHopCsrPlan requires float32 CSR values.")
        if p_crow.numel() != rows + 1 or pt_crow.numel() != rows + 1:
            raise RuntimeError("CSR row-pointer length mismatch.")
        if p_col.numel() != p_values.numel():
            raise RuntimeError("P col/value nnz mismatch.")
        if pt_col.numel() != pt_values.numel():
            raise RuntimeError("P^T col/value nnz mismatch.")
        self._p = (p_crow, p_col, p_values)
        self._pt = (pt_crow, pt_col, pt_values)
        self._rows = rows
        self._dense_cols = dense_cols
        self._algorithm = algorithm
        self._nnz = int(p_values.numel())
        self._device = dev
        self._p_sched = build_row_schedule(p_crow)
        self._pt_sched = build_row_schedule(pt_crow)
        self._part = None
        self._prepared = False

    def _check_dense(self, x: torch.Tensor, name: str) -> None:
        if not x.is_cuda:
            raise RuntimeError(f"{name} must be CUDA.")
        if x.device != self._device:
            raise RuntimeError(f"{name} is on wrong CUDA device.")
        if x.dtype not in (torch.float32, torch.bfloat16):
            raise RuntimeError(f"{name} must be float32 (or bfloat16).")
        if x.dim() != 2:
            raise RuntimeError(f"{name} must be 2-D.")
        if x.size(0) != self._rows or x.size(1) != self._dense_cols:
            raise RuntimeError(f"{name} shape mismatch, expected [{self._rows}, {self._dense_cols}], "
                               f"got [{x.size(0)}, {x.size(1)}].")
        if not x.is_contiguous():
            raise RuntimeError(f"{name} must be contiguous row-major.")

    def prepare(self, x: torch.Tensor) -> None:
        """Sizes and allocates the SpMM scratch (the cuSPARSE workspace of the
        reference, multihop_csr_pipeline_cuda.cu:246-262)."""
        self._check_dense(x, "prepare input")
        n_seg = max(self._p_sched.n_seg, self._pt_sched.n_seg)
        self._part = None
        if n_seg > 0:
            nbytes = int(_lib.load_library().cign_spmm_partial_bytes(n_seg, self._dense_cols))
            self._part = torch.empty(max(1, nbytes // 4), dtype=torch.float32, device=self._device)
        self._prepared = True

    def _require_prepared(self):
        if not self._prepared:
            raise RuntimeError("MultiHopCsrPlan.prepare() must be called before timed execution.")

    def forward3(self, x: torch.Tensor):
        self._check_dense(x, "forward3 x")
        self._require_prepared()
        lib = _lib.load_library()
        y1, y2, y3 = (torch.empty_like(x) for _ in range(3))
        crow, col, val = self._p
        lib.call("cign_spmm_fwd3", _lib.stream_ptr(self._device), _lib.dtype_code(x), self._rows, self._dense_cols,
                 col.data_ptr(), val.data_ptr(), *self._p_sched.args(), x.data_ptr(),
                 y1.data_ptr(), y2.data_ptr(), y3.data_ptr(), _lib.ptr(self._part),
                 self._p_sched.counters.data_ptr())
        return [y1, y2, y3]

    def backward3(self, grad_y1: torch.Tensor, grad_y2: torch.Tensor, grad_y3: torch.Tensor) -> torch.Tensor:
        self._check_dense(grad_y1, "backward3 g1")
        self._check_dense(grad_y2, "backward3 g2")
        self._check_dense(grad_y3, "backward3 g3")
        self._require_prepared()
        if not (grad_y1.dtype == grad_y2.dtype == grad_y3.dtype):
            raise RuntimeError("backward3 gradients must share a dtype.")
        lib = _lib.load_library()
        t2, t1, gx = (torch.empty_like(grad_y1) for _ in range(3))
        crow, col, val = self._pt
        lib.call("cign_spmm_bwd3", _lib.stream_ptr(self._device), _lib.dtype_code(grad_y1), self._rows,
                 self._dense_cols, col.data_ptr(), val.data_ptr(), *self._pt_sched.args(),
                 grad_y1.data_ptr(), grad_y2.data_ptr(), grad_y3.data_ptr(), t2.data_ptr(), t1.data_ptr(),
                 gx.data_ptr(), _lib.ptr(self._part), self._pt_sched.counters.data_ptr())
        return gx

    def algorithm(self) -> int:
        return self._algorithm

    def workspace_bytes(self) -> int:
        return 0 if self._part is None else int(self._part.numel() * 4)

    def info(self) -> str:
        return (f"HIP MultiHopCSR3 (gfx950 degree-bucketed SpMM), schedule_hint={self._algorithm}, "
                f"shape=[{self._rows},{self._rows}], nnz={self._nnz}, dense_cols={self._dense_cols}, "
                f"workspace={self.workspace_bytes()} bytes, heavy_rows={self._p_sched.n_hrow}, "
                f"segments={self._p_sched.n_seg}, device={self._device}")


_MultihopExt.MultiHopCsrPlan = MultiHopCsrPlan


class MultiHopCSR3Function(torch.autograd.Function):
    """multihop_csr_pipeline.py:59-86. The dense input is cast to the
    operator's dense dtype (float32 by default, as in the reference) and the
    gradient is returned in the input dtype; missing grads become zeros."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, operator: "MultiHopCSR3GraphOperator"):
        ctx.input_dtype = x.dtype
        ctx.operator = operator
        xd = x.to(dtype=operator.dense_dtype).contiguous()
        y1, y2, y3 = operator.plan.forward3(xd)
        return y1, y2, y3

    @staticmethod
    def backward(ctx, grad_y1, grad_y2, grad_y3):
        ref = grad_y1 if grad_y1 is not None else (grad_y2 if grad_y2 is not None else grad_y3)
        if ref is None:
            return None, None
        if grad_y1 is None:
            grad_y1 = torch.zeros_like(ref)
        if grad_y2 is None:
            grad_y2 = torch.zeros_like(ref)
        if grad_y3 is None:
            grad_y3 = torch.zeros_like(ref)
        dt = ctx.operator.dense_dtype
        grad_x = ctx.operator.plan.backward3(grad_y1.to(dtype=dt).contiguous(), grad_y2.to(dtype=dt).contiguous(),
                                             grad_y3.to(dtype=dt).contiguous())
        if grad_x.dtype != ctx.input_dtype:
            grad_x = grad_x.to(ctx.input_dtype)
        return grad_x, None


class MultiHopCSR3GraphOperator:
    """multihop_csr_pipeline.py:89-140. ``dense_dtype`` (float32 default, the
    reference's behaviour; bfloat16 opt-in) is the storage dtype the three
    hops run in."""

    __slots__ = ("base", "plan", "_storage_p", "_storage_pt", "shape", "nnz", "dtype", "device", "dense_cols",
                 "algorithm", "powers", "info", "dense_dtype")

    def __init__(self, base_fixed_csr, dense_cols: int, algorithm: int = 2, dense_dtype=torch.float32):
        if int(dense_cols) <= 0:
            raise ValueError("dense_cols must be positive.")
        if int(algorithm) not in (1, 2, 3):
            raise ValueError("MultiHop algorithm must be 1, 2, or 3.")
        if not hasattr(base_fixed_csr, "csr") or not hasattr(base_fixed_csr, "csr_t"):
            raise TypeError("MultiHopCSR3 expects an already prepared FixedCSRGraphOperator.")
        if dense_dtype not in (torch.float32, torch.bfloat16):
            raise TypeError(f"dense_dtype must be float32 or bfloat16, got {dense_dtype}")
        self.base = base_fixed_csr
        self.shape = tuple(base_fixed_csr.shape)
        self.nnz = int(base_fixed_csr.nnz)
        self.dtype = base_fixed_csr.dtype
        self.device = base_fixed_csr.device
        self.dense_cols = int(dense_cols)
        self.algorithm = int(algorithm)
        self.powers = (1, 2, 3)
        self.dense_dtype = dense_dtype
        ensure_multihop_csr_loaded()
        p = _csr_parts_int32(base_fixed_csr.csr)
        pt = _csr_parts_int32(base_fixed_csr.csr_t)
        self._storage_p = p
        self._storage_pt = pt
        self.plan = MultiHopCsrPlan(p[0], p[1], p[2], pt[0], pt[1], pt[2], int(self.shape[0]), self.dense_cols,
                                    self.algorithm)
        dummy = torch.empty((self.shape[0], self.dense_cols), device=self.device, dtype=torch.float32)
        self.plan.prepare(dummy)
        torch.cuda.synchronize(self.device)
        self.info: Dict[str, object] = {
            "backend": "HIP_MultiHopCSR3",
            "powers": list(self.powers),
            "shape": self.shape,
            "nnz": self.nnz,
            "dense_cols": self.dense_cols,
            "index_dtype": "torch.int32",
            "algorithm": self.algorithm,
            "dense_dtype": str(self.dense_dtype),
            "workspace_bytes": int(self.plan.workspace_bytes()),
            "native_info": self.plan.info(),
        }

    @property
    def csr(self):
        return self.base.csr

    @property
    def csr_t(self):
        return self.base.csr_t


def _csr_mm(csr: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """One HIP SpMM in the operator dtype (multihop_csr_pipeline.py:51-56)."""
    return _hip_parts(csr).spmm(x.to(dtype=csr.dtype).contiguous())


class _TailFixedCSRFunction(torch.autograd.Function):
    """One exact fixed-CSR propagation step after the native 3-hop prefix
    (multihop_csr_pipeline.py:143-157)."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, csr: torch.Tensor, csr_t: torch.Tensor):
        ctx.csr_t = csr_t
        ctx.input_dtype = x.dtype
        return _csr_mm(csr, x)

    @staticmethod
    def backward(ctx, grad_y):
        grad_x = _csr_mm(ctx.csr_t, grad_y)
        if grad_x.dtype != ctx.input_dtype:
            grad_x = grad_x.to(ctx.input_dtype)
        return grad_x, None, None


class HybridNative3TailCSRGraphOperator:
    """Arbitrary-K propagation: native first 3 powers + exact CSR tail
    (multihop_csr_pipeline.py:160-211)."""

    __slots__ = ("base", "native3", "shape", "nnz", "dtype", "device", "dense_cols", "algorithm", "powers",
                 "positive_powers", "max_power", "info")

    def __init__(self, base_fixed_csr, dense_cols: int, powers, algorithm: int = 2):
        powers = tuple(sorted(set(int(p) for p in powers)))
        if not powers or min(powers) < 0:
            raise ValueError(f"powers must be non-empty non-negative integers, got {powers}")
        positive = tuple(p for p in powers if p > 0)
        if not positive or max(positive) < 3:
            raise ValueError("HybridNative3TailCSR requires at least one positive requested power >= 3; "
                             f"got powers={powers}")
        self.base = base_fixed_csr
        self.native3 = MultiHopCSR3GraphOperator(base_fixed_csr, dense_cols=dense_cols, algorithm=algorithm)
        self.shape = tuple(base_fixed_csr.shape)
        self.nnz = int(base_fixed_csr.nnz)
        self.dtype = base_fixed_csr.dtype
        self.device = base_fixed_csr.device
        self.dense_cols = int(dense_cols)
        self.algorithm = int(algorithm)
        self.powers = powers
        self.positive_powers = positive
        self.max_power = max(positive)
        self.info = {
            "backend": "HybridNative3TailCSR",
            "powers": list(self.powers),
            "shape": self.shape,
            "nnz": self.nnz,
            "dense_cols": self.dense_cols,
            "algorithm": self.algorithm,
            "prefix": "HIP_MultiHopCSR3",
            "tail_steps": max(0, self.max_power - 3),
            "implementation": "native forward3/backward3 prefix + exact HIP CSR tail",
            "native_info": self.native3.info,
        }

    @property
    def csr(self):
        return self.base.csr

    @property
    def csr_t(self):
        return self.base.csr_t


def hybrid_native3_tail_csr(operator: HybridNative3TailCSRGraphOperator, x: torch.Tensor):
    """multihop_csr_pipeline.py:214-230."""
    y1, y2, y3 = multihop_csr3(operator.native3, x)
    requested = set(operator.positive_powers)
    out = {}
    if 1 in requested:
        out[1] = y1
    if 2 in requested:
        out[2] = y2
    if 3 in requested:
        out[3] = y3
    current = y3
    for power in range(4, operator.max_power + 1):
        current = _TailFixedCSRFunction.apply(current, operator.csr, operator.csr_t)
        if power in requested:
            out[power] = current
    return out


class GenericMultiHopCSRFunction(torch.autograd.Function):
    """Cached CSR recurrence with one autograd node
    (multihop_csr_pipeline.py:233-265)."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, operator: "GenericMultiHopCSRGraphOperator"):
        ctx.operator = operator
        ctx.input_dtype = x.dtype
        current = x.to(dtype=operator.dtype).contiguous()
        outputs = []
        wanted = set(operator.positive_powers)
        for p in range(1, operator.max_power + 1):
            current = _csr_mm(operator.csr, current)
            if p in wanted:
                outputs.append(current)
        return tuple(outputs)

    @staticmethod
    def backward(ctx, *grad_outputs):
        op = ctx.operator
        if not grad_outputs:
            return None, None
        ref = next((g for g in grad_outputs if g is not None), None)
        if ref is None:
            return None, None
        grad_by_power = {p: g for p, g in zip(op.positive_powers, grad_outputs) if g is not None}
        pt = _hip_parts(op.csr_t)
        acc = torch.zeros_like(ref, dtype=op.dtype)
        for p in range(op.max_power, 0, -1):
            g = grad_by_power.get(p)
            if g is not None:
                acc = acc + g.to(dtype=op.dtype).contiguous()
            acc = pt.spmm(acc)
        if acc.dtype != ctx.input_dtype:
            acc = acc.to(ctx.input_dtype)
        return acc, None


class GenericMultiHopCSRGraphOperator:
    """multihop_csr_pipeline.py:268-306."""

    __slots__ = ("base", "shape", "nnz", "dtype", "device", "dense_cols", "algorithm", "powers", "positive_powers",
                 "max_power", "info")

    def __init__(self, base_fixed_csr, dense_cols: int, powers, algorithm: int = 2):
        if not hasattr(base_fixed_csr, "csr") or not hasattr(base_fixed_csr, "csr_t"):
            raise TypeError("GenericMultiHopCSR expects an already prepared FixedCSRGraphOperator.")
        powers = tuple(sorted(set(int(p) for p in powers)))
        if not powers or min(powers) < 0:
            raise ValueError(f"powers must be non-empty non-negative integers, got {powers}")
        self.base = base_fixed_csr
        self.shape = tuple(base_fixed_csr.shape)
        self.nnz = int(base_fixed_csr.nnz)
        self.dtype = base_fixed_csr.dtype
        self.device = base_fixed_csr.device
        self.dense_cols = int(dense_cols)
        self.algorithm = int(algorithm)
        self.powers = powers
        self.positive_powers = tuple(p for p in powers if p > 0)
        self.max_power = max(self.positive_powers) if self.positive_powers else 0
        self.info = {
            "backend": "GenericMultiHopCSR_Autograd",
            "powers": list(self.powers),
            "shape": self.shape,
            "nnz": self.nnz,
            "dense_cols": self.dense_cols,
            "value_dtype": str(self.dtype),
            "implementation": "cached CSR recurrence (HIP SpMM) + single custom autograd node",
        }

    @property
    def csr(self):
        return self.base.csr

    @property
    def csr_t(self):
        return self.base.csr_t


def prepare_multihop_csr_operator(base_fixed_csr, dense_cols: int, algorithm: int = 2, powers=(1, 2, 3),
                                  prefer_native_three_hop: bool = True, strategy: str = "auto"):
    """multihop_csr_pipeline.py:309-337."""
    pset = tuple(sorted(set(int(p) for p in powers)))
    positive = tuple(p for p in pset if p > 0)
    max_power = max(positive) if positive else 0
    strategy = str(strategy).strip().lower()
    if strategy not in {"auto", "native3_tail", "generic"}:
        raise ValueError(f"Unknown MultiHop strategy={strategy!r}")
    if prefer_native_three_hop and pset == (1, 2, 3):
        return MultiHopCSR3GraphOperator(base_fixed_csr, dense_cols=dense_cols, algorithm=algorithm)
    if strategy in {"auto", "native3_tail"} and max_power >= 3:
        return HybridNative3TailCSRGraphOperator(base_fixed_csr, dense_cols=dense_cols, powers=pset,
                                                 algorithm=algorithm)
    return GenericMultiHopCSRGraphOperator(base_fixed_csr, dense_cols=dense_cols, powers=pset, algorithm=algorithm)


def multihop_csr3(operator: MultiHopCSR3GraphOperator, x: torch.Tensor):
    return MultiHopCSR3Function.apply(x, operator)


def generic_multihop_csr(operator: GenericMultiHopCSRGraphOperator, x: torch.Tensor):
    if not operator.positive_powers:
        return {}
    vals = GenericMultiHopCSRFunction.apply(x, operator)
    if len(operator.positive_powers) == 1 and torch.is_tensor(vals):
        vals = (vals,)
    return {p: y for p, y in zip(operator.positive_powers, vals)}
