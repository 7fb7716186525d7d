"""Degree-bucketed row schedules (host side of csrc/schedule.h).

A schedule is built once per fixed CSR/CSC row pointer, like the reference's
one-time graph preparation (MultiHopCsrPlan::prepare,
multihop_csr_ext/multihop_csr_pipeline_cuda.cu:246-262;
GraphCliffordNet.prepare_fused_gat_graph, generic_engine/model_cign.py:1069-1158),
and cached per row-pointer tensor for the stateless GAT entry points.
"""
from __future__ import annotations

import ctypes as C
import weakref
from dataclasses import dataclass

import numpy as np
import torch

from ._lib import load_library

# SpMM schedules: rows with at most LIGHT_MAX edges get one wavefront (or a
# lane group), heavier rows are cut into segments of seg_edges edges, one
# 512-thread workgroup each, processed in rounds of 512 edges. Rows longer
# than one segment merge their partial sums across workgroups (partials
# stored and loaded write-through, the last workgroup to arrive adds them in
# segment order); long segments instead serialise rounds inside one
# workgroup. segment_edges_for() balances the two by graph size.
LIGHT_MAX = 64
# Smallest segment (small graphs), for every row width. Gathers of narrow rows
# (at most 256 bytes: D = 64 fp32, the c2/c3 GAT's 4 x 16) once started at
# 1024 edges, when a cross-workgroup merge cost an L2 write-back and
# invalidate on the XCDs involved (c2 SpMM hop 9.9 -> 9.2 us against 512).
# With write-through merges 512 is ahead for them too: c2 layer step 0.0912
# -> 0.0864 ms, the SpMM hops 26.2 / 27.6 -> 24.9 / 25.8 us per three, the
# GAT forward unchanged (256, 1024 and 2048 measured too).
SEG_EDGES = 512
SEG_EDGES_MAX = 16384


def segment_edges_for(nnz: int, floor: int = SEG_EDGES) -> int:
    """Segment length for a graph of nnz edges: the power of two nearest
    above nnz / 4096, clamped to [floor, 16384]. One segment is then at most
    ~1/16 of the edges a CU handles, so the longest workgroup stays short
    against the whole launch, while rows that need a cross-workgroup merge
    become rare (at 62M edges a 512-edge segment leaves 9,250 merging rows
    and takes 2.2x longer per hop than 16,384)."""
    want = max(1, int(nnz) // 4096)
    seg = floor
    while seg < want and seg < SEG_EDGES_MAX:
        seg *= 2
    return seg
# Collapsed-GAT pair-layout schedules: one wavefront takes at most 16 edges
# of a row, segments are 64 edges (16 per wave). The feature-layout forward
# uses the SpMM geometry; cign_gat_schedule_params says which.
GAT_LIGHT_MAX = 16
GAT_SEG_EDGES = 64


@dataclass
class RowSchedule:
    buf: torch.Tensor        # int32 device buffer (csrc/schedule.h layout)
    header: np.ndarray       # host copy of its 12-int header (passed to every launch)
    counters: torch.Tensor   # int32 [n_hrow + 1], zero; kernels leave it zero (last slot: spare global counter)
    n_rows: int
    n_light: int
    n_seg: int
    n_hrow: int
    max_degree: int

    def args(self):
        """(device schedule, host header) pointers of the C-ABI."""
        return (self.buf.data_ptr(), self.header.ctypes.data)


def build_row_schedule(rowptr: torch.Tensor, device=None, light_max: int = LIGHT_MAX,
                       seg_edges: int | None = None, seg_floor: int = SEG_EDGES) -> RowSchedule:
    """Builds the schedule of a row pointer (any integer dtype, any device).
    seg_edges None picks segment_edges_for(nnz, seg_floor). One host copy of the row
    pointer is taken (a synchronisation when it lives on the GPU); this
    happens once per graph, outside timed regions."""
    lib = load_library(require_gpu=False)
    rp = np.ascontiguousarray(rowptr.detach().to("cpu", torch.int64).numpy())
    n_rows = int(rp.shape[0]) - 1
    if n_rows < 0:
        raise ValueError("row pointer must have at least one entry")
    if seg_edges is None:
        seg_edges = segment_edges_for(int(rp[-1]) if rp.size else 0, seg_floor)
    nl, ns, nh = C.c_int32(), C.c_int32(), C.c_int32()
    tot = C.c_int64()
    lib.call("cign_row_schedule_size", rp.ctypes.data, n_rows, light_max, seg_edges,
             C.byref(nl), C.byref(ns), C.byref(nh), C.byref(tot))
    host = np.zeros(int(tot.value), dtype=np.int32)
    lib.call("cign_row_schedule_build", rp.ctypes.data, n_rows, light_max, seg_edges,
             host.ctypes.data, int(tot.value))
    dev = device if device is not None else rowptr.device
    buf = torch.from_numpy(host).to(dev)
    counters = torch.zeros(nh.value + 1, dtype=torch.int32, device=dev)
    deg = np.diff(rp)
    header = np.ascontiguousarray(host[:12].copy())
    return RowSchedule(buf, header, counters, n_rows, int(nl.value), int(ns.value), int(nh.value),
                       int(deg.max()) if deg.size else 0)


_CACHE: dict[tuple, tuple[weakref.ref, int, RowSchedule]] = {}


def cached_row_schedule(rowptr: torch.Tensor, light_max: int = LIGHT_MAX, seg_edges: int | None = None,
                        seg_floor: int = SEG_EDGES) -> RowSchedule:
    """Schedule for a row-pointer tensor, built on first use and reused while
    the tensor is alive and unmodified (checked through its version counter)."""
    key = (id(rowptr), int(light_max), None if seg_edges is None else int(seg_edges), int(seg_floor))
    hit = _CACHE.get(key)
    if hit is not None:
        ref, version, sched = hit
        if ref() is rowptr and version == rowptr._version and sched.n_rows == rowptr.numel() - 1:
            return sched
    sched = build_row_schedule(rowptr, light_max=light_max, seg_edges=seg_edges, seg_floor=seg_floor)
    _CACHE[key] = (weakref.ref(rowptr, lambda _r, k=key: _CACHE.pop(k, None)), rowptr._version, sched)
    return sched


def gat_schedule(rowptr: torch.Tensor, pass_: int, dtype_code: int, heads: int, channels: int) -> RowSchedule:
    """Schedule of a CSR/CSC pointer for a collapsed-GAT pass (0 = forward,
    1 = backward), with the geometry the library asks for that shape. When
    the library accepts any multiple of 256 as the segment length (its
    feature-layout kernels, seg_edges reported as 0 = "any"), the length
    follows the graph size like the SpMM's (from SEG_EDGES)."""
    lib = load_library(require_gpu=False)
    light, seg = C.c_int32(), C.c_int32()
    lib.call("cign_gat_schedule_params", int(pass_), int(dtype_code), int(heads), int(channels), C.byref(light),
             C.byref(seg))
    if seg.value > 0:
        return cached_row_schedule(rowptr, light.value, seg.value)
    return cached_row_schedule(rowptr, light.value, None, SEG_EDGES)
