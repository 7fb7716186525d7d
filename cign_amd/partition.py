"""Row-nnz partitioned execution of the layer on one GPU: the one-GPU part of
splitting a graph too large for one launch (or, later, for one GPU).

The reference partitions the GAT by destination rows in
generic_engine/chunked_dgnn_gat.py:104-209 (fixed runs of target nodes,
halved while a chunk's local node set exceeds max_local_nodes; every chunk
keeps all in-edges of its targets and adds the source-only nodes as feature
providers) and runs the op chunk by chunk (:214-252), leaving the source
gradients of overlapping chunks to autograd's scatter-add. Here:

* partition_rows cuts the node range into contiguous shards balanced by
  edge count (one unit per edge of each row pointer given, plus one per row),
  since power-law hubs would leave row-count shards unbalanced; shards whose
  local node set exceeds max_local_nodes are halved by edges, as the
  reference halves chunks.
* A shard owns its nodes [lo, hi) as destination rows AND as sources. Its
  RowShard lists the in-edges of its rows and the source halo (the sources
  outside [lo, hi)); its ColShard lists the out-edges of its sources and the
  destination halo.
* Forward passes (GAT forward, the SpMM hops y = P x) run per RowShard on
  halo-gathered inputs. Backward passes whose sums run over a node's
  out-edges (the GAT's source gradients) run per ColShard on gathered
  per-row inputs, so every node's sum is taken in one shard, in the whole
  graph's order; the SpMM backward is a forward pass of P^T. The gathers
  (index_select of the local node lists) stand where a multi-GPU run
  exchanges halo rows.
* Every shard schedule is built with the whole graph's schedule geometry and
  the GAT shard entry points run the whole graph's kernel variant and
  dropout indices, so each node's outputs and gradients are bit-identical to
  the unsharded layer's. Only sums over all nodes (the GAT bias gradient)
  are combined across shards, in shard order (an all-reduce on several GPUs).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import numpy as np
import torch

from . import _lib
from .schedule import RowSchedule, build_row_schedule, gat_schedule


def _host_i64(t: torch.Tensor) -> np.ndarray:
    return np.ascontiguousarray(t.detach().to("cpu", torch.int64).numpy())


def partition_rows(rowptrs: Sequence, num_shards: int, max_local_nodes: int | None = None,
                   cols: Sequence | None = None) -> list[tuple[int, int]]:
    """Contiguous node ranges [lo, hi) covering [0, n), balanced by cost(row) =
    1 + sum of the row's edges over `rowptrs` (host or device row pointers of
    the same n). With max_local_nodes (and `cols`, the column arrays of the
    same row pointers), a range whose rows plus source halo exceed it is
    halved by cost until it fits (a single row that does not fit raises, as
    chunked_dgnn_gat.py:137-141)."""
    rps = [_host_i64(torch.as_tensor(r)) for r in rowptrs]
    if not rps:
        raise ValueError("partition_rows needs at least one row pointer")
    n = int(rps[0].shape[0]) - 1
    if any(int(r.shape[0]) - 1 != n for r in rps):
        raise ValueError("row pointers must all cover the same rows")
    if num_shards < 1:
        raise ValueError("num_shards must be positive")
    cost = np.arange(n + 1, dtype=np.int64)
    for r in rps:
        cost += r - r[0]
    total = int(cost[-1])
    cuts = [0]
    for k in range(1, num_shards):
        c = int(np.searchsorted(cost, total * k / num_shards, side="left"))
        if cuts[-1] < c < n:
            cuts.append(c)
    cuts.append(n)
    ranges = [(cuts[i], cuts[i + 1]) for i in range(len(cuts) - 1) if cuts[i + 1] > cuts[i]]
    if max_local_nodes is None:
        return ranges
    if cols is None:
        raise ValueError("max_local_nodes needs the column arrays")
    cls = [_host_i64(torch.as_tensor(c)) for c in cols]
    out = []

    def fit(lo, hi):
        mark = np.zeros(n, dtype=bool)
        mark[lo:hi] = True
        for r, c in zip(rps, cls):
            mark[c[r[lo]:r[hi]]] = True
        size = int(mark.sum())
        if size <= max_local_nodes:
            out.append((lo, hi))
            return
        if hi - lo <= 1:
            raise RuntimeError(f"row {lo} needs {size} local nodes, above max_local_nodes={max_local_nodes}")
        mid = int(np.searchsorted(cost, (cost[lo] + cost[hi]) / 2, side="left"))
        mid = min(max(mid, lo + 1), hi - 1)
        fit(lo, mid)
        fit(mid, hi)

    for lo, hi in ranges:
        fit(lo, hi)
    return out


@dataclass
class RowShard:
    """Destination rows [lo, hi) of a CSR with their in-edges [e0, e1): `nodes`
    (device int64, ascending) = the rows and their source halo, `col` (device
    int32) = the in-edges' sources as positions in `nodes`, in the CSR's own
    order; `sched` = the rows' schedule with the whole graph's geometry."""
    lo: int
    hi: int
    e0: int
    e1: int
    nodes: torch.Tensor
    col: torch.Tensor
    val: torch.Tensor | None
    sched: RowSchedule

    @property
    def halo(self) -> int:
        return int(self.nodes.numel()) - (self.hi - self.lo)


@dataclass
class ColShard:
    """Source columns [lo, hi) of a graph with their out-edges: `nodes` (device
    int64, ascending) = the sources and the destination rows they reach,
    [own, own + hi - lo) = the sources' positions in `nodes`; the shard's own
    graph over `nodes` as CSR (rowptr, col; edges in whole-graph CSR order),
    CSC (colptr, row) and perm (CSC entry -> local CSR id); csr_ids (device
    int64) = each local CSR edge's id in the whole graph; schedules of both
    with the whole graph's geometry."""
    lo: int
    hi: int
    own: int
    nodes: torch.Tensor
    rowptr: torch.Tensor
    col: torch.Tensor
    colptr: torch.Tensor
    row: torch.Tensor
    perm: torch.Tensor
    csr_ids: torch.Tensor
    row_sched: RowSchedule
    col_sched: RowSchedule

    @property
    def nnz(self) -> int:
        return int(self.col.numel())


def _row_shard(rp: np.ndarray, cl: np.ndarray, val, lo: int, hi: int, light: int, seg: int, dev) -> RowShard:
    n = rp.shape[0] - 1
    e0, e1 = int(rp[lo]), int(rp[hi])
    src = cl[e0:e1]
    mark = np.zeros(n, dtype=bool)
    mark[lo:hi] = True
    mark[src] = True
    nodes = np.flatnonzero(mark)
    lid = np.cumsum(mark, dtype=np.int64) - 1
    local_rp = torch.from_numpy(rp[lo:hi + 1] - e0)
    return RowShard(lo, hi, e0, e1, torch.from_numpy(nodes).to(dev),
                    torch.from_numpy(lid[src].astype(np.int32)).to(dev),
                    None if val is None else val[e0:e1],
                    build_row_schedule(local_rp, device=dev, light_max=light, seg_edges=seg))


def _col_shard(colptr: np.ndarray, row: np.ndarray, perm: np.ndarray, lo: int, hi: int, light: int, seg_rows: int,
               seg_cols: int, dev) -> ColShard:
    n = colptr.shape[0] - 1
    c0, c1 = int(colptr[lo]), int(colptr[hi])
    dst, ids = row[c0:c1], perm[c0:c1]
    mark = np.zeros(n, dtype=bool)
    mark[lo:hi] = True
    mark[dst] = True
    nodes = np.flatnonzero(mark)
    lid = np.cumsum(mark, dtype=np.int64) - 1
    nl = nodes.shape[0]
    own = int(lid[lo])
    # CSC over the local nodes: only the own sources have entries.
    counts = np.zeros(nl, dtype=np.int64)
    counts[own:own + hi - lo] = np.diff(colptr[lo:hi + 1])
    l_colptr = np.concatenate([[0], np.cumsum(counts)])
    l_row = lid[dst]
    src_local = np.repeat(np.arange(own, own + hi - lo, dtype=np.int64), np.diff(colptr[lo:hi + 1]))
    # CSR in whole-graph edge order (rows ascend with the whole graph's ids)
    order = np.argsort(ids, kind="stable")
    l_rowptr = np.concatenate([[0], np.cumsum(np.bincount(l_row, minlength=nl))])
    l_col = src_local[order]
    l_perm = np.empty_like(order)
    l_perm[order] = np.arange(order.shape[0])
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a).astype(np.int32)).to(dev)
    return ColShard(lo, hi, own, torch.from_numpy(nodes).to(dev), i32(l_rowptr), i32(l_col), i32(l_colptr),
                    i32(l_row), i32(l_perm), torch.from_numpy(ids[order]).to(dev),
                    build_row_schedule(torch.from_numpy(l_rowptr), device=dev, light_max=light, seg_edges=seg_rows),
                    build_row_schedule(torch.from_numpy(l_colptr), device=dev, light_max=light, seg_edges=seg_cols))


def _geometry(sched: RowSchedule) -> tuple[int, int]:
    """(light_max, seg_edges) a schedule was built with (its header)."""
    return int(sched.header[4]), int(sched.header[3])


class ShardedGAT:
    """The collapsed GAT (cign_gat_fwd / cign_gat_bwd semantics) over the
    shards of `ranges`: forward per RowShard of the CSR, backward per ColShard
    of the CSC. gat_graph = ((rowptr, col), (row, colptr), perm) on the GPU,
    as prepare_fused_gat_graph returns it."""

    def __init__(self, gat_graph, ranges, heads: int, channels: int, dtype: torch.dtype = torch.float32):
        (rowptr, col), (row, colptr), perm = gat_graph
        self.gat_graph = gat_graph
        self.heads, self.channels, self.dtype = int(heads), int(channels), dtype
        self.code = _lib.dtype_code(torch.empty(0, dtype=dtype))
        self.n = int(rowptr.numel()) - 1
        self.nnz = int(col.numel())
        lib = _lib.load_library(require_gpu=False)
        if int(lib.cign_gat_row_agg_floats(self.code, 1, self.heads, self.channels)) == 0:
            raise RuntimeError(f"sharded GAT needs a feature-layout shape (per-row aggregates); H={heads} x "
                               f"C={channels} has none")
        dev = rowptr.device
        # The whole graph's schedules fix the geometry every shard uses.
        fl, fs = _geometry(gat_schedule(rowptr, 0, self.code, self.heads, self.channels))
        bl, brs = _geometry(gat_schedule(rowptr, 1, self.code, self.heads, self.channels))
        _, bcs = _geometry(gat_schedule(colptr, 1, self.code, self.heads, self.channels))
        rp, cl = _host_i64(rowptr), _host_i64(col)
        cp, rw, pm = _host_i64(colptr), _host_i64(row), _host_i64(perm)
        self.ranges = [(int(lo), int(hi)) for lo, hi in ranges]
        if not self.ranges or self.ranges[0][0] != 0 or self.ranges[-1][1] != self.n or any(
                a[1] != b[0] for a, b in zip(self.ranges, self.ranges[1:])):
            raise ValueError("shard ranges must cover [0, n) contiguously")
        self.row_shards = [_row_shard(rp, cl, None, lo, hi, fl, fs, dev) for lo, hi in self.ranges]
        self.col_shards = [_col_shard(cp, rw, pm, lo, hi, bl, brs, bcs, dev) for lo, hi in self.ranges]

    @property
    def info(self) -> dict:
        """Partition summary in the manner of ChunkedDgNNGraph.info
        (chunked_dgnn_gat.py:57-80)."""
        rs, cs = self.row_shards, self.col_shards
        return {
            "backend": "cign_amd row-nnz shards",
            "num_nodes": self.n,
            "num_edges": self.nnz,
            "num_chunks": len(rs),
            "max_local_nodes_observed": max(int(s.nodes.numel()) for s in rs),
            "total_local_node_references": sum(int(s.nodes.numel()) for s in rs),
            "total_real_edges": sum(s.e1 - s.e0 for s in rs),
            "chunks": [{"target_lo": s.lo, "target_hi": s.hi, "targets": s.hi - s.lo,
                        "local_nodes": int(s.nodes.numel()), "halo_nodes": s.halo, "real_edges": s.e1 - s.e0,
                        "backward_local_nodes": int(c.nodes.numel()), "backward_edges": c.nnz}
                       for s, c in zip(rs, cs)],
        }

    def forward(self, attn_row, attn_col, in_feat, bias, negative_slope: float, attn_drop: float, seed: int):
        """Outputs of cign_gat_fwd for the whole graph ([out, pre, edge_max,
        edge_sum, edge_mask], row_agg), computed shard by shard."""
        lib = _lib.load_library()
        n, H, C = self.n, self.heads, self.channels
        dev = in_feat.device
        out = torch.empty((n, C), dtype=in_feat.dtype, device=dev)
        pre = torch.empty((n, C), dtype=torch.float32, device=dev)
        emax = torch.empty((n, H), dtype=torch.float32, device=dev)
        esum = torch.empty((n, H), dtype=torch.float32, device=dev)
        mask = torch.empty((self.nnz, H), dtype=torch.uint8, device=dev)
        F = H * C
        agg = torch.empty(n * (2 * F + H), dtype=torch.float32, device=dev)
        a_s, a_l, a_b = agg[:n * F].view(n, F), agg[n * F:2 * n * F].view(n, F), agg[2 * n * F:].view(n, H)
        st = _lib.stream_ptr(dev)
        for s in self.row_shards:
            t = s.hi - s.lo
            if t == 0:
                continue
            # halo exchange: the shard's sources
            x_l = in_feat.index_select(0, s.nodes).contiguous()
            ac_l = attn_col.index_select(0, s.nodes).contiguous()
            agg_l = torch.empty(t * (2 * F + H), dtype=torch.float32, device=dev)
            ws_bytes = int(lib.cign_gat_fwd_workspace_bytes(s.sched.n_seg, H, C))
            ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
            lib.call("cign_gat_fwd_shard", st, self.code, t, s.e1 - s.e0, H, C, attn_row[s.lo:s.hi].data_ptr(),
                     ac_l.data_ptr(), s.col.data_ptr(), *s.sched.args(), s.sched.counters.data_ptr(),
                     float(negative_slope), x_l.data_ptr(), bias.data_ptr(), float(attn_drop),
                     int(seed) & ((1 << 64) - 1), out[s.lo:s.hi].data_ptr(), pre[s.lo:s.hi].data_ptr(),
                     emax[s.lo:s.hi].data_ptr(), esum[s.lo:s.hi].data_ptr(), mask[s.e0:s.e1].data_ptr(),
                     ws.data_ptr(), ws_bytes, agg_l.data_ptr(), s.e0, self.nnz)
            a_s[s.lo:s.hi].copy_(agg_l[:t * F].view(t, F))
            a_l[s.lo:s.hi].copy_(agg_l[t * F:2 * t * F].view(t, F))
            a_b[s.lo:s.hi].copy_(agg_l[2 * t * F:].view(t, H))
        return [out, pre, emax, esum, mask], agg

    def backward(self, negative_slope: float, attn_drop: float, edge_max, edge_sum, edge_mask, in_feat, attn_row,
                 attn_col, pre, grad_y, row_agg):
        """[grad_feat, grad_attn_row, grad_attn_col, grad_bias] of cign_gat_bwd
        for the whole graph, computed per source-column shard from the
        forward's per-row outputs (row_agg required)."""
        lib = _lib.load_library()
        n, H, C = self.n, self.heads, self.channels
        F = H * C
        dev = in_feat.device
        grad_feat = torch.empty_like(in_feat)
        grad_ar = torch.empty_like(attn_row)
        grad_ac = torch.empty_like(attn_col)
        bias_parts = torch.zeros((len(self.col_shards), C), dtype=torch.float32, device=dev)
        a_s, a_l = row_agg[:n * F].view(n, F), row_agg[n * F:2 * n * F].view(n, F)
        a_b = row_agg[2 * n * F:].view(n, H)
        st = _lib.stream_ptr(dev)
        for k, s in enumerate(self.col_shards):
            t = s.hi - s.lo
            if t == 0:
                continue
            nodes, nl = s.nodes, int(s.nodes.numel())
            g = lambda v: v.index_select(0, nodes).contiguous()
            agg_l = torch.cat([g(a_s).view(-1), g(a_l).view(-1), g(a_b).view(-1)])
            mask_l = edge_mask.index_select(0, s.csr_ids).contiguous()
            x_l, ar_l, ac_l, pre_l, gy_l = g(in_feat), g(attn_row), g(attn_col), g(pre), g(grad_y)
            em_l, es_l = g(edge_max), g(edge_sum)
            row_blocks = s.row_sched.n_seg + (s.row_sched.n_light + 3) // 4
            ws_bytes = int(lib.cign_gat_bwd_workspace_bytes(nl, s.nnz, H, C, row_blocks, s.row_sched.n_seg,
                                                            s.col_sched.n_seg))
            ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
            gf_l = torch.empty_like(x_l)
            gar_l, gac_l = torch.empty_like(ar_l), torch.empty_like(ac_l)
            lib.call("cign_gat_bwd_shard", st, self.code, nl, s.nnz, H, C, float(negative_slope), float(attn_drop),
                     s.col.data_ptr(), s.row.data_ptr(), s.perm.data_ptr(), em_l.data_ptr(), es_l.data_ptr(),
                     mask_l.data_ptr(), x_l.data_ptr(), ar_l.data_ptr(), ac_l.data_ptr(), pre_l.data_ptr(),
                     gy_l.data_ptr(), *s.row_sched.args(), s.row_sched.counters.data_ptr(), *s.col_sched.args(),
                     s.col_sched.counters.data_ptr(), ws.data_ptr(), ws_bytes, gf_l.data_ptr(), gar_l.data_ptr(),
                     gac_l.data_ptr(), bias_parts[k].data_ptr(), agg_l.data_ptr(), s.own, t, self.nnz)
            own = slice(s.own, s.own + t)
            grad_feat[s.lo:s.hi].copy_(gf_l[own])
            grad_ar[s.lo:s.hi].copy_(gar_l[own])
            grad_ac[s.lo:s.hi].copy_(gac_l[own])
        # sum over shards in shard order (the all-reduce of several GPUs)
        grad_bias = bias_parts[0].clone()
        for k in range(1, bias_parts.size(0)):
            grad_bias += bias_parts[k]
        return [grad_feat, grad_ar, grad_ac, grad_bias]


class ShardedMultiHop:
    """The 3-hop pipeline of MultiHopCsrPlan (forward3 / backward3: y_k =
    P y_(k-1); t2 = g2 + P^T g3, t1 = g1 + P^T t2, gx = P^T t1) over the
    shards of `ranges`: each hop runs per RowShard of P (forward) or P^T
    (backward) on the previous hop's rows gathered for the shard's halo.
    operator = FixedCSRGraphOperator on the GPU."""

    def __init__(self, operator, ranges, dense_cols: int):
        from .multihop_csr_pipeline import _csr_parts_int32
        from .schedule import LIGHT_MAX, segment_edges_for

        self.dense_cols = int(dense_cols)
        self.ranges = [(int(lo), int(hi)) for lo, hi in ranges]
        self.n = int(operator.shape[0])
        self.p_shards, self.pt_shards = [], []
        n_seg = 0
        for csr, dst in ((operator.csr, self.p_shards), (operator.csr_t, self.pt_shards)):
            crow, col, val = _csr_parts_int32(csr)
            # the whole operator's schedule geometry, as MultiHopCsrPlan builds it
            light, seg = LIGHT_MAX, segment_edges_for(int(col.numel()))
            rp, cl = _host_i64(crow), _host_i64(col)
            for lo, hi in self.ranges:
                sh = _row_shard(rp, cl, val.contiguous(), lo, hi, light, seg, crow.device)
                dst.append(sh)
                n_seg = max(n_seg, sh.sched.n_seg)
        lib = _lib.load_library(require_gpu=False)
        self._part_floats = max(1, int(lib.cign_spmm_partial_bytes(n_seg, self.dense_cols)) // 4) if n_seg else 1

    def _hop(self, shards, x, add, y, part):
        lib = _lib.load_library()
        st = _lib.stream_ptr(x.device)
        for s in shards:
            if s.hi == s.lo:
                continue
            x_l = x.index_select(0, s.nodes).contiguous()  # halo exchange
            lib.call("cign_spmm", st, _lib.dtype_code(x), s.hi - s.lo, self.dense_cols, s.col.data_ptr(),
                     s.val.data_ptr(), *s.sched.args(), x_l.data_ptr(),
                     None if add is None else add[s.lo:s.hi].data_ptr(), y[s.lo:s.hi].data_ptr(), part.data_ptr(),
                     s.sched.counters.data_ptr())

    def forward3(self, x):
        part = torch.empty(self._part_floats, dtype=torch.float32, device=x.device)
        y1, y2, y3 = (torch.empty_like(x) for _ in range(3))
        self._hop(self.p_shards, x, None, y1, part)
        self._hop(self.p_shards, y1, None, y2, part)
        self._hop(self.p_shards, y2, None, y3, part)
        return y1, y2, y3

    def backward3(self, g1, g2, g3):
        part = torch.empty(self._part_floats, dtype=torch.float32, device=g1.device)
        t2, t1, gx = (torch.empty_like(g1) for _ in range(3))
        self._hop(self.pt_shards, g3, g2, t2, part)
        self._hop(self.pt_shards, t2, g1, t1, part)
        self._hop(self.pt_shards, t1, None, gx, part)
        return gx


def prepare_sharded_gat_graph(gat_graph, heads: int, channels: int, dtype: torch.dtype = torch.float32,
                              max_local_nodes: int | None = 45000, target_chunk_nodes: int = 8192) -> ShardedGAT:
    """The partitioned GAT graph for `gat_graph` (prepare_fused_gat_graph's
    format on the GPU), with the knobs of prepare_chunked_dgnn_graph
    (chunked_dgnn_gat.py:104-110): ceil(n / target_chunk_nodes) shards,
    balanced by in- plus out-edges, each then halved until its local node set
    (rows, source halo and destination halo) is at most max_local_nodes."""
    (rowptr, col), (row, colptr), _ = gat_graph
    n = int(rowptr.numel()) - 1
    if target_chunk_nodes <= 0:
        raise ValueError("target_chunk_nodes must be positive")
    if max_local_nodes is not None and max_local_nodes <= 0:
        raise ValueError("max_local_nodes must be positive")
    shards = max(1, -(-n // int(target_chunk_nodes)))
    ranges = partition_rows([rowptr, colptr], shards, max_local_nodes, cols=[col, row])
    return ShardedGAT(gat_graph, ranges, heads, channels, dtype)


class _ShardedCollapsedGATFn(torch.autograd.Function):
    """_CollapsedGATFn (collapsed_gat.py:57-161) over a ShardedGAT."""

    @staticmethod
    def forward(ctx, attn_row, attn_col, in_feat, bias, sharded, negative_slope, attn_drop, seed):
        attn_row, attn_col = attn_row.contiguous(), attn_col.contiguous()
        in_feat, bias = in_feat.contiguous(), bias.contiguous()
        (y, pre, emax, esum, mask), agg = sharded.forward(attn_row, attn_col, in_feat, bias, negative_slope,
                                                          attn_drop, seed)
        ctx.save_for_backward(emax, esum, mask, in_feat, attn_row, attn_col, pre, agg)
        ctx.sharded = sharded
        ctx.negative_slope, ctx.attn_drop = float(negative_slope), float(attn_drop)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        emax, esum, mask, in_feat, attn_row, attn_col, pre, agg = ctx.saved_tensors
        gf, gar, gac, gb = ctx.sharded.backward(ctx.negative_slope, ctx.attn_drop, emax, esum, mask, in_feat,
                                                attn_row, attn_col, pre,
                                                grad_y.to(dtype=in_feat.dtype).contiguous(), agg)
        return gar, gac, gf, gb, None, None, None, None


def sharded_collapsed_gat_mean_bias_silu(attn_row: torch.Tensor, attn_col: torch.Tensor, sharded: ShardedGAT,
                                         negative_slope: float, in_feat: torch.Tensor, bias: torch.Tensor,
                                         attn_drop: float) -> torch.Tensor:
    """collapsed_gat_mean_bias_silu run shard by shard over `sharded` (the
    same dropout seeds: one shared call counter)."""
    from .collapsed_gat import next_seed

    if in_feat.dim() != 3 or int(in_feat.size(1)) != sharded.heads or int(in_feat.size(2)) != sharded.channels:
        raise ValueError(f"in_feat must be [N,{sharded.heads},{sharded.channels}] for this sharded graph, got "
                         f"{tuple(in_feat.shape)}")
    if in_feat.dtype != sharded.dtype or int(in_feat.size(0)) != sharded.n:
        raise ValueError(f"in_feat must be {sharded.dtype} with {sharded.n} rows for this sharded graph")
    if bias is None:
        raise ValueError("collapsed GAT currently requires bias=True")
    return _ShardedCollapsedGATFn.apply(attn_row, attn_col, in_feat, bias, sharded, float(negative_slope),
                                        float(attn_drop), next_seed(attn_drop))
