"""CPU oracle for the CIGN sparse message-passing hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (``cign_amd``) imports this
module; only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` use it, and only as the checker (or the timed CPU
baseline), never as a code path of the product.

Every function is a numpy restatement (float64 by default) of the reference
algorithm, citing the reference file:line it follows. Backward formulas are
written out explicitly from the reference kernels (not by autograd) so that
the tests can pin them independently against finite differences of the
forward. Integer work (CSR/CSC/perm, dropout bits) is exact.

Parity status of each function is stated in its docstring ("pinned by ...").
"""
from __future__ import annotations

import numpy as np
import scipy.sparse as sp

NEG_BIG = -1.0e38  # initial running max of the reference (collapsed_gat_cuda.cu:87)

# ---------------------------------------------------------------------------
# splitmix64 dropout bits
# ---------------------------------------------------------------------------
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_IDX_MUL = np.uint64(0xD2B74407B1CE6E93)


def splitmix64(x: np.ndarray) -> np.ndarray:
    """splitmix64 finaliser, collapsed_gat_cuda.cu:27-32 and
    fused_block_ops_ext/fused_block_ops_cuda.cu:14-19 (Vigna's public-domain
    generator). Pinned by Vigna's published output sequence (tests)."""
    x = np.asarray(x, dtype=np.uint64)
    with np.errstate(over="ignore"):
        x = x + _GOLDEN
        x = (x ^ (x >> np.uint64(30))) * _M1
        x = (x ^ (x >> np.uint64(27))) * _M2
        return x ^ (x >> np.uint64(31))


def gat_dropout_keep(seed: int, total: int, p: float) -> np.ndarray:
    """Keep bits [total] of the collapsed-GAT edge dropout,
    collapsed_gat_cuda.cu:34-47: u = ((r >> 32) + 0.5f) * 2^-32 in float32,
    keep = u > p (p as float32). Index = csr_edge * H + head."""
    idx = np.arange(total, dtype=np.uint64)
    with np.errstate(over="ignore"):
        r = splitmix64(np.uint64(seed) ^ (idx * _IDX_MUL))
    hi = (r >> np.uint64(32)).astype(np.uint32)
    u = (hi.astype(np.float32) + np.float32(0.5)) * np.float32(2.3283064365386963e-10)
    return u > np.float32(p)


def block_dropout_keep(seed: int, total: int, p: float) -> np.ndarray:
    """Keep bits of the block ops (dropout-LN, gamma residual),
    fused_block_ops_ext/fused_block_ops_cuda.cu:20-26: 53-bit uniform in
    double, keep = u >= (double)(float)p; p <= 0 keeps everything."""
    if float(np.float32(p)) <= 0.0:
        return np.ones(total, dtype=bool)
    idx = np.arange(total, dtype=np.uint64)
    with np.errstate(over="ignore"):
        r = splitmix64(np.uint64(seed) ^ (idx * _IDX_MUL))
    u = (r >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    return u >= float(np.float32(p))


def collapsed_gat_seed(initial_seed: int, call_id: int, attn_drop: float) -> int:
    """Per-call dropout seed of collapsed_gat_mean_bias_silu,
    collapsed_gat.py:204-211 (call_id = value of the module call counter)."""
    if float(attn_drop) <= 0.0:
        return 0
    base = int(initial_seed) & ((1 << 63) - 1)
    return (base + 0x9E3779B97F4A7C15 * (call_id + 1)) & ((1 << 63) - 1)


def block_ops_seed(initial_seed: int, call: int, tag: int, dropout_p: float) -> int:
    """fused_block_ops.py:46-50 (call = counter value + 1)."""
    if float(dropout_p) <= 0.0:
        return 0
    base = int(initial_seed) & ((1 << 63) - 1)
    return (base + 0x9E3779B97F4A7C15 * call + 0xD2B74407B1CE6E93 * int(tag)) & ((1 << 63) - 1)


# ---------------------------------------------------------------------------
# Graph preparation
# ---------------------------------------------------------------------------
def coalesce(row: np.ndarray, col: np.ndarray, n: int, values: np.ndarray | None = None):
    """Sort by (row, col) and merge duplicates (summing values), the
    semantics of torch COO .coalesce() / PyG coalesce used at
    generic_engine/train_cign.py:1572,1587 and model.py:161,183."""
    key = row.astype(np.int64) * n + col.astype(np.int64)
    order = np.argsort(key, kind="stable")
    key = key[order]
    uniq, start = np.unique(key, return_index=True)
    r = (uniq // n).astype(np.int64)
    c = (uniq % n).astype(np.int64)
    if values is None:
        return r, c, None
    v = np.add.reduceat(values[order], start) if len(key) else values[:0]
    return r, c, v


def normalized_adjacency(edge_index: np.ndarray, n: int, use_undirected: bool = True,
                         add_self_loop: bool = True):
    """P = D^-1/2 (A + I) D^-1/2, generic_engine/train_cign.py:1558-1590:
    to_undirected (coalesced), append one self-loop per node, deg = count of
    col entries (float32), clamp(min=1).pow(-0.5), w = dis[row] * dis[col]
    (float32), then COO coalesce (duplicates summed). Returns
    (edge_index_used [2,E'], P as (row, col, val float32), coalesced)."""
    row, col = edge_index[0].astype(np.int64), edge_index[1].astype(np.int64)
    if use_undirected:
        r2 = np.concatenate([row, col])
        c2 = np.concatenate([col, row])
        row, col, _ = coalesce(r2, c2, n)
    if add_self_loop:
        loop = np.arange(n, dtype=np.int64)
        row = np.concatenate([row, loop])
        col = np.concatenate([col, loop])
    deg = np.bincount(col, minlength=n).astype(np.float32)
    # torch's float32 pow(x, -0.5) is evaluated as 1 / sqrt(x) with two float32
    # roundings (not a correctly rounded rsqrt); restated exactly.
    dis = (np.float32(1.0) / np.sqrt(np.maximum(deg, np.float32(1.0)))).astype(np.float32)
    w = (dis[row] * dis[col]).astype(np.float32)
    pr, pc, pv = coalesce(row, col, n, w)
    return np.stack([row, col]), (pr, pc, pv.astype(np.float32))


def normalized_laplacian(edge_index: np.ndarray, n: int, use_undirected: bool = True):
    """L = I - D^-1/2 A D^-1/2, generic_engine/train_cign.py:1518-1555 with
    PyG get_laplacian(normalization="sym"): to_undirected (coalesced), self
    loops dropped, deg = count of row entries (float32), deg^-1/2 (0 for
    isolated nodes), off-diagonal -dis[row] * dis[col] (float32), a unit
    diagonal appended, COO coalesce. Returns (edge_index_used, L as (row,
    col, val float32)). Pinned by a dense float64 construction, L sqrt(deg)
    = 0 and the spectrum in [0, 2] (tests)."""
    row, col = edge_index[0].astype(np.int64), edge_index[1].astype(np.int64)
    if use_undirected:
        row, col, _ = coalesce(np.concatenate([row, col]), np.concatenate([col, row]), n)
    used = np.stack([row, col])
    keep = row != col
    r, c = row[keep], col[keep]
    deg = np.bincount(r, minlength=n).astype(np.float32)
    with np.errstate(divide="ignore"):
        dis = (np.float32(1.0) / np.sqrt(deg)).astype(np.float32)
    dis[deg == 0] = 0.0
    off = -(dis[r] * dis[c]).astype(np.float32)
    loop = np.arange(n, dtype=np.int64)
    lr, lc, lv = coalesce(np.concatenate([r, loop]), np.concatenate([c, loop]), n,
                          np.concatenate([off, np.ones(n, np.float32)]))
    return used, (lr, lc, lv.astype(np.float32))


def roc_auc_pairs(y_true: np.ndarray, score: np.ndarray) -> float:
    """ROC AUC by its definition: the fraction of (positive, negative) pairs
    ranked correctly, ties counted half (the quantity
    generic_engine/train_cign.py:1810 takes from sklearn). O(P*N): small
    inputs only."""
    y_true = np.asarray(y_true)
    pos = score[y_true == y_true.max()].astype(np.float64)
    neg = score[y_true != y_true.max()].astype(np.float64)
    d = pos[:, None] - neg[None, :]
    return float(((d > 0).sum() + 0.5 * (d == 0).sum()) / d.size)


def gat_edge_index(edge_index: np.ndarray, n: int) -> np.ndarray:
    """remove_self_loops + add_self_loops, generic_engine/train_cign.py:1759-1771."""
    row, col = edge_index[0].astype(np.int64), edge_index[1].astype(np.int64)
    keep = row != col
    loop = np.arange(n, dtype=np.int64)
    return np.stack([np.concatenate([row[keep], loop]), np.concatenate([col[keep], loop])])


def csr_from_coo(row: np.ndarray, col: np.ndarray, n: int):
    """Row pointer / column index of edges sorted by (row, col) (stable for
    duplicates). Returns (rowptr int64 [n+1], col int64 [E], order [E]) with
    order[k] = input position of the k-th CSR entry."""
    key = row.astype(np.int64) * n + col.astype(np.int64)
    order = np.argsort(key, kind="stable")
    rowptr = np.zeros(n + 1, dtype=np.int64)
    np.add.at(rowptr, row[order] + 1, 1)
    return np.cumsum(rowptr), col[order].astype(np.int64), order


def gat_graph_format(edge_index: np.ndarray, n: int):
    """CSR by destination / CSC by source / perm, the graph format consumed by
    the collapsed GAT (generic_engine/model_cign.py:1117-1133: edge_index is
    flipped to target->source, then the fused-GAT graph format is built).
    Canonical definition: CSR entries sorted by (dst, src); CSC entries
    sorted by (src, dst); perm[k] = CSR index of the k-th CSC entry
    (consumed at collapsed_gat_cuda.cu:247). Returns int64 arrays
    (rowptr, col, row, colptr, perm)."""
    src, dst = edge_index[0].astype(np.int64), edge_index[1].astype(np.int64)
    rowptr, col, order_csr = csr_from_coo(dst, src, n)
    colptr, row, order_csc = csr_from_coo(src, dst, n)
    pos_in_csr = np.empty(len(order_csr), dtype=np.int64)
    pos_in_csr[order_csr] = np.arange(len(order_csr))
    perm = pos_in_csr[order_csc]
    return rowptr, col, row, colptr, perm


def transpose_csr(rowptr: np.ndarray, col: np.ndarray, val: np.ndarray, n: int):
    """CSR of P^T by index flip + coalesce, model.py:176-184."""
    rows = np.repeat(np.arange(n, dtype=np.int64), np.diff(rowptr))
    tr, tc, tv = coalesce(col, rows, n, val)
    rp = np.zeros(n + 1, dtype=np.int64)
    np.add.at(rp, tr + 1, 1)
    return np.cumsum(rp), tc, tv


# ---------------------------------------------------------------------------
# SpMM / multihop
# ---------------------------------------------------------------------------
def csr_matrix(rowptr, col, val, n, dtype=np.float64):
    return sp.csr_matrix((np.asarray(val, dtype=dtype), np.asarray(col), np.asarray(rowptr)), shape=(n, n))


def spmm(rowptr, col, val, x, add=None):
    """y = P x (+ add): cusparseSpMM at multihop_csr_pipeline_cuda.cu:264-285
    and torch.sparse.mm at model.py:91. Pinned by dense matmul and the
    circulant known answer of validate_a3v5.py:11-19 (tests)."""
    n = len(rowptr) - 1
    y = csr_matrix(rowptr, col, val, n, dtype=np.float64) @ np.asarray(x, dtype=np.float64)
    return y if add is None else y + add


def multihop3_forward(p_csr, x):
    """forward3, multihop_csr_pipeline_cuda.cu:287-297: y1=Px, y2=Py1, y3=Py2."""
    y1 = spmm(*p_csr, x)
    y2 = spmm(*p_csr, y1)
    y3 = spmm(*p_csr, y2)
    return y1, y2, y3


def multihop3_backward(pt_csr, g1, g2, g3):
    """backward3, multihop_csr_pipeline_cuda.cu:307-320:
    t2 = g2 + P^T g3, t1 = g1 + P^T t2, gx = P^T t1. Pinned by the adjoint
    identity against multihop3_forward (tests)."""
    t2 = spmm(*pt_csr, g3, add=g2)
    t1 = spmm(*pt_csr, t2, add=g1)
    return spmm(*pt_csr, t1)


def multihop_generic_forward(p_csr, x, powers):
    """GenericMultiHopCSRFunction.forward, multihop_csr_pipeline.py:235-246."""
    wanted = sorted(set(int(p) for p in powers if int(p) > 0))
    out, cur = {}, np.asarray(x, dtype=np.float64)
    for p in range(1, (max(wanted) if wanted else 0) + 1):
        cur = spmm(*p_csr, cur)
        if p in wanted:
            out[p] = cur
    return out


def multihop_generic_backward(pt_csr, grads: dict, max_power: int, shape):
    """GenericMultiHopCSRFunction.backward, multihop_csr_pipeline.py:249-265:
    acc = 0; for p = K..1: acc += g_p; acc = P^T acc."""
    acc = np.zeros(shape, dtype=np.float64)
    for p in range(max_power, 0, -1):
        if p in grads and grads[p] is not None:
            acc = acc + grads[p]
        acc = spmm(*pt_csr, acc)
    return acc


# ---------------------------------------------------------------------------
# Collapsed GAT
# ---------------------------------------------------------------------------
def _leaky(x, slope):
    return np.where(x > 0, x, x * slope)


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _silu_grad(x):
    s = 1.0 / (1.0 + np.exp(-x))
    return s * (1.0 + x * (1.0 - s))


def _segment_reduce(ufunc, values, rowptr, empty):
    """Row-wise reduce of CSR-ordered values [E, ...] -> [N, ...]."""
    n = len(rowptr) - 1
    out = np.full((n,) + values.shape[1:], empty, dtype=values.dtype)
    nonempty = np.nonzero(np.diff(rowptr) > 0)[0]
    if len(nonempty):
        out[nonempty] = ufunc.reduceat(values, rowptr[:-1][nonempty], axis=0)
    return out


def gat_softmax(attn_row, attn_col, rowptr, col, slope):
    """Per-destination edge softmax of the collapsed GAT,
    collapsed_gat_cuda.cu:84-131: raw = attn_row[i] + attn_col[j],
    sc = LeakyReLU(raw), max over in-edges (empty rows: -1e38), sum of
    exp(sc - max). Returns (raw [E,H], soft [E,H], emax [N,H], esum [N,H])."""
    n = len(rowptr) - 1
    rows = np.repeat(np.arange(n), np.diff(rowptr))
    raw = attn_row[rows] + attn_col[col]
    sc = _leaky(raw, slope)
    emax = _segment_reduce(np.maximum, sc, rowptr, NEG_BIG)
    ex = np.exp(sc - emax[rows])
    esum = _segment_reduce(np.add, ex, rowptr, 0.0)
    denom = esum[rows]
    soft = np.where(denom > 0, ex / np.where(denom > 0, denom, 1.0), 0.0)
    return raw, soft, emax, esum


def _edge_weights(soft, keep, p):
    """w = s * keep / (1 - p) (p > 0), collapsed_gat_cuda.cu:140-146."""
    if p > 0:
        return np.where(keep, soft / (1.0 - p), 0.0)
    return soft


def collapsed_gat_forward(attn_row, attn_col, rowptr, col, slope, x, bias, p=0.0, keep=None):
    """Collapsed GAT forward, collapsed_gat_cuda.cu:52-174 (semantics of
    collapsed_gat.py:164-225 / dgNN GATConvFuse(...).mean(1) + bias -> SiLU).
    x [N,H,C], attn_* [N,H], keep [E,H] bool (dropout mask, CSR order).
    Returns dict(out, pre, emax, esum). Pinned by: finite differences (its
    backward), degree-1 / uniform-score closed forms, the dense textbook GAT
    (H=1) and brute-force loops (tests)."""
    x = np.asarray(x, dtype=np.float64)
    n, H, C = x.shape
    raw, soft, emax, esum = gat_softmax(np.asarray(attn_row, np.float64), np.asarray(attn_col, np.float64),
                                        rowptr, col, slope)
    w = _edge_weights(soft, keep, p)
    agg = np.zeros((n, C), dtype=np.float64)
    for h in range(H):
        W = sp.csr_matrix((w[:, h], col, rowptr), shape=(n, n))
        agg += W @ x[:, h, :]
    pre = agg / H + np.asarray(bias, dtype=np.float64)
    return {"out": _silu(pre), "pre": pre, "emax": emax, "esum": esum}


def collapsed_gat_backward(attn_row, attn_col, rowptr, col, slope, x, bias, grad_y, p=0.0, keep=None):
    """Collapsed GAT backward, the reference kernels restated in order:
    grad_pre (collapsed_gat_cuda.cu:176-186), grad_bias (:188-206),
    grad_feat by CSC walk (:211-277) written here as W_h^T g_pre / H,
    grad_edge SDDMM (:295-359), softmax + LeakyReLU backward with
    grad_attn_row / grad_attn_col (:362-430). Returns dict(grad_feat,
    grad_attn_row, grad_attn_col, grad_bias, grad_pre, grad_raw)."""
    x = np.asarray(x, dtype=np.float64)
    n, H, C = x.shape
    raw, soft, emax, esum = gat_softmax(np.asarray(attn_row, np.float64), np.asarray(attn_col, np.float64),
                                        rowptr, col, slope)
    w = _edge_weights(soft, keep, p)
    agg = np.zeros((n, C))
    for h in range(H):
        agg += sp.csr_matrix((w[:, h], col, rowptr), shape=(n, n)) @ x[:, h, :]
    pre = agg / H + np.asarray(bias, dtype=np.float64)
    g_pre = np.asarray(grad_y, dtype=np.float64) * _silu_grad(pre)
    g_bias = g_pre.sum(axis=0)
    rows = np.repeat(np.arange(n), np.diff(rowptr))
    g_feat = np.zeros_like(x)
    g_edge = np.zeros((len(col), H))
    for h in range(H):
        W = sp.csr_matrix((w[:, h], col, rowptr), shape=(n, n))
        g_feat[:, h, :] = (W.T @ g_pre) / H
        g_edge[:, h] = np.einsum("ec,ec->e", g_pre[rows], x[col, h, :]) / H
    if p > 0:
        ge = np.where(keep, g_edge, 0.0) / (1.0 - p)
    else:
        ge = g_edge
    wsum = _segment_reduce(np.add, soft * ge, rowptr, 0.0)
    g_sc = soft * (ge - wsum[rows])
    g_raw = np.where(raw < 0, g_sc * slope, g_sc)
    g_row = _segment_reduce(np.add, g_raw, rowptr, 0.0)
    g_col = np.zeros((n, H))
    np.add.at(g_col, col, g_raw)
    return {"grad_feat": g_feat, "grad_attn_row": g_row, "grad_attn_col": g_col, "grad_bias": g_bias,
            "grad_pre": g_pre, "grad_raw": g_raw}


def _sub_rows(rowptr, rows):
    """Row pointer [len(rows)+1] and CSR edge ids of the given rows."""
    rows = np.asarray(rows, dtype=np.int64)
    deg = rowptr[rows + 1] - rowptr[rows]
    sub = np.zeros(len(rows) + 1, dtype=np.int64)
    sub[1:] = np.cumsum(deg)
    start = np.repeat(rowptr[rows] - sub[:-1], deg)
    return sub, start + np.arange(sub[-1], dtype=np.int64)


def _rows_softmax_agg(attn_row, attn_col, rowptr, col, slope, x, rows):
    """Softmax statistics and the aggregates sum_e s x[j] and sum_e s l' x[j]
    ([R,H,C]) of the given destination rows, over their complete in-edge
    lists, with the edge arrays of those rows only (no [E,C] gathers)."""
    x = np.asarray(x, dtype=np.float64)
    n, H, C = x.shape
    sub, eid = _sub_rows(rowptr, rows)
    cols = np.asarray(col, dtype=np.int64)[eid]
    ar = np.asarray(attn_row, np.float64)[np.asarray(rows, dtype=np.int64)]
    # Local destinations 0..R-1 over the sources' global ids.
    raw, soft, emax, esum = gat_softmax(ar, np.asarray(attn_col, np.float64), sub, cols, slope)
    lp = np.where(raw < 0, slope, 1.0)
    R = len(sub) - 1
    agg = np.zeros((R, H, C))
    agg_l = np.zeros((R, H, C))
    for h in range(H):
        agg[:, h, :] = sp.csr_matrix((soft[:, h], cols, sub), shape=(R, n)) @ x[:, h, :]
        agg_l[:, h, :] = sp.csr_matrix((soft[:, h] * lp[:, h], cols, sub), shape=(R, n)) @ x[:, h, :]
    return dict(sub=sub, cols=cols, raw=raw, soft=soft, lp=lp, emax=emax, esum=esum, agg=agg, agg_l=agg_l)


def collapsed_gat_forward_rows(attn_row, attn_col, rowptr, col, slope, x, bias, rows):
    """collapsed_gat_forward (p = 0) evaluated at the given destination rows
    only: each row's output needs only its own in-edges, so the cost is that
    of those rows' edges (for full-size graphs). Returns dict(out, pre, emax,
    esum) of shape [len(rows), ...]. Pinned against collapsed_gat_forward on
    graphs with hubs and empty rows (tests)."""
    H = np.asarray(x).shape[1]
    r = _rows_softmax_agg(attn_row, attn_col, rowptr, col, slope, x, rows)
    pre = r["agg"].sum(axis=1) / H + np.asarray(bias, dtype=np.float64)
    return {"out": _silu(pre), "pre": pre, "emax": r["emax"], "esum": r["esum"]}


def collapsed_gat_backward_columns(attn_row, attn_col, rowptr, col, slope, x, bias, grad_y, cols):
    """collapsed_gat_backward (p = 0) evaluated at the given source columns:
    grad_feat and grad_attn_col of those columns, plus grad_attn_row and
    grad_pre of every destination row that reads one of them. The rows that
    read a column are found by scanning `col`; their complete in-edge lists
    give the softmax, pre and grad_pre; then, with g = grad_pre[i],
      wsum[i,h]  = <g, sum_e s x[j_e,h]>/H,
      g_raw[e,h] = l'_e s_e (<g, x[j_e,h]>/H - wsum[i,h]),
      grad_attn_row[i,h] = <g, sum_e s l' x[j_e,h]>/H - wsum[i,h] sum_e s l',
    and each requested column sums s g/H (grad_feat) and g_raw (grad_attn_col)
    over its edges. Returns dict(cols, grad_feat [J,H,C], grad_attn_col [J,H],
    rows, grad_attn_row [R,H], grad_pre [R,C]). Pinned against
    collapsed_gat_backward on graphs with hubs and empty rows (tests)."""
    x = np.asarray(x, dtype=np.float64)
    n, H, C = x.shape
    cols = np.asarray(cols, dtype=np.int64)
    col = np.asarray(col, dtype=np.int64)
    want = np.zeros(n, dtype=bool)
    want[cols] = True
    all_rows = np.repeat(np.arange(n, dtype=np.int64), np.diff(rowptr))
    rows = np.unique(all_rows[want[col]])
    r = _rows_softmax_agg(attn_row, attn_col, rowptr, col, slope, x, rows)
    pre = r["agg"].sum(axis=1) / H + np.asarray(bias, dtype=np.float64)
    g_pre = np.asarray(grad_y, dtype=np.float64)[rows] * _silu_grad(pre)
    wsum = np.einsum("rc,rhc->rh", g_pre, r["agg"]) / H
    b_l = _segment_reduce(np.add, r["soft"] * r["lp"], r["sub"], 0.0)
    g_row = np.einsum("rc,rhc->rh", g_pre, r["agg_l"]) / H - wsum * b_l
    # Edges of those rows whose source is a requested column.
    local = np.repeat(np.arange(len(rows), dtype=np.int64), np.diff(r["sub"]))
    hit = np.nonzero(want[r["cols"]])[0]
    ei, ej = local[hit], r["cols"][hit]
    s, lp = r["soft"][hit], r["lp"][hit]
    dot = np.einsum("ec,ehc->eh", g_pre[ei], x[ej]) / H
    g_raw = lp * s * (dot - wsum[ei])
    slot = np.searchsorted(np.sort(cols), ej)
    order = np.argsort(cols)
    g_feat = np.zeros((len(cols), H, C))
    g_col = np.zeros((len(cols), H))
    np.add.at(g_feat, order[slot], s[:, :, None] * g_pre[ei][:, None, :] / H)
    np.add.at(g_col, order[slot], g_raw)
    return {"cols": cols, "grad_feat": g_feat, "grad_attn_col": g_col, "rows": rows, "grad_attn_row": g_row,
            "grad_pre": g_pre}


def spmm_rows(rowptr, col, val, x, rows, add=None):
    """Rows `rows` of spmm(rowptr, col, val, x, add) from those rows' edges."""
    sub, eid = _sub_rows(rowptr, rows)
    n_src = np.asarray(x).shape[0]
    m = sp.csr_matrix((np.asarray(val, np.float64)[eid], np.asarray(col, np.int64)[eid], sub),
                      shape=(len(sub) - 1, n_src))
    y = m @ np.asarray(x, dtype=np.float64)
    return y if add is None else y + np.asarray(add, np.float64)[np.asarray(rows, dtype=np.int64)]


def collapsed_gat_row_aggregates(attn_row, attn_col, rowptr, col, slope, x, p=0.0, keep=None):
    """Per-destination-row aggregates the feature-layout forward saves for its
    backward (no reference counterpart; they regroup the sums of
    collapsed_gat_cuda.cu:295-430): with w = s * keep/(1-p) and l' the
    LeakyReLU slope of the raw score,
      agg[i,h]   = sum_e w x[j_e,h],   agg_l[i,h] = sum_e w l' x[j_e,h],
      b_l[i,h]   = sum_e s l'.
    Then <g_pre[i], agg_l[i,h]>/H - <g_pre[i], agg[i,h]>/H * b_l[i,h] is
    grad_attn_row[i,h] of collapsed_gat_backward (pinned in tests)."""
    x = np.asarray(x, dtype=np.float64)
    n, H, C = x.shape
    raw, soft, _, _ = gat_softmax(np.asarray(attn_row, np.float64), np.asarray(attn_col, np.float64),
                                  rowptr, col, slope)
    w = _edge_weights(soft, keep, p)
    lp = np.where(raw < 0, slope, 1.0)
    agg = np.zeros((n, H, C))
    agg_l = np.zeros((n, H, C))
    for h in range(H):
        agg[:, h, :] = sp.csr_matrix((w[:, h], col, rowptr), shape=(n, n)) @ x[:, h, :]
        agg_l[:, h, :] = sp.csr_matrix((w[:, h] * lp[:, h], col, rowptr), shape=(n, n)) @ x[:, h, :]
    b_l = _segment_reduce(np.add, soft * lp, rowptr, 0.0)
    return {"agg": agg, "agg_l": agg_l, "b_l": b_l}


# ---------------------------------------------------------------------------
# GAT side ops
# ---------------------------------------------------------------------------
def attention_logits_forward(x, att_src, att_dst):
    """alpha_src[n,h] = <x[n,h,:], att_src[h,:]>, likewise alpha_dst,
    fused_gat_sideops_cuda.cu:25-60 (att tensors [1,H,C])."""
    x = np.asarray(x, np.float64)
    return (np.einsum("nhc,hc->nh", x, np.asarray(att_src, np.float64).reshape(x.shape[1:])),
            np.einsum("nhc,hc->nh", x, np.asarray(att_dst, np.float64).reshape(x.shape[1:])))


def attention_logits_backward(grad_src, grad_dst, x, att_src, att_dst):
    """fused_gat_sideops_cuda.cu:65-167: g_x = gs*att_src + gd*att_dst;
    g_att[h,c] = sum_n g*x (returned as [1,H,C])."""
    x = np.asarray(x, np.float64)
    H, C = x.shape[1:]
    a_s = np.asarray(att_src, np.float64).reshape(H, C)
    a_d = np.asarray(att_dst, np.float64).reshape(H, C)
    gs = np.asarray(grad_src, np.float64)
    gd = np.asarray(grad_dst, np.float64)
    gx = gs[:, :, None] * a_s[None] + gd[:, :, None] * a_d[None]
    return gx, np.einsum("nh,nhc->hc", gs, x)[None], np.einsum("nh,nhc->hc", gd, x)[None]


def head_silu_forward(out, bias):
    """fused_gat_sideops_cuda.cu:171-195: pre = mean_h out + bias, y = SiLU(pre)."""
    out = np.asarray(out, np.float64)
    pre = out.mean(axis=1) + np.asarray(bias, np.float64)
    return _silu(pre), pre


def head_silu_backward(grad_y, pre, heads):
    """fused_gat_sideops_cuda.cu:197-239: g_out[n,h,c] = g*SiLU'(pre)/H, g_bias = sum_n."""
    gp = np.asarray(grad_y, np.float64) * _silu_grad(np.asarray(pre, np.float64))
    return np.repeat((gp / heads)[:, None, :], heads, axis=1), gp.sum(axis=0)


# ---------------------------------------------------------------------------
# Clifford packs
# ---------------------------------------------------------------------------
def _dw(bhr, brh, interaction):
    """compute_dw, generic_engine/fused_clifford_cign_pack_ext/
    fused_clifford_switch_pack_cuda.cu:22-58 (interaction 0 = old, 1 = new,
    2 = new with tanh, the switch_pack_ext variant at :48,51). Returns
    D, W and their partials wrt bhr, brh."""
    if interaction == 0:
        D = _silu(bhr)
        W = bhr - brh
        return D, W, _silu_grad(bhr), np.zeros_like(bhr), np.ones_like(bhr), -np.ones_like(bhr)
    sym = 0.5 * (bhr + brh)
    anti = 0.5 * (bhr - brh)
    D = _silu(sym)
    dsym = _silu_grad(sym)
    if interaction == 2:
        W = np.tanh(anti)
        dw = 1.0 - W * W
    else:
        W = anti
        dw = np.ones_like(anti)
    return D, W, 0.5 * dsym, 0.5 * dsym, 0.5 * dw, -0.5 * dw


def clifford_pack_forward(H, C, props, alpha, interaction=0, weighting=0):
    """Clifford pack forward for K hops. interaction 0 (old, A3
    fused_clifford_pack_cuda.cu:22-56 and the generic-K old kernel
    fused_clifford_pack.py:88-98), 1 (new, CIGN pack
    generic_engine/fused_clifford_cign_pack_ext/...cuda.cu:65-179 and
    generic_engine/fused_clifford_cign_generic.py:58-68), 2 (new + tanh,
    fused_clifford_switch_pack_ext). T_H = P_k[:, :D], T_C = P_k[:, D:];
    bhr = H*T_C, brh = C*T_H. weighting 0 -> [N, K*2D] = cat_k(a_k W_k,
    a_k D_k); 1 -> [N, 2D] = [sum a_k D_k, sum a_k W_k] (D first)."""
    H = np.asarray(H, np.float64)
    C = np.asarray(C, np.float64)
    D = H.shape[1]
    A = np.asarray(alpha, np.float64).reshape(H.shape[0], len(props))
    outs, Dagg, Wagg = [], 0.0, 0.0
    for k, P in enumerate(props):
        P = np.asarray(P, np.float64)
        th, tc = P[:, :D], P[:, D:]
        Dv, Wv, *_ = _dw(H * tc, C * th, interaction)
        a = A[:, k:k + 1]
        outs += [a * Wv, a * Dv]
        Dagg = Dagg + a * Dv
        Wagg = Wagg + a * Wv
    if weighting == 0:
        return np.concatenate(outs, axis=1)
    return np.concatenate([Dagg, Wagg], axis=1)


def clifford_pack_backward(grad_out, H, C, props, alpha, interaction=0, weighting=0):
    """Explicit backward of clifford_pack_forward, following
    backward_main_kernel / backward_alpha_kernel
    (generic_engine/fused_clifford_cign_pack_ext/...cuda.cu:186-368).
    Returns (gH, gC, [gP_k], gA)."""
    H = np.asarray(H, np.float64)
    C = np.asarray(C, np.float64)
    G = np.asarray(grad_out, np.float64)
    n, D = H.shape
    K = len(props)
    A = np.asarray(alpha, np.float64).reshape(n, K)
    gH = np.zeros_like(H)
    gC = np.zeros_like(C)
    gP, gA = [], np.zeros((n, K))
    for k, P in enumerate(props):
        P = np.asarray(P, np.float64)
        th, tc = P[:, :D], P[:, D:]
        bhr, brh = H * tc, C * th
        Dv, Wv, dD_bhr, dD_brh, dW_bhr, dW_brh = _dw(bhr, brh, interaction)
        a = A[:, k:k + 1]
        if weighting == 0:
            goW = G[:, k * 2 * D:k * 2 * D + D]
            goD = G[:, k * 2 * D + D:(k + 1) * 2 * D]
        else:
            goD = G[:, :D]
            goW = G[:, D:]
        gD, gW = goD * a, goW * a
        gbhr = gD * dD_bhr + gW * dW_bhr
        gbrh = gD * dD_brh + gW * dW_brh
        gH += gbhr * tc
        gC += gbrh * th
        gP.append(np.concatenate([gbrh * C, gbhr * H], axis=1))
        gA[:, k] = (goW * Wv + goD * Dv).sum(axis=1)
    return gH, gC, gP, gA


# ---------------------------------------------------------------------------
# Block ops
# ---------------------------------------------------------------------------
def dropout_layernorm_forward(x, w, b, p, eps, keep):
    """fused_block_ops_cuda.cu:45-70: q = keep*x/(1-p); LayerNorm(q)."""
    x = np.asarray(x, np.float64)
    scale = 1.0 / (1.0 - p) if p > 0 else 1.0
    q = np.where(keep, x * scale, 0.0)
    mu = q.mean(axis=1, keepdims=True)
    var = ((q - mu) ** 2).mean(axis=1, keepdims=True)
    rs = 1.0 / np.sqrt(var + eps)
    return (q - mu) * rs * w + b, mu[:, 0], rs[:, 0]


def dropout_layernorm_backward(gy, x, w, p, eps, keep):
    """fused_block_ops_cuda.cu:96-118 + param stage 1/2: dx, dw, db."""
    x = np.asarray(x, np.float64)
    gy = np.asarray(gy, np.float64)
    scale = 1.0 / (1.0 - p) if p > 0 else 1.0
    q = np.where(keep, x * scale, 0.0)
    D = x.shape[1]
    mu = q.mean(axis=1, keepdims=True)
    rs = 1.0 / np.sqrt(((q - mu) ** 2).mean(axis=1, keepdims=True) + eps)
    xhat = (q - mu) * rs
    dn = gy * w
    s1 = dn.sum(axis=1, keepdims=True)
    s2 = (dn * xhat).sum(axis=1, keepdims=True)
    dq = (rs / D) * (D * dn - s1 - xhat * s2)
    dx = np.where(keep, dq * scale, 0.0)
    return dx, (gy * xhat).sum(axis=0), gy.sum(axis=0)


def add_layernorm_forward(a, b0, w, b, eps):
    """fused_block_ops_cuda.cu:72-94: LayerNorm(a + b0)."""
    z = np.asarray(a, np.float64) + np.asarray(b0, np.float64)
    mu = z.mean(axis=1, keepdims=True)
    rs = 1.0 / np.sqrt(((z - mu) ** 2).mean(axis=1, keepdims=True) + eps)
    return (z - mu) * rs * w + b, mu[:, 0], rs[:, 0]


def add_layernorm_backward(gy, a, b0, w, eps):
    """fused_block_ops_cuda.cu:120-139: dz (returned for both inputs), dw, db."""
    z = np.asarray(a, np.float64) + np.asarray(b0, np.float64)
    gy = np.asarray(gy, np.float64)
    D = z.shape[1]
    mu = z.mean(axis=1, keepdims=True)
    rs = 1.0 / np.sqrt(((z - mu) ** 2).mean(axis=1, keepdims=True) + eps)
    xhat = (z - mu) * rs
    dn = gy * w
    dz = (rs / D) * (D * dn - dn.sum(axis=1, keepdims=True) - xhat * (dn * xhat).sum(axis=1, keepdims=True))
    return dz, (gy * xhat).sum(axis=0), gy.sum(axis=0)


def gamma_residual_forward(h, g, gamma, p, keep):
    """fused_block_ops_cuda.cu gamma_residual_forward: y = h + gamma*keep*g/(1-p)."""
    scale = 1.0 / (1.0 - p) if p > 0 else 1.0
    return np.asarray(h, np.float64) + np.asarray(gamma, np.float64) * np.where(keep, np.asarray(g, np.float64) * scale, 0.0)


def gamma_residual_backward(gy, g, gamma, p, keep):
    """gamma_backward_stage1/2: grad_h = gy, grad_g = gy*gamma*m, grad_gamma = sum_n gy*g*m."""
    scale = 1.0 / (1.0 - p) if p > 0 else 1.0
    m = np.where(keep, scale, 0.0)
    gy = np.asarray(gy, np.float64)
    return gy, gy * np.asarray(gamma, np.float64) * m, (gy * np.asarray(g, np.float64) * m).sum(axis=0)


# ---------------------------------------------------------------------------
# Hop gate (node mode)
# ---------------------------------------------------------------------------
def hop_gate_score(H, C, score_mode):
    """generic_engine/model_cign.py:731-745: old [H | C], new [H + C | |H - C|]."""
    H = np.asarray(H, np.float64)
    C = np.asarray(C, np.float64)
    if int(score_mode) == 0:
        return np.concatenate([H, C], axis=1)
    return np.concatenate([H + C, np.abs(H - C)], axis=1)


def hop_gate_forward(H, C, weight, bias, score_mode):
    """alpha = softmax_k(score @ weight.T + bias), model_cign.py:747-749."""
    s = hop_gate_score(H, C, score_mode)
    logits = s @ np.asarray(weight, np.float64).T + np.asarray(bias, np.float64)
    logits = logits - logits.max(axis=1, keepdims=True)
    e = np.exp(logits)
    return e / e.sum(axis=1, keepdims=True)


def hop_gate_backward(g_alpha, H, C, weight, bias, score_mode):
    """Gradients (gH, gC, g_weight, g_bias) of hop_gate_forward: softmax
    Jacobian, then the linear map, then the score (d|x|/dx = sign(x), 0 at 0)."""
    H = np.asarray(H, np.float64)
    C = np.asarray(C, np.float64)
    Wt = np.asarray(weight, np.float64)
    a = hop_gate_forward(H, C, weight, bias, score_mode)
    g = np.asarray(g_alpha, np.float64)
    gl = a * (g - (a * g).sum(axis=1, keepdims=True))
    s = hop_gate_score(H, C, score_mode)
    gs = gl @ Wt
    D = H.shape[1]
    g1, g2 = gs[:, :D], gs[:, D:]
    if int(score_mode) == 0:
        gH, gC = g1, g2
    else:
        sg = np.sign(H - C)
        gH, gC = g1 + sg * g2, g1 - sg * g2
    return gH, gC, gl.T @ s, gl.sum(axis=0)


# ---------------------------------------------------------------------------
# Dense projections (nn.Linear under _local_amp_linear)
# ---------------------------------------------------------------------------
def bf16_round(x):
    """Round-to-nearest-even to bfloat16, returned as float64 (the cast that
    torch.autocast applies to Linear inputs and outputs). Pinned against
    torch's own float32 -> bfloat16 conversion in tests/test_oracle.py."""
    a = np.ascontiguousarray(np.asarray(x, np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    r = np.where(nan, u | 0x400000, r).astype(np.uint32)
    return r.view(np.float32).astype(np.float64)


def linear_forward(x, w, b=None, amp=False):
    """_local_amp_linear (generic_engine/model_cign.py:86-103): y = x W^T + b
    in float64; with amp (local bf16 autocast) inputs, weight and bias are
    rounded to bf16 first and the output is rounded to bf16 (autocast output
    dtype) before the cast back to float32. Pinned by the closed form (float64
    matmul) and by the autocast rounding points."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    if amp:
        x, w = bf16_round(x), bf16_round(w)
        b = None if b is None else bf16_round(b)
    y = x @ w.T
    if b is not None:
        y = y + np.asarray(b, np.float64)
    return bf16_round(y) if amp else y


def linear_backward(gy, x, w, amp=False):
    """grad_x = gy W, grad_W = gy^T x, grad_b = sum_n gy (float64). With amp
    (the backward of _local_amp_linear's autocast region): y.float()'s
    backward hands the bf16 Linear a bf16 gradient, so gy, x and W enter the
    products rounded to bf16, and the bf16 Linear's backward returns bf16
    grad_x, grad_W and grad_b (each a float64 sum rounded once to bf16), which
    the casts of x, W and b back to float32 pass on unchanged. Pinned against
    torch CPU autocast of nn.Linear in tests/test_oracle.py."""
    gy, x, w = (np.asarray(v, np.float64) for v in (gy, x, w))
    if not amp:
        return gy @ w, gy.T @ x, gy.sum(axis=0)
    gy, x, w = bf16_round(gy), bf16_round(x), bf16_round(w)
    return bf16_round(gy @ w), bf16_round(gy.T @ x), bf16_round(gy.sum(axis=0))
