"""Pins the CPU oracle (oracle/cign_oracle.py) before it is trusted.

Each check is independent of the oracle's own formula: published vectors,
closed forms, brute-force loops, dense textbook definitions, an independent
library routine, or finite differences of the oracle's forward (which pins
the explicitly written backward formulas). CPU only.
"""
import numpy as np
import pytest
import scipy.special
import torch

from oracle import cign_oracle as O
from tests.conftest import assert_close, random_gat_graph


# ---------------------------------------------------------------- splitmix64
def test_splitmix64_published_sequence():
    # Vigna's splitmix64.c, state seeded with 1234567: first five outputs.
    seed, golden = 1234567, 0x9E3779B97F4A7C15
    states = np.array([(seed + k * golden) % 2**64 for k in range(5)], dtype=np.uint64)
    got = [int(v) for v in O.splitmix64(states)]
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
                   16408922859458223821]


def _mix_py(x):
    m = (1 << 64) - 1
    x = (x + 0x9E3779B97F4A7C15) & m
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & m
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & m
    return x ^ (x >> 31)


def test_gat_mask_bits_match_integer_restatement():
    # keep = ((hi + 0.5f) * 2^-32 > p) in float32 (collapsed_gat_cuda.cu:42-45),
    # restated with Python integers and numpy float32 scalars.
    seed, p, n = 0x1234_5678_9ABC_DEF0, 0.3, 500
    keep = O.gat_dropout_keep(seed, n, p)
    for idx in range(n):
        r = _mix_py(seed ^ ((idx * 0xD2B74407B1CE6E93) & ((1 << 64) - 1)))
        u = (np.float32(r >> 32) + np.float32(0.5)) * np.float32(2.0 ** -32)
        assert bool(u > np.float32(p)) == bool(keep[idx])
    assert abs(keep.mean() - 0.7) < 0.08


def test_block_mask_bits_match_integer_restatement():
    seed, p, n = 987654321, 0.5, 400
    keep = O.block_dropout_keep(seed, n, p)
    for idx in range(n):
        r = _mix_py(seed ^ ((idx * 0xD2B74407B1CE6E93) & ((1 << 64) - 1)))
        assert ((r >> 11) * 2.0 ** -53 >= 0.5) == bool(keep[idx])
    assert O.block_dropout_keep(seed, 10, 0.0).all()


def _golden_seeds():
    import json
    from pathlib import Path

    return json.loads((Path(__file__).resolve().parent / "golden" / "seeds.json").read_text())


def test_block_ops_seed_matches_reference_vectors():
    """O.block_ops_seed against the seeds the reference's own
    fused_block_ops._next_seed returned (tests/golden/make_seeds.py): six
    initial seeds, tags 1, 2 and 7, calls with p = 0 that must not advance
    the counter."""
    for case in _golden_seeds()["block_ops"]:
        call = 0
        for c in case["calls"]:
            if c["p"] > 0:
                call += 1
            assert O.block_ops_seed(case["initial_seed"], call, c["tag"], c["p"]) == c["seed"], (case["initial_seed"], c)


def test_collapsed_gat_seed_matches_reference_vectors():
    """O.collapsed_gat_seed against the seeds the reference's
    collapsed_gat_mean_bias_silu passed to its autograd function."""
    for case in _golden_seeds()["collapsed_gat"]:
        call_id = 0
        for c in case["calls"]:
            assert O.collapsed_gat_seed(case["initial_seed"], call_id, c["attn_drop"]) == c["seed"], c
            if c["attn_drop"] > 0:
                call_id += 1


def test_product_seed_streams_match_reference_vectors(monkeypatch):
    """The product's own per-call seeds (cign_amd.fused_block_ops._next_seed,
    the collapsed-GAT wrapper) replay the reference's call sequences exactly.
    The GAT wrapper runs up to its autograd call, which returns the seed."""
    import itertools
    from types import SimpleNamespace

    import torch

    import cign_amd.collapsed_gat as cg
    import cign_amd.fused_block_ops as fb

    gold = _golden_seeds()
    for case in gold["block_ops"]:
        torch.manual_seed(case["initial_seed"])
        monkeypatch.setattr(fb, "_CALL_COUNTER", itertools.count())
        assert [fb._next_seed(c["tag"], c["p"]) for c in case["calls"]] == [c["seed"] for c in case["calls"]]

    class Feat:
        dtype = torch.float32
        device = SimpleNamespace(type="cuda")

        def dim(self):
            return 3

        def size(self, i):
            return (4, 2, 3)[i]

    monkeypatch.setattr(cg._CollapsedGATFn, "apply", staticmethod(lambda *a: int(a[-1])))
    for case in gold["collapsed_gat"]:
        torch.manual_seed(case["initial_seed"])
        monkeypatch.setattr(cg, "_CALL_COUNTER", itertools.count())
        got = [cg.collapsed_gat_mean_bias_silu(None, None, (None, None), (None, None), None, 0.2, Feat(), object(),
                                               c["attn_drop"]) for c in case["calls"]]
        assert got == [c["seed"] for c in case["calls"]]


def test_seed_formulas():
    assert O.collapsed_gat_seed(5, 0, 0.0) == 0
    assert O.collapsed_gat_seed(5, 0, 0.1) == (5 + 0x9E3779B97F4A7C15) & ((1 << 63) - 1)
    assert O.block_ops_seed(7, 2, 1, 0.2) == (7 + 2 * 0x9E3779B97F4A7C15 + 0xD2B74407B1CE6E93) & ((1 << 63) - 1)


# ---------------------------------------------------------------- graph formats
def test_gat_graph_format_brute_force(rng):
    n = 40
    ei = random_gat_graph(rng, n, avg_deg=4)
    rowptr, col, row, colptr, perm = O.gat_graph_format(ei, n)
    src, dst = ei
    edges = sorted(zip(dst.tolist(), src.tolist()))  # CSR: by (dst, src)
    assert col.tolist() == [s for _, s in edges]
    assert rowptr.tolist() == [sum(1 for d, _ in edges if d < i) for i in range(n + 1)]
    cedges = sorted(zip(src.tolist(), dst.tolist()))  # CSC: by (src, dst)
    assert row.tolist() == [d for _, d in cedges]
    assert colptr.tolist() == [sum(1 for s, _ in cedges if s < j) for j in range(n + 1)]
    for k, (s, d) in enumerate(cedges):
        assert edges[perm[k]] == (d, s)


def test_normalized_adjacency_matches_torch_coalesce(rng):
    n = 60
    ei = np.stack([rng.integers(0, n, 300), rng.integers(0, n, 300)])
    used, (pr, pc, pv) = O.normalized_adjacency(ei, n)
    # Independent check with torch's own COO machinery (reference train_cign.py:1571-1587 ops).
    e = torch.from_numpy(ei)
    both = torch.cat([e, e.flip(0)], 1)
    key = torch.unique(both[0] * n + both[1])
    und = torch.stack([key // n, key % n])
    loops = torch.arange(n)
    full = torch.cat([und, torch.stack([loops, loops])], 1)
    deg = torch.zeros(n).scatter_add_(0, full[1], torch.ones(full.size(1)))
    dis = deg.clamp(min=1).pow(-0.5)
    w = dis[full[0]] * dis[full[1]]
    P = torch.sparse_coo_tensor(full, w, (n, n)).coalesce()
    assert np.array_equal(P.indices()[0].numpy(), pr) and np.array_equal(P.indices()[1].numpy(), pc)
    assert np.array_equal(pv, P.values().numpy()), "P values must be bit-identical"
    # Symmetric operator and row sums of D^-1/2 (A+I) D^-1/2 against dense math.
    A = np.zeros((n, n))
    A[und[0].numpy(), und[1].numpy()] = 1
    A += np.eye(n)
    d = A.sum(1)
    dense = A / np.sqrt(np.outer(d, d))
    Pd = np.zeros((n, n))
    Pd[pr, pc] = pv
    assert_close(Pd, dense, 1e-6, 1e-7, "dense P")


def test_transpose_csr(rng):
    n = 30
    r, c, v = O.coalesce(rng.integers(0, n, 120), rng.integers(0, n, 120), n, rng.standard_normal(120))
    rp = np.zeros(n + 1, np.int64)
    np.add.at(rp, r + 1, 1)
    rp = np.cumsum(rp)
    trp, tc, tv = O.transpose_csr(rp, c, v, n)
    M = O.csr_matrix(rp, c, v, n).toarray()
    assert_close(O.csr_matrix(trp, tc, tv, n).toarray(), M.T, 0, 0, "P^T")


# ---------------------------------------------------------------- SpMM / multihop
def _circulant(n):
    # validate_a3v5.py:11-19: offsets {0, +-1, +-7, +-31, +-127}, w = 1/9.
    offs = [0, 1, -1, 7, -7, 31, -31, 127, -127]
    rows = np.repeat(np.arange(n), len(offs))
    cols = (rows + np.tile(offs, n)) % n
    r, c, v = O.coalesce(rows, cols, n, np.full(len(rows), 1.0 / 9.0))
    rp = np.zeros(n + 1, np.int64)
    np.add.at(rp, r + 1, 1)
    return np.cumsum(rp), c, v, offs


def test_spmm_circulant_known_answer(rng):
    n, d = 512, 8
    rp, c, v, offs = _circulant(n)
    x = rng.standard_normal((n, d))
    expect = sum(np.roll(x, -o, axis=0) for o in offs) / 9.0
    assert_close(O.spmm(rp, c, v, x), expect, 1e-12, 1e-12, "circulant")


def test_multihop_adjoint_and_dense(rng):
    n, d = 80, 5
    r, c, v = O.coalesce(rng.integers(0, n, 500), rng.integers(0, n, 500), n, rng.standard_normal(500))
    rp = np.zeros(n + 1, np.int64)
    np.add.at(rp, r + 1, 1)
    rp = np.cumsum(rp)
    p = (rp, c, v)
    pt = O.transpose_csr(rp, c, v, n)
    M = O.csr_matrix(rp, c, v, n).toarray()
    x = rng.standard_normal((n, d))
    y = O.multihop3_forward(p, x)
    for k in range(3):
        assert_close(y[k], np.linalg.matrix_power(M, k + 1) @ x, 1e-10, 1e-10, f"y{k+1}")
    g = [rng.standard_normal((n, d)) for _ in range(3)]
    gx = O.multihop3_backward(pt, *g)
    lhs = sum((y[k] * g[k]).sum() for k in range(3))
    assert abs(lhs - (x * gx).sum()) < 1e-9 * max(1, abs(lhs))
    gen = O.multihop_generic_backward(pt, {1: g[0], 2: g[1], 3: g[2]}, 3, x.shape)
    assert_close(gen, gx, 1e-12, 1e-12, "generic == native3")
    fw = O.multihop_generic_forward(p, x, (1, 3, 5))
    assert_close(fw[5], np.linalg.matrix_power(M, 5) @ x, 1e-9, 1e-9, "P^5")


# ---------------------------------------------------------------- collapsed GAT
def _gat_inputs(rng, n, H, C, deg=5, hubs=None):
    ei = random_gat_graph(rng, n, avg_deg=deg, hubs=hubs)
    rowptr, col, row, colptr, perm = O.gat_graph_format(ei, n)
    return dict(rowptr=rowptr, col=col, x=rng.standard_normal((n, H, C)), ar=rng.standard_normal((n, H)),
                ac=rng.standard_normal((n, H)), b=rng.standard_normal(C))


def test_gat_dense_textbook_single_head(rng):
    # H=1, p=0: out_i = SiLU(sum_j softmax_j(LeakyReLU(a_dst[i] + a_src[j])) x_j + b)
    # with the softmax over the in-neighbours j of destination i (dense form).
    n, C, slope = 25, 3, 0.2
    d = _gat_inputs(rng, n, 1, C)
    A = np.zeros((n, n), bool)
    rows = np.repeat(np.arange(n), np.diff(d["rowptr"]))
    A[rows, d["col"]] = True
    S = d["ar"][:, 0][:, None] + d["ac"][:, 0][None, :]
    S = np.where(S > 0, S, slope * S)
    S = np.where(A, S, -np.inf)
    W = scipy.special.softmax(S, axis=1)
    pre = W @ d["x"][:, 0, :] + d["b"]
    got = O.collapsed_gat_forward(d["ar"], d["ac"], d["rowptr"], d["col"], slope, d["x"], d["b"])
    assert_close(got["pre"], pre, 1e-12, 1e-12, "pre")
    assert_close(got["out"], pre / (1 + np.exp(-pre)), 1e-12, 1e-12, "out")


def test_gat_sampled_rows_and_columns_match_full_oracle(rng):
    """The row-sampled forward and column-sampled backward (used at full
    size, where the whole-graph oracle does not fit) equal the whole-graph
    oracle at the sampled rows/columns, including hubs, rows with empty
    in-lists (rowptr plateaus) and columns no row reads."""
    n, H, C = 160, 3, 5
    d = _gat_inputs(rng, n, H, C, hubs={4: 120, 9: 90})
    rp, cl = d["rowptr"].copy(), d["col"].copy()
    # Empty rows 20..23: drop their edges.
    keep = ~np.isin(np.repeat(np.arange(n), np.diff(rp)), [20, 21, 22, 23])
    rows_all = np.repeat(np.arange(n), np.diff(rp))[keep]
    cl = cl[keep]
    rp = np.concatenate([[0], np.cumsum(np.bincount(rows_all, minlength=n))])
    gy = rng.standard_normal((n, C))
    f = O.collapsed_gat_forward(d["ar"], d["ac"], rp, cl, 0.2, d["x"], d["b"])
    g = O.collapsed_gat_backward(d["ar"], d["ac"], rp, cl, 0.2, d["x"], d["b"], gy)
    rows = np.array([4, 9, 0, 21, 37, 159, 100])
    fr = O.collapsed_gat_forward_rows(d["ar"], d["ac"], rp, cl, 0.2, d["x"], d["b"], rows)
    for k in ("out", "pre", "emax", "esum"):
        assert_close(fr[k], f[k][rows], 1e-12, 1e-12, k)
    unread = np.setdiff1d(np.arange(n), cl)
    cols = np.array([9, 4, 55, 0, 158] + ([int(unread[0])] if unread.size else []))
    gc = O.collapsed_gat_backward_columns(d["ar"], d["ac"], rp, cl, 0.2, d["x"], d["b"], gy, cols)
    assert_close(gc["grad_feat"], g["grad_feat"][cols], 1e-12, 1e-12, "grad_feat")
    assert_close(gc["grad_attn_col"], g["grad_attn_col"][cols], 1e-12, 1e-12, "grad_attn_col")
    assert_close(gc["grad_attn_row"], g["grad_attn_row"][gc["rows"]], 1e-12, 1e-12, "grad_attn_row")
    assert_close(gc["grad_pre"], g["grad_pre"][gc["rows"]], 1e-12, 1e-12, "grad_pre")
    assert set(gc["rows"].tolist()) == set(np.repeat(np.arange(n), np.diff(rp))[np.isin(cl, cols)].tolist())
    # Row-sampled SpMM.
    val = rng.standard_normal(len(cl))
    X = rng.standard_normal((n, 7))
    A = rng.standard_normal((n, 7))
    assert_close(O.spmm_rows(rp, cl, val, X, rows, add=A), O.spmm(rp, cl, val, X, add=A)[rows], 1e-12, 1e-12,
                 "spmm_rows")


def test_gat_closed_forms(rng):
    n, H, C = 20, 3, 4
    d = _gat_inputs(rng, n, H, C)
    # attn_col = 0: every in-edge of a row has the same score -> uniform
    # weights, whatever attn_row is. (A swapped row/col operand fails this.)
    got = O.collapsed_gat_forward(d["ar"], np.zeros((n, H)), d["rowptr"], d["col"], 0.2, d["x"], d["b"])
    deg = np.diff(d["rowptr"])
    rows = np.repeat(np.arange(n), deg)
    mean = np.zeros((n, C))
    np.add.at(mean, rows, d["x"][d["col"]].mean(axis=1))
    assert_close(got["pre"], mean / deg[:, None] + d["b"], 1e-12, 1e-12, "uniform")
    # Only self-loops: softmax == 1.
    self_only = np.arange(n + 1), np.arange(n)
    got = O.collapsed_gat_forward(d["ar"], d["ac"], *self_only, 0.2, d["x"], d["b"])
    assert_close(got["pre"], d["x"].mean(axis=1) + d["b"], 1e-12, 1e-12, "degree 1")
    assert_close(got["esum"], np.ones((n, H)), 1e-12, 0, "esum")
    # Empty row: pre = bias, max = -1e38, sum = 0 (collapsed_gat_cuda.cu:87-130).
    rp = np.concatenate([[0], np.arange(n)])  # row 0 empty
    got = O.collapsed_gat_forward(d["ar"], d["ac"], rp, np.arange(n - 1), 0.2, d["x"], d["b"])
    assert_close(got["pre"][0], d["b"], 0, 0, "empty row")
    assert got["emax"][0, 0] == O.NEG_BIG and got["esum"][0, 0] == 0


def test_gat_brute_force_loops(rng):
    n, H, C, slope, p = 12, 2, 3, 0.15, 0.4
    d = _gat_inputs(rng, n, H, C, deg=3)
    E = len(d["col"])
    keep = rng.random((E, H)) > p
    got = O.collapsed_gat_forward(d["ar"], d["ac"], d["rowptr"], d["col"], slope, d["x"], d["b"], p, keep)
    for i in range(n):
        acc = np.zeros(C)
        for h in range(H):
            es = range(d["rowptr"][i], d["rowptr"][i + 1])
            sc = {e: d["ar"][i, h] + d["ac"][d["col"][e], h] for e in es}
            sc = {e: (s if s > 0 else s * slope) for e, s in sc.items()}
            m = max(sc.values())
            z = sum(np.exp(s - m) for s in sc.values())
            for e in es:
                w = np.exp(sc[e] - m) / z
                w = w / (1 - p) if keep[e, h] else 0.0
                acc += w * d["x"][d["col"][e], h]
        assert_close(got["pre"][i], acc / H + d["b"], 1e-12, 1e-12, f"row {i}")


@pytest.mark.parametrize("p", [0.0, 0.35])
def test_gat_backward_finite_differences(rng, p):
    n, H, C, slope = 18, 3, 4, 0.2
    d = _gat_inputs(rng, n, H, C, deg=4)
    E = len(d["col"])
    keep = rng.random((E, H)) > p if p > 0 else None
    gy = rng.standard_normal((n, C))
    g = O.collapsed_gat_backward(d["ar"], d["ac"], d["rowptr"], d["col"], slope, d["x"], d["b"], gy, p, keep)

    def f(ar, ac, x, b):
        out = O.collapsed_gat_forward(ar, ac, d["rowptr"], d["col"], slope, x, b, p, keep)["out"]
        return (out * gy).sum()

    base = dict(ar=d["ar"], ac=d["ac"], x=d["x"], b=d["b"])
    grads = dict(ar=g["grad_attn_row"], ac=g["grad_attn_col"], x=g["grad_feat"], b=g["grad_bias"])
    eps = 1e-6
    for name in base:
        v = rng.standard_normal(base[name].shape)
        plus = dict(base)
        minus = dict(base)
        plus[name] = base[name] + eps * v
        minus[name] = base[name] - eps * v
        fd = (f(**plus) - f(**minus)) / (2 * eps)
        an = (grads[name] * v).sum()
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (name, fd, an)


@pytest.mark.parametrize("p", [0.0, 0.35])
def test_gat_row_aggregates_give_backward(rng, p):
    """The saved per-row aggregates reproduce the (finite-difference pinned)
    backward: grad_attn_row = <g, agg_l>/H - <g, agg>/H * b_l, and the head
    mean of agg is pre - bias. A dropped slope, keep factor or head index in
    the aggregates fails one of the two."""
    n, H, C, slope = 30, 3, 4, 0.2
    d = _gat_inputs(rng, n, H, C, deg=5, hubs={2: 20})
    E = len(d["col"])
    keep = rng.random((E, H)) > p if p > 0 else None
    gy = rng.standard_normal((n, C))
    g = O.collapsed_gat_backward(d["ar"], d["ac"], d["rowptr"], d["col"], slope, d["x"], d["b"], gy, p, keep)
    f = O.collapsed_gat_forward(d["ar"], d["ac"], d["rowptr"], d["col"], slope, d["x"], d["b"], p, keep)
    a = O.collapsed_gat_row_aggregates(d["ar"], d["ac"], d["rowptr"], d["col"], slope, d["x"], p, keep)
    gp = g["grad_pre"]
    wsum = np.einsum("nc,nhc->nh", gp, a["agg"]) / H
    A = np.einsum("nc,nhc->nh", gp, a["agg_l"]) / H
    assert_close(A - wsum * a["b_l"], g["grad_attn_row"], 1e-10, 1e-12, "grad_attn_row from aggregates")
    assert_close(a["agg"].mean(axis=1), f["pre"] - d["b"], 1e-12, 1e-12, "head mean of agg")


# ---------------------------------------------------------------- side ops
def test_attention_logits_and_head_silu(rng):
    n, H, C = 7, 3, 5
    x = rng.standard_normal((n, H, C))
    a_s, a_d = rng.standard_normal((1, H, C)), rng.standard_normal((1, H, C))
    s, dd = O.attention_logits_forward(x, a_s, a_d)
    for i in range(n):
        for h in range(H):
            assert abs(s[i, h] - sum(x[i, h, c] * a_s[0, h, c] for c in range(C))) < 1e-12
            assert abs(dd[i, h] - sum(x[i, h, c] * a_d[0, h, c] for c in range(C))) < 1e-12
    gs, gd = rng.standard_normal((n, H)), rng.standard_normal((n, H))
    gx, gas, gad = O.attention_logits_backward(gs, gd, x, a_s, a_d)
    eps = 1e-6
    f = lambda x_, s_, d_: (O.attention_logits_forward(x_, s_, d_)[0] * gs).sum() + \
        (O.attention_logits_forward(x_, s_, d_)[1] * gd).sum()
    for arg, an in ((0, gx), (1, gas), (2, gad)):
        base = [x, a_s, a_d]
        v = rng.standard_normal(base[arg].shape)
        up = list(base); dn = list(base)
        up[arg] = base[arg] + eps * v
        dn[arg] = base[arg] - eps * v
        assert abs((f(*up) - f(*dn)) / (2 * eps) - (an * v).sum()) < 1e-6
    out = rng.standard_normal((n, H, C))
    b = rng.standard_normal(C)
    y, pre = O.head_silu_forward(out, b)
    gy = rng.standard_normal((n, C))
    go, gb = O.head_silu_backward(gy, pre, H)
    v = rng.standard_normal(out.shape)
    fd = ((O.head_silu_forward(out + eps * v, b)[0] - O.head_silu_forward(out - eps * v, b)[0]) * gy).sum() / (2 * eps)
    assert abs(fd - (go * v).sum()) < 1e-6
    vb = rng.standard_normal(C)
    fdb = ((O.head_silu_forward(out, b + eps * vb)[0] - O.head_silu_forward(out, b - eps * vb)[0]) * gy).sum() / (2 * eps)
    assert abs(fdb - (gb * vb).sum()) < 1e-6


# ---------------------------------------------------------------- packs
@pytest.mark.parametrize("interaction", [0, 1, 2])
@pytest.mark.parametrize("weighting", [0, 1])
@pytest.mark.parametrize("K", [1, 3, 4])
def test_pack_backward_finite_differences(rng, interaction, weighting, K):
    n, D = 6, 5
    H, C = rng.standard_normal((n, D)), rng.standard_normal((n, D))
    props = [rng.standard_normal((n, 2 * D)) for _ in range(K)]
    A = rng.random((n, K))
    out = O.clifford_pack_forward(H, C, props, A, interaction, weighting)
    G = rng.standard_normal(out.shape)
    gH, gC, gP, gA = O.clifford_pack_backward(G, H, C, props, A, interaction, weighting)

    def f(H_, C_, P_, A_):
        return (O.clifford_pack_forward(H_, C_, P_, A_, interaction, weighting) * G).sum()

    eps = 1e-6
    for which in range(4):
        base = [H, C, props, A]
        an_grad = [gH, gC, gP, gA][which]
        if which == 2:
            v = [rng.standard_normal(p.shape) for p in props]
            up = [p + eps * w for p, w in zip(props, v)]
            dn = [p - eps * w for p, w in zip(props, v)]
            an = sum((g * w).sum() for g, w in zip(gP, v))
        else:
            v = rng.standard_normal(base[which].shape)
            up, dn = base[which] + eps * v, base[which] - eps * v
            an = (an_grad * v).sum()
        bu, bd = list(base), list(base)
        bu[which], bd[which] = up, dn
        fd = (f(*bu) - f(*bd)) / (2 * eps)
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (which, fd, an)


def test_pack_closed_forms(rng):
    n, D = 4, 3
    H, C = rng.standard_normal((n, D)), rng.standard_normal((n, D))
    P = rng.standard_normal((n, 2 * D))
    A = np.ones((n, 1))
    th, tc = P[:, :D], P[:, D:]
    old = O.clifford_pack_forward(H, C, [P], A, 0, 0)  # validate_a3.py:8-19 legacy_pack
    z = H * tc
    assert_close(old, np.concatenate([z - th * C, z / (1 + np.exp(-z))], 1), 1e-12, 1e-12, "old")
    new = O.clifford_pack_forward(H, C, [P], A, 1, 1)  # validate_cign_acceleration.py:10-18
    s, a = 0.5 * (H * tc + C * th), 0.5 * (H * tc - C * th)
    assert_close(new, np.concatenate([s / (1 + np.exp(-s)), a], 1), 1e-12, 1e-12, "new/new")
    tanh = O.clifford_pack_forward(H, C, [P], A, 2, 0)
    assert_close(tanh, np.concatenate([np.tanh(a), s / (1 + np.exp(-s))], 1), 1e-12, 1e-12, "tanh/old")


# ---------------------------------------------------------------- block ops
def test_block_ops_against_torch_layer_norm(rng):
    n, D, eps, p = 9, 7, 1e-5, 0.25
    x = rng.standard_normal((n, D))
    w, b = rng.standard_normal(D), rng.standard_normal(D)
    keep = rng.random((n, D)) >= p
    y, mu, rs = O.dropout_layernorm_forward(x, w, b, p, eps, keep)
    xt = torch.tensor(np.where(keep, x / (1 - p), 0.0), requires_grad=True)
    wt = torch.tensor(w, requires_grad=True)
    bt = torch.tensor(b, requires_grad=True)
    yt = torch.nn.functional.layer_norm(xt, (D,), wt, bt, eps)
    assert_close(y, yt.detach().numpy(), 1e-12, 1e-12, "dropout-LN fwd")
    gy = rng.standard_normal((n, D))
    yt.backward(torch.tensor(gy))
    dx, dw, db = O.dropout_layernorm_backward(gy, x, w, p, eps, keep)
    assert_close(dx, np.where(keep, xt.grad.numpy() / (1 - p), 0), 1e-10, 1e-12, "dx")
    assert_close(dw, wt.grad.numpy(), 1e-10, 1e-12, "dw")
    assert_close(db, bt.grad.numpy(), 1e-10, 1e-12, "db")
    a, b0 = rng.standard_normal((n, D)), rng.standard_normal((n, D))
    y2, _, _ = O.add_layernorm_forward(a, b0, w, b, eps)
    zt = torch.tensor(a + b0, requires_grad=True)
    y2t = torch.nn.functional.layer_norm(zt, (D,), torch.tensor(w), torch.tensor(b), eps)
    assert_close(y2, y2t.detach().numpy(), 1e-12, 1e-12, "add-LN fwd")
    y2t.backward(torch.tensor(gy))
    dz, _, _ = O.add_layernorm_backward(gy, a, b0, w, eps)
    assert_close(dz, zt.grad.numpy(), 1e-10, 1e-12, "add-LN dz")
    h, g, gamma = rng.standard_normal((n, D)), rng.standard_normal((n, D)), rng.standard_normal(D)
    yr = O.gamma_residual_forward(h, g, gamma, p, keep)
    assert_close(yr, h + gamma * np.where(keep, g / (1 - p), 0), 1e-12, 1e-12, "gamma residual")
    gh, gg, ggam = O.gamma_residual_backward(gy, g, gamma, p, keep)
    eps2 = 1e-6
    v = rng.standard_normal(D)
    fd = ((O.gamma_residual_forward(h, g, gamma + eps2 * v, p, keep) -
           O.gamma_residual_forward(h, g, gamma - eps2 * v, p, keep)) * gy).sum() / (2 * eps2)
    assert abs(fd - (ggam * v).sum()) < 1e-6


# ---------------------------------------------------------------------------
# Hop gate
# ---------------------------------------------------------------------------
def test_hop_gate_oracle_against_torch_autograd_and_closed_forms():
    """Pins hop_gate_forward/backward: torch fp64 autograd of the reference
    expression (model_cign.py:731-749), rows summing to one, uniform alpha for
    zero weights, and the old score reducing to the plain concatenation."""
    import torch

    rng = np.random.default_rng(7)
    n, D, K = 40, 6, 3
    H, C = rng.standard_normal((n, D)), rng.standard_normal((n, D))
    C[0, 0] = H[0, 0]  # |H - C| at 0: gradient convention sign(0) = 0
    W, b = rng.standard_normal((K, 2 * D)), rng.standard_normal(K)
    g = rng.standard_normal((n, K))
    for mode in (0, 1):
        a = O.hop_gate_forward(H, C, W, b, mode)
        assert np.allclose(a.sum(axis=1), 1.0)
        Ht, Ct = torch.tensor(H, requires_grad=True), torch.tensor(C, requires_grad=True)
        Wt, bt = torch.tensor(W, requires_grad=True), torch.tensor(b, requires_grad=True)
        s = torch.cat([Ht, Ct], -1) if mode == 0 else torch.cat([Ht + Ct, torch.abs(Ht - Ct)], -1)
        at = torch.softmax(torch.nn.functional.linear(s, Wt, bt), dim=-1)
        (at * torch.tensor(g)).sum().backward()
        assert np.allclose(a, at.detach().numpy(), rtol=1e-12, atol=1e-14)
        gH, gC, gW, gb = O.hop_gate_backward(g, H, C, W, b, mode)
        for mine, ref in ((gH, Ht.grad), (gC, Ct.grad), (gW, Wt.grad), (gb, bt.grad)):
            assert np.allclose(mine, ref.numpy(), rtol=1e-10, atol=1e-12)
    assert np.allclose(O.hop_gate_forward(H, C, np.zeros((K, 2 * D)), np.zeros(K), 1), 1.0 / K)
    assert np.array_equal(O.hop_gate_score(H, C, 0), np.concatenate([H, C], 1))


# ---------------------------------------------------------------------------
# Block composition oracle (oracle/block_oracle.py)
# ---------------------------------------------------------------------------
def test_block_oracle_stages_match_numpy_oracle():
    """The torch fp64 block restatement's GAT and pack stages equal the numpy
    oracle's collapsed GAT and Clifford pack (every interaction x weighting,
    with and without alpha), so the composition is pinned stage by stage."""
    import torch
    from oracle import block_oracle as B

    rng = np.random.default_rng(11)
    n, Hh, C = 60, 3, 5
    ei = []
    for i in range(n):
        for j in rng.choice(n, size=int(rng.integers(0, 6)), replace=False):
            ei.append((int(j), i))
    ei = np.array(ei, dtype=np.int64).T
    ge = O.gat_edge_index(ei, n)
    r, c, _ = O.coalesce(ge[0], ge[1], n)
    # rows = destinations: CSR of the flipped edge list
    rowptr, col = O.csr_from_coo(c, r, n)[:2]
    x = rng.standard_normal((n, Hh, C))
    a_s, a_d, b = rng.standard_normal((n, Hh)), rng.standard_normal((n, Hh)), rng.standard_normal(C)
    y = B._gat(torch.tensor(x), torch.tensor(a_s), torch.tensor(a_d), rowptr, col, 0.2, torch.tensor(b))
    ref = O.collapsed_gat_forward(a_d, a_s, rowptr, col, 0.2, x, b)
    assert np.allclose(y.numpy(), ref["out"], rtol=1e-12, atol=1e-12)
    D, K = 4, 3
    Hn, Cn = rng.standard_normal((n, D)), rng.standard_normal((n, D))
    props = [rng.standard_normal((n, 2 * D)) for _ in range(K)]
    alpha = rng.random((n, K))
    for inter in (0, 1, 2):
        for w in (0, 1):
            for a in (alpha, None):
                got = B._pack(torch.tensor(Hn), torch.tensor(Cn), [torch.tensor(p) for p in props],
                              None if a is None else torch.tensor(a)[:, :, None], inter, w)
                want = O.clifford_pack_forward(Hn, Cn, props, np.ones((n, K)) if a is None else a, inter, w)
                assert np.allclose(got.numpy(), want, rtol=1e-12, atol=1e-12), (inter, w, a is None)


def test_bf16_round_matches_torch_cast():
    """The oracle's bf16 rounding is torch's float32 -> bfloat16 cast (RNE),
    including ties, subnormals, infinities and NaN."""
    import torch

    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-40, 38, 20000),
                           np.array([0.0, -0.0, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 1e-45, -3e-39, np.inf, -np.inf,
                                     3.3895314e38], dtype=np.float32)]).astype(np.float32)
    got = O.bf16_round(vals)
    want = torch.from_numpy(vals).to(torch.bfloat16).double().numpy()
    assert np.array_equal(got, want)
    assert np.isnan(O.bf16_round(np.array([np.nan], np.float32)))[0]


def test_linear_oracle_amp_rounding_points():
    """amp: operands and output rounded to bf16 (torch CPU autocast of
    F.linear gives the same within one bf16 ulp of the output)."""
    import torch

    rng = np.random.default_rng(1)
    x = rng.standard_normal((64, 48)).astype(np.float32)
    w = rng.standard_normal((24, 48)).astype(np.float32) / 7
    b = rng.standard_normal(24).astype(np.float32)
    y = O.linear_forward(x, w, b, amp=True)
    assert np.array_equal(O.bf16_round(y), y)
    with torch.autocast("cpu", dtype=torch.bfloat16):
        t = torch.nn.functional.linear(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b))
    assert t.dtype == torch.bfloat16
    np.testing.assert_allclose(t.double().numpy(), y, rtol=2 ** -7, atol=2 ** -7)
    gx, gw, gb = O.linear_backward(np.ones((64, 24)), x, w)
    np.testing.assert_allclose(gw, np.tile(x.astype(np.float64).sum(0), (24, 1)), rtol=1e-12)
    np.testing.assert_allclose(gb, np.full(24, 64.0))
    np.testing.assert_allclose(gx, np.tile(w.astype(np.float64).sum(0), (64, 1)), rtol=1e-12)


def test_linear_oracle_amp_backward_matches_torch_autocast():
    """amp backward: torch CPU autocast of nn.Linear, whose output goes on as
    float32 (y.float(), as _local_amp_linear returns it), gives bf16-valued
    grad_x, grad_W and grad_b, grad_b being the sum of the bf16-rounded
    grad_y. O.linear_backward(amp=True) matches grad_x and grad_b bit for bit
    and grad_W within one bf16 ulp (torch accumulates the 64 rows in another
    order); an oracle that left the gradients unrounded, or summed the
    unrounded grad_y for grad_b, fails this."""
    import torch

    torch.manual_seed(0)
    lin = torch.nn.Linear(48, 24)
    x = torch.randn(64, 48, requires_grad=True)
    with torch.autocast("cpu", dtype=torch.bfloat16):
        y = lin(x)
    gy = torch.randn(64, 24)
    y.float().backward(gy)
    gx, gw, gb = O.linear_backward(gy.numpy(), x.detach().numpy(), lin.weight.detach().numpy(), amp=True)
    for name, got in (("grad_x", gx), ("grad_w", gw), ("grad_b", gb)):
        assert np.array_equal(O.bf16_round(got), got), name
    assert np.array_equal(gx, x.grad.double().numpy())
    assert np.array_equal(gb, lin.bias.grad.double().numpy())
    assert not np.array_equal(O.bf16_round(gy.double().numpy().sum(0)), gb)
    tw = lin.weight.grad.double().numpy()
    assert np.mean(gw == tw) > 0.99
    assert np.all(np.abs(gw - tw) <= 2.0 ** -7 * np.abs(tw))


def test_net_oracle_closed_forms():
    """net_forward's outer composition: with gamma = 0 every block is the
    identity (H + 0 * G), so the logits are classifier(LN([H0]*(L+1))) with H0
    = SiLU(lin0 x) + eta SiLU(lin1 x); with eta = 0 the second projection
    drops out and 'last' combine keeps one state. A swapped projection, a
    missing SiLU or a wrong concat count fails one of these."""
    import torch
    import torch.nn.functional as F
    from oracle import block_oracle as B

    rng = np.random.default_rng(5)
    n, D, heads, in_dim, L = 40, 8, 2, 6, 2
    ei = np.array([[j, i] for i in range(n) for j in rng.choice(n, 3, replace=False)], dtype=np.int64).T
    ge = O.gat_edge_index(ei, n)
    r, c, _ = O.coalesce(ge[0], ge[1], n)
    rowptr, col = O.csr_from_coo(c, r, n)[:2]
    prow, pcol, _ = O.csr_from_coo(r, c, n)
    pval = np.full(pcol.size, 0.1)
    t = lambda *s: torch.tensor(rng.standard_normal(s))
    g = {"input_proj_0.weight": t(D, in_dim), "input_proj_0.bias": t(D), "input_proj_1.weight": t(D, in_dim),
         "input_proj_1.bias": t(D), "input_eta": torch.tensor(0.3, dtype=torch.float64),
         "output_norm.weight": t((L + 1) * D), "output_norm.bias": t((L + 1) * D),
         "classifier.weight": t(5, (L + 1) * D), "classifier.bias": t(5)}
    for i in range(L):
        for k, shape in {"h_norm.weight": (D,), "h_norm.bias": (D,), "c_norm.weight": (D,), "c_norm.bias": (D,),
                         "context_gat.lin.weight": (heads * D, D), "context_gat.att_src": (1, heads, D),
                         "context_gat.att_dst": (1, heads, D), "context_gat.bias": (D,),
                         "proj.weight": (D, 6 * D), "proj.bias": (D,), "hop_gate_mlp.weight": (3, 2 * D),
                         "hop_gate_mlp.bias": (3,)}.items():
            g[f"blocks.{i}.{k}"] = t(*shape)
        g[f"blocks.{i}.gamma"] = torch.zeros(D, dtype=torch.float64)
    x = t(n, in_dim)
    kw = dict(num_layers=L, dual=True, layer_combine="concat", score_mode=1, interaction=1, weighting=0,
              gate_mode="node", heads=heads)
    got = B.net_forward(g, x, rowptr, col, (prow, pcol, pval), (1, 2, 3), **kw)
    h0 = F.silu(x @ g["input_proj_0.weight"].T + g["input_proj_0.bias"]) + \
        0.3 * F.silu(x @ g["input_proj_1.weight"].T + g["input_proj_1.bias"])
    z = torch.cat([h0] * (L + 1), dim=1)
    z = (z - z.mean(1, keepdim=True)) / torch.sqrt(z.var(1, unbiased=False, keepdim=True) + 1e-5)
    z = z * g["output_norm.weight"] + g["output_norm.bias"]
    want = z @ g["classifier.weight"].T + g["classifier.bias"]
    assert torch.allclose(got, want, rtol=1e-10, atol=1e-10)
    g2 = dict(g, input_eta=torch.tensor(0.0, dtype=torch.float64))
    g2["output_norm.weight"], g2["output_norm.bias"] = t(D), t(D)
    g2["classifier.weight"] = t(5, D)
    got2 = B.net_forward(g2, x, rowptr, col, (prow, pcol, pval), (1, 2, 3), **dict(kw, layer_combine="last"))
    h = F.silu(x @ g["input_proj_0.weight"].T + g["input_proj_0.bias"])
    z = F.layer_norm(h, (D,), g2["output_norm.weight"], g2["output_norm.bias"], 1e-5)
    assert torch.allclose(got2, z @ g2["classifier.weight"].T + g["classifier.bias"], rtol=1e-10, atol=1e-10)


def test_block_oracle_amp_linear_matches_autocast_rounding_points():
    """block_oracle._AmpLinear (the selective-AMP projections of the block and
    net oracles) equals the pinned O.linear_forward(amp=True) forward and
    O.linear_backward(amp=True), in float64."""
    import torch

    from oracle import block_oracle as B

    rng = np.random.default_rng(9)
    x, w, b = rng.standard_normal((37, 19)), rng.standard_normal((11, 19)), rng.standard_normal(11)
    gy = rng.standard_normal((37, 11))
    xt, wt, bt = (torch.from_numpy(v).requires_grad_() for v in (x, w, b))
    y = B._AmpLinear.apply(xt, wt, bt)
    assert np.array_equal(y.detach().numpy(), O.linear_forward(x, w, b, amp=True))
    y.backward(torch.from_numpy(gy))
    gx, gw, gb = O.linear_backward(gy, x, w, amp=True)
    assert np.array_equal(xt.grad.numpy(), gx)
    assert np.array_equal(wt.grad.numpy(), gw)
    assert np.array_equal(bt.grad.numpy(), gb)


def test_cpu_path_layer_matches_oracle(rng):
    """The float32 torch restatement of the reference's CPU path (the timed
    CPU baseline) computes the oracle's GAT and three hops, forward and
    backward, to float32 accuracy."""
    import torch

    from oracle import cpu_path

    n, H, C, D = 120, 3, 5, 7
    ei = random_gat_graph(rng, n, avg_deg=6, hubs={2: 90})
    rowptr, col, _, _, _ = O.gat_graph_format(ei, n)
    val = rng.random(len(col))
    p_csr = (rowptr, col, val)
    pt_csr = O.transpose_csr(rowptr, col, val, n)
    L = cpu_path.LayerCPU(rowptr, col, p_csr, pt_csr, n, H, C, D, seed=3)
    L.step()
    d = lambda t: t.detach().double().numpy()
    f = O.collapsed_gat_forward(d(L.ar), d(L.ac), rowptr, col, 0.2, d(L.x), d(L.b))
    y = cpu_path.gat_concat_false(L.x, L.ac, L.ar, L.rows, L.src, n, 0.2, L.b)
    assert_close(d(y), f["out"], 1e-4, 1e-5, "gat out")
    g = O.collapsed_gat_backward(d(L.ar), d(L.ac), rowptr, col, 0.2, d(L.x), d(L.b), d(L.gy))
    for name, t in (("grad_feat", L.x), ("grad_attn_row", L.ar), ("grad_attn_col", L.ac), ("grad_bias", L.b)):
        assert_close(d(t.grad), g[name], 1e-4, 1e-5, name)
    ys = O.multihop3_forward(p_csr, d(L.X))
    gx = O.multihop3_backward(pt_csr, *(d(t) for t in L.G))
    assert_close(d(L.X.grad), gx, 1e-4, 1e-5, "multihop grad_x")
    y1 = cpu_path._FixedCsrMM.apply(L.X, L.P, L.PT)
    assert_close(d(y1), ys[0], 1e-4, 1e-5, "hop 1")
    assert cpu_path.host_threads() >= 1


def test_assert_close_rejects_nan():
    """The comparison helpers fail on a NaN where a number is expected (a
    NaN compares false against any tolerance); assert_close accepts NaN
    against NaN."""
    from tests.conftest import assert_close, assert_close_fp32_derived

    e = np.array([1.0, 2.0, 3.0])
    a = e.copy()
    a[1] = np.nan
    with pytest.raises(AssertionError):
        assert_close(a, e, rtol=1e-4, atol=1e-5)
    with pytest.raises(AssertionError):
        assert_close_fp32_derived(a, e, e)
    assert_close(a, a, rtol=1e-4, atol=1e-5)


def test_fp32_derived_per_row_spread():
    """per_row takes the spread term over each row: an element off by 3e-4
    in a row whose float32 error is 1e-7 fails, though another row's 1e-3
    float32 error would have covered it tensor-wide."""
    from tests.conftest import assert_close_fp32_derived

    e = np.linspace(-1.0, 1.0, 40).reshape(4, 10)
    e32 = e.copy()
    e32[0, :] += 1e-3
    e32[1:, :] += 1e-7
    a = e.copy()
    a[2, 3] += 3e-4
    assert_close_fp32_derived(a, e, e32)
    with pytest.raises(AssertionError):
        assert_close_fp32_derived(a, e, e32, per_row=True)
    a[2, 3] = e[2, 3]
    a[0, 5] += 2.5e-3
    assert_close_fp32_derived(a, e, e32, per_row=True)


def test_bf16_store_bound_covers_fp32_sums_stored_in_bf16(rng):
    """conftest.bf16_store_bound: float32 sums of products (row sums of a
    random sparse-like matrix, sequential and pairwise orders) rounded once to
    bf16 lie within the bound around the float64 sum; a result two bf16
    spacings away (a rounding too many, or a dropped term of that size)
    does not; and an input error carried through |P| widens it exactly by
    that propagated amount."""
    import torch

    from tests.conftest import assert_within, bf16_store_bound

    n, k = 400, 37
    P = rng.random((n, k)) * (rng.random((n, k)) < 0.5)
    x = O.bf16_round(rng.standard_normal(k))
    exact = P @ x
    terms = np.abs(P) @ np.abs(x)
    bound = bf16_store_bound(exact, terms, k)
    P32, x32 = P.astype(np.float32), x.astype(np.float32)
    for sums in (np.array([np.float32(sum(np.float32(p) * np.float32(v) for p, v in zip(row, x32))) for row in P32]),
                 (P32 @ x32).astype(np.float32)):
        stored = torch.from_numpy(sums).to(torch.bfloat16).double().numpy()
        assert_within(stored, exact, bound, "fp32 sum stored in bf16")
    off = exact + 2 * 2.0 ** -7 * np.abs(exact) + 1e-3
    with pytest.raises(AssertionError, match="outside the derived bound"):
        assert_within(off, exact, bound, "two spacings off")
    carried = np.full(k, 1e-3)
    wider = bf16_store_bound(exact, terms, k, np.abs(P) @ carried)
    assert np.all(wider > bound)
    assert np.allclose(wider - bound, (1 + 2.0 ** -8) * (np.abs(P) @ carried))
