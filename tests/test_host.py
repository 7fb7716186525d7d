"""CPU tests of the product's host logic: graph preparation (bit-exact
against the oracle), synthetic generators, row schedules, and the C-ABI
library (loads, exports every declared symbol; host-only entry points)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from cign_amd import _lib, graph, graphgen
from cign_amd.schedule import LIGHT_MAX, SEG_EDGES, build_row_schedule
from oracle import cign_oracle as O
from tests.conftest import random_gat_graph

ROOT = Path(__file__).resolve().parents[1]


def test_normalized_adjacency_bit_exact(rng):
    n = 300
    ei = np.stack([rng.integers(0, n, 2000), rng.integers(0, n, 2000)])
    used, P = graph.build_sparse_normalized_adjacency(torch.from_numpy(ei), n)
    o_used, (pr, pc, pv) = O.normalized_adjacency(ei, n)
    assert np.array_equal(used.numpy(), o_used)
    assert np.array_equal(P.indices()[0].numpy(), pr)
    assert np.array_equal(P.indices()[1].numpy(), pc)
    assert np.array_equal(P.values().numpy(), pv)


def test_fixed_csr_operator_and_transpose(rng):
    n = 200
    ei = np.stack([rng.integers(0, n, 900), rng.integers(0, n, 900)])
    _, P = graph.build_sparse_normalized_adjacency(torch.from_numpy(ei), n)
    op = graph.prepare_fixed_csr_operator(P)
    _, (pr, pc, pv) = O.normalized_adjacency(ei, n)
    rp, c, order = O.csr_from_coo(pr, pc, n)
    assert np.array_equal(op.csr.crow_indices().numpy(), rp)
    assert np.array_equal(op.csr.col_indices().numpy(), c)
    assert np.array_equal(op.csr.values().numpy(), pv[order])
    trp, tc, tv = O.transpose_csr(rp, c, pv[order], n)
    assert np.array_equal(op.csr_t.crow_indices().numpy(), trp)
    assert np.array_equal(op.csr_t.col_indices().numpy(), tc)
    assert np.array_equal(op.csr_t.values().numpy(), tv.astype(np.float32))


def test_gat_graph_format_bit_exact(rng):
    n = 500
    ei = random_gat_graph(rng, n, avg_deg=7, hubs={3: 300})
    # prepare_fused_gat_graph takes PyG source->target edges.
    (rowptr, col), (row, colptr), perm = graph.prepare_fused_gat_graph(torch.from_numpy(ei), n)
    o = O.gat_graph_format(ei, n)
    for got, want in zip((rowptr, col, row, colptr, perm), o):
        assert got.dtype == torch.int32
        assert np.array_equal(got.numpy(), want)


def test_prepare_gat_edge_index():
    ei = torch.tensor([[0, 1, 1, 2, 2], [1, 1, 0, 2, 0]])
    out = graph.prepare_gat_edge_index(ei, 3)
    assert np.array_equal(out.numpy(), O.gat_edge_index(ei.numpy(), 3))
    assert out.tolist() == [[0, 1, 2, 0, 1, 2], [1, 0, 0, 0, 1, 2]]


def test_chung_lu_c2_shape():
    ei = graphgen.chung_lu_directed(24492, 186100, gamma=2.5, max_degree=1100, seed=0)
    assert ei.shape == (2, 186100)
    assert (ei[0] != ei[1]).all()
    key = ei[0] * 24492 + ei[1]
    assert np.unique(key).size == key.size
    deg = np.bincount(ei[1], minlength=24492)
    assert (np.diff(deg) <= 0).all()  # relabelled by descending degree
    assert 900 <= deg.max() <= 1100
    again = graphgen.chung_lu_directed(24492, 186100, gamma=2.5, max_degree=1100, seed=0)
    assert np.array_equal(ei, again)


def test_uniform_out_degree():
    ei = graphgen.uniform_out_degree(200, 8, seed=0)
    assert ei.shape == (2, 1600)
    assert (ei[0] != ei[1]).all()
    assert (np.bincount(ei[0], minlength=200) == 8).all()


def _sched_host(rowptr):
    s = build_row_schedule(torch.from_numpy(rowptr), device="cpu")
    return s, s.buf.numpy()


def test_row_schedule_layout(rng):
    deg = rng.integers(0, 40, 300)
    deg[5], deg[9], deg[11] = 1000, 257, 65
    rowptr = np.concatenate([[0], np.cumsum(deg)])
    s, b = _sched_host(rowptr)
    assert (s.n_light, s.n_hrow) == ((deg <= LIGHT_MAX).sum(), (deg > LIGHT_MAX).sum())
    assert s.n_seg == sum(-(-d // SEG_EDGES) for d in deg if d > LIGHT_MAX)
    lt = deg[deg <= LIGHT_MAX]
    assert tuple(b[:12]) == (s.n_light, s.n_seg, s.n_hrow, SEG_EDGES, LIGHT_MAX, 0,
                             *((lt > (1 << k)).sum() for k in range(6)))
    assert np.array_equal(s.header, b[:12])
    rec = b[12:12 + 4 * s.n_light].reshape(-1, 4)
    light = rec[:, 0]
    assert sorted(light.tolist()) == sorted(np.nonzero(deg <= LIGHT_MAX)[0].tolist())
    assert np.array_equal(rec[:, 1], rowptr[light]) and np.array_equal(rec[:, 2], rowptr[light + 1])
    assert (np.diff(deg[light]) <= 0).all()
    off = 12 + 4 * s.n_light
    seg = b[off:off + 4 * s.n_seg].reshape(-1, 4)
    hrow = b[off + 4 * s.n_seg:].reshape(-1, 2)
    covered = {}
    for r, beg, end, h in seg:
        assert rowptr[r] <= beg < end <= rowptr[r + 1] and end - beg <= SEG_EDGES
        covered.setdefault(r, []).append((beg, end))
        first, cnt = hrow[h]
        assert seg[first][0] == r
    for r, spans in covered.items():
        spans.sort()
        assert spans[0][0] == rowptr[r] and spans[-1][1] == rowptr[r + 1]
        assert all(a[1] == b_[0] for a, b_ in zip(spans, spans[1:]))


def test_library_exports_declared_symbols():
    lib = _lib.load_library(require_gpu=False)
    header = (ROOT / "include" / "cign_amd.h").read_text()
    declared = set(re.findall(r"\b(cign_[a-z0-9_]+)\s*\(", header))
    assert declared, "no declarations parsed"
    assert declared == set(_lib.exported_symbols()), declared ^ set(_lib.exported_symbols())
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared:
        assert hasattr(raw, name), name
    assert lib.cign_version() >= 1


def test_host_entry_points_reject_bad_arguments():
    lib = _lib.load_library(require_gpu=False)
    rp = np.array([0, 2, 1], dtype=np.int64)  # not monotone
    a, b, c = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    t = ctypes.c_int64()
    rc = lib.cign_row_schedule_size(rp.ctypes.data, 2, 64, 256, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c),
                                    ctypes.byref(t))
    assert rc == 1 and b"monotone" in lib.cign_last_error()


def test_product_never_imports_oracle():
    for p in (ROOT / "cign_amd").rglob("*.py"):
        text = p.read_text()
        assert not re.search(r"^\s*(from|import)\s+(\.\.)?oracle", text, re.M), p
        assert "cign_oracle" not in text, p


def _gat_wave_ranges(rowptr):
    """Edge ranges walked by the GAT kernels' wavefronts (light rows and the
    four 16-edge waves of each segment), from the real schedule."""
    from cign_amd.schedule import GAT_LIGHT_MAX, GAT_SEG_EDGES

    s = build_row_schedule(torch.from_numpy(rowptr.astype(np.int64)), device="cpu", light_max=GAT_LIGHT_MAX,
                           seg_edges=GAT_SEG_EDGES)
    b = s.buf.numpy()
    rec = b[12:12 + 4 * s.n_light].reshape(-1, 4)
    seg = b[12 + 4 * s.n_light:12 + 4 * s.n_light + 4 * s.n_seg].reshape(-1, 4)
    out = [(r[1], r[2]) for r in rec]
    for _, beg, end, _ in seg:
        for w in range(4):
            eb = min(beg + 16 * w, end)
            out.append((eb, min(end, eb + 16)))
    return out


def test_gat_edge_index_reads_stay_in_bounds(rng):
    # Emulates the clamped index arithmetic of gat_kernels.h: a wave reads
    # col/rowind/perm at t < ee ? t : eb for every lane and tile, and reads
    # nothing when its range is empty (an empty range may start at nnz).
    rowptr = np.array([0, 0, 1, 1, 3, 3])  # rows 0, 2, 4 empty; row 4 starts at nnz
    graphs = [rowptr]
    ei = random_gat_graph(rng, 300, avg_deg=5, hubs={4: 800})
    (rp, _), (_, cp), _ = graph.to_graph_format(torch.from_numpy(ei).flip(0), size=(300, 300))
    graphs += [rp.numpy(), cp.numpy()]
    for H in (1, 4, 6, 12):
        HP = 4 if H <= 4 else (8 if H <= 8 else 32)
        epw = 64 // HP
        for rp in graphs:
            nnz = int(rp[-1])
            for eb, ee in _gat_wave_ranges(rp):
                if ee <= eb:
                    continue
                nt = -(-(ee - eb) // epw)
                assert nt <= max(1, 16 // epw)
                for el in range(epw):
                    for k in range(nt):
                        t = eb + el + k * epw
                        assert 0 <= (t if t < ee else eb) < nnz


def test_segment_edges_for_graph_size():
    """Segment length: 512 on small graphs (c2/c3), 16384 at c5 (62.4M
    edges), a power of two in between that grows with nnz, never below the
    floor asked for."""
    from cign_amd.schedule import SEG_EDGES, SEG_EDGES_MAX, segment_edges_for

    assert segment_edges_for(0) == SEG_EDGES == 512
    assert segment_edges_for(210_592) == 512
    assert segment_edges_for(210_592, 1024) == 1024
    assert segment_edges_for(62_400_000) == segment_edges_for(62_400_000, 1024) == SEG_EDGES_MAX == 16384
    prev = 0
    for nnz in np.logspace(3, 9, 40).astype(np.int64):
        s = segment_edges_for(int(nnz))
        assert s >= prev and s & (s - 1) == 0 and s % 256 == 0
        prev = s


def test_gat_schedules_take_the_graph_size_segment(rng):
    """The GAT feature-layout schedules (the library accepts any multiple of
    256) get the SpMM's segment length for the graph size: 512 on a small
    graph for every pass and row width (header word 3 is the schedule's
    segment length); the SpMM plan's schedules likewise."""
    from cign_amd import schedule as S

    deg = rng.integers(0, 30, 400)
    deg[7] = 3000
    rowptr = torch.from_numpy(np.concatenate([[0], np.cumsum(deg)]).astype(np.int32))
    seg = lambda sch: int(sch.header[3])
    assert seg(S.gat_schedule(rowptr, 0, 0, 4, 16)) == 512  # 4 x 16 fp32: 256-byte rows
    assert seg(S.gat_schedule(rowptr, 0, 1, 4, 32)) == 512  # 4 x 32 bf16: 256-byte rows
    assert seg(S.gat_schedule(rowptr, 0, 0, 6, 256)) == 512  # wide rows
    assert seg(S.gat_schedule(rowptr, 1, 0, 4, 16)) == 512  # backward passes
    assert seg(S.build_row_schedule(rowptr)) == 512


def test_spmm_noalloc_rejects_schedules_beyond_its_scratch():
    """The no-allocation SpMM checks its fixed scratch size on the host, before
    any HIP call: a schedule needing more partial sums or counters is refused
    with the sizes in the error text."""
    lib = _lib.load_library(require_gpu=False)
    hdr = np.zeros(12, dtype=np.int32)
    hdr[0], hdr[1], hdr[2] = 10, 1_000_000, 10  # 10^6 segments x 512 columns of fp32 partials
    rc = lib.cign_spmm_fwd3_noalloc(None, 0, 20, 512, None, None, None, hdr.ctypes.data, None, None, None, None)
    assert rc == 1 and b"scratch holds" in lib.cign_last_error()
    hdr[1], hdr[2] = 1, 300_000  # more merge counters than the scratch holds
    rc = lib.cign_spmm_fwd3_noalloc(None, 0, 300_010, 4, None, None, None, hdr.ctypes.data, None, None, None, None)
    assert rc == 1 and b"262144 counters" in lib.cign_last_error()


def test_dispatch_signatures_match_reference_vectors(monkeypatch):
    """canonical_config / cign_speed_signature give the reference's keys and
    dicts (vectors recorded from the reference by
    tests/golden/make_dispatch_signatures.py): option forms --a v / --a=v,
    list options, booleans, repeated options, the switch environment."""
    import json

    from cign_amd.cign_dispatch_utils import cign_speed_signature
    from cign_amd.generic_dispatch import canonical_config

    cases = json.loads((ROOT / "tests" / "golden" / "dispatch_signatures.json").read_text())["cases"]
    assert len(cases) >= 20
    keys = ("CIGN_ALPHA_SCORE_MODE", "CIGN_INTERACTION_MODE", "CIGN_ALPHA_WEIGHTING_MODE", "CIGN_OUTER_NONLINEARITY",
            "CLIFFORD_EDGE_DROP_RATIO")
    for c in cases:
        for k in keys:
            monkeypatch.delenv(k, raising=False)
        for k, v in c["env"].items():
            monkeypatch.setenv(k, v)
        assert canonical_config(c["argv"]) == (c["canonical_key"], c["canonical_cfg"]), c["argv"]
        assert cign_speed_signature(c["argv"]) == (c["cign_key"], c["cign_cfg"]), (c["argv"], c["env"])
    monkeypatch.setenv("CIGN_INTERACTION_MODE", "sideways")
    with pytest.raises(ValueError, match="old/new"):
        cign_speed_signature([])


def _header_prototypes():
    """{name: (return type, [parameter types])} of include/cign_amd.h."""
    text = (ROOT / "include" / "cign_amd.h").read_text()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    protos = {}
    for ret, name, params in re.findall(r"([A-Za-z_][\w ]*?\**)\s*\b(cign_\w+)\s*\(([^)]*)\)\s*;", text):
        params = " ".join(params.split())
        types = [] if params in ("", "void") else [p.strip().rsplit(" ", 1)[0] if "*" not in p.rsplit(" ", 1)[-1]
                                                  else p.strip() for p in params.split(",")]
        protos[name] = (" ".join(ret.split()), types)
    return protos


def test_ctypes_signatures_match_header():
    """Every entry point's ctypes argument list has the header's length and,
    argument by argument, the same kind (pointer, int32, int64, uint64,
    float), and the same return kind: a mismatch would pass arguments in the
    wrong registers without any error."""
    def kind(t):
        t = t.replace("const ", "").strip()
        if "*" in t:
            return C.c_void_p
        return {"int": C.c_int32, "int32_t": C.c_int32, "int64_t": C.c_int64, "uint64_t": C.c_uint64,
                "float": C.c_float}[t]

    import ctypes as C

    protos = _header_prototypes()
    assert set(protos) == set(_lib._SIGNATURES), set(protos) ^ set(_lib._SIGNATURES)
    for name, (ret, params) in protos.items():
        sig_ret, sig_args = _lib._SIGNATURES[name]
        assert len(params) == len(sig_args), f"{name}: header {len(params)} arguments, ctypes {len(sig_args)}"
        for i, (p, a) in enumerate(zip(params, sig_args)):
            assert C.sizeof(kind(p)) == C.sizeof(a) and (kind(p) is C.c_float) == (a is C.c_float), \
                f"{name} argument {i}: header {p!r}, ctypes {a}"
        if ret.endswith("*"):
            assert sig_ret in (C.c_void_p, C.c_char_p), name
        else:
            assert C.sizeof(kind(ret)) == C.sizeof(sig_ret), f"{name}: returns {ret}, ctypes {sig_ret}"
