"""GPU parity of the collapsed GAT (forward + backward) against the oracle,
through the drop-in API (collapsed_gat.ensure_collapsed_gat_loaded().forward/
backward and collapsed_gat_mean_bias_silu with autograd), which calls the
C-ABI. Tolerances: fp32 1e-4 rel / 1e-5 abs; outputs stored in bf16 (from
fp32 math on bf16 inputs, the oracle on the same rounded inputs) 2e-2
relative with a 1e-5 absolute floor (one bf16 rounding is 2^-8 relative;
the floor covers fp32 rounding near zero). Dropout masks and CSR/CSC/perm
are bit-exact."""
import numpy as np
import pytest
import torch

from oracle import cign_oracle as O
from tests.conftest import assert_close, random_gat_graph

pytestmark = pytest.mark.gpu
TOL = {torch.float32: dict(rtol=1e-4, atol=1e-5), torch.bfloat16: dict(rtol=2e-2, atol=1e-5)}


def _graph(rng, n, hubs):
    ei = random_gat_graph(rng, n, avg_deg=5, hubs=hubs)
    # also give two nodes a large out-degree (heavy CSC columns)
    for j in list(hubs)[:2]:
        extra = np.stack([np.full(min(600, n), j), rng.choice(n, size=min(600, n), replace=False)])
        ei = np.concatenate([ei, extra], 1)
    r, c, _ = O.coalesce(ei[0], ei[1], n)
    return np.stack([r, c])


def _dev_graph(ei, n):
    from cign_amd.graph import prepare_fused_gat_graph

    (rowptr, col), (row, colptr), perm = prepare_fused_gat_graph(torch.from_numpy(ei), n)
    return tuple(t.cuda() for t in (rowptr, col, row, colptr, perm))


def _inputs(rng, n, H, C, dtype):
    x = torch.from_numpy(rng.standard_normal((n, H, C)).astype(np.float32)).to(dtype).cuda()
    ar = torch.from_numpy(rng.standard_normal((n, H)).astype(np.float32)).cuda()
    ac = torch.from_numpy(rng.standard_normal((n, H)).astype(np.float32)).cuda()
    b = torch.from_numpy(rng.standard_normal(C).astype(np.float32)).cuda()
    gy = torch.from_numpy(rng.standard_normal((n, C)).astype(np.float32)).to(dtype).cuda()
    return x, ar, ac, b, gy


CASES = [
    (4, 16, 0.0, torch.float32, 600, {3: 1000, 7: 300}),
    (4, 16, 0.3, torch.float32, 600, {3: 1000, 7: 300}),
    (1, 3, 0.0, torch.float32, 500, {1: 900}),
    (6, 40, 0.2, torch.float32, 400, {0: 700, 2: 260}),
    (8, 32, 0.0, torch.float32, 256, {5: 513}),
    (12, 8, 0.1, torch.float32, 200, {9: 257}),
    (6, 256, 0.0, torch.float32, 300, {4: 800}),
    (32, 16, 0.1, torch.float32, 64, {}),
    (2, 5, 0.0, torch.float32, 100, {}),
    (4, 16, 0.0, torch.bfloat16, 600, {3: 1000}),
    (4, 32, 0.25, torch.bfloat16, 400, {0: 700}),
    (6, 256, 0.0, torch.bfloat16, 200, {2: 300}),
    (3, 8, 0.1, torch.float32, 300, {1: 2000}),
    (1, 256, 0.0, torch.float32, 200, {0: 600}),
    (5, 32, 0.0, torch.bfloat16, 300, {2: 520}),
    (1, 4, 0.1, torch.float32, 300, {2: 400}),
    (4, 4, 0.0, torch.float32, 300, {1: 700}),
    (2, 8, 0.2, torch.bfloat16, 300, {1: 500}),
    # four heads of 32 and 64 channels: the channel-major columns kernel with
    # 8 and 16 lanes per column (large-graph kernels)
    (4, 32, 0.0, torch.float32, 400, {2: 900}),
    (4, 64, 0.1, torch.float32, 300, {1: 700}),
    (4, 64, 0.0, torch.bfloat16, 300, {0: 600, 5: 70}),
    # wide rows (several chunks per lane): V = H*C/(W*64) = 4, 4, 8, 2, 2 and
    # a narrow bf16 row of 64 chunks
    (4, 256, 0.1, torch.float32, 300, {2: 700}),
    (8, 128, 0.0, torch.float32, 300, {1: 400}),
    (8, 256, 0.2, torch.float32, 150, {0: 300}),
    (8, 64, 0.3, torch.float32, 300, {3: 600}),
    (4, 256, 0.2, torch.bfloat16, 300, {2: 500}),
    (2, 256, 0.0, torch.bfloat16, 300, {1: 400}),
]


def _forward(ext, agg_mode, *args):
    """ext.forward, or with agg_mode ext.forward_agg (the autograd path): the
    outputs and the per-row aggregate buffer (None for shapes without one)."""
    if agg_mode:
        return ext.forward_agg(*args, True)
    return ext.forward(*args), None


@pytest.mark.parametrize("big", [False, True], ids=["small-graph-kernels", "large-graph-kernels"])
@pytest.mark.parametrize("agg_mode", [False, True])
@pytest.mark.parametrize("H,C,p,dtype,n,hubs", CASES)
def test_ext_forward_backward_matches_oracle(H, C, p, dtype, n, hubs, agg_mode, big, monkeypatch):
    """big: the kernel variants the library runs from 4M edges up (the lanes
    of a head sharing the softmax work, other batch caps), forced at these
    sizes through CIGN_GAT_BIG_GRAPH_EDGES=0."""
    from cign_amd import _lib
    from cign_amd.collapsed_gat import ensure_collapsed_gat_loaded

    if big:
        monkeypatch.setenv("CIGN_GAT_BIG_GRAPH_EDGES", "0")
    print(f"gat ext H={H} C={C} p={p} dtype={dtype} n={n} agg={agg_mode} big={big}", flush=True)
    rng = np.random.default_rng(H * 1000 + C)
    ei = _graph(rng, n, hubs)
    rowptr, col, row, colptr, perm = _dev_graph(ei, n)
    x, ar, ac, b, gy = _inputs(rng, n, H, C, dtype)
    ext = ensure_collapsed_gat_loaded()
    seed = 0x5EED_1234
    (out, pre, emax, esum, mask), agg = _forward(ext, agg_mode, ar, ac, rowptr, col, 0.2, x, b, p, seed)
    floats = int(_lib.load_library().cign_gat_row_agg_floats(_lib.dtype_code(x), n, H, C))
    assert (agg is None) == (not agg_mode or floats == 0)
    grads = ext.backward(0.2, p, rowptr, col, colptr, row, perm, emax, esum, mask, x, ar, ac, pre, gy, agg)
    rp, cl = rowptr.cpu().numpy().astype(np.int64), col.cpu().numpy().astype(np.int64)
    E = cl.size
    keep = O.gat_dropout_keep(seed, E * H, p).reshape(E, H) if p > 0 else None
    if p > 0:
        assert np.array_equal(mask.cpu().numpy() != 0, keep), "dropout mask must be bit-exact"
    xn, gyn = x.double().cpu().numpy(), gy.double().cpu().numpy()
    arn, acn, bn = ar.double().cpu().numpy(), ac.double().cpu().numpy(), b.double().cpu().numpy()
    f = O.collapsed_gat_forward(arn, acn, rp, cl, 0.2, xn, bn, p, keep)
    g = O.collapsed_gat_backward(arn, acn, rp, cl, 0.2, xn, bn, gyn, p, keep)
    tol, t32 = TOL[dtype], TOL[torch.float32]
    assert_close(out.double().cpu().numpy(), f["out"], name="out", **tol)
    assert_close(pre.cpu().numpy(), f["pre"], name="pre", **t32)
    assert_close(emax.cpu().numpy(), f["emax"], name="edge_max", **t32)
    assert_close(esum.cpu().numpy(), f["esum"], name="edge_sum", **t32)
    gx, gar, gac, gb = grads
    assert gx.dtype == dtype and gar.dtype == torch.float32
    assert_close(gx.double().cpu().numpy(), g["grad_feat"], name="grad_feat", **tol)
    assert_close(gar.cpu().numpy(), g["grad_attn_row"], name="grad_attn_row", **t32)
    assert_close(gac.cpu().numpy(), g["grad_attn_col"], name="grad_attn_col", **t32)
    assert_close(gb.cpu().numpy(), g["grad_bias"], name="grad_bias", **t32)
    if agg is not None:
        # The aggregates themselves: per (row, head) softmax-weighted sums of
        # the source rows, with and without the LeakyReLU slope, and sum s l'.
        F = H * C
        a = agg.double().cpu().numpy()
        ref = O.collapsed_gat_row_aggregates(arn, acn, rp, cl, 0.2, xn, p, keep)
        assert_close(a[:n * F].reshape(n, H, C), ref["agg"], name="agg", **tol)
        assert_close(a[n * F:2 * n * F].reshape(n, H, C), ref["agg_l"], name="agg_l", **tol)
        assert_close(a[2 * n * F:].reshape(n, H), ref["b_l"], name="b_l", **t32)


@pytest.fixture(scope="module")
def c2():
    from cign_amd import workloads

    return workloads.build(workloads.C2, device="cuda")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_autograd_full_c2(c2, dtype):
    """BASELINE config c2 at full size (N = 24,492, E = 210,592, 4 heads x
    16) through the autograd wrapper, fp32 and bf16 features, against the
    float64 oracle on the same (bf16-rounded) values. bf16 stores the output
    and grad_feat in bf16 from fp32 math, so they sit within half a bf16
    spacing (2^-8 relative) of the oracle plus fp32 rounding: 2e-2 relative
    with a 1e-5 absolute floor; the fp32 outputs (attention gradients, grad
    bias) keep 1e-4 / 1e-5."""
    from cign_amd.collapsed_gat import collapsed_gat_mean_bias_silu

    print(f"gat autograd c2 full size H=4 C=16 dtype={dtype}", flush=True)
    (rowptr, col), (row, colptr), perm = c2.gat_graph
    rng = np.random.default_rng(0)
    n, H, C = c2.n, 4, 16
    x, ar, ac, b, gy = _inputs(rng, n, H, C, dtype)
    for t in (x, ar, ac, b):
        t.requires_grad_(True)
    y = collapsed_gat_mean_bias_silu(ar, ac, (rowptr, col), (row, colptr), perm, 0.2, x, b, 0.0)
    assert y.dtype == dtype
    y.backward(gy)
    rp, cl = rowptr.cpu().numpy().astype(np.int64), col.cpu().numpy().astype(np.int64)
    args = (ar.detach().double().cpu().numpy(), ac.detach().double().cpu().numpy(), rp, cl, 0.2,
            x.detach().double().cpu().numpy(), b.detach().double().cpu().numpy())
    f = O.collapsed_gat_forward(*args)
    g = O.collapsed_gat_backward(*args, gy.double().cpu().numpy())
    t = TOL[torch.float32]
    tl = TOL[dtype]
    assert_close(y.detach().double().cpu().numpy(), f["out"], name="out", **tl)
    assert x.grad.dtype == dtype
    assert_close(x.grad.double().cpu().numpy(), g["grad_feat"], name="grad_feat", **tl)
    assert_close(ar.grad.cpu().numpy(), g["grad_attn_row"], name="grad_attn_row", **t)
    assert_close(ac.grad.cpu().numpy(), g["grad_attn_col"], name="grad_attn_col", **t)
    assert_close(b.grad.cpu().numpy(), g["grad_bias"], name="grad_bias", **t)
    # Size-independent properties at full size: sum over edges of the softmax
    # is 1 per (row, head) -> constant features give out = SiLU(mean_h v_h + b).
    v = torch.from_numpy(rng.standard_normal((1, H, C)).astype(np.float32)).to(dtype).cuda()
    yc = collapsed_gat_mean_bias_silu(ar.detach(), ac.detach(), (rowptr, col), (row, colptr), perm, 0.2,
                                      v.expand(n, H, C).contiguous(), b.detach(), 0.0)
    pre = (v.double().mean(1) + b.detach().double()).cpu().numpy()
    assert_close(yc.double().cpu().numpy(), np.broadcast_to(pre / (1 + np.exp(-pre)), (n, C)), name="constant", **tl)


def test_dropout_seed_stream_matches_reference_formula(c2):
    import cign_amd.collapsed_gat as cg

    (rowptr, col), (row, colptr), perm = c2.gat_graph
    rng = np.random.default_rng(1)
    n, H, C = c2.n, 4, 16
    x, ar, ac, b, _ = _inputs(rng, n, H, C, torch.float32)
    torch.manual_seed(1234)
    start = next(cg._CALL_COUNTER)  # consume one id so the next call uses start + 1
    seen = []
    orig = cg._CollapsedGATFn.apply

    def spy(*a):
        seen.append(a[-1])
        return orig(*a)

    cg._CollapsedGATFn.apply = spy
    try:
        cg.collapsed_gat_mean_bias_silu(ar, ac, (rowptr, col), (row, colptr), perm, 0.2, x, b, 0.5)
        cg.collapsed_gat_mean_bias_silu(ar, ac, (rowptr, col), (row, colptr), perm, 0.2, x, b, 0.0)
    finally:
        cg._CollapsedGATFn.apply = orig
    assert seen[0] == O.collapsed_gat_seed(1234, start + 1, 0.5)
    assert seen[1] == 0
    # The mask drawn with that seed is the reference's bit for bit.
    ext = cg.ensure_collapsed_gat_loaded()
    _, _, _, _, mask = ext.forward(ar, ac, rowptr, col, 0.2, x, b, 0.5, seen[0])
    E = col.numel()
    assert np.array_equal(mask.cpu().numpy() != 0, O.gat_dropout_keep(seen[0], E * H, 0.5).reshape(E, H))


def test_rows_without_edges_and_single_node():
    from cign_amd.collapsed_gat import ensure_collapsed_gat_loaded

    ext = ensure_collapsed_gat_loaded()
    n, H, C = 5, 2, 4
    rowptr = torch.tensor([0, 0, 1, 1, 3, 3], dtype=torch.int32, device="cuda")  # rows 0, 2, 4 empty
    col = torch.tensor([2, 0, 1], dtype=torch.int32, device="cuda")
    rng = np.random.default_rng(2)
    x, ar, ac, b, gy = _inputs(rng, n, H, C, torch.float32)
    out, pre, emax, esum, _ = ext.forward(ar, ac, rowptr, col, 0.2, x, b, 0.0, 0)
    assert torch.allclose(pre[0], b) and torch.allclose(pre[2], b) and torch.allclose(pre[4], b)
    assert float(esum[0, 0]) == 0.0 and float(emax[0, 0]) == float(np.float32(-1.0e38))
    from cign_amd.graph import to_graph_format

    rows = torch.repeat_interleave(torch.arange(n), torch.diff(rowptr.cpu().long()))
    (_, _), (row, colptr), perm = to_graph_format(torch.stack([rows, col.cpu().long()]), size=(n, n))
    gx, gar, gac, gb = ext.backward(0.2, 0.0, rowptr, col, colptr.cuda(), row.cuda(), perm.cuda(), emax, esum,
                                    torch.empty(3, H, dtype=torch.uint8, device="cuda"), x, ar, ac, pre, gy)
    g = O.collapsed_gat_backward(ar.double().cpu().numpy(), ac.double().cpu().numpy(), rowptr.cpu().numpy(),
                                 col.cpu().numpy(), 0.2, x.double().cpu().numpy(), b.double().cpu().numpy(),
                                 gy.double().cpu().numpy())
    assert_close(gx.cpu().numpy(), g["grad_feat"], name="gx", **TOL[torch.float32])
    assert_close(gb.cpu().numpy(), g["grad_bias"], name="gb", **TOL[torch.float32])
    # One node with its self-loop.
    one = torch.tensor([0, 1], dtype=torch.int32, device="cuda")
    z = torch.zeros(1, dtype=torch.int32, device="cuda")
    x1, ar1, ac1, b1, _ = _inputs(rng, 1, 3, 7, torch.float32)
    out1, pre1, _, _, _ = ext.forward(ar1, ac1, one, z, 0.2, x1, b1, 0.0, 0)
    assert_close(pre1.cpu().numpy(), (x1.double().mean(1) + b1.double()).cpu().numpy(), name="one",
                 **TOL[torch.float32])


def test_deterministic_bitwise(c2):
    from cign_amd.collapsed_gat import ensure_collapsed_gat_loaded

    (rowptr, col), (row, colptr), perm = c2.gat_graph
    rng = np.random.default_rng(3)
    x, ar, ac, b, gy = _inputs(rng, c2.n, 4, 16, torch.float32)
    ext = ensure_collapsed_gat_loaded()
    r1 = ext.forward(ar, ac, rowptr, col, 0.2, x, b, 0.1, 77)
    r2 = ext.forward(ar, ac, rowptr, col, 0.2, x, b, 0.1, 77)
    for a, c in zip(r1, r2):
        assert torch.equal(a, c)
    g1 = ext.backward(0.2, 0.1, rowptr, col, colptr, row, perm, r1[2], r1[3], r1[4], x, ar, ac, r1[1], gy)
    g2 = ext.backward(0.2, 0.1, rowptr, col, colptr, row, perm, r1[2], r1[3], r1[4], x, ar, ac, r1[1], gy)
    for a, c in zip(g1, g2):
        assert torch.equal(a, c)


def test_argument_errors(c2):
    from cign_amd.collapsed_gat import collapsed_gat_mean_bias_silu

    (rowptr, col), (row, colptr), perm = c2.gat_graph
    n = c2.n
    ar = torch.zeros(n, 33, device="cuda")
    with pytest.raises(ValueError, match="H<=32"):
        collapsed_gat_mean_bias_silu(ar, ar, (rowptr, col), (row, colptr), perm, 0.2,
                                     torch.zeros(n, 33, 4, device="cuda"), torch.zeros(4, device="cuda"), 0.0)
    with pytest.raises(TypeError):
        collapsed_gat_mean_bias_silu(ar, ar, (rowptr, col), (row, colptr), perm, 0.2, torch.zeros(n, 4, 4),
                                     torch.zeros(4), 0.0)
    with pytest.raises(ValueError, match="bias"):
        collapsed_gat_mean_bias_silu(ar[:, :4], ar[:, :4], (rowptr, col), (row, colptr), perm, 0.2,
                                     torch.zeros(n, 4, 4, device="cuda"), None, 0.0)


@pytest.mark.parametrize("big", [False, True], ids=["small-graph-kernels", "large-graph-kernels"])
@pytest.mark.parametrize("agg_mode", [False, True])
@pytest.mark.parametrize("seg", [256, 1024, 4096])
@pytest.mark.parametrize("dtype,p", [(torch.float32, 0.0), (torch.float32, 0.2), (torch.bfloat16, 0.0)])
def test_long_segments_multi_round(seg, dtype, p, agg_mode, big, monkeypatch):
    """Hub rows/columns of 2,500-6,000 edges cut into segments of `seg` edges
    (several 256-edge rounds per workgroup, several workgroups per row)."""
    import cign_amd.schedule as S

    if big:
        monkeypatch.setenv("CIGN_GAT_BIG_GRAPH_EDGES", "0")
    print(f"gat long segments seg={seg} dtype={dtype} p={p} agg={agg_mode} big={big}", flush=True)
    monkeypatch.setattr(S, "segment_edges_for", lambda nnz, floor=512: seg)
    S._CACHE.clear()
    rng = np.random.default_rng(seg)
    n, H, C = 7000, 4, 16
    ei = random_gat_graph(rng, n, avg_deg=4, hubs={3: 6000, 40: 2500})
    ei = np.concatenate([ei, np.stack([np.full(5000, 11), rng.choice(n, 5000, replace=False)])], 1)
    r, c, _ = O.coalesce(ei[0], ei[1], n)
    rowptr, col, row, colptr, perm = _dev_graph(np.stack([r, c]), n)
    x, ar, ac, b, gy = _inputs(rng, n, H, C, dtype)
    ext = __import__("cign_amd.collapsed_gat", fromlist=["x"]).ensure_collapsed_gat_loaded()
    (out, pre, emax, esum, mask), agg = _forward(ext, agg_mode, ar, ac, rowptr, col, 0.2, x, b, p, 99)
    assert (agg is not None) == agg_mode
    gf, gar, gac, gb = ext.backward(0.2, p, rowptr, col, colptr, row, perm, emax, esum, mask, x, ar, ac, pre, gy,
                                    agg)
    rp, cl = rowptr.cpu().numpy().astype(np.int64), col.cpu().numpy().astype(np.int64)
    keep = mask.cpu().numpy().astype(bool) if p > 0 else None
    if p > 0:
        assert np.array_equal(keep.reshape(-1), O.gat_dropout_keep(99, cl.size * H, p))
    args = (ar.double().cpu().numpy(), ac.double().cpu().numpy(), rp, cl, 0.2, x.double().cpu().numpy(),
            b.double().cpu().numpy())
    f = O.collapsed_gat_forward(*args, p=p, keep=keep)
    gr = O.collapsed_gat_backward(*args, gy.double().cpu().numpy(), p=p, keep=keep)
    tol = TOL[dtype]
    assert_close(pre.cpu().numpy(), f["pre"], name="pre", **tol)
    assert_close(gf.double().cpu().numpy(), gr["grad_feat"], name="grad_feat", **tol)
    assert_close(gar.cpu().numpy(), gr["grad_attn_row"], name="grad_attn_row", **tol)
    assert_close(gac.cpu().numpy(), gr["grad_attn_col"], name="grad_attn_col", **tol)
    assert_close(gb.cpu().numpy(), gr["grad_bias"], name="grad_bias", **tol)
    S._CACHE.clear()


@pytest.mark.parametrize("agg_mode", [False, True])
@pytest.mark.parametrize("H,C,dtype,p", [(6, 256, torch.float32, 0.0), (6, 256, torch.float32, 0.3),
                                         (6, 256, torch.bfloat16, 0.0)])
def test_wide_rows_long_segments(H, C, dtype, p, agg_mode, monkeypatch):
    """Production-shape rows (H=6 x C=256: 6 chunks per lane in fp32, 3 in
    bf16) with hub rows and columns split into several 512-edge segments."""
    import cign_amd.schedule as S

    print(f"gat wide long segments H={H} C={C} dtype={dtype} p={p} agg={agg_mode}", flush=True)
    monkeypatch.setattr(S, "segment_edges_for", lambda nnz, floor=512: 512)
    S._CACHE.clear()
    rng = np.random.default_rng(H * C)
    n = 2500
    ei = random_gat_graph(rng, n, avg_deg=4, hubs={5: 2400, 17: 1100})
    ei = np.concatenate([ei, np.stack([np.full(1800, 9), rng.choice(n, 1800, replace=False)])], 1)
    r, c, _ = O.coalesce(ei[0], ei[1], n)
    rowptr, col, row, colptr, perm = _dev_graph(np.stack([r, c]), n)
    x, ar, ac, b, gy = _inputs(rng, n, H, C, dtype)
    ext = __import__("cign_amd.collapsed_gat", fromlist=["x"]).ensure_collapsed_gat_loaded()
    (out, pre, emax, esum, mask), agg = _forward(ext, agg_mode, ar, ac, rowptr, col, 0.2, x, b, p, 7)
    assert (agg is not None) == agg_mode
    gf, gar, gac, gb = ext.backward(0.2, p, rowptr, col, colptr, row, perm, emax, esum, mask, x, ar, ac, pre, gy,
                                    agg)
    rp, cl = rowptr.cpu().numpy().astype(np.int64), col.cpu().numpy().astype(np.int64)
    keep = mask.cpu().numpy().astype(bool) if p > 0 else None
    if p > 0:
        assert np.array_equal(keep.reshape(-1), O.gat_dropout_keep(7, cl.size * H, p))
    args = (ar.double().cpu().numpy(), ac.double().cpu().numpy(), rp, cl, 0.2, x.double().cpu().numpy(),
            b.double().cpu().numpy())
    f = O.collapsed_gat_forward(*args, p=p, keep=keep)
    gr = O.collapsed_gat_backward(*args, gy.double().cpu().numpy(), p=p, keep=keep)
    tol, t32 = TOL[dtype], TOL[torch.float32]
    assert_close(pre.cpu().numpy(), f["pre"], name="pre", **tol)
    assert_close(emax.cpu().numpy(), f["emax"], name="edge_max", **t32)
    assert_close(esum.cpu().numpy(), f["esum"], name="edge_sum", **t32)
    assert_close(gf.double().cpu().numpy(), gr["grad_feat"], name="grad_feat", **tol)
    assert_close(gar.cpu().numpy(), gr["grad_attn_row"], name="grad_attn_row", **tol)
    assert_close(gac.cpu().numpy(), gr["grad_attn_col"], name="grad_attn_col", **tol)
    assert_close(gb.cpu().numpy(), gr["grad_bias"], name="grad_bias", **tol)
    S._CACHE.clear()
