"""GPU parity of the CSR SpMM / multihop pipeline against the oracle, through
the drop-in Python API (multihop_csr_pipeline, graph) and the C-ABI.
Tolerances: fp32 1e-4 rel / 1e-5 abs. bf16 (inputs rounded to bf16 first, the
oracle on the rounded values): a hop stores one float32 sum in bf16, so it
sits within 2^-8 of the float64 sum plus the float32 summation bound of its
terms (conftest.bf16_store_bound); a chain of hops adds each earlier
rounding carried through |P| (_bf16_chain_bound)."""
import numpy as np
import pytest
import torch

from oracle import cign_oracle as O
from tests.conftest import assert_close, assert_within, bf16_store_bound

pytestmark = pytest.mark.gpu

F32_TOL = dict(rtol=1e-4, atol=1e-5)


@pytest.fixture(scope="module")
def c3():
    from cign_amd import workloads

    return workloads.build(workloads.C2, device="cuda")


def _np_csr(csr):
    return (csr.crow_indices().cpu().numpy().astype(np.int64), csr.col_indices().cpu().numpy().astype(np.int64),
            csr.values().cpu().numpy().astype(np.float64))


def _abs_csr(p):
    import scipy.sparse as sp

    crow, col, val = p
    n = len(crow) - 1
    return sp.csr_matrix((np.abs(val), col, crow), shape=(n, n))


def _bf16_hop_bound(p, x, ref, add=None, carried=None):
    """Bound of one bf16 hop y = P x (+ add) against the float64 oracle ref
    (x, add: the exact inputs; carried: a bound on the error the stored x
    already holds)."""
    A = _abs_csr(p)
    terms = A @ np.abs(x) + (0.0 if add is None else np.abs(add))
    extra = 0.0
    if carried is not None:
        terms = terms + A @ carried
        extra = A @ carried
    n_terms = np.diff(p[0])[:, None] + (0 if add is None else 1)
    return bf16_store_bound(ref, terms, n_terms, extra)


def _rand(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype).cuda()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("d", [1, 3, 64, 100, 256, 512])
def test_spmm_full_c3_matches_oracle(c3, dtype, d):
    from cign_amd.graph import _hip_parts

    print(f"spmm c3 dtype={dtype} d={d}", flush=True)
    p = _np_csr(c3.operator.csr)
    x = _rand((c3.n, d), dtype, 10 + d)
    add = _rand((c3.n, d), dtype, 20 + d)
    y = _hip_parts(c3.operator.csr).spmm(x, add=add)
    ref = O.spmm(*p, x.double().cpu().numpy(), add=add.double().cpu().numpy())
    if dtype == torch.float32:
        assert_close(y.cpu().numpy(), ref, name="spmm", **F32_TOL)
    else:
        xn, an = x.double().cpu().numpy(), add.double().cpu().numpy()
        assert_within(y.double().cpu().numpy(), ref, _bf16_hop_bound(p, xn, ref, add=an), "spmm bf16")


def test_multihop3_autograd_c3_d64(c3):
    from cign_amd.multihop_csr_pipeline import MultiHopCSR3GraphOperator, multihop_csr3

    print("multihop3 c3 d=64 fwd+bwd", flush=True)
    op = MultiHopCSR3GraphOperator(c3.operator, dense_cols=64)
    x = _rand((c3.n, 64), torch.float32, 1).requires_grad_(True)
    y1, y2, y3 = multihop_csr3(op, x)
    g = [_rand((c3.n, 64), torch.float32, 2 + k) for k in range(3)]
    torch.autograd.backward([y1, y2, y3], g)
    p, pt = _np_csr(c3.operator.csr), _np_csr(c3.operator.csr_t)
    ref = O.multihop3_forward(p, x.detach().double().cpu().numpy())
    for k, y in enumerate((y1, y2, y3)):
        assert_close(y.detach().cpu().numpy(), ref[k], name=f"y{k+1}", **F32_TOL)
    gref = O.multihop3_backward(pt, *(t.double().cpu().numpy() for t in g))
    assert_close(x.grad.cpu().numpy(), gref, name="grad_x", **F32_TOL)
    # Size-independent property: the adjoint identity sum_k <y_k, g_k> = <x, grad_x>.
    lhs = sum(float((y.double() * gk.double()).sum()) for y, gk in zip((y1, y2, y3), g))
    rhs = float((x.detach().double() * x.grad.double()).sum())
    assert abs(lhs - rhs) <= 1e-4 * abs(lhs)


def test_multihop3_bf16_and_missing_grads(c3):
    from cign_amd.multihop_csr_pipeline import MultiHopCSR3GraphOperator, multihop_csr3

    print("multihop3 c3 bf16 d=256", flush=True)
    op = MultiHopCSR3GraphOperator(c3.operator, dense_cols=256, dense_dtype=torch.bfloat16)
    x = _rand((c3.n, 256), torch.bfloat16, 3).requires_grad_(True)
    y1, y2, y3 = multihop_csr3(op, x)
    assert y1.dtype == torch.bfloat16
    p = _np_csr(c3.operator.csr)
    xn = x.detach().double().cpu().numpy()
    ref1 = O.spmm(*p, xn)
    assert_within(y1.detach().double().cpu().numpy(), ref1, _bf16_hop_bound(p, xn, ref1), "y1 bf16")
    # Only y3 receives a gradient: missing grads become zeros (multihop_csr_pipeline.py:70-78).
    g3 = _rand((c3.n, 256), torch.bfloat16, 4)
    y3.backward(g3)
    pt = _np_csr(c3.operator.csr_t)
    z = np.zeros((c3.n, 256))
    g3n = g3.double().cpu().numpy()
    gref = O.multihop3_backward(pt, z, z, g3n)
    assert x.grad.dtype == torch.bfloat16
    # t2 = P^T g3 (+ 0), t1 = P^T t2 (+ 0), grad = P^T t1, each stored in bf16
    t2 = O.spmm(*pt, g3n)
    b2 = _bf16_hop_bound(pt, g3n, t2, add=z)
    t1 = O.spmm(*pt, t2)
    b1 = _bf16_hop_bound(pt, t2, t1, add=z, carried=b2)
    assert np.allclose(O.spmm(*pt, t1), gref, rtol=1e-12, atol=1e-12)
    assert_within(x.grad.double().cpu().numpy(), gref, _bf16_hop_bound(pt, t1, gref, carried=b1), "grad bf16")


def test_reference_dtype_rule_fp32_default(c3):
    from cign_amd.multihop_csr_pipeline import MultiHopCSR3GraphOperator, multihop_csr3

    op = MultiHopCSR3GraphOperator(c3.operator, dense_cols=8)
    x = _rand((c3.n, 8), torch.bfloat16, 5).requires_grad_(True)
    y1, _, _ = multihop_csr3(op, x)
    assert y1.dtype == torch.float32  # cast to fp32 like the reference
    y1.sum().backward()
    assert x.grad.dtype == torch.bfloat16


def _small_operator(seed=0, n=300):
    from cign_amd import graph

    rng = np.random.default_rng(seed)
    ei = np.stack([rng.integers(0, n, 1500), rng.integers(0, n, 1500)])
    ei = np.concatenate([ei, np.stack([np.zeros(400, np.int64), rng.integers(0, n, 400)])], 1)  # a hub
    _, P = graph.build_sparse_normalized_adjacency(torch.from_numpy(ei), n)
    op = graph.prepare_fixed_csr_operator(P)
    dev = lambda c: torch.sparse_csr_tensor(c.crow_indices().cuda(), c.col_indices().cuda(), c.values().cuda(),
                                            size=c.shape)
    return graph.FixedCSRGraphOperator(dev(op.csr), dev(op.csr_t)), n


@pytest.mark.parametrize("powers,strategy", [((1, 3, 5), "auto"), ((2, 4), "generic"), ((0, 1, 2), "auto"),
                                             ((1, 2, 3), "auto")])
def test_operator_strategies_match_oracle(powers, strategy):
    from cign_amd.graph import selected_sparse_powers
    from cign_amd.multihop_csr_pipeline import prepare_multihop_csr_operator

    print(f"strategy powers={powers} {strategy}", flush=True)
    base, n = _small_operator()
    op = prepare_multihop_csr_operator(base, dense_cols=16, powers=powers, strategy=strategy)
    x = _rand((n, 16), torch.float32, 7).requires_grad_(True)
    out = selected_sparse_powers(op, x, powers)
    assert sorted(out) == sorted(set(powers))
    p = _np_csr(base.csr)
    fw = O.multihop_generic_forward(p, x.detach().double().cpu().numpy(), powers)
    grads = {}
    loss = 0
    for k in sorted(out):
        if k == 0:
            continue
        assert_close(out[k].detach().cpu().numpy(), fw[k], name=f"P^{k}", **F32_TOL)
        gk = _rand((n, 16), torch.float32, 30 + k)
        grads[k] = gk.double().cpu().numpy()
        loss = loss + (out[k] * gk).sum()
    loss.backward()
    gref = O.multihop_generic_backward(_np_csr(base.csr_t), grads, max(grads), (n, 16))
    assert_close(x.grad.cpu().numpy(), gref, name="grad", **F32_TOL)


def test_fixed_sparse_mm_autograd():
    from cign_amd.graph import fixed_sparse_mm

    base, n = _small_operator(3)
    x = _rand((n, 5), torch.float32, 9).requires_grad_(True)
    y = fixed_sparse_mm(base, x)
    g = _rand((n, 5), torch.float32, 10)
    y.backward(g)
    assert_close(y.detach().cpu().numpy(), O.spmm(*_np_csr(base.csr), x.detach().double().cpu().numpy()),
                 name="y", **F32_TOL)
    assert_close(x.grad.cpu().numpy(), O.spmm(*_np_csr(base.csr_t), g.double().cpu().numpy()), name="gx", **F32_TOL)


def test_circulant_known_answer_gpu():
    from cign_amd.graph import _hip_parts

    n, d = 4096, 128  # validate_a3v5.py:11-19
    offs = [0, 1, -1, 7, -7, 31, -31, 127, -127]
    rows = np.repeat(np.arange(n), len(offs))
    cols = (rows + np.tile(offs, n)) % n
    A = torch.sparse_coo_tensor(torch.from_numpy(np.stack([rows, cols])), torch.full((len(rows),), 1.0 / 9.0),
                                (n, n)).coalesce().to_sparse_csr()
    A = torch.sparse_csr_tensor(A.crow_indices().cuda(), A.col_indices().cuda(), A.values().cuda(), size=(n, n))
    x = _rand((n, d), torch.float32, 11)
    y = _hip_parts(A).spmm(x).cpu().numpy()
    xn = x.double().cpu().numpy()
    expect = sum(np.roll(xn, -o, axis=0) for o in offs) / 9.0
    assert_close(y, expect, name="circulant", **F32_TOL)


def test_deterministic_and_counters_reset(c3):
    from cign_amd.graph import _hip_parts

    parts = _hip_parts(c3.operator.csr)
    x = _rand((c3.n, 64), torch.float32, 12)
    a = parts.spmm(x)
    b = parts.spmm(x)
    assert torch.equal(a, b)
    assert int(parts.sched.counters.abs().sum()) == 0


def test_plan_errors(c3):
    from cign_amd.multihop_csr_pipeline import MultiHopCSR3GraphOperator

    op = MultiHopCSR3GraphOperator(c3.operator, dense_cols=8)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        op.plan.forward3(torch.zeros(c3.n, 9, device="cuda"))
    with pytest.raises(RuntimeError, match="must be CUDA"):
        op.plan.forward3(torch.zeros(c3.n, 8))
    with pytest.raises(RuntimeError, match="contiguous"):
        op.plan.forward3(torch.zeros(8, c3.n, device="cuda").t())
    with pytest.raises(ValueError):
        MultiHopCSR3GraphOperator(c3.operator, dense_cols=8, algorithm=4)


@pytest.mark.parametrize("seg_edges", [256, 512, 1024, 2048])
@pytest.mark.parametrize("dtype,d", [(torch.float32, 64), (torch.float32, 1100), (torch.bfloat16, 256),
                                     (torch.bfloat16, 24)])
def test_spmm_big_hubs_segment_sizes(seg_edges, dtype, d):
    """Rows of 3,000-6,000 edges: many segments merged across workgroups, and
    segments longer than one 256-edge round of a workgroup."""
    from cign_amd.graph import HipCsr
    from cign_amd.schedule import build_row_schedule

    print(f"spmm big hubs seg={seg_edges} dtype={dtype} d={d}", flush=True)
    rng = np.random.default_rng(seg_edges + d)
    n = 7000
    deg = rng.integers(0, 12, n)
    deg[[5, 100, 6999]] = [3000, 6000, 1500]
    deg[[7, 8]] = [65, 257]
    rp = np.zeros(n + 1, np.int64)
    rp[1:] = np.cumsum(deg)
    col = np.concatenate([np.sort(rng.choice(n, size=int(k), replace=False)) for k in deg]).astype(np.int64)
    # positive weights normalised per row, like the propagation operator
    # (random-sign weights over 6,000 terms cancel below fp32's reach)
    val = rng.random(col.size) / np.repeat(np.maximum(deg, 1), deg)
    crow = torch.from_numpy(rp).cuda()
    A = torch.sparse_csr_tensor(crow, torch.from_numpy(col).cuda(), torch.from_numpy(val).float().cuda(),
                                size=(n, n))
    parts = HipCsr(A)
    parts.sched = build_row_schedule(crow, seg_edges=seg_edges)
    x = _rand((n, d), dtype, 3)
    y = parts.spmm(x)
    ref = O.spmm(rp, col, val.astype(np.float32).astype(np.float64), x.double().cpu().numpy())
    if dtype == torch.float32:
        assert_close(y.cpu().numpy(), ref, name="spmm", **F32_TOL)
    else:
        pv = (rp, col, val.astype(np.float32).astype(np.float64))
        xn = x.double().cpu().numpy()
        assert_within(y.double().cpu().numpy(), ref, _bf16_hop_bound(pv, xn, ref), "spmm bf16")
    assert int(parts.sched.counters.abs().sum()) == 0
