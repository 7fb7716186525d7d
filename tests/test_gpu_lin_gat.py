"""bf16 features with fp32 outputs and gradients (library dtype 2) and the
context GAT's lin + logits + collapsed GAT as one autograd function
(lin_gat), which under bf16 AMP holds its projection output in bf16.

Dtype 2 runs the bf16 kernels' lane geometry with fp32 outputs, so on the
same values it must give the bf16 (dtype 1) launch's fp32 results bit for
bit and its bf16 outputs before rounding; against fp32 features holding the
same values (dtype 0, another lane geometry) it agrees to the fp32
tolerance. The module path is checked against the three autograd functions
it replaces (CIGN_GAT_FUSED_LIN=0): the same rounding points, so the fp32
tolerance plus, under AMP where an operand is rounded to bf16, one bf16 ulp;
against the oracle it is covered by the block and net tests."""
import numpy as np
import pytest
import torch

from tests.conftest import assert_close as _assert_close
from tests.test_gpu_gat import _dev_graph, _graph

pytestmark = pytest.mark.gpu
F32 = dict(rtol=1e-4, atol=1e-5)


def assert_close(a, e, **kw):
    _assert_close(a.double().cpu().numpy(), e.double().cpu().numpy(), **kw)

# (H, C, p, n, hubs): wide rows (V = 3, 2), narrow rows, heavy columns
CASES = [
    (6, 256, 0.0, 300, {4: 800}),
    (6, 256, 0.32, 200, {1: 500}),
    (4, 128, 0.1, 300, {2: 700}),
    (4, 16, 0.0, 600, {3: 1000}),
    (2, 64, 0.2, 300, {1: 400}),
]


def _match(a32, e, same_lanes):
    """A dtype-2 result against dtype 1's: bit for bit (a bf16 output: the
    fp32 result rounded) on the same lane geometry, else to the fp32
    tolerance (a bf16 output: one bf16 ulp)."""
    if e.dtype == torch.bfloat16:
        if same_lanes:
            assert torch.equal(a32.to(torch.bfloat16), e)
        else:
            assert_close(a32, e.float(), rtol=2.0 ** -7, atol=1e-5)
    elif same_lanes:
        assert torch.equal(a32, e)
    else:
        assert_close(a32, e, **F32)


def _bf16_exact(rng, *shape):
    return torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(torch.bfloat16).float().cuda()


@pytest.mark.parametrize("big", [False, True])
@pytest.mark.parametrize("H,C,p,n,hubs", CASES)
def test_gat_bf16_f32_dtype(H, C, p, n, hubs, big, monkeypatch):
    from cign_amd.collapsed_gat import bf16_f32_supported, ensure_collapsed_gat_loaded

    if big:
        monkeypatch.setenv("CIGN_GAT_BIG_GRAPH_EDGES", "0")
    assert bf16_f32_supported(H, C)
    rng = np.random.default_rng(H * 1000 + C + int(100 * p))
    ei = _graph(rng, n, hubs)
    rowptr, col, row, colptr, perm = _dev_graph(ei, n)
    x = _bf16_exact(rng, n, H, C)
    ar = torch.from_numpy(rng.standard_normal((n, H)).astype(np.float32)).cuda()
    ac = torch.from_numpy(rng.standard_normal((n, H)).astype(np.float32)).cuda()
    b = torch.from_numpy(rng.standard_normal(C).astype(np.float32)).cuda()
    gy = _bf16_exact(rng, n, C)
    ext = ensure_collapsed_gat_loaded()
    seed = 1234
    x16, gy16 = x.to(torch.bfloat16), gy.to(torch.bfloat16)
    print(f"case H={H} C={C} p={p} n={n} big={big}", flush=True)
    f2, agg2 = ext.forward_agg(ar, ac, rowptr, col, 0.2, x16, b, p, seed, True, f32_out=True)
    f1, agg1 = ext.forward_agg(ar, ac, rowptr, col, 0.2, x16, b, p, seed, True)
    f0, agg0 = ext.forward_agg(ar, ac, rowptr, col, 0.2, x, b, p, seed, True)
    assert f2[0].dtype == torch.float32 and f1[0].dtype == torch.bfloat16
    # Below the large-graph threshold, rows of at most 64 four-value chunks
    # run bf16 features four values per lane; dtype 2 keeps eight.
    same_lanes = big or H * C // 4 > 64
    _match(f2[0], f1[0], same_lanes)
    for a, e in zip(f2[1:4], f1[1:4]):
        _match(a, e, same_lanes)
    if p > 0:
        assert torch.equal(f2[4], f1[4])
        assert torch.equal(f2[4], f0[4])
    assert agg2 is not None
    _match(agg2, agg1, same_lanes)
    # against fp32 features holding the same values
    for a, e in zip(f2[:4], f0[:4]):
        assert_close(a, e, **F32)
    assert_close(agg2, agg0, **F32)

    b2 = ext.backward(0.2, p, rowptr, col, colptr, row, perm, f2[2], f2[3], f2[4], x16, ar, ac, f2[1], gy, agg2,
                      f32_out=True)
    b1 = ext.backward(0.2, p, rowptr, col, colptr, row, perm, f1[2], f1[3], f1[4], x16, ar, ac, f1[1], gy16, agg1)
    b0 = ext.backward(0.2, p, rowptr, col, colptr, row, perm, f0[2], f0[3], f0[4], x, ar, ac, f0[1], gy, agg0)
    assert b2[0].dtype == torch.float32
    for a, e in zip(b2, b1):
        _match(a, e, same_lanes)
    # without the aggregates: the rows pass gathers x again (another order)
    b2g = ext.backward(0.2, p, rowptr, col, colptr, row, perm, f2[2], f2[3], f2[4], x16, ar, ac, f2[1], gy, None,
                       f32_out=True)
    for a, e in zip(b2g, b2):
        assert_close(a, e, **F32)
    for a, e in zip(b2, b0):
        assert_close(a, e, **F32)


def test_gat_bf16_f32_rejects_pair_layout_shapes():
    from cign_amd import _lib
    from cign_amd.collapsed_gat import bf16_f32_supported, ensure_collapsed_gat_loaded

    assert not bf16_f32_supported(6, 40)
    rng = np.random.default_rng(3)
    n = 50
    ei = _graph(rng, n, {})
    rowptr, col, row, colptr, perm = _dev_graph(ei, n)
    x16 = torch.randn(n, 6, 40, device="cuda").to(torch.bfloat16)
    z = torch.zeros(n, 6, device="cuda")
    with pytest.raises(RuntimeError):
        ensure_collapsed_gat_loaded().forward_agg(z, z, rowptr, col, 0.2, x16, torch.zeros(40, device="cuda"), 0.0,
                                                  0, True, f32_out=True)
    assert _lib.load_library() is not None


@pytest.mark.parametrize("C,amp", [(256, True), (64, True), (256, False), (64, False), (40, False), (40, True)])
def test_lin_gat_matches_three_functions(C, amp, monkeypatch):
    """The module forward + backward as one function against the lin, the
    logits and the collapsed GAT as three, with GAT dropout, in fp32 and
    under bf16 AMP (x_proj held in bf16 where the shape allows: C 256 and 64;
    C = 40 takes the pair-layout GAT on a float32 x_proj). Under AMP the GAT
    runs another lane geometry on each path (fp32 reassociation), so grad x
    and grad W, which round their operand to bf16, also allow one bf16 ulp."""
    import itertools

    from cign_amd import collapsed_gat
    from cign_amd.graph import prepare_fused_gat_graph
    from cign_amd.model_cign import CompatibleCollapsedFusedGATConv
    from tests.conftest import bf16_flip_atol

    H, n, K = (6 if C == 256 else 4), 300, 48
    rng = np.random.default_rng(C)
    ei = _graph(rng, n, {2: 500})
    (rowptr, col), (row, colptr), perm = prepare_fused_gat_graph(torch.from_numpy(ei), n)
    csr, csc, perm = (rowptr.cuda(), col.cuda()), (row.cuda(), colptr.cuda()), perm.cuda()
    torch.manual_seed(0)
    mod = CompatibleCollapsedFusedGATConv(K, C, heads=H, dropout=0.32).cuda().train()
    with torch.no_grad():
        mod.bias.normal_()
    mod._selective_amp_enabled = amp
    mod._selective_amp_dtype = torch.bfloat16
    x0 = torch.from_numpy(rng.standard_normal((n, K)).astype(np.float32)).cuda()
    gy = torch.from_numpy(rng.standard_normal((n, C)).astype(np.float32)).cuda()
    res = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("CIGN_GAT_FUSED_LIN", mode)
        # the same dropout seed for both runs
        torch.manual_seed(5)
        monkeypatch.setattr(collapsed_gat, "_CALL_COUNTER", itertools.count())
        x = x0.clone().requires_grad_(True)
        mod.zero_grad(set_to_none=True)
        y = mod(x, csr, csc, perm)
        y.backward(gy)
        res[mode] = {"y": y.detach().clone(), "x": x.grad.clone()}
        res[mode].update({k: v.grad.clone() for k, v in mod.named_parameters()})
    assert set(res["1"]) == {"y", "x", "lin.weight", "att_src", "att_dst", "bias"}
    for k, e in res["0"].items():
        a = res["1"][k]
        extra = bf16_flip_atol(e.cpu().numpy()) if amp and k in ("x", "lin.weight") else 0.0
        assert_close(a, e, rtol=1e-4, atol=1e-5 * max(1.0, float(e.abs().max())) + extra, name=k)
