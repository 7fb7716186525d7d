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
against the oracle it is covered by the block and net tests. Its backward's
bf16 gradient entry points are checked bit for bit against their float32
counterparts on the same values: the logits backward's bf16 grad_x against
its float32 grad_x rounded to nearest even, and cign_linear_bwd_bf16gy
against cign_linear_bwd with bf16 math."""
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


@pytest.mark.parametrize("M,N,K", [(1000, 256, 48), (777, 1536, 256), (130, 64, 300), (37, 24, 20), (0, 64, 32)])
def test_linear_bwd_bf16_grad_y(M, N, K):
    """cign_linear_bwd_bf16gy on bf16 grad_y against cign_linear_bwd (math 1)
    on the same values in float32: bit for bit (both GEMMs read the bf16
    values and run the same tiles)."""
    from cign_amd import _lib

    print(f"linear bwd bf16 grad_y M={M} N={N} K={K}", flush=True)
    lib = _lib.load_library()
    rng = np.random.default_rng(M + N + K)
    gy16 = torch.from_numpy((rng.standard_normal((M, N)) / 30).astype(np.float32)).cuda().to(torch.bfloat16)
    gy = gy16.float()
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
    w = torch.from_numpy((rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)).cuda()
    st = _lib.stream_ptr(x.device)
    ws_bytes = int(lib.cign_linear_bwd_workspace_bytes(M, N, K, 0))
    ws = _lib.workspace(ws_bytes, x.device)
    outs = []
    for name, g in (("cign_linear_bwd", gy), ("cign_linear_bwd_bf16gy", gy16)):
        gx = torch.full((M, K), float("nan"), device="cuda")
        gw = torch.full((N, K), float("nan"), device="cuda")
        args = (g.data_ptr(), x.data_ptr(), w.data_ptr(), gx.data_ptr(), gw.data_ptr())
        if name == "cign_linear_bwd":
            lib.call(name, st, M, N, K, 1, *args, None, ws.data_ptr(), ws_bytes)
        else:
            lib.call(name, st, M, N, K, *args, ws.data_ptr(), ws_bytes)
        outs.append((gx, gw))
    torch.cuda.synchronize()
    for a, e, what in ((outs[1][0], outs[0][0], "grad_x"), (outs[1][1], outs[0][1], "grad_w")):
        assert torch.equal(a, e), what
    # grad_x may be skipped
    gw = torch.empty((N, K), device="cuda")
    lib.call("cign_linear_bwd_bf16gy", st, M, N, K, gy16.data_ptr(), x.data_ptr(), w.data_ptr(), None,
             gw.data_ptr(), ws.data_ptr(), ws_bytes)
    torch.cuda.synchronize()
    assert torch.equal(gw, outs[0][1])


@pytest.mark.parametrize("H,C", [(6, 256), (4, 64), (2, 8), (3, 1040)])
def test_attn_logits_bwd_acc_bf16_grad_x(H, C):
    """cign_attn_logits_bwd_acc writing a bf16 grad_x: the float32 grad_x of
    the same call rounded to nearest even, bit for bit; the logits'
    gradients unchanged."""
    from cign_amd import _lib

    print(f"logits bwd acc bf16 grad_x H={H} C={C}", flush=True)
    lib = _lib.load_library()
    n = 517
    rng = np.random.default_rng(H * C)
    xp = torch.from_numpy(rng.standard_normal((n, H, C)).astype(np.float32)).cuda().to(torch.bfloat16)
    s = torch.from_numpy(rng.standard_normal((H, C)).astype(np.float32)).cuda()
    d = torch.from_numpy(rng.standard_normal((H, C)).astype(np.float32)).cuda()
    gs = torch.from_numpy(rng.standard_normal((n, H)).astype(np.float32)).cuda()
    gd = torch.from_numpy(rng.standard_normal((n, H)).astype(np.float32)).cuda()
    gin = torch.from_numpy((rng.standard_normal((n, H, C)) / 7).astype(np.float32)).cuda()
    st = _lib.stream_ptr(xp.device)
    ws_bytes = int(lib.cign_colsum_workspace_bytes(n, H * C, 2))
    ws = _lib.workspace(ws_bytes, xp.device)
    res = []
    for code, dt in ((0, torch.float32), (1, torch.bfloat16)):
        gx = torch.empty((n, H, C), dtype=dt, device="cuda")
        g_s, g_d = torch.empty_like(s), torch.empty_like(d)
        lib.call("cign_attn_logits_bwd_acc", st, n, H, C, 1, code, gs.data_ptr(), gd.data_ptr(), xp.data_ptr(),
                 s.data_ptr(), d.data_ptr(), gin.data_ptr(), gx.data_ptr(), g_s.data_ptr(), g_d.data_ptr(),
                 ws.data_ptr(), ws_bytes)
        res.append((gx, g_s, g_d))
    torch.cuda.synchronize()
    assert torch.equal(res[1][0], res[0][0].to(torch.bfloat16))
    assert torch.equal(res[1][1], res[0][1]) and torch.equal(res[1][2], res[0][2])


def test_bf16_gradient_entry_points_reject():
    from cign_amd import _lib

    lib = _lib.load_library()
    n, H, C = 10, 2, 12
    x32 = torch.zeros((n, H, C), device="cuda")
    x16 = x32.to(torch.bfloat16)
    v = torch.zeros((H, C), device="cuda")
    g = torch.zeros((n, H), device="cuda")
    out16 = torch.empty_like(x16)
    ws = _lib.workspace(int(lib.cign_colsum_workspace_bytes(n, H * C, 2)), x32.device)
    st = _lib.stream_ptr(x32.device)
    for xd, x, gin, gdt in ((0, x32, x32, 1), (1, x16, x32, 1), (1, x16, x32, 2)):
        # float32 x, channels not a multiple of 8, an unknown code
        with pytest.raises(RuntimeError):
            lib.call("cign_attn_logits_bwd_acc", st, n, H, C, xd, gdt, g.data_ptr(), g.data_ptr(), x.data_ptr(),
                     v.data_ptr(), v.data_ptr(), gin.data_ptr(), out16.data_ptr(), v.data_ptr(), v.data_ptr(),
                     ws.data_ptr(), ws.numel())
    w = torch.zeros((16, 8), device="cuda")
    gw = torch.empty_like(w)
    lws = _lib.workspace(int(lib.cign_linear_bwd_workspace_bytes(n, 16, 8, 0)), w.device)
    with pytest.raises(RuntimeError, match="N must exceed"):
        lib.call("cign_linear_bwd_bf16gy", st, n, 16, 8, x16.data_ptr(), w.data_ptr(), w.data_ptr(), None,
                 gw.data_ptr(), lws.data_ptr(), lws.numel())
    with pytest.raises(RuntimeError, match="workspace too small"):
        lib.call("cign_linear_bwd_bf16gy", st, n, 24, 8, x16.data_ptr(), torch.zeros((n, 8), device="cuda").data_ptr(),
                 torch.zeros((24, 8), device="cuda").data_ptr(), None, gw.data_ptr(), lws.data_ptr(), 0)


@pytest.mark.parametrize("amp", [False, True])
@pytest.mark.parametrize("n,K", [(300, 48), (24492, 300)])
def test_lin_gat_data_input_fused_wgrad(n, K, amp):
    """Input features that need no gradient (config c2: x is data) take
    cign_lin_logits_wgrad, the logits' backward fused into the weight
    gradient; with x requiring a gradient the module runs the logits
    backward and the Linear backward apart. Same forward (bit for bit), the
    GAT bias gradient bit for bit, the weight and attention-vector gradients
    to the fp32 tolerance of another summation order (under AMP the weight
    gradient, a bf16 output, within one bf16 ulp)."""
    from cign_amd.graph import prepare_fused_gat_graph
    from cign_amd.model_cign import CompatibleCollapsedFusedGATConv
    from tests.conftest import bf16_flip_atol

    H, C = 4, 16
    print(f"fused lin wgrad n={n} K={K} amp={amp}", flush=True)
    from oracle import cign_oracle as O

    rng = np.random.default_rng(n + K)
    if n <= 1000:
        ei = _graph(rng, n, {2: min(500, n - 1)})
    else:  # about 8.6 edges a node, as the c2 graph, plus a hub column
        src = np.concatenate([rng.integers(0, n, 8 * n), np.full(2000, 7)])
        dst = np.concatenate([rng.integers(0, n, 8 * n), rng.integers(0, n, 2000)])
        ei = O.gat_edge_index(np.stack([src, dst]).astype(np.int64), n)
        r, c, _ = O.coalesce(ei[0], ei[1], n)
        ei = np.stack([r, c])
    (rowptr, col), (row, colptr), perm = prepare_fused_gat_graph(torch.from_numpy(ei), n)
    csr, csc, perm = (rowptr.cuda(), col.cuda()), (row.cuda(), colptr.cuda()), perm.cuda()
    torch.manual_seed(0)
    mod = CompatibleCollapsedFusedGATConv(K, C, heads=H, dropout=0.0).cuda().train()
    with torch.no_grad():
        mod.bias.normal_()
        mod.att_src.normal_()
        mod.att_dst.normal_()
    mod._selective_amp_enabled = amp
    mod._selective_amp_dtype = torch.bfloat16
    x0 = torch.from_numpy(rng.standard_normal((n, K)).astype(np.float32)).cuda()
    gy = torch.from_numpy((rng.standard_normal((n, C)) / np.sqrt(n)).astype(np.float32)).cuda()
    res = {}
    for data in (True, False):
        x = x0.clone().requires_grad_(not data)
        mod.zero_grad(set_to_none=True)
        y = mod(x, csr, csc, perm)
        y.backward(gy)
        res[data] = {"y": y.detach().clone()}
        res[data].update({k: v.grad.clone() for k, v in mod.named_parameters()})
    assert torch.equal(res[True]["y"], res[False]["y"])
    assert torch.equal(res[True]["bias"], res[False]["bias"])
    for k in ("lin.weight", "att_src", "att_dst"):
        a, e = res[True][k], res[False][k]
        extra = bf16_flip_atol(e.cpu().numpy()) if amp and k == "lin.weight" else 0.0
        assert_close(a, e, rtol=1e-4, atol=1e-5 * max(1.0, float(e.abs().max())) + extra, name=k)
