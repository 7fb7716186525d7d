"""The layer run shard by shard (cign_amd.partition: nnz-balanced row shards
with source halos for the forward passes, column shards with destination
halos for the GAT's source gradients) against the unsharded layer on the same
inputs: the collapsed GAT forward (outputs, softmax statistics, dropout mask,
per-row aggregates) and backward (feature and attention gradients), and the
3-hop SpMM forward and backward, bit for bit. grad_bias, a sum over all
nodes, is combined across shards in shard order and checked to the fp32
bound of a reordered column sum. c2 (24.5K nodes, 211K edges) here; the
c5 graph in test_gpu_c5.py."""
import numpy as np
import pytest
import torch

from tests.conftest import colsum_atol

pytestmark = pytest.mark.gpu

SLOPE = 0.2


def _rand(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype).cuda()


def check_sharded_layer(w, ranges, dtype, H, C, D, p, seed=7, hops=True):
    """Runs the layer whole and by the shards of `ranges`; asserts per-node
    results equal bit for bit and grad_bias to the reordered-sum bound."""
    from cign_amd.collapsed_gat import ensure_collapsed_gat_loaded
    from cign_amd.multihop_csr_pipeline import MultiHopCSR3GraphOperator
    from cign_amd.partition import ShardedGAT, ShardedMultiHop

    (rowptr, col), (row, colptr), perm = w.gat_graph
    n = w.n
    ext = ensure_collapsed_gat_loaded()
    x = _rand((n, H, C), dtype, 1)
    ar, ac, bias = _rand((n, H), torch.float32, 2), _rand((n, H), torch.float32, 3), _rand((C,), torch.float32, 4)
    gy = _rand((n, C), dtype, 5)
    outs, agg = ext.forward_agg(ar, ac, rowptr, col, SLOPE, x, bias, p, seed, True)
    out, pre, emax, esum, mask = outs
    grads = ext.backward(SLOPE, p, rowptr, col, colptr, row, perm, emax, esum, mask, x, ar, ac, pre, gy, agg)

    sg = ShardedGAT(w.gat_graph, ranges, H, C, dtype)
    s_outs, s_agg = sg.forward(ar, ac, x, bias, SLOPE, p, seed)
    s_grads = sg.backward(SLOPE, p, s_outs[2], s_outs[3], s_outs[4], x, ar, ac, s_outs[1], gy, s_agg)
    torch.cuda.synchronize()
    names = ["out", "pre", "edge_max", "edge_sum"] + (["edge_mask"] if p > 0 else [])
    for name, a, b in zip(names, s_outs, outs):
        assert torch.equal(a, b), f"{name}: {int((a != b).sum())} of {a.numel()} differ"
    assert torch.equal(s_agg, agg), "row_agg differs"
    for name, a, b in zip(["grad_feat", "grad_attn_row", "grad_attn_col"], s_grads[:3], grads[:3]):
        assert torch.equal(a, b), f"{name}: {int((a != b).sum())} of {a.numel()} differ"
    # grad_bias = sum over nodes of grad_pre: reordered fp32 sums agree to the bound
    gp = (gy.float() * torch.sigmoid(pre) * (1 + pre * (1 - torch.sigmoid(pre)))).double()
    tol = colsum_atol(gp.abs().sum(0).cpu().numpy(), n)
    err = (s_grads[3].double() - grads[3].double()).abs().cpu().numpy()
    assert np.all(err <= 2 * tol), f"grad_bias: max err {err.max()} vs bound {2 * tol.max()}"

    if not hops:
        return
    dt = dtype
    X, g1, g2, g3 = (_rand((n, D), dt, 10 + k) for k in range(4))
    plan = MultiHopCSR3GraphOperator(w.operator, dense_cols=D, dense_dtype=dt).plan
    ys = plan.forward3(X)
    gx = plan.backward3(g1, g2, g3)
    sm = ShardedMultiHop(w.operator, ranges, D)
    s_ys = sm.forward3(X)
    s_gx = sm.backward3(g1, g2, g3)
    torch.cuda.synchronize()
    for k, (a, b) in enumerate(zip(s_ys, ys)):
        assert torch.equal(a, b), f"hop {k + 1}: {int((a != b).sum())} of {a.numel()} differ"
    assert torch.equal(s_gx, gx), f"grad_x of the hops: {int((s_gx != gx).sum())} differ"


@pytest.fixture(scope="module")
def c2():
    from cign_amd import workloads

    return workloads.build(workloads.C2, device="cuda")


@pytest.mark.parametrize("dtype,H,C,D", [(torch.float32, 4, 16, 64), (torch.bfloat16, 4, 32, 256)])
@pytest.mark.parametrize("shards,p", [(1, 0.0), (3, 0.3), (8, 0.0), (8, 0.3)])
def test_sharded_layer_c2_bit_identical(c2, dtype, H, C, D, shards, p):
    from cign_amd.partition import partition_rows

    (rowptr, _), (_, colptr), _ = c2.gat_graph
    ranges = partition_rows([rowptr, colptr, c2.operator.csr.crow_indices()], shards)
    print(f"c2 shards={len(ranges)} dtype={dtype} H={H} C={C} D={D} p={p}", flush=True)
    check_sharded_layer(c2, ranges, dtype, H, C, D, p)


def test_sharded_layer_c2_local_node_cap(c2):
    """Shards cut further by a local-node cap (the reference's max_local_nodes)."""
    from cign_amd.partition import partition_rows

    (rowptr, col), _, _ = c2.gat_graph
    ranges = partition_rows([rowptr], 2, max_local_nodes=6000, cols=[col])
    assert len(ranges) > 2
    check_sharded_layer(c2, ranges, torch.float32, 4, 16, 64, 0.3, hops=False)


def test_sharded_gat_runs_the_whole_graphs_variant(c2, monkeypatch):
    """With the large-graph threshold at the whole graph's edge count, the
    whole-graph launch runs the large-graph variants while every shard is
    below it: the shards still match bit for bit because they select the
    variant by the whole graph's count."""
    from cign_amd.partition import partition_rows

    monkeypatch.setenv("CIGN_GAT_BIG_GRAPH_EDGES", str(c2.nnz_gat))
    (rowptr, _), (_, colptr), _ = c2.gat_graph
    ranges = partition_rows([rowptr, colptr], 4)
    check_sharded_layer(c2, ranges, torch.bfloat16, 4, 32, 256, 0.3, hops=False)


@pytest.mark.parametrize("amp", [False, True])
def test_net_with_chunked_gat_matches_whole_graph(amp):
    """GraphCliffordNet at c1 with use_chunked_fused_gat (the graph prepared
    as nnz-balanced shards by its dgnn_chunk_* knobs) against the same model on
    the whole graph: logits, loss and every parameter gradient bit for bit,
    except the GAT biases (sums over all nodes, combined across shards), which
    agree to fp32 rounding. Under selective AMP the whole graph holds x_proj
    in bf16 and runs the bf16-feature GAT kernels (lin_gat), while the shards
    take float32 features holding the same bf16 values: the two sum in other
    lane orders, so they agree to fp32 reassociation carried through the
    later bf16 roundings, the bf16 bar (2e-2 relative plus one bf16 ulp of
    each tensor's scale)."""
    from tests.conftest import assert_close, bf16_flip_atol

    import torch.nn.functional as F

    from cign_amd import graph as G
    from cign_amd import workloads
    from cign_amd.model_cign import GraphCliffordNet
    from cign_amd.multihop_csr_pipeline import prepare_multihop_csr_operator
    from tests.test_gpu_net import _randomize

    w = workloads.build(workloads.C1, device="cuda")
    n, D, heads, in_dim, classes = w.n, 64, 4, 64, 5
    used, _ = G.build_sparse_normalized_adjacency(w.edge_index, n)
    gat_ei = G.prepare_gat_edge_index(used, n)
    mh = prepare_multihop_csr_operator(w.operator, dense_cols=2 * D, powers=(1, 2))
    models = []
    for chunked in (False, True):
        m = GraphCliffordNet(in_dim, D, classes, num_layers=2, order_set=(1, 2), gat_heads=heads, use_fused_gat=True,
                             use_chunked_fused_gat=chunked, dgnn_chunk_max_nodes=1500,
                             dgnn_chunk_target_nodes=300, use_selective_amp=amp).cuda().eval()
        _randomize(m, 3)
        info = m.prepare_fused_gat_graph(gat_ei, n)
        if chunked:
            assert info["num_chunks"] >= 7 and info["max_local_nodes_observed"] <= 1500
            assert info["total_real_edges"] == info["num_edges"] == w.nnz_gat
        models.append(m)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(n, in_dim, generator=g).cuda()
    y = torch.randint(0, classes, (n,), generator=g).cuda()
    outs = []
    for m in models:
        logits = m(x, None, mh)
        loss = F.cross_entropy(logits, y)
        loss.backward()
        outs.append((logits, loss))
    torch.cuda.synchronize()
    if amp:
        np_ = lambda t: t.detach().double().cpu().numpy()
        for i, name in enumerate(("logits", "loss")):
            e = np_(outs[0][i])
            assert_close(np_(outs[1][i]), e, rtol=2e-2, atol=1e-5 + bf16_flip_atol(e), name=name)
        for (name, a), (_, b) in zip(models[0].named_parameters(), models[1].named_parameters()):
            e = np_(a.grad)
            assert_close(np_(b.grad), e, rtol=2e-2, atol=1e-5 + bf16_flip_atol(e), name=f"grad {name}")
        return
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    for (name, a), (_, b) in zip(models[0].named_parameters(), models[1].named_parameters()):
        if name.endswith("context_gat.bias"):
            assert torch.allclose(a.grad, b.grad, rtol=1e-4, atol=1e-5), name
        else:
            assert torch.equal(a.grad, b.grad), f"grad {name} differs"
