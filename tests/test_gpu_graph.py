"""HIP graph capture of the layer step (collapsed GAT forward/backward with
dropout + the 3-hop SpMM forward/backward) through the drop-in API: every
replay, with the program's own eager work and synchronisations between
replays, reproduces the eager results bit for bit (the kernels record no
memset nodes and their cross-workgroup counters return to zero)."""
import numpy as np
import pytest
import torch

from tests.conftest import random_gat_graph

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,p", [(torch.float32, 0.0), (torch.float32, 0.3), (torch.bfloat16, 0.2)])
def test_graph_replays_match_eager(dtype, p):
    from cign_amd import graph
    from cign_amd.collapsed_gat import ensure_collapsed_gat_loaded
    from cign_amd.multihop_csr_pipeline import MultiHopCSR3GraphOperator

    rng = np.random.default_rng(11)
    n, H, C, D = 700, 4, 16, 64
    ei = random_gat_graph(rng, n, avg_deg=6, hubs={3: 650, 9: 300})
    (rowptr, col), (row, colptr), perm = graph.prepare_fused_gat_graph(torch.from_numpy(ei), n)
    rowptr, col, row, colptr, perm = (t.cuda() for t in (rowptr, col, row, colptr, perm))
    _, P = graph.build_sparse_normalized_adjacency(torch.from_numpy(ei), n)
    op_cpu = graph.prepare_fixed_csr_operator(P)
    mv = lambda c: torch.sparse_csr_tensor(c.crow_indices().cuda(), c.col_indices().cuda(), c.values().cuda(),
                                           size=c.shape)
    op = graph.FixedCSRGraphOperator(mv(op_cpu.csr), mv(op_cpu.csr_t))
    mh = MultiHopCSR3GraphOperator(op, dense_cols=D, dense_dtype=dtype)
    plan = mh.plan
    ext = ensure_collapsed_gat_loaded()

    g = torch.Generator().manual_seed(5)
    rnd = lambda *s: torch.randn(*s, generator=g).cuda()
    x, gy = rnd(n, H, C).to(dtype), rnd(n, C).to(dtype)
    ar, ac, bias = rnd(n, H), rnd(n, H), rnd(C)
    X, g1, g2, g3 = (rnd(n, D).to(dtype) for _ in range(4))
    seed = 12345

    def step():
        out, pre, emax, esum, mask = ext.forward(ar, ac, rowptr, col, 0.2, x, bias, p, seed)
        gf, gar, gac, gb = ext.backward(0.2, p, rowptr, col, colptr, row, perm, emax, esum, mask, x, ar, ac, pre, gy)
        ys = plan.forward3(X)
        gx = plan.backward3(g1, g2, g3)
        res = [out, pre, emax, esum, gf, gar, gac, gb, *ys, gx]
        if p > 0:
            res.append(mask)
        return res

    eager = [t.clone() for t in step()]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        static = step()
    scratch = torch.zeros(1 << 20, device="cuda")
    for r in range(4):
        for t in static:
            t.fill_(float("nan")) if t.is_floating_point() else t.fill_(7)
        gr.replay()
        scratch.add_(1.0)  # eager work between replays
        torch.cuda.synchronize()
        for i, (a, e) in enumerate(zip(static, eager)):
            assert torch.equal(a, e), f"replay {r}: output {i} differs from the eager result"
