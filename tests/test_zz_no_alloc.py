"""cign_spmm_fwd3_noalloc (partial sums and merge counters in the library's
own per-GPU scratch) against cign_spmm_fwd3 (caller workspace), through the
C-ABI: bit-identical outputs on two calls in a row, the second smaller, on
graphs whose hub rows are cut into several merging segments."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _graph(n, hub_deg, seed):
    from cign_amd import graph

    rng = np.random.default_rng(seed)
    ei = np.stack([rng.integers(0, n, 8 * n), rng.integers(0, n, 8 * n)])
    hub = np.stack([np.full(hub_deg, 3), rng.choice(n, hub_deg, replace=False)])
    _, P = graph.build_sparse_normalized_adjacency(torch.from_numpy(np.concatenate([ei, hub], 1)), n)
    return graph.prepare_fixed_csr_operator(P).csr


def _run_pair(lib, csr, d, dtype, seed):
    from cign_amd import _lib
    from cign_amd.schedule import build_row_schedule

    n = csr.shape[0]
    crow = csr.crow_indices()
    # 512-edge segments: the hub row spans several segments that merge
    # through the partial sums and counters.
    sched = build_row_schedule(crow, device="cuda", seg_edges=512)
    assert sched.n_seg > 1 and sched.n_seg > sched.n_hrow, "case must have multi-segment rows"
    col = csr.col_indices().to(torch.int32).cuda()
    val = csr.values().to(torch.float32).cuda()
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, d, generator=g).to(dtype).cuda()
    code = _lib.dtype_code(x)
    st = _lib.stream_ptr()
    ref = [torch.empty_like(x) for _ in range(3)]
    partial = torch.empty(max(1, int(lib.cign_spmm_partial_bytes(sched.n_seg, d))), dtype=torch.uint8, device="cuda")
    lib.call("cign_spmm_fwd3", st, code, n, d, col.data_ptr(), val.data_ptr(), *sched.args(), x.data_ptr(),
             *(t.data_ptr() for t in ref), partial.data_ptr(), sched.counters.data_ptr())
    out = [torch.full_like(x, float("nan")) for _ in range(3)]
    lib.call("cign_spmm_fwd3_noalloc", st, code, n, d, col.data_ptr(), val.data_ptr(), *sched.args(), x.data_ptr(),
             *(t.data_ptr() for t in out))
    torch.cuda.synchronize()
    for k in range(3):
        assert torch.equal(out[k], ref[k]), f"hop {k + 1} differs (n={n}, d={d}, {dtype})"
    assert int(sched.counters.abs().sum()) == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_spmm_fwd3_noalloc_matches_workspace_entry(dtype):
    from cign_amd import _lib

    lib = _lib.load_library()
    print(f"noalloc fwd3 {dtype}: n=4000 d=256 hub 3000, then n=900 d=64 hub 850", flush=True)
    _run_pair(lib, _graph(4000, 3000, 1), 256, dtype, 11)
    _run_pair(lib, _graph(900, 850, 2), 64, dtype, 12)
