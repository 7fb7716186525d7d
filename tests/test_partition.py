"""CPU tests of the row-nnz partitioner and the shard structures (the
partitioned execution that replaces chunked_dgnn_gat.py:104-209): coverage,
balance, the local-node cap, and every shard's local graph mapped back to the
whole graph edge by edge (brute force)."""
import numpy as np
import pytest
import torch

from cign_amd import graph
from cign_amd.partition import ShardedGAT, partition_rows
from tests.conftest import random_gat_graph


def _gat(rng, n=600, hubs=None):
    ei = random_gat_graph(rng, n, avg_deg=6, hubs=hubs or {5: 400, 300: 250})
    return graph.prepare_fused_gat_graph(torch.from_numpy(ei), n), n


def _local_nodes(rp, col, lo, hi):
    return np.union1d(np.arange(lo, hi), col[rp[lo]:rp[hi]])


@pytest.mark.parametrize("shards", [1, 2, 5, 16])
def test_partition_covers_and_balances(rng, shards):
    ((rowptr, col), _, _), n = _gat(rng)
    rp = rowptr.numpy().astype(np.int64)
    ranges = partition_rows([rowptr], shards)
    assert ranges[0][0] == 0 and ranges[-1][1] == n
    assert all(a[1] == b[0] for a, b in zip(ranges, ranges[1:]))
    assert all(hi > lo for lo, hi in ranges)
    assert len(ranges) <= shards
    cost = np.arange(n + 1) + rp
    per = [cost[hi] - cost[lo] for lo, hi in ranges]
    # each cut lands within one row of its target
    heaviest = int((np.diff(rp) + 1).max())
    assert max(per) <= cost[-1] / shards + heaviest
    if shards > 1:
        # a hub row makes a shard of its own rather than dragging its neighbours in
        assert min(per) >= 1


def test_partition_two_row_pointers_and_edge_cases(rng):
    ((rowptr, col), (row, colptr), _), n = _gat(rng)
    ranges = partition_rows([rowptr, colptr], 4)
    cost = np.arange(n + 1) + rowptr.numpy() + colptr.numpy()
    per = [cost[hi] - cost[lo] for lo, hi in ranges]
    assert max(per) - min(per) <= 2 * int(np.diff(cost).max())
    # more shards than rows: one row each at most
    tiny = torch.tensor([0, 1, 3, 4], dtype=torch.int32)
    assert partition_rows([tiny], 10) == [(0, 1), (1, 2), (2, 3)]
    with pytest.raises(ValueError):
        partition_rows([tiny, torch.tensor([0, 1])], 2)
    with pytest.raises(ValueError):
        partition_rows([tiny], 0)


def test_partition_local_node_cap(rng):
    ((rowptr, col), _, _), n = _gat(rng)
    rp, cl = rowptr.numpy().astype(np.int64), col.numpy().astype(np.int64)
    cap = 450  # above the 401-node hub row, below most nnz-balanced shards' local sets
    ranges = partition_rows([rowptr], 2, max_local_nodes=cap, cols=[col])
    assert ranges[0][0] == 0 and ranges[-1][1] == n
    assert all(a[1] == b[0] for a, b in zip(ranges, ranges[1:]))
    assert len(ranges) > 2
    for lo, hi in ranges:
        assert _local_nodes(rp, cl, lo, hi).size <= cap
    # a single row that cannot fit raises (chunked_dgnn_gat.py:137-141)
    with pytest.raises(RuntimeError, match="local nodes"):
        partition_rows([rowptr], 2, max_local_nodes=300, cols=[col])
    with pytest.raises(ValueError):
        partition_rows([rowptr], 2, max_local_nodes=cap)


@pytest.mark.parametrize("shards", [1, 3, 7])
def test_shard_graphs_map_back_to_the_whole_graph(rng, shards):
    gg, n = _gat(rng)
    (rowptr, col), (row, colptr), perm = gg
    rp, cl = rowptr.numpy().astype(np.int64), col.numpy().astype(np.int64)
    cp, rw, pm = colptr.numpy().astype(np.int64), row.numpy().astype(np.int64), perm.numpy().astype(np.int64)
    erow = np.repeat(np.arange(n), np.diff(rp))  # destination of each CSR edge
    sg = ShardedGAT(gg, partition_rows([rowptr, colptr], shards), heads=4, channels=16)
    seen_fwd = np.zeros(cl.size, dtype=int)
    seen_bwd = np.zeros(cl.size, dtype=int)
    for s in sg.row_shards:
        nodes = s.nodes.numpy()
        assert np.array_equal(nodes, _local_nodes(rp, cl, s.lo, s.hi))
        assert (s.e0, s.e1) == (rp[s.lo], rp[s.hi])
        assert np.array_equal(nodes[s.col.numpy()], cl[s.e0:s.e1])  # same edges, same order
        assert s.sched.n_rows == s.hi - s.lo
        assert s.halo == np.setdiff1d(cl[s.e0:s.e1], np.arange(s.lo, s.hi)).size
        seen_fwd[s.e0:s.e1] += 1
    for c in sg.col_shards:
        nodes = c.nodes.numpy()
        want = np.union1d(np.arange(c.lo, c.hi), rw[cp[c.lo]:cp[c.hi]])
        assert np.array_equal(nodes, want)
        assert np.array_equal(nodes[c.own:c.own + c.hi - c.lo], np.arange(c.lo, c.hi))
        l_cp, l_row, l_perm = c.colptr.numpy(), c.row.numpy(), c.perm.numpy()
        l_rp, l_col, ids = c.rowptr.numpy(), c.col.numpy(), c.csr_ids.numpy()
        nl = nodes.size
        assert l_cp.size == nl + 1 and l_rp.size == nl + 1
        # CSC: the own sources' columns, entries in the whole graph's CSC order
        for j in range(c.lo, c.hi):
            a, b = l_cp[c.own + j - c.lo], l_cp[c.own + j - c.lo + 1]
            assert np.array_equal(nodes[l_row[a:b]], rw[cp[j]:cp[j + 1]])
            assert np.array_equal(ids[l_perm[a:b]], pm[cp[j]:cp[j + 1]])
        assert l_cp[c.own] == 0 and l_cp[c.own + c.hi - c.lo] == l_cp[-1] == c.nnz
        # CSR: whole-graph edge order; each local edge is the same (dst, src)
        assert np.all(np.diff(ids) > 0)
        l_erow = np.repeat(np.arange(nl), np.diff(l_rp))
        assert np.array_equal(nodes[l_erow], erow[ids])
        assert np.array_equal(nodes[l_col], cl[ids])
        assert np.array_equal(np.sort(l_perm), np.arange(c.nnz))
        assert c.row_sched.n_rows == nl and c.col_sched.n_rows == nl
        seen_bwd[ids] += 1
    # every edge in exactly one shard each way
    assert np.all(seen_fwd == 1) and np.all(seen_bwd == 1)
    info = sg.info
    assert info["num_chunks"] == len(sg.row_shards) and info["total_real_edges"] == cl.size


def test_shards_use_the_whole_graph_geometry(rng):
    gg, n = _gat(rng)
    (rowptr, col), (row, colptr), perm = gg
    from cign_amd.schedule import gat_schedule

    whole_f = gat_schedule(rowptr, 0, 0, 4, 16)
    whole_r = gat_schedule(rowptr, 1, 0, 4, 16)
    whole_c = gat_schedule(colptr, 1, 0, 4, 16)
    sg = ShardedGAT(gg, partition_rows([rowptr], 4), heads=4, channels=16)
    for s in sg.row_shards:
        assert tuple(s.sched.header[3:5]) == tuple(whole_f.header[3:5])
    for c in sg.col_shards:
        assert tuple(c.row_sched.header[3:5]) == tuple(whole_r.header[3:5])
        assert tuple(c.col_sched.header[3:5]) == tuple(whole_c.header[3:5])
    with pytest.raises(RuntimeError, match="feature-layout"):
        ShardedGAT(gg, partition_rows([rowptr], 2), heads=3, channels=10)
    with pytest.raises(ValueError, match="cover"):
        ShardedGAT(gg, [(0, 10), (20, n)], heads=4, channels=16)
