"""The training driver's host side: operators P (Laplacian, hybrid), the
heterophilous .npz loader, splits and metrics (generic_engine/train_cign.py).
CPU only; the GPU training step is in test_gpu_net.py."""
from __future__ import annotations

import types

import numpy as np
import pytest
import torch

from cign_amd import graph
from cign_amd import train_cign as T
from oracle import cign_oracle as O


def _random_edges(rng, n, e, isolated=()):
    src = rng.integers(0, n, e)
    dst = rng.integers(0, n, e)
    keep = ~np.isin(src, isolated) & ~np.isin(dst, isolated)
    return np.stack([src[keep], dst[keep]])


def _coo_parts(P):
    P = P.coalesce()
    return P.indices()[0].numpy(), P.indices()[1].numpy(), P.values().numpy()


def test_laplacian_bit_exact_against_oracle(rng):
    n = 300
    ei = _random_edges(rng, n, 1500, isolated=(7, 11))
    ei = np.concatenate([ei, [[3, 5], [3, 3]]], axis=1)  # an explicit self-loop is dropped
    used, L = graph.build_sparse_laplacian(torch.from_numpy(ei), n)
    o_used, (r, c, v) = O.normalized_laplacian(ei, n)
    assert np.array_equal(used.numpy(), o_used)
    lr, lc, lv = _coo_parts(L)
    assert np.array_equal(lr, r) and np.array_equal(lc, c)
    assert np.array_equal(lv, v)  # float32 bit for bit


def test_laplacian_oracle_pinned_by_dense_definition(rng):
    n = 120
    ei = _random_edges(rng, n, 500, isolated=(0, 9))
    _, (r, c, v) = O.normalized_laplacian(ei, n)
    L = np.zeros((n, n))
    np.add.at(L, (r, c), v.astype(np.float64))
    # independent dense construction: A from the symmetrised edge set
    A = np.zeros((n, n))
    A[ei[0], ei[1]] = 1.0
    A[ei[1], ei[0]] = 1.0
    np.fill_diagonal(A, 0.0)
    d = A.sum(1)
    dis = np.where(d > 0, 1.0 / np.sqrt(np.maximum(d, 1.0)), 0.0)
    ref = np.eye(n) - dis[:, None] * A * dis[None, :]
    np.testing.assert_allclose(L, ref, rtol=1e-6, atol=1e-7)
    # L sqrt(deg) = 0, L symmetric, spectrum in [0, 2]
    np.testing.assert_allclose(L @ np.sqrt(d), 0.0, atol=1e-5)
    np.testing.assert_allclose(L, L.T, atol=0)
    ev = np.linalg.eigvalsh(L)
    assert ev.min() > -1e-6 and ev.max() < 2 + 1e-6
    # isolated nodes keep a unit diagonal and nothing else
    assert L[0, 0] == 1.0 and np.count_nonzero(L[0]) == 1


def test_laplacian_unnormalised_and_random_walk(rng):
    n = 50
    ei = torch.from_numpy(graph.to_undirected(torch.from_numpy(_random_edges(rng, n, 200)), n).numpy())
    A = np.zeros((n, n))
    A[ei[0].numpy(), ei[1].numpy()] = 1.0
    np.fill_diagonal(A, 0.0)
    d = A.sum(1)
    for norm, ref in ((None, np.diag(d) - A),
                      ("rw", np.eye(n) - np.where(d > 0, 1.0 / np.maximum(d, 1.0), 0.0)[:, None] * A)):
        idx, w = graph.get_laplacian(ei, n, normalization=norm)
        L = np.zeros((n, n))
        np.add.at(L, (idx[0].numpy(), idx[1].numpy()), w.numpy().astype(np.float64))
        np.testing.assert_allclose(L, ref, rtol=1e-6, atol=1e-7)
    with pytest.raises(ValueError):
        graph.get_laplacian(ei, n, normalization="bad")


def test_graph_operator_modes(rng):
    n = 200
    ei = torch.from_numpy(_random_edges(rng, n, 900))
    dense = lambda P: P.to_dense().double().numpy()
    u_a, P_a = graph.build_graph_operator(ei, n, True, "adjacency", 0.3)
    u_l, P_l = graph.build_graph_operator(ei, n, True, "laplacian", 0.3)
    u_h, P_h = graph.build_graph_operator(ei, n, True, "hybrid", 0.3)
    # adjacency returns its index with the self-loops appended; the
    # Laplacian and hybrid modes return the undirected index alone
    assert torch.equal(u_l, u_h) and torch.equal(u_a[:, :u_l.size(1)], u_l)
    assert torch.equal(u_a[:, u_l.size(1):], torch.arange(n).repeat(2, 1))
    _, (r, c, v) = O.normalized_adjacency(ei.numpy(), n)
    assert np.array_equal(_coo_parts(P_a)[2], v)
    np.testing.assert_allclose(dense(P_h), 0.3 * dense(P_l) + 0.7 * dense(P_a), rtol=1e-6, atol=1e-7)
    # alpha = 1 and 0 reduce to the two operators
    np.testing.assert_array_equal(dense(graph.build_graph_operator(ei, n, True, "hybrid", 1.0)[1]), dense(P_l))
    np.testing.assert_array_equal(dense(graph.build_graph_operator(ei, n, True, "hybrid", 0.0)[1]), dense(P_a))
    with pytest.raises(ValueError):
        graph.build_graph_operator(ei, n, True, "hybrid", 1.5)
    with pytest.raises(ValueError):
        graph.build_graph_operator(ei, n, True, "other", 0.5)
    with pytest.raises(ValueError):
        graph.sparse_linear_combination(P_a, torch.eye(3).to_sparse(), 0.5)


def _write_npz(path, rng, n=64, f=12, e=150, splits=10, classes=5):
    x = rng.standard_normal((n, f)).astype(np.float32)
    y = rng.integers(0, classes, n).astype(np.int64)
    edges = rng.integers(0, n, (e, 2)).astype(np.int64)
    masks = {k: rng.random((splits, n)) < 0.3 for k in ("train_masks", "val_masks", "test_masks")}
    path.parent.mkdir(parents=True, exist_ok=True)
    np.savez(path, node_features=x, node_labels=y, edges=edges, **masks)
    return x, y, edges, masks


def test_heterophilous_npz_loader(tmp_path, rng):
    path = tmp_path / "amazon_ratings" / "raw" / "amazon_ratings.npz"
    x, y, edges, masks = _write_npz(path, rng)
    ds, data = T.load_dataset("Amazon-ratings", str(tmp_path))
    assert ds[0] is data and data.num_nodes == 64
    assert np.array_equal(data.x.numpy(), x) and np.array_equal(data.y.numpy(), y)
    # undirected and coalesced: both directions, sorted by (row, col), no duplicates
    r, c, _ = O.coalesce(np.concatenate([edges[:, 0], edges[:, 1]]), np.concatenate([edges[:, 1], edges[:, 0]]), 64)
    assert np.array_equal(data.edge_index.numpy(), np.stack([r, c]))
    for k in ("train", "val", "test"):
        m = getattr(data, f"{k}_mask")
        assert m.shape == (64, 10) and m.dtype == torch.bool
        assert np.array_equal(m.numpy(), masks[f"{k}_masks"].T)
    assert T.get_raw_mask_shape(data) == (64, 10)
    with pytest.raises(FileNotFoundError):
        T.load_dataset("Tolokers", str(tmp_path))
    with pytest.raises(NotImplementedError):
        T.load_dataset("Cora", str(tmp_path))
    with pytest.raises(ValueError):
        T.load_dataset("NoSuchGraph", str(tmp_path))


def test_splits():
    m = torch.tensor([[True, False], [False, True], [True, True]])
    assert torch.equal(T.select_mask(m, 1), m[:, 1])
    assert torch.equal(T.select_mask(m[:, 0], 5), m[:, 0])
    with pytest.raises(ValueError):
        T.select_mask(m, 2)
    n = 1003
    tr, va, te = T.generate_random_ratio_split(n, 0.5, 0.25, 0.25, split_seed=7)
    assert int(tr.sum()) == int(n * 0.5) and int(va.sum()) == int(n * 0.25)
    assert int(te.sum()) == n - int(n * 0.5) - int(n * 0.25)  # the remainder goes to test
    assert not (tr & va).any() and not (tr & te).any() and not (va & te).any()
    assert bool((tr | va | te).all())
    again = T.generate_random_ratio_split(n, 0.5, 0.25, 0.25, split_seed=7)
    assert all(torch.equal(a, b) for a, b in zip((tr, va, te), again))
    other = T.generate_random_ratio_split(n, 0.5, 0.25, 0.25, split_seed=8)
    assert not torch.equal(tr, other[0])
    with pytest.raises(ValueError):
        T.generate_random_ratio_split(n, 0.5, 0.3, 0.3, split_seed=0)
    data = types.SimpleNamespace(num_nodes=3, train_mask=m, val_mask=m, test_mask=m)
    args = types.SimpleNamespace(split_mode="original", split_index=1)
    T.apply_split(data, args)
    assert torch.equal(data.train_mask, m[:, 1])
    args = types.SimpleNamespace(split_mode="random_ratio", train_ratio=0.6, val_ratio=0.2, test_ratio=0.2,
                                 split_seed=0)
    T.apply_split(data, args)
    assert data.train_mask.shape == (3,)
    with pytest.raises(ValueError):
        T.apply_split(data, types.SimpleNamespace(split_mode="other"))
    with pytest.raises(ValueError):
        T.apply_split(types.SimpleNamespace(num_nodes=3), types.SimpleNamespace(split_mode="original",
                                                                                  split_index=0))


def test_metrics(rng):
    n = 400
    logits = torch.from_numpy(rng.standard_normal((n, 2)).astype(np.float32))
    y = torch.from_numpy(rng.integers(0, 2, n))
    mask = torch.from_numpy(rng.random(n) < 0.5)
    acc = T.accuracy(logits, y, mask)
    assert acc == float(((logits.argmax(1) == y) & mask).sum()) / float(mask.sum())
    assert T.accuracy(logits, y, torch.zeros(n, dtype=torch.bool)) == 0.0
    # the AUC is the pairwise ranking fraction of the softmax column 1
    score = torch.softmax(logits[mask], dim=-1)[:, 1].numpy()
    auc = T.binary_roc_auc(logits, y, mask)
    assert abs(auc - O.roc_auc_pairs(y[mask].numpy(), score)) < 1e-12
    # single logit: sigmoid; ties count half
    one = torch.tensor([0.0, 0.0, 1.0, -1.0])
    yy = torch.tensor([1, 0, 1, 0])
    assert T.binary_roc_auc(one, yy, torch.ones(4, dtype=torch.bool)) == O.roc_auc_pairs(yy.numpy(),
                                                                                          torch.sigmoid(one).numpy())
    assert T.binary_roc_auc(one[:, None], yy, torch.ones(4, dtype=torch.bool)) == 0.875
    assert T.binary_roc_auc(one, torch.ones(4, dtype=torch.long), torch.ones(4, dtype=torch.bool)) == 0.0
    bad = logits.clone()
    bad[mask.nonzero()[0, 0], 0] = float("nan")
    assert np.isnan(T.binary_roc_auc(bad, y, mask))
    assert T.compute_metric(logits, y, mask, "Tolokers") == auc
    assert T.compute_metric(logits, y, mask, "Amazon-ratings") == acc
    assert T.get_metric_name(" Questions ") == "ROC AUC" and T.get_metric_name("Roman-empire") == "Accuracy"


def test_auc_oracle_pinned_by_known_answers():
    # perfect, reversed and all-tied rankings; one mis-ordered pair of four
    y = np.array([0, 0, 1, 1])
    assert O.roc_auc_pairs(y, np.array([0.1, 0.2, 0.8, 0.9])) == 1.0
    assert O.roc_auc_pairs(y, np.array([0.9, 0.8, 0.2, 0.1])) == 0.0
    assert O.roc_auc_pairs(y, np.array([0.5, 0.5, 0.5, 0.5])) == 0.5
    assert O.roc_auc_pairs(y, np.array([0.1, 0.85, 0.8, 0.9])) == 0.75
