"""Seeded synthetic graphs for the benchmark configurations.

The reference ships no generator (its runs load Amazon-ratings through PyG);
these are this build's own, fixed by seed:

* ``chung_lu_pairs``: undirected Chung-Lu power-law graph. Node weights
  w_i = (i + i0)^(-1/(gamma-1)); pair endpoints are drawn independently with
  probability proportional to w (numpy PCG64), self-pairs dropped, duplicates
  removed, until ``n_pairs`` distinct unordered pairs exist (first ones in
  draw order). i0 is chosen by bisection so the expected maximum degree is
  ``max_degree``. Nodes are relabelled by descending degree
  ("in-degree-sorted"), ties by original id.
* ``uniform_out_degree``: every node gets ``out_degree`` distinct random
  targets (c1 of the benchmark), edges as (source, target).
"""
from __future__ import annotations

import numpy as np


def _expected_max_degree(i0: float, n: int, n_pairs: int, gamma: float) -> float:
    w = (np.arange(n, dtype=np.float64) + i0) ** (-1.0 / (gamma - 1.0))
    return 2.0 * n_pairs * w[0] / w.sum()


def _solve_offset(n: int, n_pairs: int, gamma: float, max_degree: float) -> float:
    lo, hi = 1e-6, float(n)
    for _ in range(200):
        mid = np.sqrt(lo * hi)
        if _expected_max_degree(mid, n, n_pairs, gamma) > max_degree:
            lo = mid
        else:
            hi = mid
    return float(np.sqrt(lo * hi))


def chung_lu_pairs(n: int, n_pairs: int, gamma: float = 2.5, max_degree: float = 1000.0, seed: int = 0):
    """Returns int64 [2, n_pairs] unordered pairs (u < v) of the relabelled graph."""
    rng = np.random.Generator(np.random.PCG64(seed))
    i0 = _solve_offset(n, n_pairs, gamma, max_degree)
    w = (np.arange(n, dtype=np.float64) + i0) ** (-1.0 / (gamma - 1.0))
    cdf = np.cumsum(w / w.sum())
    cdf[-1] = 1.0
    keys = np.empty(0, dtype=np.int64)
    seen_first: np.ndarray | None = None
    batch = int(n_pairs * 1.3) + 1024
    while True:
        a = np.searchsorted(cdf, rng.random(batch), side="right")
        b = np.searchsorted(cdf, rng.random(batch), side="right")
        a = np.minimum(a, n - 1)
        b = np.minimum(b, n - 1)
        ok = a != b
        u, v = np.minimum(a[ok], b[ok]), np.maximum(a[ok], b[ok])
        keys = np.concatenate([keys, u.astype(np.int64) * n + v])
        uniq, first = np.unique(keys, return_index=True)
        if uniq.size >= n_pairs:
            seen_first = np.sort(first)[:n_pairs]
            break
        batch = max(1024, int((n_pairs - uniq.size) * 1.5))
    chosen = keys[seen_first]
    u, v = chosen // n, chosen % n
    deg = np.bincount(u, minlength=n) + np.bincount(v, minlength=n)
    order = np.lexsort((np.arange(n), -deg))  # descending degree, ties by id
    relabel = np.empty(n, dtype=np.int64)
    relabel[order] = np.arange(n)
    u, v = relabel[u], relabel[v]
    return np.stack([np.minimum(u, v), np.maximum(u, v)])


def chung_lu_directed(n: int, n_directed: int, gamma: float = 2.5, max_degree: float = 1000.0, seed: int = 0):
    """Both directions of ``n_directed // 2`` Chung-Lu pairs: int64 [2, E]."""
    pairs = chung_lu_pairs(n, n_directed // 2, gamma=gamma, max_degree=max_degree, seed=seed)
    return np.concatenate([pairs, pairs[::-1]], axis=1)


def uniform_out_degree(n: int, out_degree: int = 8, seed: int = 0):
    """int64 [2, n*out_degree] (source, target) with distinct non-self targets."""
    rng = np.random.Generator(np.random.PCG64(seed))
    src = np.repeat(np.arange(n, dtype=np.int64), out_degree)
    dst = np.empty(n * out_degree, dtype=np.int64)
    for i in range(n):
        t = rng.choice(n - 1, size=out_degree, replace=False)
        dst[i * out_degree:(i + 1) * out_degree] = t + (t >= i)
    return np.stack([src, dst])
