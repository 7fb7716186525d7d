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

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

# Host threads for the elementwise parts (numpy releases the GIL in
# searchsorted and ufunc loops); chunking keeps every element's result, and
# so the graph, identical to the single-threaded computation.
_THREADS = 8


def _chunked(fn, n: int, out: np.ndarray, parts: int = 4 * _THREADS) -> np.ndarray:
    step = max(1, -(-n // parts))
    with ThreadPoolExecutor(_THREADS) as pool:
        list(pool.map(lambda i: fn(slice(i, min(n, i + step)), out), range(0, n, step)))
    return out


def _weights(n: int, i0: float, gamma: float) -> np.ndarray:
    """w_i = (i + i0)^(-1/(gamma-1)), float64."""
    base = np.arange(n, dtype=np.float64) + i0
    expo = -1.0 / (gamma - 1.0)

    def fn(sl, out):
        out[sl] = base[sl] ** expo

    return _chunked(fn, n, np.empty(n, dtype=np.float64))


def _draw(cdf: np.ndarray, u: np.ndarray) -> np.ndarray:
    """searchsorted(cdf, u, side="right") over host threads."""

    def fn(sl, out):
        out[sl] = np.searchsorted(cdf, u[sl], side="right")

    return _chunked(fn, u.size, np.empty(u.size, dtype=np.int64))


def _first_occurrences(keys: np.ndarray) -> np.ndarray:
    """Sorted indices of the first occurrence of each distinct key (what
    np.unique(keys, return_index=True)[1] sorted gives), by a stable sort."""
    k = torch.from_numpy(keys)
    srt, order = torch.sort(k, stable=True)
    head = torch.ones(srt.numel(), dtype=torch.bool)
    head[1:] = srt[1:] != srt[:-1]
    return torch.sort(order[head]).values.numpy()


def _expected_max_degree(i0: float, n: int, n_pairs: int, gamma: float) -> float:
    w = _weights(n, i0, gamma)
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
    w = _weights(n, i0, gamma)
    cdf = np.cumsum(w / w.sum())
    cdf[-1] = 1.0
    keys = np.empty(0, dtype=np.int64)
    seen_first: np.ndarray | None = None
    batch = int(n_pairs * 1.3) + 1024
    while True:
        a = _draw(cdf, rng.random(batch))
        b = _draw(cdf, rng.random(batch))
        a = np.minimum(a, n - 1)
        b = np.minimum(b, n - 1)
        ok = a != b
        u, v = np.minimum(a[ok], b[ok]), np.maximum(a[ok], b[ok])
        keys = np.concatenate([keys, u.astype(np.int64) * n + v])
        first = _first_occurrences(keys)
        if first.size >= n_pairs:
            seen_first = first[:n_pairs]
            break
        batch = max(1024, int((n_pairs - first.size) * 1.5))
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
