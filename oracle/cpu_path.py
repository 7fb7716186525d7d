"""The reference's CPU path for the hot path, restated in float32 torch on the
host -- TEST INFRASTRUCTURE AND BASELINE ONLY (bench.py's cpu_baseline legs;
nothing in cign_amd imports it).

With no CUDA device the reference turns every CUDA backend off and keeps the
fixed-CSR operator (generic_engine/train_cign.py:1199-1212), so its layer runs
  * the GAT as PyG GATConv computes it (concat=False): per-edge logits
    LeakyReLU(a_dst[i] + a_src[j]), a scatter softmax over each destination's
    in-edges (max detached, as torch_geometric.utils.softmax does), messages
    s * x[j] scatter-added per destination, the head mean, bias and SiLU
    (collapsed_gat.py:176-180 names this composition; model.py:591 the
    GATConv);
  * the hops as torch.sparse.mm on CSR(P) with the backward on CSR(P^T)
    (FixedCSRSpMMFunction, model.py:57-106);
and autograd for every backward. The timing follows generic_engine/
train_cign.py:2137-2144 (time.perf_counter around forward + backward) with
the warmup / median of backend_autotune_cign.py:228-229 (3 warmup, median).
"""
from __future__ import annotations

import os
import time

import numpy as np
import torch
import torch.nn.functional as F


def host_threads() -> int:
    """Threads for the host baseline: every core torch may use, capped by
    OMP_NUM_THREADS when set (the GPU box's CPU share)."""
    n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return n


class _FixedCsrMM(torch.autograd.Function):
    """FixedCSRSpMMFunction (model.py:57-106): y = P x, grad = P^T g."""

    @staticmethod
    def forward(ctx, x, p, pt):
        ctx.pt = pt
        return torch.sparse.mm(p, x)

    @staticmethod
    def backward(ctx, g):
        return torch.sparse.mm(ctx.pt, g.contiguous()), None, None


def _csr(crow, col, val, n):
    return torch.sparse_csr_tensor(torch.as_tensor(np.asarray(crow, np.int64)), torch.as_tensor(np.asarray(col, np.int64)),
                                   torch.as_tensor(np.asarray(val, np.float32)), size=(n, n))


def gat_concat_false(x, a_src, a_dst, rows, src, n, slope, bias):
    """GATConv message passing (concat=False) + head mean + bias + SiLU."""
    e = F.leaky_relu(a_dst[rows] + a_src[src], slope)  # [E,H]
    idx = rows[:, None].expand_as(e)
    m = torch.full((n, e.size(1)), float("-inf"), dtype=e.dtype).scatter_reduce(0, idx, e.detach(), "amax",
                                                                                include_self=True)
    ex = torch.exp(e - m[rows])
    den = torch.zeros(n, e.size(1), dtype=e.dtype).index_add_(0, rows, ex)
    s = ex / (den[rows] + 1e-16)
    out = torch.zeros_like(x).index_add_(0, rows, s.unsqueeze(-1) * x[src])
    return F.silu(out.mean(dim=1) + bias)


class LayerCPU:
    """The c2+c3 layer of the benchmark on the host: the GAT core (H x C) and
    the three hops of P over D columns, forward + backward, float32."""

    def __init__(self, rowptr, col, p_csr, pt_csr, n, H, C, D, seed=0):
        g = torch.Generator().manual_seed(seed)
        self.n = n
        self.rows = torch.repeat_interleave(torch.arange(n), torch.as_tensor(np.diff(np.asarray(rowptr, np.int64))))
        self.src = torch.as_tensor(np.asarray(col, np.int64))
        self.P, self.PT = _csr(*p_csr, n), _csr(*pt_csr, n)
        self.x = torch.randn(n, H, C, generator=g).requires_grad_()
        self.ar = torch.randn(n, H, generator=g).requires_grad_()
        self.ac = torch.randn(n, H, generator=g).requires_grad_()
        self.b = torch.randn(C, generator=g).requires_grad_()
        self.gy = torch.randn(n, C, generator=g)
        self.X = torch.randn(n, D, generator=g).requires_grad_()
        self.G = [torch.randn(n, D, generator=g) for _ in range(3)]

    def step(self):
        for t in (self.x, self.ar, self.ac, self.b, self.X):
            t.grad = None
        y = gat_concat_false(self.x, self.ac, self.ar, self.rows, self.src, self.n, 0.2, self.b)
        y1 = _FixedCsrMM.apply(self.X, self.P, self.PT)
        y2 = _FixedCsrMM.apply(y1, self.P, self.PT)
        y3 = _FixedCsrMM.apply(y2, self.P, self.PT)
        torch.autograd.backward([y, y1, y2, y3], [self.gy, *self.G])


def time_steps(step, seconds: float, warmup: int = 3, min_steps: int = 3):
    """Median seconds per step over as many steps as fit in `seconds`
    (at least min_steps), after `warmup` steps; and the count."""
    for _ in range(warmup):
        step()
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < min_steps or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)
