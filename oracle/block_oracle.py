"""CPU oracle of the Clifford block composition -- TEST INFRASTRUCTURE ONLY.

A float64 torch (CPU) restatement of GraphCliffordBlock.forward in eval mode
(no dropout), following the reference's own unfused formulas
(generic_engine/model_cign.py:751-937, the torch fallback at :878-925,
compute_hop_gate :721-749, CompatibleCollapsedFusedGATConv :524-567 with the
textbook GAT of collapsed_gat_cuda.cu:84-173). Gradients come from torch
autograd in float64. Each stage is pinned against oracle/cign_oracle.py in
tests/test_oracle.py. Only tests/ may import this module.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def _bf16(t):
    """Round to bfloat16 (nearest even) and back to t's dtype: torch's own
    float32 -> bfloat16 cast, the cast autocast applies."""
    return t.to(torch.float32).to(torch.bfloat16).to(t.dtype)


class _AmpLinear(torch.autograd.Function):
    """y = x W^T + b under the local bf16 autocast of _local_amp_linear
    (generic_engine/model_cign.py:86-103), rounding where the GPU path rounds:
    x, W and b to bf16, the output to bf16 (autocast's output dtype, handed on
    as float32); backward products on bf16-rounded operands (grad_y, W, x),
    grad_b the sum of the rounded grad_y, and grad_x, grad_W, grad_b each
    rounded to bf16 (the bf16 Linear's backward outputs, which the casts of
    x, W and b back to float32 hand on unchanged). Arithmetic between the
    rounding points is exact in the tensors' dtype."""

    @staticmethod
    def forward(ctx, x, w, b):
        xr, wr = _bf16(x), _bf16(w)
        ctx.save_for_backward(xr, wr)
        ctx.has_bias = b is not None
        y = xr @ wr.T
        if b is not None:
            y = y + _bf16(b)
        return _bf16(y)

    @staticmethod
    def backward(ctx, gy):
        xr, wr = ctx.saved_tensors
        gr = _bf16(gy)
        return _bf16(gr @ wr), _bf16(gr.T @ xr), (_bf16(gr.sum(0)) if ctx.has_bias else None)


def _linear(x, w, b, amp):
    """F.linear, or its bf16-autocast rounding points when amp."""
    if amp:
        return _AmpLinear.apply(x, w, b)
    return F.linear(x, w, b)


def _gat(xp, a_src, a_dst, rowptr, col, slope, bias):
    """Collapsed GAT (concat=False) + head mean + bias + SiLU, float64."""
    n = xp.size(0)
    deg = torch.from_numpy(np.diff(rowptr)).long()
    rows = torch.repeat_interleave(torch.arange(n), deg)
    src = torch.from_numpy(np.asarray(col, np.int64))
    e = F.leaky_relu(a_dst[rows] + a_src[src], slope)  # [E,H]
    m = torch.full((n, e.size(1)), -torch.inf, dtype=e.dtype).scatter_reduce(0, rows[:, None].expand_as(e), e,
                                                                             "amax", include_self=True)
    ex = torch.exp(e - m.detach()[rows])
    den = torch.zeros(n, e.size(1), dtype=e.dtype).index_add(0, rows, ex)
    s = ex / den[rows]
    out = torch.zeros_like(xp).index_add(0, rows, s[:, :, None] * xp[src])
    pre = out.mean(dim=1) + bias
    return F.silu(pre)


def _pack(Hn, Cn, props, alpha, interaction, weighting):
    D = Hn.size(1)
    Ds, Ws = [], []
    for P in props:
        th, tc = P[:, :D], P[:, D:]
        bhr, brh = Hn * tc, Cn * th
        if interaction == 0:
            Dv, Wv = F.silu(bhr), bhr - brh
        else:
            Dv = F.silu(0.5 * (bhr + brh))
            Wv = 0.5 * (bhr - brh)
            if interaction == 2:
                Wv = torch.tanh(Wv)
        Ds.append(Dv)
        Ws.append(Wv)
    Dh, Wh = torch.stack(Ds, 1), torch.stack(Ws, 1)  # [N,K,D]
    if weighting == 0:
        feats = torch.cat([Wh, Dh], dim=-1)
        if alpha is not None:
            feats = feats * alpha
        return feats.reshape(Hn.size(0), -1)
    if alpha is not None:
        Dh, Wh = Dh * alpha, Wh * alpha
    return torch.cat([Dh.sum(1), Wh.sum(1)], dim=-1)


def block_forward(params: dict, H, rowptr, col, p_csr, order_set, *, score_mode, interaction, weighting,
                  gate_mode, heads, slope=0.2, eps=1e-5, amp=False):
    """Eval-mode block forward. params: leaf tensors named like the module's
    parameters (h_norm.weight, ..., context_gat.lin.weight, ...), float64 for
    the oracle (float32 to measure the rounding error of the same arithmetic
    in float32); p_csr: (rowptr, col, val) of the normalized adjacency P
    (numpy), used in H's dtype. amp: the GAT lin and proj under selective
    bf16 autocast (_AmpLinear)."""
    g = params
    D = H.size(1)
    Hn = F.layer_norm(H, (D,), g["h_norm.weight"], g["h_norm.bias"], eps)
    xp = _linear(Hn, g["context_gat.lin.weight"], None, amp).view(H.size(0), heads, -1)
    a_src = (xp * g["context_gat.att_src"]).sum(-1)
    a_dst = (xp * g["context_gat.att_dst"]).sum(-1)
    Cg = _gat(xp, a_src, a_dst, rowptr, col, slope, g["context_gat.bias"])
    Cn = F.layer_norm(Cg + Hn, (D,), g["c_norm.weight"], g["c_norm.bias"], eps)
    X = torch.cat([Hn, Cn], dim=-1)
    prow, pcol, pval = p_csr
    P = torch.sparse_csr_tensor(torch.from_numpy(np.asarray(prow, np.int64)),
                                torch.from_numpy(np.asarray(pcol, np.int64)),
                                torch.from_numpy(np.asarray(pval, np.float64)).to(H.dtype),
                                size=(H.size(0), H.size(0)))
    powers, cur = {}, X
    for k in range(1, max(order_set) + 1):
        cur = P @ cur
        powers[k] = cur
    powers[0] = X
    props = [powers[s] for s in order_set]
    if gate_mode == "none":
        alpha = None
    elif gate_mode == "global":
        alpha = torch.softmax(g["hop_gate_logits"], 0).view(1, -1, 1)
    else:
        s = torch.cat([Hn, Cn], -1) if score_mode == 0 else torch.cat([Hn + Cn, torch.abs(Hn - Cn)], -1)
        alpha = torch.softmax(F.linear(s, g["hop_gate_mlp.weight"], g["hop_gate_mlp.bias"]), -1).unsqueeze(-1)
    G = _pack(Hn, Cn, props, alpha, interaction, weighting)
    Gf = _linear(G, g["proj.weight"], g["proj.bias"], amp)
    gamma = g["gamma"]
    return H + (gamma.unsqueeze(0) if gamma.dim() == 1 else gamma) * Gf


def net_forward(params: dict, x, rowptr, col, p_csr, order_set, *, num_layers, dual, layer_combine, score_mode,
                interaction, weighting, gate_mode, heads, slope=0.2, eps=1e-5, amp=False):
    """Eval-mode GraphCliffordNet._forward_impl (generic_engine/model_cign.py:
    1160-1204) in float64: dual input projection H = SiLU(lin0 x) + eta
    SiLU(lin1 x) (or one projection), the blocks (block_forward on each
    block's parameters), concatenated (or last) layer states, output
    LayerNorm, classifier (float32 in the model, exact here). amp: the input
    projections and every block's lin and proj under selective bf16 autocast.
    Returns the logits."""
    g = params
    if dual:
        hb = F.silu(_linear(x, g["input_proj_0.weight"], g.get("input_proj_0.bias"), amp))
        hv = F.silu(_linear(x, g["input_proj_1.weight"], g.get("input_proj_1.bias"), amp))
        H = hb + g["input_eta"] * hv
    else:
        H = F.silu(_linear(x, g["input_proj.weight"], g.get("input_proj.bias"), amp))
    states = [H]
    for i in range(num_layers):
        pre = f"blocks.{i}."
        bp = {k[len(pre):]: v for k, v in g.items() if k.startswith(pre)}
        H = block_forward(bp, H, rowptr, col, p_csr, order_set, score_mode=score_mode, interaction=interaction,
                          weighting=weighting, gate_mode=gate_mode, heads=heads, slope=slope, eps=eps, amp=amp)
        states.append(H)
    out = torch.cat(states, dim=-1) if layer_combine == "concat" else states[-1]
    out = F.layer_norm(out, (out.size(1),), g["output_norm.weight"], g["output_norm.bias"], eps)
    return F.linear(out, g["classifier.weight"], g.get("classifier.bias"))
