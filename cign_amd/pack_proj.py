"""The tail of the Clifford block as one fused pair of kernels: the pack
(weighting old), the projection proj, its bias, dropout and the gamma
residual (generic_engine/model_cign.py:803-846 then :927-933):

    G   = cat_k alpha_k [W_k, D_k]           (never stored)
    out = h + gamma * dropout(G Wp^T + bp)

cign_pack_proj_fwd builds G's tiles inside the projection's MFMA operand
load; cign_pack_proj_bwd computes grad_G tile by tile and runs the pack's
backward on it in the same kernel, rebuilds G in the grad_Wp reduction, and
adds the node gate's backward. Values and gradients are those of
gated_clifford_pack / clifford_pack_any followed by linear_gamma_residual,
up to the order of the fp32 sums inside the products.
"""
from __future__ import annotations

import ctypes
import os

import torch

from . import _lib

MAX_HOPS = 4
DIMS = (64, 128, 256)


def supported(D: int, K: int, weighting: int) -> bool:
    """Shapes the fused kernels take: weighting old, D in {64, 128, 256}, K <= 4."""
    return int(weighting) == 0 and int(D) in DIMS and 1 <= int(K) <= MAX_HOPS


def use_fused(D: int, K: int, weighting: int, amp: bool) -> bool:
    """Whether GraphCliffordBlock runs its tail as the fused pack projection:
    for the shapes it takes, under the math CIGN_PACK_PROJ names ("all", the
    default; "bf16"; "none"). At the production block it is the faster tail
    in both maths (bf16 1.757 against 1.768 ms, fp32 2.452 against 2.490 ms
    per block step) and stores neither G_raw nor its gradient."""
    mode = os.environ.get("CIGN_PACK_PROJ", "all").strip().lower()
    if mode not in ("bf16", "all", "none"):
        raise ValueError("CIGN_PACK_PROJ must be all, bf16 or none")
    if mode == "none" or (mode == "bf16" and not amp):
        return False
    return supported(D, K, weighting)


class _PackProjFn(torch.autograd.Function):
    """out = h + gamma * drop(pack(H, C, props, alpha) Wp^T + bp).
    gate_mode: "node" (alpha from the gate Linear gw/gb on [H, C] scores,
    computed here), "global" (alpha_vec [K], shared by every node) or "none"
    (alpha 1)."""

    @staticmethod
    def forward(ctx, h, H, C, gw, gb, alpha_vec, w, bias, gamma, interaction, score_mode, gate_mode, p, seed, math,
                *props):
        lib = _lib.load_library()
        N, D = H.shape
        K = len(props)
        dev = H.device
        st = _lib.stream_ptr(dev)
        if gate_mode == "node":
            alpha = torch.empty((N, K), dtype=torch.float32, device=dev)
            lib.call("cign_hop_gate_fwd", st, N, D, K, int(score_mode), H.data_ptr(), C.data_ptr(), gw.data_ptr(),
                     gb.data_ptr(), alpha.data_ptr())
            a_stride = K
        else:
            alpha = alpha_vec.detach().float().contiguous() if gate_mode == "global" else torch.ones(
                K, dtype=torch.float32, device=dev)
            a_stride = 0
        g_out = torch.empty((N, D), dtype=torch.float32, device=dev)
        out = torch.empty((N, D), dtype=torch.float32, device=dev)
        mask = torch.empty((N, D), dtype=torch.uint8, device=dev)
        arr = _lib.ptr_array([t.data_ptr() for t in props])
        ws_bytes = int(lib.cign_pack_proj_fwd_workspace_bytes(D, K, int(math)))
        ws = _lib.workspace(ws_bytes, dev)
        lib.call("cign_pack_proj_fwd", st, N, D, K, int(interaction), int(math), H.data_ptr(), C.data_ptr(),
                 ctypes.addressof(arr), 2 * D, alpha.data_ptr(), a_stride, w.data_ptr(), _lib.ptr(bias),
                 h.data_ptr(), gamma.data_ptr(), float(p), int(seed) & ((1 << 64) - 1), g_out.data_ptr(),
                 out.data_ptr(), mask.data_ptr(), ws.data_ptr(), ws_bytes)
        ctx.save_for_backward(H, C, alpha, w, g_out, gamma, mask, gw, *props)
        ctx.meta = (int(interaction), int(score_mode), gate_mode, float(p), int(math), a_stride, bias is not None)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        H, C, alpha, w, g_out, gamma, mask, gw, *props = ctx.saved_tensors
        interaction, score_mode, gate_mode, p, math, a_stride, has_bias = ctx.meta
        lib = _lib.load_library()
        N, D = H.shape
        K = len(props)
        dev = H.device
        st = _lib.stream_ptr(dev)
        go = grad_out.float().contiguous()
        grad_g = torch.empty_like(g_out)
        grad_gamma = torch.empty((D,), dtype=torch.float32, device=dev)
        ws_bytes = int(lib.cign_colsum_workspace_bytes(N, D, 1))
        ws = _lib.workspace(ws_bytes, dev)
        lib.call("cign_gamma_residual_bwd", st, N, D, go.data_ptr(), g_out.data_ptr(), gamma.data_ptr(),
                 mask.data_ptr(), p, grad_g.data_ptr(), grad_gamma.data_ptr(), ws.data_ptr(), ws_bytes)
        gH, gC = torch.empty_like(H), torch.empty_like(C)
        gP = [torch.empty_like(t) for t in props]
        g_alpha = torch.empty((N, K), dtype=torch.float32, device=dev)
        gw_out = torch.empty_like(w)
        gb_out = torch.empty((D,), dtype=torch.float32, device=dev) if has_bias else None
        node = gate_mode == "node"
        ggw = torch.empty_like(gw) if node else None
        ggb = torch.empty((K,), dtype=torch.float32, device=dev) if node else None
        pws_bytes = int(lib.cign_pack_proj_bwd_workspace_bytes(N, D, K))
        pws = _lib.workspace(pws_bytes, dev)
        arr = _lib.ptr_array([t.data_ptr() for t in props])
        garr = _lib.ptr_array([t.data_ptr() for t in gP])
        lib.call("cign_pack_proj_bwd", st, N, D, K, interaction, math, grad_g.data_ptr(), H.data_ptr(), C.data_ptr(),
                 ctypes.addressof(arr), 2 * D, alpha.data_ptr(), a_stride, w.data_ptr(), score_mode,
                 gw.data_ptr() if node else None, gH.data_ptr(), gC.data_ptr(), ctypes.addressof(garr), 2 * D,
                 g_alpha.data_ptr(), gw_out.data_ptr(), _lib.ptr(gb_out), _lib.ptr(ggw), _lib.ptr(ggb),
                 pws.data_ptr(), pws_bytes)
        g_alpha_vec = g_alpha.sum(0) if gate_mode == "global" else None
        return (go, gH, gC, ggw, ggb, g_alpha_vec, gw_out, gb_out, grad_gamma, None, None, None, None, None, None,
                *gP)


def pack_proj_gamma_residual(h: torch.Tensor, H_norm: torch.Tensor, C_norm: torch.Tensor, propagated,
                             gate_mode: str, gate_linear, global_logits, score_mode: str, interaction: int,
                             proj: torch.nn.Linear, gamma: torch.Tensor, dropout_p: float, amp: bool,
                             amp_dtype: torch.dtype = torch.bfloat16, seed: int | None = None) -> torch.Tensor:
    """The block's `proj` output, h + gamma * dropout(proj(G_raw)), with G_raw
    the weighting-old pack of (H_norm, C_norm, propagated) under the hop gate
    of gate_mode ("node": gate_linear on the score_mode scores; "global":
    softmax(global_logits); "none": alpha 1). The dropout seed follows the
    block-op stream as linear_gamma_residual's does."""
    from .fused_block_ops import _next_seed
    from .linear import _math_code

    if seed is None:
        seed = _next_seed(2, dropout_p)

    def f32(t):
        t = t.to(dtype=torch.float32).contiguous()
        return t if t.data_ptr() % 16 == 0 else t.clone()  # rows start 16-byte aligned
    H, C = f32(H_norm), f32(C_norm)
    props = [f32(t) for t in propagated]
    K = len(props)
    dev = H.device
    if gate_mode == "node":
        gw = f32(gate_linear.weight)
        gb = f32(gate_linear.bias) if gate_linear.bias is not None else torch.zeros(K, device=dev)
        alpha_vec = None
    elif gate_mode == "global":
        gw = gb = None
        alpha_vec = torch.softmax(global_logits, dim=0)
    else:
        gw = gb = alpha_vec = None
    bias = proj.bias.float().contiguous() if proj.bias is not None else None
    return _PackProjFn.apply(f32(h), H, C, gw, gb, alpha_vec, proj.weight.float().contiguous(), bias,
                             gamma.float().contiguous(), int(interaction), {"old": 0, "new": 1}[str(score_mode)],
                             gate_mode, float(dropout_p), int(seed), _math_code(bool(amp), amp_dtype), *props)
