"""Hop gate of the Clifford block on gfx950 (generic_engine/model_cign.py:
721-749): alpha[n, :] = softmax_k(Linear(2D -> K)(score[n, :])) with score
[H | C] (alpha_score_mode "old") or [H + C | |H - C|] ("new"), computed by
one fused kernel (cign_hop_gate_fwd) and its backward (cign_hop_gate_bwd).
"global" mode is softmax of K parameters (no kernel needed) and "none"
returns None, as in the reference.
"""
from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F

from . import _lib
from ._lib import check, check_input


class HopGateFunction(torch.autograd.Function):
    """alpha [N,K] from (H_norm, C_norm, weight [K,2D], bias [K])."""

    @staticmethod
    def forward(ctx, H, C, weight, bias, score_mode: int):
        for t, n in ((H, "H_norm"), (C, "C_norm"), (weight, "weight"), (bias, "bias")):
            check_input(t, n)
        check(H.dim() == 2 and C.shape == H.shape, "H_norm/C_norm must be [N,D]")
        N, D = H.shape
        K = weight.size(0)
        check(weight.dim() == 2 and weight.size(1) == 2 * D, "hop gate weight must be [K,2D]")
        check(bias.dim() == 1 and bias.numel() == K, "hop gate bias must be [K]")
        lib = _lib.load_library()
        alpha = torch.empty((N, K), dtype=torch.float32, device=H.device)
        lib.call("cign_hop_gate_fwd", _lib.stream_ptr(H.device), N, D, K, int(score_mode), H.data_ptr(),
                 C.data_ptr(), weight.data_ptr(), bias.data_ptr(), alpha.data_ptr())
        ctx.save_for_backward(H, C, weight, alpha)
        ctx.score_mode = int(score_mode)
        return alpha

    @staticmethod
    def backward(ctx, grad_alpha):
        H, C, weight, alpha = ctx.saved_tensors
        N, D = H.shape
        K = weight.size(0)
        lib = _lib.load_library()
        g = grad_alpha.to(dtype=torch.float32).contiguous()
        gH, gC = torch.empty_like(H), torch.empty_like(C)
        gW = torch.empty_like(weight)
        gb = torch.empty((K,), dtype=torch.float32, device=H.device)
        ws_bytes = int(lib.cign_hop_gate_bwd_workspace_bytes(N, D, K))
        ws = _lib.workspace(ws_bytes, H.device)
        lib.call("cign_hop_gate_bwd", _lib.stream_ptr(H.device), N, D, K, ctx.score_mode, H.data_ptr(), C.data_ptr(),
                 weight.data_ptr(), alpha.data_ptr(), g.data_ptr(), gH.data_ptr(), gC.data_ptr(), gW.data_ptr(),
                 gb.data_ptr(), ws.data_ptr(), ws_bytes)
        return gH, gC, gW, gb, None


class PackGateFunction(torch.autograd.Function):
    """The node-mode hop gate fused into the Clifford pack: G_raw from (H_norm,
    C_norm, gate weight [K,2D], gate bias [K], K propagated [N,2D] tensors)
    in one kernel each way (cign_pack_gate_fwd / cign_pack_gate_bwd). Alpha
    exists only inside (saved for the backward); grad_H / grad_C come out
    with the pack's and the gate's terms already summed."""

    @staticmethod
    def forward(ctx, interaction, weighting, score_mode, H, C, weight, bias, *props):
        from ._pack import _out_width
        for t, n in ((H, "H_norm"), (C, "C_norm"), (weight, "weight"), (bias, "bias")):
            check_input(t, n)
        for k, p in enumerate(props):
            check_input(p, f"P{k}")
        check(H.dim() == 2 and C.shape == H.shape, "H_norm/C_norm must be [N,D]")
        N, D = H.shape
        K = len(props)
        check(1 <= K <= 16, "hop count must be in [1, 16]")
        check(weight.dim() == 2 and tuple(weight.shape) == (K, 2 * D), "hop gate weight must be [K,2D]")
        check(bias.dim() == 1 and bias.numel() == K, "hop gate bias must be [K]")
        for k, p in enumerate(props):
            check(tuple(p.shape) == (N, 2 * D), f"P{k} must be [N,2D]")
        lib = _lib.load_library()
        alpha = torch.empty((N, K), dtype=torch.float32, device=H.device)
        out = torch.empty((N, _out_width(D, K, int(weighting))), dtype=torch.float32, device=H.device)
        arr = _lib.ptr_array([p.data_ptr() for p in props])
        lib.call("cign_pack_gate_fwd", _lib.stream_ptr(H.device), N, D, K, int(interaction), int(weighting),
                 int(score_mode), H.data_ptr(), C.data_ptr(), ctypes.addressof(arr), 2 * D, weight.data_ptr(),
                 bias.data_ptr(), alpha.data_ptr(), out.data_ptr())
        ctx.modes = (int(interaction), int(weighting), int(score_mode))
        ctx.save_for_backward(H, C, weight, alpha, *props)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        H, C, weight, alpha, *props = ctx.saved_tensors
        interaction, weighting, score_mode = ctx.modes
        N, D = H.shape
        K = len(props)
        lib = _lib.load_library()
        g = grad_out.to(dtype=torch.float32).contiguous()
        gH, gC = torch.empty_like(H), torch.empty_like(C)
        gP = [torch.empty_like(p) for p in props]
        gW = torch.empty_like(weight)
        gb = torch.empty((K,), dtype=torch.float32, device=H.device)
        ws_bytes = int(lib.cign_hop_gate_bwd_workspace_bytes(N, D, K))
        ws = _lib.workspace(ws_bytes, H.device)
        arr = _lib.ptr_array([p.data_ptr() for p in props])
        garr = _lib.ptr_array([t.data_ptr() for t in gP])
        lib.call("cign_pack_gate_bwd", _lib.stream_ptr(H.device), N, D, K, interaction, weighting, score_mode,
                 g.data_ptr(), H.data_ptr(), C.data_ptr(), ctypes.addressof(arr), 2 * D, alpha.data_ptr(),
                 weight.data_ptr(), gH.data_ptr(), gC.data_ptr(), ctypes.addressof(garr), 2 * D, gW.data_ptr(),
                 gb.data_ptr(), ws.data_ptr(), ws_bytes)
        return (None, None, None, gH, gC, gW, gb, *gP)


def gated_clifford_pack(H_norm: torch.Tensor, C_norm: torch.Tensor, propagated, linear: torch.nn.Linear,
                        score_mode: str, interaction: int, weighting: int) -> torch.Tensor:
    """G_raw of the Clifford block with the node-mode gate: the same value as
    clifford_pack_any(H_norm, C_norm, propagated, node_hop_gate(...)), from
    one fused kernel per direction. Inputs become float32 as both of those
    functions make them."""
    mode = {"old": 0, "new": 1}[str(score_mode)]
    H = H_norm.to(dtype=torch.float32).contiguous()
    C = C_norm.to(dtype=torch.float32).contiguous()
    props = [p.to(dtype=torch.float32).contiguous() for p in propagated]
    bias = linear.bias if linear.bias is not None else torch.zeros(linear.out_features, device=H.device)
    return PackGateFunction.apply(int(interaction), int(weighting), mode, H, C, linear.weight.float().contiguous(),
                                  bias.float().contiguous(), *props)


def node_hop_gate(H_norm: torch.Tensor, C_norm: torch.Tensor, linear: torch.nn.Linear, score_mode: str) -> torch.Tensor:
    """Node-mode gate -> [N,K,1]. The MLP and softmax stay fp32, as in the
    reference (model_cign.py:746-749)."""
    mode = {"old": 0, "new": 1}[str(score_mode)]
    H = H_norm.float().contiguous()
    C = C_norm.float().contiguous()
    bias = linear.bias if linear.bias is not None else torch.zeros(linear.out_features, device=H.device)
    alpha = HopGateFunction.apply(H, C, linear.weight.float().contiguous(), bias.float().contiguous(), mode)
    return alpha.unsqueeze(-1)


def global_hop_gate(logits: torch.Tensor, num_nodes: int) -> torch.Tensor:
    """Global mode: one softmax over K parameters broadcast to [N,K,1]
    (model_cign.py:727-731)."""
    alpha = F.softmax(logits, dim=0)
    return alpha.view(1, -1, 1).expand(num_nodes, -1, -1)
