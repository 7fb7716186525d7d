"""Hop gate of the Clifford block on gfx950 (generic_engine/model_cign.py:
721-749): alpha[n, :] = softmax_k(Linear(2D -> K)(score[n, :])) with score
[H | C] (alpha_score_mode "old") or [H + C | |H - C|] ("new"), computed by
one fused kernel (cign_hop_gate_fwd) and its backward (cign_hop_gate_bwd).
"global" mode is softmax of K parameters (no kernel needed) and "none"
returns None, as in the reference.
"""
from __future__ import annotations

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
