"""The CIGN switch-aware K=3 fused Clifford pack behind both reference
modules generic_engine/fused_clifford_cign_pack.py and
generic_engine/fused_clifford_switch_pack.py (:18-183 in each). The two
differ only in what interaction mode "new" computes for W: (B_HR-B_RH)/2,
or tanh of it (fused_clifford_switch_pack_cuda.cu:48,51) -- C-ABI
interaction code 1 or 2 of cign_pack_fwd / cign_pack_bwd. make() builds one
module's public objects for a given code:

interaction_mode "old":  D = SiLU(B_HR),            W = B_HR - B_RH
interaction_mode "new":  D = SiLU((B_HR+B_RH)/2),   W = (B_HR-B_RH)/2 [tanh]
alpha_weighting_mode "old": output = cat_k(alpha_k * [W_k, D_k]) -> [N,6D]
alpha_weighting_mode "new": output = [sum_k alpha_k D_k, sum_k alpha_k W_k] -> [N,2D]
with B_HR = H*T_C, B_RH = C*T_H, T_H = P_k[:, :D], T_C = P_k[:, D:]. The
extension object has the reference's ``forward(H, C, P0, P1, P2, alpha,
interaction, weighting)`` and ``backward(grad_out, H, C, P0, P1, P2, alpha,
interaction, weighting) -> [gH, gC, gP0, gP1, gP2, gA]``
(fused_clifford_switch_pack.cpp:69-126).
"""
from __future__ import annotations

from types import SimpleNamespace
from typing import Sequence

import torch

from . import _pack
from ._lib import check


def mode_to_int(name: str, kind: str) -> int:
    """'old' -> 0, 'new' -> 1 (fused_clifford_cign_pack.py:58-64)."""
    value = str(name).strip().lower()
    if value == "old":
        return 0
    if value == "new":
        return 1
    raise ValueError(f"{kind} must be old/new, got {name!r}")


def make(new_interaction_code: int, extension_name: str) -> SimpleNamespace:
    """Public objects of one switch-pack module whose interaction mode "new"
    is C-ABI interaction code new_interaction_code."""
    state = {"ext": None, "err": None}

    def abi_interaction(mode: int) -> int:
        return 0 if int(mode) == 0 else int(new_interaction_code)

    def check_modes(interaction_mode, weighting_mode):
        check(int(interaction_mode) in (0, 1), "interaction_mode must be 0(old) or 1(new)")
        check(int(weighting_mode) in (0, 1), "weighting_mode must be 0(old) or 1(new)")

    class SwitchExt:
        @staticmethod
        def forward(H, C, P0, P1, P2, alpha, interaction_mode, weighting_mode):
            _pack._validate(H, C, [P0, P1, P2], alpha, K_expected=3)
            check_modes(interaction_mode, weighting_mode)
            return _pack.forward_list(H, C, [P0, P1, P2], alpha, abi_interaction(interaction_mode),
                                      int(weighting_mode))

        @staticmethod
        def backward(grad_out, H, C, P0, P1, P2, alpha, interaction_mode, weighting_mode):
            _pack._validate(H, C, [P0, P1, P2], alpha, K_expected=3)
            check_modes(interaction_mode, weighting_mode)
            N, D = H.shape
            old = int(weighting_mode) == 0
            check(grad_out.dim() == 2 and grad_out.size(0) == N and grad_out.size(1) == (6 * D if old else 2 * D),
                  "old weighting grad_out must be [N,6D]" if old else "new weighting grad_out must be [N,2D]")
            gH, gC, gP, gA = _pack.backward_list(grad_out, H, C, [P0, P1, P2], alpha,
                                                 abi_interaction(interaction_mode), int(weighting_mode))
            return [gH, gC, gP[0], gP[1], gP[2], gA]

    state["factory"] = SwitchExt

    def ensure_loaded(verbose: bool = False):
        """Loader semantics of the reference modules (:18-55): cached object,
        RuntimeError without a GPU, first failure cached and re-raised."""
        return _pack.ensure_loaded(state, "CIGN switch fused Clifford pack")

    class FusedCliffordSwitchPackFunction(torch.autograd.Function):
        """Autograd of the pack (fused_clifford_cign_pack.py:78-121)."""

        @staticmethod
        def forward(ctx, H, C, P0, P1, P2, alpha, interaction_mode_int: int, weighting_mode_int: int):
            ext = ensure_loaded(False)
            out = ext.forward(H, C, P0, P1, P2, alpha, int(interaction_mode_int), int(weighting_mode_int))
            ctx.interaction_mode_int = int(interaction_mode_int)
            ctx.weighting_mode_int = int(weighting_mode_int)
            ctx.save_for_backward(H, C, P0, P1, P2, alpha)
            return out

        @staticmethod
        def backward(ctx, grad_output):
            ext = ensure_loaded(False)
            H, C, P0, P1, P2, alpha = ctx.saved_tensors
            grads = ext.backward(grad_output.to(dtype=torch.float32).contiguous(), H, C, P0, P1, P2, alpha,
                                 ctx.interaction_mode_int, ctx.weighting_mode_int)
            return (*grads, None, None)

    def fused_clifford_switch_pack(H_norm: torch.Tensor, C_norm: torch.Tensor, propagated: Sequence[torch.Tensor],
                                   alpha: torch.Tensor | None, interaction_mode: str,
                                   alpha_weighting_mode: str) -> torch.Tensor:
        """Fused K=3 Clifford interaction + alpha weighting (:124-183)."""
        if len(propagated) != 3:
            raise ValueError("CIGN switch fused pack is specialized for exactly 3 hops; "
                             f"got {len(propagated)}.")
        if H_norm.dim() != 2 or C_norm.shape != H_norm.shape:
            raise ValueError("H_norm/C_norm must both be [N,D]")
        N, D = H_norm.shape
        H = H_norm.to(dtype=torch.float32).contiguous()
        C = C_norm.to(dtype=torch.float32).contiguous()
        props = [p.to(dtype=torch.float32).contiguous() for p in propagated]
        for p in props:
            if tuple(p.shape) != (N, 2 * D):
                raise ValueError(f"Every propagated tensor must be {(N, 2 * D)}, got {tuple(p.shape)}")
        A = _pack.normalize_alpha(alpha, int(N), 3, H.device)
        return FusedCliffordSwitchPackFunction.apply(H, C, props[0], props[1], props[2], A,
                                                     mode_to_int(interaction_mode, "interaction_mode"),
                                                     mode_to_int(alpha_weighting_mode, "alpha_weighting_mode"))

    return SimpleNamespace(ensure_loaded=ensure_loaded, function=FusedCliffordSwitchPackFunction,
                           pack=fused_clifford_switch_pack, extension_name=lambda: extension_name)
