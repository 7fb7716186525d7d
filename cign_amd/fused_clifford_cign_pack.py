"""CIGN switch-aware K=3 fused Clifford pack on gfx950: a drop-in for the
reference module generic_engine/fused_clifford_cign_pack.py, with the same public names,
extension entry points, mode strings and errors.

interaction_mode "old":  D = SiLU(B_HR),            W = B_HR - B_RH
interaction_mode "new":  D = SiLU((B_HR+B_RH)/2),   W = (B_HR-B_RH)/2
alpha_weighting_mode "old": output = cat_k(alpha_k * [W_k, D_k]) -> [N,6D]
alpha_weighting_mode "new": output = [sum_k alpha_k D_k, sum_k alpha_k W_k] -> [N,2D]
with B_HR = H*T_C, B_RH = C*T_H, T_H = P_k[:, :D], T_C = P_k[:, D:]
(generic_engine/fused_clifford_cign_pack.py:124-183; kernels
generic_engine/fused_clifford_cign_pack_ext/fused_clifford_switch_pack_cuda.cu).
The extension's ``forward(H, C, P0, P1, P2, alpha, interaction, weighting)``
and ``backward(grad_out, H, C, P0, P1, P2, alpha, interaction, weighting) ->
[gH, gC, gP0, gP1, gP2, gA]`` (fused_clifford_switch_pack.cpp:69-126) call
cign_pack_fwd / cign_pack_bwd.
"""
from __future__ import annotations

from typing import Sequence

import torch

from . import _pack
from ._lib import check

_STATE = {"ext": None, "err": None}
_NEW_INTERACTION = 1  # C-ABI interaction code of mode "new"


def _extension_name() -> str:
    return "cign_amd_fused_clifford_cign_pack_hip"


def _abi_interaction(interaction_mode: int) -> int:
    return 0 if int(interaction_mode) == 0 else _NEW_INTERACTION


class _SwitchExt:
    @staticmethod
    def _modes(interaction_mode, weighting_mode):
        check(int(interaction_mode) in (0, 1), "interaction_mode must be 0(old) or 1(new)")
        check(int(weighting_mode) in (0, 1), "weighting_mode must be 0(old) or 1(new)")

    @staticmethod
    def forward(H, C, P0, P1, P2, alpha, interaction_mode, weighting_mode):
        _pack._validate(H, C, [P0, P1, P2], alpha, K_expected=3)
        _SwitchExt._modes(interaction_mode, weighting_mode)
        return _pack.forward_list(H, C, [P0, P1, P2], alpha, _abi_interaction(interaction_mode), int(weighting_mode))

    @staticmethod
    def backward(grad_out, H, C, P0, P1, P2, alpha, interaction_mode, weighting_mode):
        _pack._validate(H, C, [P0, P1, P2], alpha, K_expected=3)
        _SwitchExt._modes(interaction_mode, weighting_mode)
        N, D = H.shape
        want = 6 * D if int(weighting_mode) == 0 else 2 * D
        which = "old weighting grad_out must be [N,6D]" if int(weighting_mode) == 0 else \
            "new weighting grad_out must be [N,2D]"
        check(grad_out.dim() == 2 and grad_out.size(0) == N and grad_out.size(1) == want, which)
        gH, gC, gP, gA = _pack.backward_list(grad_out, H, C, [P0, P1, P2], alpha, _abi_interaction(interaction_mode),
                                             int(weighting_mode))
        return [gH, gC, gP[0], gP[1], gP[2], gA]


_STATE["factory"] = _SwitchExt


def ensure_fused_clifford_switch_pack_loaded(verbose: bool = False):
    """generic_engine/fused_clifford_cign_pack.py:18-55 loader semantics."""
    return _pack.ensure_loaded(_STATE, "CIGN switch fused Clifford pack")


def _mode_to_int(name: str, kind: str) -> int:
    """generic_engine/fused_clifford_cign_pack.py:58-64."""
    value = str(name).strip().lower()
    if value == "old":
        return 0
    if value == "new":
        return 1
    raise ValueError(f"{kind} must be old/new, got {name!r}")


def _normalize_alpha(alpha, N: int, device) -> torch.Tensor:
    return _pack.normalize_alpha(alpha, N, 3, device)


class FusedCliffordSwitchPackFunction(torch.autograd.Function):
    """generic_engine/fused_clifford_cign_pack.py:78-121."""

    @staticmethod
    def forward(ctx, H, C, P0, P1, P2, alpha, interaction_mode_int: int, weighting_mode_int: int):
        ext = ensure_fused_clifford_switch_pack_loaded(False)
        out = ext.forward(H, C, P0, P1, P2, alpha, int(interaction_mode_int), int(weighting_mode_int))
        ctx.interaction_mode_int = int(interaction_mode_int)
        ctx.weighting_mode_int = int(weighting_mode_int)
        ctx.save_for_backward(H, C, P0, P1, P2, alpha)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        ext = ensure_fused_clifford_switch_pack_loaded(False)
        H, C, P0, P1, P2, alpha = ctx.saved_tensors
        grads = ext.backward(grad_output.to(dtype=torch.float32).contiguous(), H, C, P0, P1, P2, alpha,
                             ctx.interaction_mode_int, ctx.weighting_mode_int)
        return (*grads, None, None)


def fused_clifford_switch_pack(H_norm: torch.Tensor, C_norm: torch.Tensor, propagated: Sequence[torch.Tensor],
                               alpha: torch.Tensor | None, interaction_mode: str,
                               alpha_weighting_mode: str) -> torch.Tensor:
    """Fused K=3 Clifford interaction + alpha weighting
    (generic_engine/fused_clifford_cign_pack.py:124-183)."""
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
    A = _normalize_alpha(alpha, int(N), H.device)
    interaction_int = _mode_to_int(interaction_mode, "interaction_mode")
    weighting_int = _mode_to_int(alpha_weighting_mode, "alpha_weighting_mode")
    return FusedCliffordSwitchPackFunction.apply(H, C, props[0], props[1], props[2], A, interaction_int,
                                                 weighting_int)
