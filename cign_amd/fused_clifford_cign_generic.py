"""CIGN generic-K fused Clifford pack (new interaction, old weighting) on
gfx950: a drop-in for the reference module
generic_engine/fused_clifford_cign_generic.py.

out[n, k*2D + d] = a_k (B_HR - B_RH)/2, out[n, k*2D + D + d] = a_k SiLU((B_HR + B_RH)/2),
B_HR = H*T_C, B_RH = C*T_H (kernels generic_engine/fused_clifford_cign_generic.py:
58-109). The propagated hops are stacked to [N,K,2D] as in the reference
(:189); the extension's ``forward(H, C, P, alpha) -> [out]`` and
``backward(grad_out, H, C, P, alpha) -> [gH, gC, gP, gA]`` call cign_pack_fwd /
cign_pack_bwd with interaction 1 and weighting 0 (no atomics: the backward is
deterministic).
"""
from __future__ import annotations

from typing import Sequence

import torch

from . import _pack

_GENERIC = {"ext": None, "err": None}


class _GenericExt:
    @staticmethod
    def forward(H, C, P, alpha):
        _pack._validate_stacked(H, C, P, alpha)
        return [_pack.forward_stacked(H, C, P, alpha, 1)]

    @staticmethod
    def backward(grad_out, H, C, P, alpha):
        _pack._validate_stacked(H, C, P, alpha)
        return list(_pack.backward_stacked(grad_out, H, C, P, alpha, 1))


_GENERIC["factory"] = _GenericExt


def ensure_generic_fused_clifford_pack_loaded(verbose: bool = False):
    """generic_engine/fused_clifford_cign_generic.py:113-135 loader semantics."""
    return _pack.ensure_loaded(_GENERIC, "generic CIGN Clifford pack")


class GenericFusedCliffordPackFunction(torch.autograd.Function):
    """generic_engine/fused_clifford_cign_generic.py:138-152."""

    @staticmethod
    def forward(ctx, H, C, P, alpha):
        ext = ensure_generic_fused_clifford_pack_loaded(False)
        (out,) = ext.forward(H, C, P, alpha)
        ctx.save_for_backward(H, C, P, alpha)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        ext = ensure_generic_fused_clifford_pack_loaded(False)
        H, C, P, alpha = ctx.saved_tensors
        gh, gc, gp, ga = ext.backward(grad_output.to(dtype=torch.float32).contiguous(), H, C, P, alpha)
        return gh, gc, gp, ga


def _normalize_alpha(alpha, N: int, K: int, device) -> torch.Tensor:
    return _pack.normalize_alpha(alpha, N, K, device)


def fused_clifford_pack(H_norm: torch.Tensor, C_norm: torch.Tensor, propagated: Sequence[torch.Tensor],
                        alpha: torch.Tensor | None) -> torch.Tensor:
    """New-interaction Clifford pack for any K -> [N, K*2D]
    (generic_engine/fused_clifford_cign_generic.py:166-190)."""
    H, C, props, A = _pack.prepare(H_norm, C_norm, propagated, alpha)
    P = torch.stack(props, dim=1).contiguous()  # [N,K,2D]
    return GenericFusedCliffordPackFunction.apply(H, C, P, A)
