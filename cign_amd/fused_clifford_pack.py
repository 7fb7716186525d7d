"""Fused Clifford pack (old interaction, old weighting) on gfx950: a drop-in
for the reference module fused_clifford_pack.py, with the same public names,
extension entry points and errors.

The special K=3 extension (fused_clifford_pack_ext/fused_clifford_pack.cpp:
50-86) has ``forward(H, C, P0, P1, P2, alpha) -> out [N,6D]`` and
``backward(grad_out, H, C, P0, P1, P2, alpha) -> [gH, gC, gP0, gP1, gP2, gA]``.
The generic-K extension (fused_clifford_pack.py:46-63) has
``forward(H, C, P[N,K,2D], alpha) -> [out]`` and
``backward(grad_out, H, C, P, alpha) -> [gH, gC, gP, gA]``. Both run
cign_pack_fwd / cign_pack_bwd with interaction 0 and weighting 0:
  out[n, k*2D + d] = a_k (bhr - brh),  out[n, k*2D + D + d] = a_k SiLU(bhr),
  bhr = H * T_C, brh = C * T_H, T_H = P_k[:, :D], T_C = P_k[:, D:].
"""
from __future__ import annotations

from typing import Sequence

import torch

from . import _pack

_SPECIAL = {"ext": None, "err": None}
_GENERIC = {"ext": None, "err": None}


def _extension_name() -> str:
    return "cign_amd_fused_clifford_pack_hip"


class _SpecialExt:
    @staticmethod
    def forward(H, C, P0, P1, P2, alpha):
        _pack._validate(H, C, [P0, P1, P2], alpha, K_expected=3)
        return _pack.forward_list(H, C, [P0, P1, P2], alpha, 0, 0)

    @staticmethod
    def backward(grad_out, H, C, P0, P1, P2, alpha):
        _pack._validate(H, C, [P0, P1, P2], alpha, K_expected=3)
        gH, gC, gP, gA = _pack.backward_list(grad_out, H, C, [P0, P1, P2], alpha, 0, 0)
        return [gH, gC, gP[0], gP[1], gP[2], gA]


class _GenericExt:
    @staticmethod
    def forward(H, C, P, alpha):
        _pack._validate_stacked(H, C, P, alpha)
        return [_pack.forward_stacked(H, C, P, alpha, 0)]

    @staticmethod
    def backward(grad_out, H, C, P, alpha):
        _pack._validate_stacked(H, C, P, alpha)
        return list(_pack.backward_stacked(grad_out, H, C, P, alpha, 0))


_SPECIAL["factory"] = _SpecialExt
_GENERIC["factory"] = _GenericExt


def ensure_special_fused_clifford_pack_loaded(verbose: bool = False):
    return _pack.ensure_loaded(_SPECIAL, "fused Clifford pack")


def ensure_generic_fused_clifford_pack_loaded(verbose: bool = False):
    return _pack.ensure_loaded(_GENERIC, "generic Clifford pack")


def ensure_fused_clifford_pack_loaded(verbose: bool = False, hop_count: int = 3):
    """fused_clifford_pack.py:168-171."""
    if int(hop_count) == 3:
        return ensure_special_fused_clifford_pack_loaded(verbose)
    return ensure_generic_fused_clifford_pack_loaded(verbose)


class FusedCliffordPack3Function(torch.autograd.Function):
    """fused_clifford_pack.py:174-189."""

    @staticmethod
    def forward(ctx, H, C, P0, P1, P2, alpha):
        ext = ensure_special_fused_clifford_pack_loaded(False)
        out = ext.forward(H, C, P0, P1, P2, alpha)
        ctx.save_for_backward(H, C, P0, P1, P2, alpha)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        ext = ensure_special_fused_clifford_pack_loaded(False)
        H, C, P0, P1, P2, alpha = ctx.saved_tensors
        grads = ext.backward(grad_output.to(dtype=torch.float32).contiguous(), H, C, P0, P1, P2, alpha)
        return tuple(grads)


class GenericFusedCliffordPackFunction(torch.autograd.Function):
    """fused_clifford_pack.py:192-207."""

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
    """Old-interaction Clifford pack -> [N, K*2D] (fused_clifford_pack.py:220-244)."""
    H, C, props, A = _pack.prepare(H_norm, C_norm, propagated, alpha)
    if len(props) == 3:
        return FusedCliffordPack3Function.apply(H, C, props[0], props[1], props[2], A)
    P = torch.stack(props, dim=1).contiguous()  # [N,K,2D]
    return GenericFusedCliffordPackFunction.apply(H, C, P, A)
