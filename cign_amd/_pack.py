"""Shared host side of the Clifford pack mirrors (fused_clifford_pack,
fused_clifford_cign_pack, fused_clifford_switch_pack,
fused_clifford_cign_generic): argument checks of the reference bindings and
the calls into cign_pack_fwd / cign_pack_bwd.

Interaction codes on the C-ABI: 0 old, 1 new, 2 new with tanh on W.
Weighting codes: 0 old ([N, K*2D]), 1 new ([N, 2D], D first).
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from . import _lib
from ._lib import check, check_input

MAX_HOPS = 16


def _validate(H, C, props: Sequence[torch.Tensor], alpha, K_expected: int | None = None):
    """fused_clifford_pack.cpp:26-48 / fused_clifford_switch_pack.cpp:32-66."""
    for t, n in ((H, "H"), (C, "C"), (alpha, "alpha")):
        check_input(t, n)
    for k, p in enumerate(props):
        check_input(p, f"P{k}")
    check(H.dim() == 2, "H must be [N,D]")
    check(C.shape == H.shape, "C must match H")
    N, D = H.shape
    check(props[0].dim() == 2 and props[0].size(0) == N and props[0].size(1) == 2 * D, "P0 must be [N,2D]")
    for k in range(1, len(props)):
        check(props[k].shape == props[0].shape, f"P{k} must match P0")
    K = len(props) if K_expected is None else K_expected
    check(alpha.dim() == 2 and alpha.size(0) == N and alpha.size(1) == K, f"alpha must be [N,{K}]")
    check(1 <= len(props) <= MAX_HOPS, f"hop count must be in [1, {MAX_HOPS}]")


def _validate_stacked(H, C, P, alpha):
    """The generic-K bindings (fused_clifford_pack.py:56-63)."""
    for t, n in ((H, "H"), (C, "C"), (P, "P"), (alpha, "alpha")):
        check_input(t, n)
    check(H.dim() == 2 and C.shape == H.shape, "H/C must be [N,D]")
    check(P.dim() == 3 and P.size(0) == H.size(0) and P.size(2) == 2 * H.size(1), "P must be [N,K,2D]")
    check(alpha.dim() == 2 and alpha.size(0) == H.size(0) and alpha.size(1) == P.size(1), "alpha must be [N,K]")
    check(1 <= P.size(1) <= MAX_HOPS, f"hop count must be in [1, {MAX_HOPS}]")


def _out_width(D: int, K: int, weighting: int) -> int:
    return 2 * K * D if weighting == 0 else 2 * D


def forward_list(H, C, props, alpha, interaction: int, weighting: int) -> torch.Tensor:
    lib = _lib.load_library()
    N, D = H.shape
    K = len(props)
    out = torch.empty((N, _out_width(D, K, weighting)), dtype=torch.float32, device=H.device)
    arr = _lib.ptr_array([p.data_ptr() for p in props])
    lib.call("cign_pack_fwd", _lib.stream_ptr(H.device), N, D, K, int(interaction), int(weighting), H.data_ptr(),
             C.data_ptr(), ctypes.addressof(arr), 2 * D, alpha.data_ptr(), out.data_ptr())
    return out


def backward_list(grad_out, H, C, props, alpha, interaction: int, weighting: int):
    lib = _lib.load_library()
    N, D = H.shape
    K = len(props)
    check_input(grad_out, "grad_out")
    check(grad_out.dim() == 2 and grad_out.size(0) == N and grad_out.size(1) == _out_width(D, K, weighting),
          f"grad_out must have shape [N,{_out_width(D, K, weighting) // max(D, 1)}D]")
    gH, gC = torch.empty_like(H), torch.empty_like(C)
    gP = [torch.empty_like(p) for p in props]
    gA = torch.empty_like(alpha)
    arr = _lib.ptr_array([p.data_ptr() for p in props])
    garr = _lib.ptr_array([g.data_ptr() for g in gP])
    lib.call("cign_pack_bwd", _lib.stream_ptr(H.device), N, D, K, int(interaction), int(weighting),
             grad_out.data_ptr(), H.data_ptr(), C.data_ptr(), ctypes.addressof(arr), 2 * D, alpha.data_ptr(),
             gH.data_ptr(), gC.data_ptr(), ctypes.addressof(garr), 2 * D, gA.data_ptr())
    return gH, gC, gP, gA


def forward_stacked(H, C, P, alpha, interaction: int) -> torch.Tensor:
    lib = _lib.load_library()
    N, D = H.shape
    K = P.size(1)
    out = torch.empty((N, 2 * K * D), dtype=torch.float32, device=H.device)
    base, es = P.data_ptr(), P.element_size()
    arr = _lib.ptr_array([base + k * 2 * D * es for k in range(K)])
    lib.call("cign_pack_fwd", _lib.stream_ptr(H.device), N, D, K, int(interaction), 0, H.data_ptr(), C.data_ptr(),
             ctypes.addressof(arr), 2 * K * D, alpha.data_ptr(), out.data_ptr())
    return out


def backward_stacked(grad_out, H, C, P, alpha, interaction: int):
    lib = _lib.load_library()
    N, D = H.shape
    K = P.size(1)
    check_input(grad_out, "grad_out")
    check(grad_out.dim() == 2 and grad_out.size(0) == N and grad_out.size(1) == 2 * K * D,
          "grad_out must be [N,K*2D]")
    gH, gC, gP, gA = torch.empty_like(H), torch.empty_like(C), torch.empty_like(P), torch.empty_like(alpha)
    es = P.element_size()
    arr = _lib.ptr_array([P.data_ptr() + k * 2 * D * es for k in range(K)])
    garr = _lib.ptr_array([gP.data_ptr() + k * 2 * D * es for k in range(K)])
    lib.call("cign_pack_bwd", _lib.stream_ptr(H.device), N, D, K, int(interaction), 0, grad_out.data_ptr(),
             H.data_ptr(), C.data_ptr(), ctypes.addressof(arr), 2 * K * D, alpha.data_ptr(), gH.data_ptr(),
             gC.data_ptr(), ctypes.addressof(garr), 2 * K * D, gA.data_ptr())
    return gH, gC, gP, gA


def normalize_alpha(alpha, N: int, K: int, device) -> torch.Tensor:
    """_normalize_alpha of the reference modules (fused_clifford_pack.py:210-217):
    None -> ones; [N,K,1] -> [N,K]; float32 contiguous; shape checked."""
    if alpha is None:
        return torch.ones((N, K), device=device, dtype=torch.float32)
    if alpha.dim() == 3 and alpha.size(-1) == 1:
        alpha = alpha.squeeze(-1)
    if tuple(alpha.shape) != (N, K):
        raise ValueError(f"Expected alpha {(N, K)}, got {tuple(alpha.shape)}")
    return alpha.to(dtype=torch.float32).contiguous()


def prepare(H_norm, C_norm, propagated, alpha, K_fixed: int | None = None):
    """Shared Python-level checks of the reference wrappers
    (fused_clifford_pack.py:220-244, fused_clifford_cign_pack.py:148-183)."""
    if K_fixed is not None and len(propagated) != K_fixed:
        raise ValueError(f"fused pack is specialized for exactly {K_fixed} hops; got {len(propagated)}.")
    if H_norm.dim() != 2 or C_norm.shape != H_norm.shape:
        raise ValueError("H_norm and C_norm must both be [N,D]")
    N, D = H_norm.shape
    K = len(propagated)
    if K <= 0:
        raise ValueError("propagated cannot be empty")
    H = H_norm.to(dtype=torch.float32).contiguous()
    C = C_norm.to(dtype=torch.float32).contiguous()
    A = normalize_alpha(alpha, int(N), int(K), H.device)
    props = [p.to(dtype=torch.float32).contiguous() for p in propagated]
    for p in props:
        if tuple(p.shape) != (N, 2 * D):
            raise ValueError(f"Every propagated tensor must be {(N, 2 * D)}, got {tuple(p.shape)}")
    return H, C, props, A


def ensure_loaded(state: dict, what: str):
    """Loader semantics of the reference modules: RuntimeError without a GPU,
    first load error cached and re-raised."""
    if state.get("ext") is not None:
        return state["ext"]
    if state.get("err") is not None:
        raise RuntimeError(f"{what} extension previously failed to load") from state["err"]
    if not torch.cuda.is_available():
        raise RuntimeError(f"{what} requires a HIP GPU")
    try:
        _lib.load_library()
        state["ext"] = state["factory"]()
        return state["ext"]
    except Exception as exc:
        state["err"] = exc
        raise


class CliffordPackFunction(torch.autograd.Function):
    """Any interaction (0 old, 1 new, 2 new + tanh) x weighting (0 old, 1 new)
    over K separate [N,2D] hops: the single HIP route the Clifford block uses
    for every mode combination (the reference dispatches the same math over
    its four pack modules and a torch fallback, model_cign.py:803-925)."""

    @staticmethod
    def forward(ctx, interaction, weighting, H, C, alpha, *props):
        _validate(H, C, list(props), alpha)
        ctx.modes = (int(interaction), int(weighting))
        ctx.save_for_backward(H, C, alpha, *props)
        return forward_list(H, C, list(props), alpha, int(interaction), int(weighting))

    @staticmethod
    def backward(ctx, grad_out):
        H, C, alpha, *props = ctx.saved_tensors
        gH, gC, gP, gA = backward_list(grad_out.to(dtype=torch.float32).contiguous(), H, C, props, alpha, *ctx.modes)
        return (None, None, gH, gC, gA, *gP)


def clifford_pack_any(H_norm, C_norm, propagated, alpha, interaction: int, weighting: int) -> torch.Tensor:
    H, C, props, A = prepare(H_norm, C_norm, propagated, alpha)
    return CliffordPackFunction.apply(int(interaction), int(weighting), H, C, A, *props)
