"""ctypes binding of libcign_amd.so, the C-ABI declared in include/cign_amd.h.

The library is loaded after ``import torch`` so that it binds to the HIP
runtime torch already loaded (same soname, one runtime per process). Every
entry point returns an int status; non-zero raises ``RuntimeError`` carrying
``cign_last_error()``. There is no CPU fallback: a missing library or a
missing GPU raises.
"""
from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libcign_amd.so"

_P = C.c_void_p
_I32 = C.c_int32
_I64 = C.c_int64
_F32 = C.c_float
_U64 = C.c_uint64

# name -> (restype, argtypes)
_SIGNATURES = {
    "cign_last_error": (C.c_char_p, []),
    "cign_version": (C.c_int, []),
    "cign_row_schedule_size": (C.c_int, [_P, _I32, _I32, _I32, _P, _P, _P, _P]),
    "cign_row_schedule_build": (C.c_int, [_P, _I32, _I32, _I32, _P, _I64]),
    "cign_spmm_partial_bytes": (_I64, [_I32, _I32]),
    "cign_spmm": (C.c_int, [_P, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "cign_spmm_fwd3": (C.c_int, [_P, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "cign_spmm_bwd3": (C.c_int, [_P, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "cign_spmm_fwd3_noalloc": (C.c_int, [_P, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P]),
    "cign_gat_schedule_params": (C.c_int, [_I32, _I32, _I32, _I32, _P, _P]),
    "cign_gat_fwd_workspace_bytes": (_I64, [_I32, _I32, _I32]),
    "cign_gat_fwd": (C.c_int, [_P, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _F32, _P, _P, _F32, _U64,
                               _P, _P, _P, _P, _P, _P, _I64, _P]),
    "cign_gat_row_agg_floats": (_I64, [_I32, _I32, _I32, _I32]),
    "cign_gat_bwd_workspace_bytes": (_I64, [_I32, _I32, _I32, _I32, _I32, _I32, _I32]),
    "cign_gat_bwd": (C.c_int, [_P, _I32, _I32, _I32, _I32, _I32, _F32, _F32] + [_P] * 11
                     + [_P, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P]),
    "cign_gat_fwd_shard": (C.c_int, [_P, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _F32, _P, _P, _F32,
                                     _U64, _P, _P, _P, _P, _P, _P, _I64, _P, _I64, _I64]),
    "cign_gat_bwd_shard": (C.c_int, [_P, _I32, _I32, _I32, _I32, _I32, _F32, _F32] + [_P] * 11
                           + [_P, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _I32, _I32, _I64]),
    # GAT side ops and block ops (nodeops.hip)
    "cign_colsum_workspace_bytes": (_I64, [_I64, _I32, _I32]),
    "cign_attn_logits_fwd": (C.c_int, [_P, _I64, _I32, _I32, _P, _P, _P, _P, _P]),
    "cign_attn_logits_bwd": (C.c_int, [_P, _I64, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64]),
    "cign_attn_logits_fwd_bf16": (C.c_int, [_P, _I64, _I32, _I32, _P, _P, _P, _P, _P]),
    "cign_attn_logits_bwd_acc": (C.c_int, [_P, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                           _P, _I64]),
    "cign_head_silu_fwd": (C.c_int, [_P, _I64, _I32, _I32, _P, _P, _P, _P]),
    "cign_head_silu_bwd": (C.c_int, [_P, _I64, _I32, _I32, _P, _P, _P, _P, _P, _I64]),
    "cign_dropout_ln_fwd": (C.c_int, [_P, _I64, _I32, _P, _P, _P, _F32, _F32, _U64, _P, _P, _P, _P]),
    "cign_dropout_ln_bwd": (C.c_int, [_P, _I64, _I32, _P, _P, _P, _P, _P, _P, _F32, _P, _P, _P, _P, _I64]),
    "cign_add_ln_fwd": (C.c_int, [_P, _I64, _I32, _P, _P, _P, _P, _F32, _P, _P, _P]),
    "cign_add_ln_bwd": (C.c_int, [_P, _I64, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64]),
    "cign_gamma_residual_fwd": (C.c_int, [_P, _I64, _I32, _P, _P, _P, _F32, _U64, _P, _P]),
    "cign_gamma_residual_bwd": (C.c_int, [_P, _I64, _I32, _P, _P, _P, _P, _F32, _P, _P, _P, _I64]),
    "cign_add_ln_cat_fwd": (C.c_int, [_P, _I64, _I32, _P, _P, _P, _P, _F32, _P, _P, _P, _P]),
    "cign_add_ln_cat_bwd": (C.c_int, [_P, _I64, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64]),
    # hop gate (gate.hip)
    "cign_hop_gate_bwd_workspace_bytes": (_I64, [_I64, _I32, _I32]),
    "cign_hop_gate_fwd": (C.c_int, [_P, _I64, _I32, _I32, _I32, _P, _P, _P, _P, _P]),
    "cign_hop_gate_bwd": (C.c_int, [_P, _I64, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64]),
    # MFMA projections (gemm.hip)
    "cign_linear_fwd": (C.c_int, [_P, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _P]),
    "cign_linear_logits_fwd": (C.c_int, [_P, _I64, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P]),
    "cign_linear_fwd_bf16y": (C.c_int, [_P, _I64, _I32, _I32, _I32, _P, _P, _P, _P]),
    "cign_linear_logits_fwd_bf16y": (C.c_int, [_P, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P]),
    "cign_linear_gamma_fwd": (C.c_int, [_P, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _F32, _U64, _P, _P,
                                        _P]),
    "cign_linear_bwd_workspace_bytes": (_I64, [_I64, _I32, _I32, _I32]),
    "cign_linear_bwd": (C.c_int, [_P, _I64, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _I64]),
    "cign_linear_bwd_bf16gy": (C.c_int, [_P, _I64, _I32, _I32, _P, _P, _P, _P, _P, _P, _I64]),
    "cign_lin_logits_wgrad_workspace_bytes": (_I64, [_I64, _I32, _I32]),
    "cign_lin_logits_wgrad": (C.c_int, [_P, _I64, _I32, _I32, _I32, _I32, _I32] + [_P] * 11 + [_I64]),
    "cign_pack_proj_fwd_workspace_bytes": (_I64, [_I32, _I32, _I32]),
    "cign_pack_proj_fwd": (C.c_int, [_P, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _I64, _P, _I64, _P, _P, _P, _P,
                                     _F32, _U64, _P, _P, _P, _P, _I64]),
    "cign_pack_proj_bwd_workspace_bytes": (_I64, [_I64, _I32, _I32]),
    "cign_pack_proj_bwd": (C.c_int, [_P, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _I64, _P, _I64, _P, _I32, _P,
                                     _P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _I64]),
    # Clifford packs (pack.hip) and the gate fused into them (gate.hip)
    "cign_pack_gate_fwd": (C.c_int, [_P, _I64, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _I64, _P, _P, _P, _P]),
    "cign_pack_gate_bwd": (C.c_int, [_P, _I64, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _I64, _P, _P, _P, _P,
                                     _P, _I64, _P, _P, _P, _I64]),
    "cign_pack_fwd": (C.c_int, [_P, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _I64, _P, _P]),
    "cign_pack_bwd": (C.c_int, [_P, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _I64,
                                _P]),
}

_LOCK = threading.Lock()
_LIB = None
_LIB_ERROR: BaseException | None = None


class _Lib:
    def __init__(self, handle: C.CDLL):
        self._h = handle
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
            setattr(self, name, fn)

    def call(self, name: str, *args) -> None:
        rc = getattr(self, name)(*args)
        if rc != 0:
            msg = self.cign_last_error().decode(errors="replace")
            raise RuntimeError(f"{name} failed (status {rc}): {msg}")


def load_library(require_gpu: bool = True) -> _Lib:
    """Loads libcign_amd.so once. Raises RuntimeError if it is not built or,
    when ``require_gpu``, if no HIP device is visible."""
    global _LIB, _LIB_ERROR
    with _LOCK:
        if _LIB is None:
            if _LIB_ERROR is not None:
                raise RuntimeError("libcign_amd previously failed to load") from _LIB_ERROR
            try:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"{LIB_PATH} is not built; run `python -m cign_amd._build` (hipcc, gfx950)"
                    )
                _LIB = _Lib(C.CDLL(str(LIB_PATH)))
            except BaseException as exc:  # cached and re-raised, like the reference loaders
                _LIB_ERROR = exc
                raise
    if require_gpu and not torch.cuda.is_available():
        raise RuntimeError("libcign_amd kernels require a HIP GPU (torch.cuda.is_available() is False)")
    return _LIB


def exported_symbols() -> list[str]:
    return sorted(_SIGNATURES)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def ptr_array(ptrs) -> C.Array:
    """Host array of device pointers (the hop pointer arrays of the packs);
    pass ``C.addressof(arr)`` and keep ``arr`` alive for the call."""
    return (C.c_void_p * len(ptrs))(*ptrs)


def check(cond: bool, msg: str) -> None:
    """TORCH_CHECK equivalent of the reference bindings: RuntimeError."""
    if not cond:
        raise RuntimeError(msg)


def check_input(t: torch.Tensor, name: str, dtype: torch.dtype = torch.float32) -> None:
    """CHECK_INPUT of the reference bindings: CUDA, contiguous, dtype."""
    check(isinstance(t, torch.Tensor) and t.is_cuda, f"{name} must be CUDA")
    check(t.is_contiguous(), f"{name} must be contiguous")
    check(t.dtype == dtype, f"{name} must be {str(dtype).replace('torch.', '')}")


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Caller-owned scratch from torch's caching allocator (at least 1 byte)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def stream_ptr(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1}


def dtype_code(t: torch.Tensor) -> int:
    try:
        return DTYPE_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32 or bfloat16") from None
