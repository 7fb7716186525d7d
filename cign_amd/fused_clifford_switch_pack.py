"""Drop-in for the reference module generic_engine/fused_clifford_switch_pack.py
(same public names, extension entry points, mode strings and errors): the
CIGN switch-aware K=3 fused Clifford pack whose interaction mode "new" is
W = tanh((B_HR-B_RH)/2), D = SiLU((B_HR+B_RH)/2) (C-ABI interaction code 2;
fused_clifford_switch_pack_cuda.cu:48,51). The implementation, shared with
fused_clifford_cign_pack, is in _switch_pack.py."""
from __future__ import annotations

from . import _switch_pack

_impl = _switch_pack.make(2, "cign_amd_fused_clifford_switch_pack_hip")

_extension_name = _impl.extension_name
_mode_to_int = _switch_pack.mode_to_int
ensure_fused_clifford_switch_pack_loaded = _impl.ensure_loaded
FusedCliffordSwitchPackFunction = _impl.function
fused_clifford_switch_pack = _impl.pack
