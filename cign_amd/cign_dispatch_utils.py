"""CIGN speed signature of the reference (cign_dispatch_utils.py:10-51): the
run-configuration signature of generic_dispatch.canonical_config plus the
outer nonlinearity and the three old/new switches (alpha score,
interaction, alpha weighting) that change the timed computation, read from
the same environment variables. Keys match the reference's for the same
command line and environment (same dict keys and revision string)."""
from __future__ import annotations

import os

from .generic_dispatch import _signature, canonical_config

CIGN_SWITCH_ENGINE_REVISION = "cign_fullaccel_v5_collapsed_dispatch"

_SWITCH_ENV = {"alpha_score": "CIGN_ALPHA_SCORE_MODE", "interaction": "CIGN_INTERACTION_MODE",
               "alpha_weighting": "CIGN_ALPHA_WEIGHTING_MODE"}


def _mode(env_name: str, default: str = "old") -> str:
    value = os.environ.get(env_name, default).strip().lower()
    if value not in ("old", "new"):
        raise ValueError(f"{env_name} must be old/new, got {value!r}")
    return value


def current_switch_modes() -> dict:
    """{'alpha_score', 'interaction', 'alpha_weighting'} -> 'old' | 'new'."""
    return {k: _mode(v) for k, v in _SWITCH_ENV.items()}


def all_old() -> bool:
    return all(v == "old" for v in current_switch_modes().values())


def cign_speed_signature(argv):
    """(key, cfg): canonical_config's dict plus CIGN_OUTER_NONLINEARITY
    (default tanh), the switch-engine revision and the three switches."""
    _, cfg = canonical_config(argv)
    cfg = dict(cfg)
    modes = current_switch_modes()
    cfg["outer_nonlinearity"] = os.environ.get("CIGN_OUTER_NONLINEARITY", "tanh")
    cfg["cign_switch_engine_revision"] = CIGN_SWITCH_ENGINE_REVISION
    cfg["cign_alpha_score_mode"] = modes["alpha_score"]
    cfg["cign_interaction_mode"] = modes["interaction"]
    cfg["cign_alpha_weighting_mode"] = modes["alpha_weighting"]
    return _signature(cfg), cfg
