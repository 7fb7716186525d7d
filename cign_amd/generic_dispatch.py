"""Run-configuration signature of the reference's dispatcher
(generic_dispatch.py:10-89), kept so that callers which key results or
registries by it find the same keys. There is one HIP route, so the
reference's backend registry, environment fingerprint and autotune
certificates (generic_dispatch.py:92-200) have nothing to choose between
and are not carried over.

The key is the first 20 hex digits of the SHA-1 of the configuration dict
serialised as compact JSON with sorted keys; the dict's keys, defaults,
normalisations and revision string are the reference's, since the key must
match its keys for the same command line.
"""
from __future__ import annotations

import hashlib
import json
import os
import re

ENGINE_REVISION = "amazon_stage3_collapsed_v1"

DEFAULTS = {
    "dataset_name": "Amazon-ratings",
    "use_undirected": True,
    "split_mode": "random_ratio",
    "train_ratio": 0.50,
    "val_ratio": 0.25,
    "test_ratio": 0.25,
    "hidden_dim": 256,
    "num_layers": 4,
    "dropout": 0.28,
    "hop_scales": [1, 2, 3],
    "gat_heads": 6,
    "gat_dropout": 0.32,
    "gamma_mode": "vector",
    "hop_gate_mode": "node",
    "operator_mode": "adjacency",
    "hybrid_alpha": 0.5,
    "layer_combine": "concat",
    "fast_backend_policy": "auto",
    "generic_backend_profile": "auto",
}


def str2bool(v) -> bool:
    """'1', 'true', 'yes', 'y', 'on' (any case, stripped) are true."""
    if isinstance(v, bool):
        return v
    return str(v).strip().lower() in ("1", "true", "yes", "y", "on")


def _option(argv, name, default, cast=str):
    """Value of the first --name VALUE or --name=VALUE in argv, cast; the
    default (uncast) when absent."""
    flag = f"--{name}"
    for pos, tok in enumerate(argv):
        if tok == flag and pos + 1 < len(argv):
            return cast(argv[pos + 1])
        if tok.startswith(flag + "="):
            return cast(tok[len(flag) + 1:])
    return default


def _int_list(argv, name, default):
    """--name=1,2,3 (commas or spaces) or --name 1 2 3 (up to the next
    --option); a bare --name with no values gives the default."""
    flag = f"--{name}"
    for pos, tok in enumerate(argv):
        if tok.startswith(flag + "="):
            return [int(v) for v in re.split(r"[, ]+", tok[len(flag) + 1:].strip()) if v]
        if tok == flag:
            vals = []
            for nxt in argv[pos + 1:]:
                if nxt.startswith("--"):
                    break
                vals.append(int(nxt))
            return vals or list(default)
    return list(default)


def _signature(cfg: dict) -> str:
    raw = json.dumps(cfg, sort_keys=True, separators=(",", ":"))
    return hashlib.sha1(raw.encode("utf-8")).hexdigest()[:20]


def canonical_config(argv):
    """(key, cfg) of a command line: the options that change the timed
    computation, normalised (generic_dispatch.py:65-89)."""
    d = DEFAULTS
    cfg = {
        "engine_revision": ENGINE_REVISION,
        "dataset": str(_option(argv, "dataset_name", d["dataset_name"])).strip().lower().replace("_", "-"),
        "use_undirected": bool(_option(argv, "use_undirected", d["use_undirected"], str2bool)),
        "split_mode": str(_option(argv, "split_mode", d["split_mode"])),
        "train_ratio": float(_option(argv, "train_ratio", d["train_ratio"], float)),
        "val_ratio": float(_option(argv, "val_ratio", d["val_ratio"], float)),
        "test_ratio": float(_option(argv, "test_ratio", d["test_ratio"], float)),
        "hidden_dim": int(_option(argv, "hidden_dim", d["hidden_dim"], int)),
        "num_layers": int(_option(argv, "num_layers", d["num_layers"], int)),
        "dropout": float(_option(argv, "dropout", d["dropout"], float)),
        "hop_scales": _int_list(argv, "hop_scales", d["hop_scales"]),
        "gat_heads": int(_option(argv, "gat_heads", d["gat_heads"], int)),
        "gat_dropout": float(_option(argv, "gat_dropout", d["gat_dropout"], float)),
        "gamma_mode": str(_option(argv, "gamma_mode", d["gamma_mode"])),
        "hop_gate_mode": str(_option(argv, "hop_gate_mode", d["hop_gate_mode"])),
        "operator_mode": str(_option(argv, "operator_mode", d["operator_mode"])),
        "hybrid_alpha": float(_option(argv, "hybrid_alpha", d["hybrid_alpha"], float)),
        "layer_combine": str(_option(argv, "layer_combine", d["layer_combine"])),
        "edge_drop_ratio": float(os.environ.get("CLIFFORD_EDGE_DROP_RATIO", "0") or 0.0),
    }
    return _signature(cfg), cfg
