"""Writes tests/golden/dispatch_signatures.json: (key, cfg) of the reference's
generic_dispatch.canonical_config and cign_dispatch_utils.cign_speed_signature
for a set of command lines and switch environments, recorded by importing the
reference's own modules in this container (plain Python: hashlib, json, os,
re). A SHA-1 key over a serialised dict has no closed form to check a
restatement against; these vectors pin it.

Run: python tests/golden/make_dispatch_signatures.py (needs /root/reference)."""
from __future__ import annotations

import json
import os
import sys
from pathlib import Path

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent / "dispatch_signatures.json"

ARGVS = [
    [],
    ["--dataset_name", "Amazon_ratings", "--hidden_dim", "128", "--num_layers=2"],
    ["--hop_scales", "1", "2", "--gat_heads", "4", "--dropout=0.1", "--use_undirected", "false"],
    ["--hop_scales=1,3 5", "--layer_combine", "last", "--operator_mode", "hybrid", "--hybrid_alpha", "0.25"],
    ["--hop_scales", "--train_ratio", "0.6", "--val_ratio=0.2", "--test_ratio", "0.2", "--gamma_mode", "scalar"],
    ["--split_mode", "public", "--hop_gate_mode", "global", "--gat_dropout", "0.5", "--dataset_name=Roman-empire"],
    ["--hidden_dim", "64", "--hidden_dim", "32", "--use_undirected=YES", "--extra", "x"],
]
ENVS = [
    {},
    {"CIGN_ALPHA_SCORE_MODE": "new", "CIGN_INTERACTION_MODE": "New", "CIGN_ALPHA_WEIGHTING_MODE": " old "},
    {"CIGN_OUTER_NONLINEARITY": "none", "CLIFFORD_EDGE_DROP_RATIO": "0.1", "CIGN_INTERACTION_MODE": "new"},
]
KEYS = ("CIGN_ALPHA_SCORE_MODE", "CIGN_INTERACTION_MODE", "CIGN_ALPHA_WEIGHTING_MODE", "CIGN_OUTER_NONLINEARITY",
        "CLIFFORD_EDGE_DROP_RATIO")


def main() -> None:
    sys.path.insert(0, str(REF))
    import cign_dispatch_utils as ref_cign  # noqa: E402  (reference module, imported here only)
    import generic_dispatch as ref_gen  # noqa: E402

    saved = {k: os.environ.pop(k) for k in KEYS if k in os.environ}
    cases = []
    try:
        for env in ENVS:
            for k in KEYS:
                os.environ.pop(k, None)
            os.environ.update(env)
            for argv in ARGVS:
                gk, gcfg = ref_gen.canonical_config(argv)
                ck, ccfg = ref_cign.cign_speed_signature(argv)
                cases.append({"env": env, "argv": argv, "canonical_key": gk, "canonical_cfg": gcfg,
                              "cign_key": ck, "cign_cfg": ccfg})
    finally:
        for k in KEYS:
            os.environ.pop(k, None)
        os.environ.update(saved)
    OUT.write_text(json.dumps({"cases": cases}, indent=1) + "\n")
    print(f"wrote {OUT} ({len(cases)} cases)")


if __name__ == "__main__":
    main()
