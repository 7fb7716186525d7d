"""Writes tests/golden/seeds.json: the dropout seeds the reference derives
per call, recorded by importing the reference's own Python in this container
(the only place /root/reference exists). Nothing else pins these functions:
they are plain Python over torch.initial_seed() and per-process call
counters, with no closed form or library routine to check against.

  * fused_block_ops._next_seed(tag, dropout_p) (fused_block_ops.py:46-50):
    0 when p <= 0 (counter not advanced), else a value from the initial seed,
    the call number and the tag;
  * the seed collapsed_gat_mean_bias_silu passes to _CollapsedGATFn.apply
    (collapsed_gat.py:204-211): 0 when attn_drop <= 0 (counter not
    advanced), else a value from the initial seed and the call number. The
    function is called with stand-in inputs that pass its dtype/device checks
    (a duck-typed feature object reporting float32 on cuda) and with
    _CollapsedGATFn.apply replaced by one that returns its last argument, the
    seed; no kernel is built or run.

Run: python tests/golden/make_seeds.py (needs /root/reference; not run by the
tests, which read the JSON it wrote)."""
from __future__ import annotations

import itertools
import json
import sys
from pathlib import Path
from types import SimpleNamespace

import torch

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent / "seeds.json"

INITIAL_SEEDS = [0, 1, 12345, (1 << 40) + 7, (1 << 63) - 25, 2 ** 64 - 3]
BLOCK_CALLS = [(1, 0.3), (2, 0.3), (1, 0.0), (2, 0.0), (2, 0.5), (1, 0.1), (7, 0.9), (1, 1e-9), (2, 0.3)]
GAT_CALLS = [0.3, 0.0, 0.5, 0.0, 0.2, 1e-9, 0.0, 0.32]


class _Feat:
    """Duck-typed in_feat: float32 [N, H, C] on a cuda device."""

    dtype = torch.float32
    device = SimpleNamespace(type="cuda")

    def __init__(self, n=4, h=2, c=3):
        self.shape = (n, h, c)

    def dim(self):
        return 3

    def size(self, i):
        return self.shape[i]


def main() -> None:
    sys.path.insert(0, str(REF))
    import collapsed_gat as ref_gat  # noqa: E402  (reference module, imported here only)
    import fused_block_ops as ref_block  # noqa: E402

    out = {"source": "reference fused_block_ops._next_seed and collapsed_gat_mean_bias_silu seed derivation",
           "block_ops": [], "collapsed_gat": []}
    for s0 in INITIAL_SEEDS:
        torch.manual_seed(s0)
        assert torch.initial_seed() == s0 % (1 << 64)
        ref_block._CALL_COUNTER = itertools.count()
        calls = [{"tag": t, "p": p, "seed": int(ref_block._next_seed(t, p))} for t, p in BLOCK_CALLS]
        out["block_ops"].append({"initial_seed": int(torch.initial_seed()), "calls": calls})

    ref_gat._CollapsedGATFn.apply = staticmethod(lambda *args: int(args[-1]))
    feat, bias = _Feat(), object()
    for s0 in INITIAL_SEEDS:
        torch.manual_seed(s0)
        ref_gat._CALL_COUNTER = itertools.count()
        calls = []
        for p in GAT_CALLS:
            seed = ref_gat.collapsed_gat_mean_bias_silu(None, None, (None, None), (None, None), None, 0.2, feat, bias,
                                                        p)
            calls.append({"attn_drop": p, "seed": int(seed)})
        out["collapsed_gat"].append({"initial_seed": int(torch.initial_seed()), "calls": calls})
    OUT.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
