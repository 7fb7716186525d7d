import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built libcign_amd.so")


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def assert_close(actual, expected, rtol, atol, name=""):
    """|a - e| <= atol + rtol * |e| elementwise (the torch.allclose rule)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, f"{name}: shape {a.shape} != {e.shape}"
    err = np.abs(a - e)
    bad = err > atol + rtol * np.abs(e)
    if bad.any():
        i = np.unravel_index(np.argmax(err - (atol + rtol * np.abs(e))), a.shape)
        raise AssertionError(f"{name}: {int(bad.sum())} of {a.size} outside rtol={rtol} atol={atol}; "
                             f"worst at {i}: got {a[i]!r} expected {e[i]!r}")


def random_gat_graph(rng, n, avg_deg=6, hubs=None):
    """Unique (src, dst) edges + one self-loop per node, as the GAT sees them
    after prepare_gat_edge_index."""
    from oracle import cign_oracle as O

    src, dst = [], []
    for i in range(n):
        k = int(rng.integers(0, 2 * avg_deg + 1))
        if hubs and i in hubs:
            k = hubs[i]
        s = rng.choice(n, size=min(k, n), replace=False)
        src.extend(s.tolist())
        dst.extend([i] * len(s))
    ei = O.gat_edge_index(np.stack([np.array(src, dtype=np.int64), np.array(dst, dtype=np.int64)]), n)
    r, c, _ = O.coalesce(ei[0], ei[1], n)
    return np.stack([r, c])
