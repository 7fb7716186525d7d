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
    """|a - e| <= atol + rtol * |e| elementwise (the torch.allclose rule); a
    NaN matches only a NaN."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, f"{name}: shape {a.shape} != {e.shape}"
    err = np.abs(a - e)
    bad = ~(err <= atol + rtol * np.abs(e)) & ~(np.isnan(a) & np.isnan(e))
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


def assert_close_fp32_derived(actual, expected64, expected32, name="", rtol=1e-4, atol=1e-5, k=4.0, per_row=False):
    """Tolerance for float32 results that sum over many nodes (parameter
    gradients): |a - e64| <= atol + rtol |e64| + k |e32 - e64| + max |e32 -
    e64| elementwise, where e32 is the same oracle computation carried out in
    float32 on the same inputs. |e32 - e64| is the rounding error float32
    arithmetic incurs on exactly this computation; k allows for a different
    summation order, and the tensor's largest such error covers the elements
    where the oracle's own order happened to round well (the GPU's order
    rounds differently: at D = 128 a GAT attention gradient the fp32 oracle
    got within 7e-6 was 2.3e-4 off on the GPU, inside the 5.6e-4 the oracle
    itself missed by elsewhere in that tensor).

    per_row: for tensors whose first axis is the node (outputs, gradients of
    node features), the last term is 2 max |e32 - e64| over the element's own
    row instead of over the tensor: a node's row comes from that node's sums
    (its neighbours, its LayerNorm row), so the row's worst float32 error is
    the scale of the rounding a different order gives there. Over the block,
    pack-projection, net and c4 tests on the GPU the results reached at most
    1.07 times that row maximum beyond atol + rtol |e64| + 4 |e32 - e64|
    (grad H at D = 256), where the tensor-wide maximum was 13 times larger
    than what was needed."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected64, dtype=np.float64)
    e32 = np.asarray(expected32, dtype=np.float64)
    assert a.shape == e.shape == e32.shape, f"{name}: shapes {a.shape} {e.shape} {e32.shape}"
    err32 = np.abs(e32 - e)
    if not err32.size:
        spread = 0.0
    elif per_row and err32.ndim >= 2:
        spread = 2.0 * err32.reshape(err32.shape[0], -1).max(axis=1).reshape((-1,) + (1,) * (err32.ndim - 1))
    elif per_row:
        spread = 2.0 * err32
    else:
        spread = err32.max()
    bound = atol + rtol * np.abs(e) + k * err32 + spread
    err = np.abs(a - e)
    bad = ~(err <= bound) & ~(np.isnan(a) & np.isnan(e))
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), a.shape)
        raise AssertionError(f"{name}: {int(bad.sum())} of {a.size} outside the fp32-derived bound; worst at {i}: "
                             f"got {a[i]!r} expected {e[i]!r} (fp32 oracle {e32[i]!r}, bound {bound[i]!r})")


def colsum_atol(terms_abs_sum, n_rows):
    """Absolute error bound of a float32 sum over n_rows rows whose terms have
    the given sum of magnitudes (per output element): the kernels add rows in
    chunks and then the chunk partials in order, so the longest chain of
    dependent float32 additions is at most about 2 sqrt(n) + 8 long, each
    adding at most 2^-24 of the running magnitude; plus 1e-5 absolute."""
    return 1e-5 + (2.0 * np.sqrt(max(int(n_rows), 1)) + 8.0) * 2.0 ** -24 * np.asarray(terms_abs_sum, np.float64)


def assert_bf16_sum_close(actual, expected_rounded, abs_terms_sum, n_terms, name=""):
    """A sum formed in float32 and rounded once to bf16 (the GPU) against the
    same sum formed in float64 and rounded once to bf16 (the oracle). With
    s32, s64 the two unrounded sums, |s32 - s64| <= d = n 2^-24 sum|terms|
    (the float32 summation bound gamma_n; the products of bf16 operands are
    exact in float32), and rounding to nearest moves each by at most half a
    bf16 spacing, at most 2^-8 of its magnitude, so |a - e| <= 2^-7 |s64| +
    1.01 d <= 2^-7 (1 + 2^-8) |e| + 1.01 d elementwise. Both sides must be
    bf16 values."""
    from oracle import cign_oracle as O

    a = np.asarray(actual, np.float64)
    e = np.asarray(expected_rounded, np.float64)
    assert np.array_equal(O.bf16_round(a), a), f"{name}: not bf16-valued"
    d = float(n_terms) * 2.0 ** -24 * np.asarray(abs_terms_sum, np.float64)
    bound = 2.0 ** -7 * (1 + 2.0 ** -8) * np.abs(e) + 1.01 * d
    err = np.abs(a - e)
    bad = ~(err <= bound)
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), a.shape)
        raise AssertionError(f"{name}: {int(bad.sum())} of {a.size} outside the bf16 sum bound; worst at {i}: "
                             f"got {a[i]!r} expected {e[i]!r} bound {bound[i]!r}")


def bf16_store_bound(exact, abs_terms, n_terms, carried=0.0):
    """Elementwise bound of |a - e| for a result a that the GPU sums in
    float32 and stores once as bf16, against the float64 oracle e of the same
    sum on the same (bf16-rounded) inputs: the float32 sum s32 differs from
    e by at most d = n 2^-24 sum|terms| (the summation bound gamma_n), and
    rounding to bf16 moves it by at most half a bf16 spacing, 2^-8 |s32|, so
    |a - e| <= 2^-8 (|e| + d) + d. `carried`: an error the inputs already
    hold (earlier bf16 roundings in a chain, propagated through the sum's
    absolute weights), added to both |e| and d."""
    e = np.abs(np.asarray(exact, np.float64))
    d = np.asarray(n_terms, np.float64) * 2.0 ** -24 * np.asarray(abs_terms, np.float64) + carried
    return 2.0 ** -8 * (e + d) + d


def assert_within(actual, expected, bound, name=""):
    """|a - e| <= bound elementwise (a NaN matches only a NaN)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    b = np.broadcast_to(np.asarray(bound, np.float64), e.shape)
    assert a.shape == e.shape, f"{name}: shape {a.shape} != {e.shape}"
    err = np.abs(a - e)
    bad = ~(err <= b) & ~(np.isnan(a) & np.isnan(e))
    if bad.any():
        i = np.unravel_index(np.argmax(err - b), a.shape)
        raise AssertionError(f"{name}: {int(bad.sum())} of {a.size} outside the derived bound; worst at {i}: "
                             f"got {a[i]!r} expected {e[i]!r} bound {b[i]!r}")


def bf16_flip_atol(expected):
    """Extra absolute tolerance of a selective-bf16 result compared with an
    oracle that rounds to bf16 at the same points: where fp32 (GPU) and fp64
    (oracle) accumulation put a value on different sides of a bf16 rounding
    boundary, that value differs by one bf16 ulp, at most 2^-7 of the largest
    magnitude in its tensor, and the difference carries on to everything
    computed from it (which may cancel to far smaller values)."""
    e = np.asarray(expected, dtype=np.float64)
    return 2.0 ** -7 * (float(np.abs(e).max()) if e.size else 0.0)
