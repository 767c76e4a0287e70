"""GPU tests of bases holding NaN and infinite values.

A non-finite value makes its own row's distances NaN or infinite, and nothing else: the squared-L2
column shift and the norm extremes are taken over the finite values only, the dense first round
ranks a NaN score after every other whatever its sign bit, and a NaN k-th score filters nothing.
So with at least k finite rows, every query's results equal the oracle's search over the finite
rows alone (ids mapped back).  The reference gives such rows no defined order (its heap compares
NaN as equal to everything, knn.rs:31-43), so the finite rows' neighbours are the contract.
"""
import numpy as np
import pytest

from knn_check import check_knn

pytestmark = pytest.mark.gpu

NAMES = {"l2": "L2Squared", "dot": "DotProduct", "cosine": "CosineSimilarity", "l1": "Manhattan"}


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    assert vector_hip.CudaDeviceContext.device_count() >= 1, "no gfx950 GPU visible"
    return vector_hip


def _plant(base, rng, n_nan_rows=40, with_inf=True):
    """NaN rows (positive and negative NaN), and unless with_inf is false one +inf value, one -inf
    value and one row mixing a NaN and an infinity; returns the mask of the rows that stay finite.
    (A dot product with an infinite row is an infinite similarity, which the reference ranks like
    any other value, so the dot-product case plants NaN only.)"""
    base = base.copy()
    n, d = base.shape
    rows = rng.choice(n, n_nan_rows + 3, replace=False)
    for i, r in enumerate(rows[:n_nan_rows]):
        base[r, rng.integers(0, d)] = np.nan if i % 2 == 0 else np.copysign(np.nan, -1.0)
    if with_inf:
        base[rows[n_nan_rows], 3] = np.inf
        base[rows[n_nan_rows + 1], d - 1] = -np.inf
        base[rows[n_nan_rows + 2], 0] = np.nan
        base[rows[n_nan_rows + 2], 1] = np.inf
    return base, np.all(np.isfinite(base), 1)


def _check_finite_rows(vh, oracle, base, keep, q, k, metric, **tol):
    eng = vh.CudaKnnEngine(base, base.shape[1], vh.DistanceMetric[NAMES[metric]])
    ids, dist, lens = eng.search_batch_arrays(q, k)
    assert np.all(lens == k)
    assert np.all(keep[ids.astype(np.int64)]), "a row holding a non-finite value was returned"
    pos = np.cumsum(keep) - 1
    check_knn(oracle, np.ascontiguousarray(base[keep]), q, pos[ids.astype(np.int64)].astype(np.uint32), dist, k,
              metric, **tol)


@pytest.mark.parametrize("metric", ["l2", "dot", "cosine", "l1"])
@pytest.mark.parametrize("k", [10, 100])
def test_float_base_with_nonfinite_rows(vh, oracle, metric, k):
    """Rows at 100 + N(0, 1): the squared-L2 shift is about 100 per column, so a non-finite shift
    would turn every row NaN."""
    rng = np.random.default_rng(41)
    clean = (100.0 + rng.standard_normal((20_000, 128))).astype(np.float32)
    base, keep = _plant(clean, rng, with_inf=metric != "dot")
    q = (100.0 + rng.standard_normal((200, 128))).astype(np.float32)
    print(f"  nonfinite float metric={metric} k={k}", flush=True)
    _check_finite_rows(vh, oracle, base, keep, q, k, metric, rtol=1e-4, atol=1e-5)


def test_integer_base_with_nonfinite_rows(vh, oracle):
    """Integer rows in [0, 255]: the shift is still rounded to integers over the finite values,
    and the finite rows' distances stay exact."""
    from vector_hip import datasets as ds

    rng = np.random.default_rng(42)
    base, keep = _plant(ds.uniform_int(30_000, 128, 43), rng)
    q = ds.uniform_int(300, 128, 44)
    print("  nonfinite integer l2 k=100", flush=True)
    _check_finite_rows(vh, oracle, base, keep, q, 100, "l2", rtol=0.0, atol=0.0)


def test_mostly_nan_base(vh, oracle):
    """More NaN rows than k among the first round's rows: the k-th score is NaN there, so later
    rounds must still filter nothing out."""
    rng = np.random.default_rng(45)
    base = rng.standard_normal((6_000, 32)).astype(np.float32)
    nan_rows = rng.choice(6_000, 5_900, replace=False)
    base[nan_rows, 0] = np.nan
    keep = np.all(np.isfinite(base), 1)
    q = rng.standard_normal((50, 32)).astype(np.float32)
    print("  mostly NaN l2 k=50", flush=True)
    _check_finite_rows(vh, oracle, base, keep, q, 50, "l2", rtol=1e-4, atol=1e-5)
