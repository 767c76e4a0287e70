"""Seeded sweep of engine shapes against the oracle.

Each case draws its shape at random from a fixed seed: base rows (1 to 20,000), dimension (1 to
300, so every MFMA kernel family and tail width appears), queries (1 to 300, crossing the
128-query tile), k (1 to 300, above n as well) and metric.  The case list is fixed, so a failure
names a reproducible case.  It covers the paths the workload tests reach only at one shape:
round sizing and balanced items at small n, the norm-seeded L2 accumulators at every
K-chunk count, and the fp4 Hamming kernel at every expanded width.
"""
import numpy as np
import pytest

from knn_check import check_knn

pytestmark = pytest.mark.gpu

METRICS = ["l2", "cosine", "dot", "l1", "minkowski", "linf", "hamming", "mahalanobis", "jaccard", "hellinger"]


def _cases(count, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        n = int(rng.choice([1, 7, 255, 256, 257, 1000, 5000, 20_000]))
        dim = int(rng.choice([1, 3, 31, 32, 33, 64, 96, 100, 128, 129, 200, 256, 300]))
        nq = int(rng.choice([1, 5, 127, 128, 129, 300]))
        k = int(rng.choice([1, 10, 64, 100, 300]))
        metric = METRICS[i % len(METRICS)]
        out.append((i, n, dim, nq, k, metric))
    return out


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    assert vector_hip.CudaDeviceContext.device_count() >= 1
    return vector_hip


@pytest.mark.parametrize("case", _cases(40, 2024), ids=lambda c: f"{c[0]}-n{c[1]}-d{c[2]}-q{c[3]}-k{c[4]}-{c[5]}")
def test_float_engine_sweep(vh, oracle, case):
    i, n, dim, nq, k, metric = case
    print(f"sweep case {case}", flush=True)
    rng = np.random.default_rng(1000 + i)
    if metric in ("jaccard", "hellinger"):
        base = rng.random((n, dim), dtype=np.float32)
        q = rng.random((nq, dim), dtype=np.float32)
    elif metric == "hamming":  # thresholded float Hamming needs coincident values
        base = np.round(rng.uniform(-1, 1, (n, dim)) * 2).astype(np.float32) / 2
        q = np.round(rng.uniform(-1, 1, (nq, dim)) * 2).astype(np.float32) / 2
    else:
        base = rng.standard_normal((n, dim)).astype(np.float32)
        q = rng.standard_normal((nq, dim)).astype(np.float32)
    eng = vh.CudaKnnEngine(base, dim, vh.DistanceMetric(oracle.METRICS[metric]))
    ids, dist, lens = eng.search_batch_arrays(q, k)
    assert np.all(lens == min(k, n))
    check_knn(oracle, base, q, ids, dist, k, metric, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("case", _cases(12, 77), ids=lambda c: f"{c[0]}-n{c[1]}-q{c[3]}-k{c[4]}")
def test_packed_hamming_sweep(vh, oracle, case):
    """Bit widths 32 to 1024 (the fp4 matrix-core kernel at every chunk count), bit-exact."""
    from vector_hip import datasets as ds

    i, n, _, nq, k, _ = case
    bits = [32, 64, 96, 128, 160, 256, 512, 1024][i % 8]
    print(f"hamming sweep case {case} bits={bits}", flush=True)
    codes = ds.packed_bits(n, bits, 500 + i)
    q = ds.packed_bits(nq, bits, 600 + i)
    ids, dist, lens = vh.HammingKnnEngine(codes).search_batch_arrays(q, k)
    rids, rdist, _ = oracle.hamming_packed_knn(codes, q, k)
    kk = min(k, n)
    assert np.all(lens == kk)
    assert np.array_equal(dist[:, :kk], rdist[:, :kk]) and np.array_equal(ids[:, :kk], rids[:, :kk])


def _wide_cases(count, seed):
    """Wider shapes than _cases: rows of up to 1,100 floats (the small-batch scan's widest tiles
    included), batches on both sides of the small-batch limits (32 and 128 queries), k up to 2048,
    and data kinds that stress the selection: integers, rows far from the origin, duplicates."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        n = int(rng.choice([1, 100, 5000, 30_000, 120_000]))
        dim = int(rng.choice([1, 100, 128, 300, 512, 768, 992, 1000, 1024, 1100]))
        nq = int(rng.choice([1, 17, 32, 33, 100, 129, 700]))
        k = int(rng.choice([1, 10, 93, 160, 2048]))
        metric = METRICS[i % len(METRICS)]
        kind = ["gauss", "int", "offset", "dup"][(i // len(METRICS)) % 4]
        while n * nq * dim > 6e8 and nq > 1:
            nq //= 2
        out.append((i, n, dim, nq, k, metric, kind))
    return out


def _data(kind, rng, n, dim, pool=None):
    if kind == "int":
        return rng.integers(0, 256, (n, dim)).astype(np.float32)
    if kind == "offset":
        return (rng.standard_normal((n, dim)) * 0.5 + 1000.0).astype(np.float32)
    if kind == "dup":
        return pool[rng.integers(0, len(pool), n)]
    return rng.standard_normal((n, dim)).astype(np.float32)


@pytest.mark.parametrize("case", _wide_cases(48, 2026),
                         ids=lambda c: f"{c[0]}-n{c[1]}-d{c[2]}-q{c[3]}-k{c[4]}-{c[5]}-{c[6]}")
def test_wide_engine_sweep(vh, oracle, case):
    i, n, dim, nq, k, metric, kind = case
    print(f"wide sweep case {case}", flush=True)
    rng = np.random.default_rng(3000 + i)
    if metric == "hamming":  # thresholded float Hamming needs coincident values
        kind = "binary"
        base = rng.integers(0, 2, (n, dim)).astype(np.float32)
        q = rng.integers(0, 2, (nq, dim)).astype(np.float32)
    else:
        if metric in ("jaccard", "hellinger"):  # non-negative data for these similarity forms
            kind = "int"
        if metric == "cosine" and kind == "offset":  # near-parallel rows: ties below float resolution
            kind = "gauss"
        pool = rng.standard_normal((20, dim)).astype(np.float32)
        base = _data(kind, rng, n, dim, pool)
        q = _data(kind, rng, nq, dim, pool)
    eng = vh.CudaKnnEngine(base, dim, vh.DistanceMetric(oracle.METRICS[metric]))
    ids, dist, lens = eng.search_batch_arrays(q, k)
    kk = min(k, n)
    assert np.all(lens == kk)
    scale = float(np.abs(base).max())
    atol = 1e-3 if kind == "offset" else 1e-5
    if metric == "dot":  # a dot product's rounding grows with its terms, not with its value
        atol = max(atol, 2e-6 * dim * scale * scale)
    exact = metric == "l2" and kind == "int" and dim <= 256
    check_knn(oracle, base, q, ids[:, :kk], dist[:, :kk], k, metric, rtol=0.0 if exact else 1e-4,
              atol=0.0 if exact else atol)
