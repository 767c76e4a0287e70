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
