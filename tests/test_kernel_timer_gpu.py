"""GPU tests of the engines' kernel timers (vhip_knn_profile, vhip_kmeans_profile,
vhip_ivfpq_profile), whose start and stop events ride on the scan kernels' own dispatches.

The timers feed the roofline figures, so they are checked for what those figures assume: every
timed launch is counted, the summed algorithmic work equals one pass of the metric's work over
every base row (the search rounds cover each row exactly once), the summed kernel time is
positive and within the wall time of the calls it covers, and a timer that is switched off
records nothing.
"""
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    assert vector_hip.CudaDeviceContext.device_count() >= 1, "no gfx950 GPU visible"
    return vector_hip


def _timed(fn):
    import vector_hip

    vector_hip.synchronize()
    t0 = time.perf_counter()
    out = fn()
    vector_hip.synchronize()
    return out, (time.perf_counter() - t0) * 1e3


@pytest.mark.parametrize("metric,flops_per_elem", [("L2Squared", 2.0), ("CosineSimilarity", 2.0),
                                                   ("Manhattan", 1.0)])
def test_knn_timer_counts_every_row_once(vh, metric, flops_per_elem):
    from vector_hip import datasets as ds

    n, d, nq, k = 120_000, 96, 1500, 10
    print(f"knn timer {metric} n={n} d={d} nq={nq} k={k}", flush=True)
    base = ds.gaussian(n, d, 41)
    q = ds.gaussian(nq, d, 42)
    eng = vh.CudaKnnEngine(base, d, vh.DistanceMetric[metric])
    eng.search_batch_arrays(q, k)  # first use allocates the host path's buffers
    eng.profile(True)  # also clears what the timer held
    _, wall_ms = _timed(lambda: eng.search_batch_arrays(q, k))
    p = eng.profile_read()
    assert p["launches"] >= 2  # a dense first round and at least one filter round
    assert p["work"] == pytest.approx(flops_per_elem * nq * n * d, rel=1e-9)
    assert 0.0 < p["kernel_ms"] <= wall_ms
    # switched off, the timer records nothing more
    eng.profile(False)
    eng.search_batch_arrays(q, k)
    assert eng.profile_read()["launches"] == 0


def test_hamming_timer_counts_every_row_once(vh):
    from vector_hip import datasets as ds

    n, bits, nq, k = 300_000, 256, 2500, 10
    print(f"hamming timer n={n} bits={bits} nq={nq} k={k}", flush=True)
    codes = ds.packed_bits(n, bits, 43)
    q = ds.packed_bits(nq, bits, 44)
    eng = vh.HammingKnnEngine(codes)
    eng.search_batch_arrays(q, k)
    eng.profile(True)
    _, wall_ms = _timed(lambda: eng.search_batch_arrays(q, k))
    p = eng.profile_read()
    assert p["launches"] >= 2
    per_pair = p["work"] / (nq * n)
    assert per_pair in (bits // 32, 2.0 * bits)  # popcount words, or 2 K fp4 operations
    assert 0.0 < p["kernel_ms"] <= wall_ms


def test_kmeans_timer_counts_each_iteration(vh):
    from vector_hip import datasets as ds

    n, d, k, iters = 200_000, 64, 256, 3
    print(f"kmeans timer n={n} d={d} k={k} iters={iters}", flush=True)
    x = ds.gaussian(n, d, 45)
    st = vh.KMeansState(x)
    st.set_centroids(x[:k])
    st.run(1)
    st.profile(True)
    _, wall_ms = _timed(lambda: st.run(iters))
    p = st.profile_read()
    assert p["launches"] == iters
    assert p["work"] == pytest.approx(2.0 * n * k * d * iters, rel=1e-9)
    assert 0.0 < p["kernel_ms"] <= wall_ms


def test_ivfpq_timer_counts_the_scan(vh):
    rng = np.random.default_rng(46)
    n, d, nq = 60_000, 64, 800
    print(f"ivfpq timer n={n} d={d} nq={nq}", flush=True)
    centres = rng.standard_normal((64, d)).astype(np.float32) * 4.0
    data = (centres[rng.integers(0, 64, n)] + rng.standard_normal((n, d))).astype(np.float32)
    q = (centres[rng.integers(0, 64, nq)] + rng.standard_normal((nq, d))).astype(np.float32)
    cfg = vh.IvfPqConfig(nlist=64, nprobe=8, num_subvectors=8, sub_clusters=256)
    ix = vh.IvfPqIndex.build_with_config(data, cfg, dimension=d)
    ix.search_batch_arrays(q, 10, 8)
    ix.profile(True)
    _, wall_ms = _timed(lambda: ix.search_batch_arrays(q, 10, 8))
    p = ix.profile_read()
    assert p["launches"] >= 1
    assert 0.0 < p["kernel_ms"] <= wall_ms
