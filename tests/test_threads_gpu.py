"""Engines called from many host threads at once.

The reference engines are `&self`, Send + Sync and callable from many threads (cudarc
serialises on one stream per device; DistributedKnnEngine fans out over rayon,
distributed_knn.rs:165-187).  Here every engine serialises its calls on its own stream under
its own mutex, and the error message is thread-local.  ctypes releases the GIL around each
library call, so the threads below really do overlap inside the library.  Every concurrent
result must equal, bit for bit, the result of the same call made alone.
"""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    assert vector_hip.CudaDeviceContext.device_count() >= 1
    return vector_hip


def _same(a, b):
    return all(np.array_equal(x.view(np.uint32) if x.dtype == np.float32 else x,
                              y.view(np.uint32) if y.dtype == np.float32 else y) for x, y in zip(a, b))


def test_one_knn_engine_many_threads(vh):
    print("threads: one kNN engine, 8 threads", flush=True)
    rng = np.random.default_rng(1)
    base = rng.standard_normal((50_000, 64)).astype(np.float32)
    eng = vh.CudaKnnEngine(base, 64)
    jobs = [(rng.standard_normal((int(rng.integers(1, 700)), 64)).astype(np.float32), int(rng.integers(1, 200)))
            for _ in range(16)]
    serial = [eng.search_batch_arrays(q, k) for q, k in jobs]
    with ThreadPoolExecutor(max_workers=8) as ex:
        for _ in range(3):
            got = list(ex.map(lambda j: eng.search_batch_arrays(*j), jobs))
            assert all(_same(g, s) for g, s in zip(got, serial))


def test_independent_engines_many_threads(vh):
    """Engines of different metrics, created and searched concurrently (creation uploads
    through each engine's own pinned staging)."""
    print("threads: independent engines", flush=True)
    rng = np.random.default_rng(2)
    base = rng.standard_normal((20_000, 48)).astype(np.float32)
    q = rng.standard_normal((100, 48)).astype(np.float32)
    metrics = [vh.DistanceMetric.L2Squared, vh.DistanceMetric.CosineSimilarity, vh.DistanceMetric.DotProduct,
               vh.DistanceMetric.Manhattan, vh.DistanceMetric.Chebyshev, vh.DistanceMetric.L2Squared]

    def run(m):
        return vh.CudaKnnEngine(base, 48, m).search_batch_arrays(q, 25)

    serial = [run(m) for m in metrics]
    with ThreadPoolExecutor(max_workers=6) as ex:
        got = list(ex.map(run, metrics))
    assert all(_same(g, s) for g, s in zip(got, serial))


def test_kmeans_and_search_interleaved(vh):
    """k-means fits (their own states) and kNN searches (a shared engine) at the same time."""
    print("threads: k-means fits with searches", flush=True)
    from vector_hip import datasets as ds

    x, _, _ = ds.gaussian_mixture(40_000, 32, 64, 3)
    eng = vh.CudaKnnEngine(x, 32)
    q = x[:300] + 0.01

    def fit(seed):
        r = vh.CudaKMeansEngine().fit(x, 32, 64, 5, -1.0, seed=seed)
        return r.centroids, np.float32(r.inertia)

    def search(k):
        return eng.search_batch_arrays(q, k)

    serial_fit = [fit(s) for s in (1, 2, 3)]
    serial_search = [search(k) for k in (5, 50, 100)]
    with ThreadPoolExecutor(max_workers=6) as ex:
        fits = [ex.submit(fit, s) for s in (1, 2, 3)]
        searches = [ex.submit(search, k) for k in (5, 50, 100)]
        for f, s in zip(fits, serial_fit):
            c, i = f.result()
            assert np.array_equal(c, s[0]) and i == s[1]
        for f, s in zip(searches, serial_search):
            assert _same(f.result(), s)


def test_ivfpq_index_many_threads(vh):
    print("threads: IVF-PQ index, 4 threads", flush=True)
    from vector_hip import datasets as ds

    base = ds.uniform(30_000, 32, 5)
    cfg = vh.IvfPqConfig.new(64, 8, 8).with_sub_clusters(256).with_max_kmeans_iters(4)
    ix = vh.IvfPqIndex.build_with_config(base, cfg, vh.DistanceMetric.L2Squared)
    rng = np.random.default_rng(6)
    jobs = [(ds.uniform(int(rng.integers(1, 300)), 32, 100 + i), int(rng.integers(1, 50)), int(rng.integers(1, 64)))
            for i in range(8)]
    serial = [ix.search_batch_arrays(q, k, nprobe=p) for q, k, p in jobs]
    with ThreadPoolExecutor(max_workers=4) as ex:
        got = list(ex.map(lambda j: ix.search_batch_arrays(j[0], j[1], nprobe=j[2]), jobs))
    assert all(_same(g, s) for g, s in zip(got, serial))


def test_error_messages_stay_in_their_thread(vh):
    """Each thread sees its own failure's message (vhip_last_error is thread-local)."""
    print("threads: thread-local errors", flush=True)
    eng = vh.CudaKnnEngine(np.zeros((10, 4), np.float32), 4)

    def bad_k(i):  # rejected inside the library, which records the message for this thread
        try:
            eng.search_batch_arrays(np.zeros((3, 4), np.float32), 3000 + i)
        except vh.InvalidConfig as e:
            return str(e)
        return ""

    def bad_gpus(i):
        try:
            vh.DistributedKMeansEngine.try_new(1000 + i)
        except vh.InsufficientDevices as e:
            return str(e), e.requested
        return "", -1

    with ThreadPoolExecutor(max_workers=8) as ex:
        a = list(ex.map(bad_k, range(16)))
        b = list(ex.map(bad_gpus, range(16)))
    assert all(f"k = {3000 + i} exceeds" in m for i, m in enumerate(a))
    assert all(str(1000 + i) in m and r == 1000 + i for i, (m, r) in enumerate(b))
