"""GPU parity tests of the kNN path through the C ABI (vector_hip -> libvector_hip.so).

Mirrors the reference's own tests (knn.rs:410-542, distributed_knn.rs:270-494,
integration_tests.rs:7-161) and adds seeded, workload-shaped parity against the CPU
oracle: tie-aware recall >= 0.999, distances within 1e-4 relative, exact for the
integer-valued squared-L2 workload.
"""
import numpy as np
import pytest

from knn_check import check_knn

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    assert vector_hip.CudaDeviceContext.device_count() >= 1, "no gfx950 GPU visible"
    return vector_hip


def _knn_rs_data(n):
    i = np.arange(n, dtype=np.float32)
    return np.stack([i * i * 0.1, i * 2.0, i + 5.0, i * 3.0], 1).astype(np.float32)


# ---- reference known-answer tests (knn.rs:410-542) ------------------------------------
def test_exact_match_vs_cpu_flat(vh, oracle):
    data = _knn_rs_data(50)
    eng = vh.CudaKnnEngine(data, 4, vh.DistanceMetric.L2Squared)
    cpu_ids, cpu_d = oracle.flat_search(data, data[10], 5, "l2")
    gpu = eng.search(data[10], 5)
    assert len(gpu) == 5
    for i in range(5):
        assert gpu[i].id == cpu_ids[i] and abs(gpu[i].distance - cpu_d[i]) < 1e-4


def test_batch_queries(vh):
    eng = vh.CudaKnnEngine(np.array([0, 0, 1, 1, 2, 2], np.float32), 2)
    r = eng.search_batch(np.array([0.1, 0.1, 1.9, 1.9], np.float32), 1)
    assert len(r) == 2 and r[0][0].id == 0 and r[1][0].id == 2


def test_empty_and_zero_k(vh):
    eng = vh.CudaKnnEngine(np.array([1, 2, 3, 4], np.float32), 2)
    assert eng.search(np.zeros(0, np.float32), 5) == []
    assert eng.search_batch(np.zeros(0, np.float32), 5) == []
    assert eng.search(np.array([1, 2], np.float32), 0) == []
    r = eng.search_batch(np.array([1, 2], np.float32), 0)
    assert len(r) == 1 and r[0] == []


def test_k_greater_than_num_vectors(vh):
    eng = vh.CudaKnnEngine(np.array([0, 0, 1, 1, 2, 2], np.float32), 2)
    assert len(eng.search(np.array([0.5, 0.5], np.float32), 100)) == 3


def test_cosine_and_dot(vh):
    eng = vh.CudaKnnEngine(np.array([1, 0, 0, 1, -1, 0], np.float32), 2, vh.DistanceMetric.CosineSimilarity)
    r = eng.search(np.array([0.95, 0.05], np.float32), 3)
    assert len(r) == 3 and r[0].id == 0 and r[2].id == 2
    eng = vh.CudaKnnEngine(np.array([1, 1, 2, 2, 3, 3], np.float32), 2, vh.DistanceMetric.DotProduct)
    r = eng.search(np.array([2, 3], np.float32), 2)
    assert [x.id for x in r] == [2, 1] and abs(r[0].distance - 15.0) < 1e-5


def test_getters_and_self_query(vh):
    eng = vh.CudaKnnEngine(np.array([1, 2, 3, 4, 5, 6], np.float32), 3)
    assert (eng.dimension(), eng.num_vectors(), eng.metric(), eng.device_id()) == (3, 2, vh.DistanceMetric.L2Squared,
                                                                                   0)
    data = np.array([10, 20, 30, 40, 50, 60], np.float32)
    eng = vh.CudaKnnEngine(data, 2)
    for i in range(3):
        r = eng.search(data[2 * i:2 * i + 2], 1)
        assert r[0].id == i and abs(r[0].distance) < 1e-4


# ---- DistributedKnnEngine (distributed_knn.rs:270-467, integration_tests.rs) -------------
def test_ddp_sharded_exact_match(vh, oracle):
    data = _knn_rs_data(60)
    ddp = vh.DistributedKnnEngine.emulator(data, 4, 3, vh.GpuShardMode.Sharded, vh.DistanceMetric.L2Squared)
    assert ddp.num_gpus() == 3 and ddp.num_vectors() == 60
    ids, d = oracle.flat_search(data, data[25], 5)
    r = ddp.search(data[25], 5)
    assert [x.id for x in r] == list(ids) and np.allclose([x.distance for x in r], d, atol=1e-4)


def test_ddp_replicated_and_global_ids(vh):
    data = np.array([0, 0, 1, 1, 2, 2, 3, 3], np.float32)
    e = vh.DistributedKnnEngine.emulator(data, 2, 2, vh.GpuShardMode.Replicated)
    r = e.search_batch(np.array([0.1, 0.1, 2.9, 2.9], np.float32), 1)
    assert r[0][0].id == 0 and r[1][0].id == 3
    data = np.array([10, 10, 20, 20, 30, 30, 40, 40], np.float32)
    s = vh.DistributedKnnEngine.emulator(data, 2, 2, vh.GpuShardMode.Sharded)
    assert s.search(np.array([39.9, 40.1], np.float32), 1)[0].id == 3
    assert s.search(np.array([20.1, 19.9], np.float32), 1)[0].id == 1
    for mode in (vh.GpuShardMode.Sharded, vh.GpuShardMode.Replicated):
        e = vh.DistributedKnnEngine.emulator(np.array([1, 2, 3, 4], np.float32), 2, 2, mode)
        assert e.search(np.zeros(0, np.float32), 5) == [] and e.search(np.array([1, 2], np.float32), 0) == []


def test_ddp_more_gpus_than_vectors_and_getters(vh):
    e = vh.DistributedKnnEngine.emulator(np.array([1, 1, 2, 2], np.float32), 2, 8, vh.GpuShardMode.Sharded)
    assert e.num_gpus() == 2 and e.num_vectors() == 2
    r = e.search(np.array([1, 1], np.float32), 2)
    assert len(r) == 2 and r[0].id == 0
    e = vh.DistributedKnnEngine.emulator(np.array([1, 2, 3, 4, 5, 6], np.float32), 3, 2, vh.GpuShardMode.Sharded)
    assert (e.num_gpus(), e.num_vectors(), e.dimension(), e.mode(), e.metric()) == (
        2, 2, 3, vh.GpuShardMode.Sharded, vh.DistanceMetric.L2Squared)


def test_try_new_single_gpu(vh, oracle):
    data = _knn_rs_data(40)
    e = vh.DistributedKnnEngine.try_new(data, 4, 1, vh.GpuShardMode.Sharded, vh.DistanceMetric.L2Squared)
    assert e.num_gpus() == 1
    ids, _ = oracle.flat_search(data, data[7], 4)
    assert [x.id for x in e.search(data[7], 4)] == list(ids)


def test_single_vs_multi_rank_consistency(vh):
    i = np.arange(60, dtype=np.float32)
    data = np.stack([i * 0.5, i * i * 0.05, np.sin(i + 3.0)], 1).astype(np.float32)
    q = np.array([1.0, 2.0, 0.5, 15.0, 45.0, -0.5, 25.0, 120.0, 0.8], np.float32)
    single = vh.CudaKnnEngine(data, 3).search_batch(q, 5)
    for mode in (vh.GpuShardMode.Sharded, vh.GpuShardMode.Replicated):
        other = vh.DistributedKnnEngine.emulator(data, 3, 4, mode).search_batch(q, 5)
        for a, b in zip(single, other):
            assert [x.id for x in a] == [x.id for x in b]
            assert np.allclose([x.distance for x in a], [x.distance for x in b], atol=1e-4)


def test_end_to_end_sharded_cluster_query(vh):
    data = np.concatenate([np.tile([0.1, 0.0, -0.1, 0.05], (30, 1)), np.tile([9.9, 10.1, 10.0, 9.95], (30, 1)),
                           np.tile([20.0, 19.9, 20.1, 20.05], (30, 1))]).astype(np.float32)
    e = vh.DistributedKnnEngine.emulator(data, 4, 3, vh.GpuShardMode.Sharded)
    r = e.search(np.full(4, 10.0, np.float32), 5)
    assert len(r) == 5 and all(30 <= x.id < 60 and x.distance < 1.0 for x in r)


ALL_METRICS = ["l2", "cosine", "dot", "l1", "minkowski", "linf", "hamming", "mahalanobis", "jaccard", "hellinger"]


@pytest.mark.parametrize("metric", ALL_METRICS)
def test_all_metrics_consistency(vh, oracle, metric):
    """integration_tests.rs:121-161, plus agreement with the CPU engine values."""
    data = np.array([0.8, 0.6, 0.8, 0.0, 0.0, 0.6, 0.1, 0.1, -1.0, -1.0], np.float32).reshape(5, 2)
    q = np.array([[0.8, 0.6]], np.float32)
    m = vh.DistanceMetric(oracle.METRICS[metric])
    single = vh.CudaKnnEngine(data, 2, m).search(q, 3)
    ddp = vh.DistributedKnnEngine.emulator(data, 2, 2, vh.GpuShardMode.Sharded, m).search(q, 3)
    assert len(single) == 3 and len(ddp) == 3
    for a, b in zip(single, ddp):
        assert abs(a.distance - b.distance) < 1e-4
    ids = np.array([[x.id for x in single]], np.uint32)
    dist = np.array([[x.distance for x in single]], np.float32)
    check_knn(oracle, data, q, ids, dist, 3, metric, rtol=1e-4, atol=1e-5)


# ---- seeded workload-shaped parity against the oracle ------------------------------------
@pytest.mark.parametrize("metric", ["l2", "dot", "cosine"])
def test_gaussian_10k_x128_parity(vh, oracle, metric):
    """10k x 128 N(0,1) base, 100 queries, k=10 (the CPU-runnable workload)."""
    from vector_hip import datasets as ds

    base = ds.gaussian(10_000, 128, ds.SEED_BASE)
    q = ds.gaussian(100, 128, ds.SEED_QUERIES)
    ids, dist, lens = vh.CudaKnnEngine(base, 128, vh.DistanceMetric(oracle.METRICS[metric])).search_batch_arrays(q, 10)
    assert np.all(lens == 10)
    check_knn(oracle, base, q, ids, dist, 10, metric, rtol=1e-4, atol=1e-5)


def test_integer_l2_exact_k100(vh, oracle):
    """Integer-valued [0,255] x 128 base (the 1M x 128 workload's distribution) at
    N = 200k, 64 queries, k = 100: every fp32 intermediate is an integer < 2^24, so
    distances must equal the reference bit for bit."""
    from vector_hip import datasets as ds

    base = ds.uniform_int(200_000, 128, ds.SEED_BASE)
    q = ds.uniform_int(64, 128, ds.SEED_QUERIES)
    ids, dist, _ = vh.CudaKnnEngine(base, 128).search_batch_arrays(q, 100)
    check_knn(oracle, base, q, ids, dist, 100, "l2", rtol=0.0, atol=0.0)


@pytest.mark.parametrize("dim", [32, 96, 128])
def test_integer_l2_extremes_exact(vh, oracle, dim):
    """Entries only 0 or 255: the largest norms (128 * 255^2) and cross terms the [0, 255]
    range allows, where the register kernel's accumulators (row norm minus 2 q.x) reach their
    widest partial sums.  Distances are exact integers and must match bit for bit; the heavy
    ties (multiples of 255^2) exercise the tie-aware check."""
    rng = np.random.default_rng(dim)
    base = (rng.integers(0, 2, (30_000, dim)) * 255).astype(np.float32)
    q = (rng.integers(0, 2, (40, dim)) * 255).astype(np.float32)
    q[0] = 255.0  # all-255 query against all-0 / all-255 rows
    base[:2] = 0.0
    base[2:4] = 255.0
    ids, dist, lens = vh.CudaKnnEngine(base, dim).search_batch_arrays(q, 20)
    assert np.all(lens == 20)
    check_knn(oracle, base, q, ids, dist, 20, "l2", rtol=0.0, atol=0.0)


def test_large_k_beyond_reference_clamp(vh, oracle):
    """k = 1000 > the reference kernel's MAX_K = 128 (knn.cu:203,218)."""
    from vector_hip import datasets as ds

    base = ds.gaussian(20_000, 64, 7)
    q = ds.gaussian(8, 64, 8)
    ids, dist, lens = vh.CudaKnnEngine(base, 64).search_batch_arrays(q, 1000)
    assert np.all(lens == 1000)
    check_knn(oracle, base, q, ids, dist, 1000, "l2", rtol=1e-4, atol=1e-5)


def test_ragged_dims_and_sizes(vh, oracle):
    """Dimensions that are not multiples of the 32-float tile and row counts that are
    not multiples of the 128-row stage."""
    rng = np.random.default_rng(12)
    for dim, n, nq, k in [(3, 1, 2, 1), (17, 129, 5, 7), (33, 1000, 130, 16), (100, 4097, 3, 50), (96, 300, 1, 300)]:
        base = rng.standard_normal((n, dim)).astype(np.float32)
        q = rng.standard_normal((nq, dim)).astype(np.float32)
        for metric in ("l2", "cosine"):
            ids, dist, lens = vh.CudaKnnEngine(base, dim, vh.DistanceMetric(oracle.METRICS[metric])
                                               ).search_batch_arrays(q, k)
            check_knn(oracle, base, q, ids, dist, k, metric, rtol=1e-4, atol=1e-5)


def test_massive_ties_take_overflow_path(vh):
    """All rows identical: every row ties with the k-th, the candidate lists overflow
    and the re-run path must still return the k lowest ids (the reference's heap keeps
    the first-seen rows, knn.rs:351-366)."""
    base = np.ones((60_000, 8), np.float32)
    q = np.zeros((3, 8), np.float32)
    ids, dist, _ = vh.CudaKnnEngine(base, 8).search_batch_arrays(q, 10)
    for r in range(3):
        assert sorted(ids[r].tolist()) == list(range(10))
        assert np.all(dist[r] == 8.0)


@pytest.mark.parametrize("metric", ["l1", "linf", "minkowski", "jaccard", "hellinger", "mahalanobis", "hamming"])
def test_valu_metrics_parity(vh, oracle, metric):
    """Non-contraction metrics against the CPU engine on U[-1,1] data (the 500k x 128
    workload's distribution) at 20k rows."""
    from vector_hip import datasets as ds

    base = ds.uniform(20_000, 128, ds.SEED_BASE)
    q = ds.uniform(40, 128, ds.SEED_QUERIES)
    if metric == "hamming":  # thresholded float Hamming needs coincident values to be meaningful
        base = np.round(base * 2) / 2
        q = np.round(q * 2) / 2
    ids, dist, _ = vh.CudaKnnEngine(base, 128, vh.DistanceMetric(oracle.METRICS[metric])).search_batch_arrays(q, 10)
    check_knn(oracle, base, q, ids, dist, 10, metric, rtol=1e-4, atol=1e-5)


def test_device_pointer_entry_point(vh):
    from vector_hip import datasets as ds

    base = ds.gaussian(5000, 64, 3)
    q = ds.gaussian(20, 64, 4)
    eng = vh.CudaKnnEngine(base, 64)
    ids, dist, _ = eng.search_batch_arrays(q, 16)
    dq = vh.DeviceBuffer.from_host(q)
    di = vh.DeviceBuffer(20 * 16 * 4)
    dd = vh.DeviceBuffer(20 * 16 * 4)
    eng.search_batch_device(dq.ptr, 20, 16, di.ptr, dd.ptr)
    i2 = di.to_host(np.empty((20, 16), np.uint32))
    d2 = dd.to_host(np.empty((20, 16), np.float32))
    assert np.array_equal(ids, i2) and np.array_equal(dist, d2)


def test_repeat_runs_bit_identical(vh):
    from vector_hip import datasets as ds

    base = ds.gaussian(30_000, 128, 5)
    q = ds.gaussian(300, 128, 6)
    eng = vh.CudaKnnEngine(base, 128)
    a = eng.search_batch_arrays(q, 32)
    b = eng.search_batch_arrays(q, 32)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


@pytest.mark.parametrize("dim", [256, 384, 512, 640, 768, 896, 1024, 200, 300])
@pytest.mark.parametrize("metric", ["l2", "dot", "cosine"])
def test_high_dimension_parity(vh, oracle, metric, dim):
    """Dimensions above 128: multiples of 128 up to 896 run the narrow resident-tile kernel
    (every one of its K-chunk counts; 768 is the 1M x 768 cosine workload's shape), 1024 the
    panel kernel, others the streaming kernel.  300 queries span ten 32-column tiles (the last
    partial) and three 128-column tiles; k = 100 makes the dense first round cover 2048 rows,
    and the last round's 9,952 rows end inside a 512-row stage."""
    from vector_hip import datasets as ds

    base = ds.normalized(12_000, dim, 31) if metric == "cosine" else ds.gaussian(12_000, dim, 31)
    q = ds.normalized(300, dim, 32) if metric == "cosine" else ds.gaussian(300, dim, 32)
    for k in (10, 100):
        ids, dist, lens = vh.CudaKnnEngine(base, dim, vh.DistanceMetric(oracle.METRICS[metric])
                                           ).search_batch_arrays(q, k)
        assert np.all(lens == k)
        check_knn(oracle, base, q, ids, dist, k, metric, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("mname", ["l2", "cosine"])
def test_last_query_batch_takes_the_small_scan(vh, oracle, mname):
    """16,384 + 37 queries: the search runs in batches of 16,384 queries, and the last 37 take the
    small-batch scan (its spread candidate counters) under the round plan of the first batch.  The
    first 200 queries and the last 37 against the oracle."""
    from vector_hip import datasets as ds

    names = {"cosine": "CosineSimilarity", "l2": "L2Squared"}
    n, d, nq = 20_000, 64, 16_384 + 37
    base = ds.uniform_int(n, d, 61) if mname == "l2" else ds.uniform(n, d, 61)
    q = ds.uniform_int(nq, d, 62) if mname == "l2" else ds.uniform(nq, d, 62)
    print(f"  {mname} {n} x {d} nq={nq}", flush=True)
    ids, dist, lens = vh.CudaKnnEngine(base, d, vh.DistanceMetric[names[mname]]).search_batch_arrays(q, 10)
    assert np.all(lens == 10)
    sel = np.r_[0:200, nq - 37:nq]
    tol = dict(rtol=0.0, atol=0.0) if mname == "l2" else dict(rtol=1e-4, atol=1e-5)
    check_knn(oracle, base, q[sel], ids[sel], dist[sel], 10, mname, **tol)
