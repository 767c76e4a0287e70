"""GPU parity of the reference benchmark's batch sweep (cuda_bench.rs:41-55, 98-152).

DistributedKnnEngine::search_batch at one GPU over batch sizes 1 to 128 with k = 10: on the
benchmark's default 10,000 x 768 U[-1, 1] base under cosine (and dot product, and squared L2),
and on a 200,000 x 128 integer base under squared L2 (exact distances).  Every batch is checked
against the oracle's search_batch_cpu.
"""
import numpy as np
import pytest

from knn_check import check_knn

pytestmark = pytest.mark.gpu

BATCHES = (1, 2, 3, 4, 8, 16, 31, 32, 64, 127, 128)


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    assert vector_hip.CudaDeviceContext.device_count() >= 1, "no gfx950 GPU visible"
    return vector_hip


def _sweep(vh, oracle, base, queries, metric, mname, **tol):
    eng = vh.DistributedKnnEngine.try_new(base, base.shape[1], 1, vh.GpuShardMode.Sharded, metric)
    for b in BATCHES:
        q = np.ascontiguousarray(queries[:b])
        print(f"  {mname} {base.shape[0]} x {base.shape[1]} batch {b}", flush=True)
        ids, dist, lens = eng.search_batch_arrays(q, 10)
        assert np.all(lens == 10)
        check_knn(oracle, base, q, ids, dist, 10, mname, **tol)


@pytest.mark.parametrize("mname", ["cosine", "dot", "l2"])
def test_cuda_bench_default_shape(vh, oracle, mname):
    from vector_hip import datasets as ds

    names = {"cosine": "CosineSimilarity", "dot": "DotProduct", "l2": "L2Squared"}
    base = ds.uniform(10_000, 768, 51)
    q = ds.uniform(128, 768, 52)
    _sweep(vh, oracle, base, q, vh.DistanceMetric[names[mname]], mname, rtol=1e-4, atol=1e-5)


def test_integer_l2_batches(vh, oracle):
    from vector_hip import datasets as ds

    base = ds.uniform_int(200_000, 128, 53)
    q = ds.uniform_int(128, 128, 54)
    _sweep(vh, oracle, base, q, vh.DistanceMetric.L2Squared, "l2", rtol=0.0, atol=0.0)


@pytest.mark.parametrize("dim", [960, 992, 1000, 1024])
@pytest.mark.parametrize("mname", ["cosine", "l2", "dot"])
def test_small_batches_with_the_widest_rows(vh, oracle, dim, mname):
    """The small-batch scan keeps its 32-query tile of dim floats in LDS and, on rounds of few row
    blocks, splits K over the waves with partial sums beside the tile.  From 992 floats a row the
    two no longer fit one workgroup's LDS beside the candidate slots, so such rounds run unsplit
    (a 1,000-float cosine search of 18 queries at k = 160 once asked for 168,064 bytes)."""
    names = {"cosine": "CosineSimilarity", "dot": "DotProduct", "l2": "L2Squared"}
    rng = np.random.default_rng(dim)
    base = (rng.standard_normal((28_089, dim)) * 0.5 + 3.0).astype(np.float32)
    queries = (rng.standard_normal((100, dim)) * 0.5 + 3.0).astype(np.float32)
    eng = vh.DistributedKnnEngine.try_new(base, dim, 1, vh.GpuShardMode.Sharded, vh.DistanceMetric[names[mname]])
    for nq, k in ((18, 160), (32, 10), (100, 10)):
        print(f"  {mname} {base.shape[0]} x {dim} batch {nq} k {k}", flush=True)
        q = np.ascontiguousarray(queries[:nq])
        ids, dist, lens = eng.search_batch_arrays(q, k)
        assert np.all(lens == k)
        check_knn(oracle, base, q, ids, dist, k, mname, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("mname,k", [("l2", 10), ("l2", 100), ("cosine", 10), ("dot", 10)])
def test_mid_batches_on_a_large_base_of_short_rows(vh, oracle, mname, k):
    """Batches of 33 to 128 queries over a base of more than 262,144 rows of at most 128 floats also
    take the small-batch scan (four 32-query tiles), whose candidate counters sit one cache line
    apart; each batch against the oracle."""
    from vector_hip import datasets as ds

    names = {"cosine": "CosineSimilarity", "dot": "DotProduct", "l2": "L2Squared"}
    n, d = 300_000, 64
    base = ds.uniform_int(n, d, 55) if mname == "l2" else ds.uniform(n, d, 55)
    q = ds.uniform_int(128, d, 56) if mname == "l2" else ds.uniform(128, d, 56)
    eng = vh.CudaKnnEngine(base, d, vh.DistanceMetric[names[mname]])
    tol = dict(rtol=0.0, atol=0.0) if mname == "l2" else dict(rtol=1e-4, atol=1e-5)
    for b in (33, 64, 100, 128):
        print(f"  {mname} {n} x {d} batch {b} k={k}", flush=True)
        ids, dist, lens = eng.search_batch_arrays(np.ascontiguousarray(q[:b]), k)
        assert np.all(lens == k)
        check_knn(oracle, base, q[:b], ids, dist, k, mname, **tol)
