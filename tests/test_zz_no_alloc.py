"""GPU tests of the allocation-free kNN search (vhip_knn_search_batch_device_noalloc).

The entry point has no counterpart in the reference: it serves callers that cannot allocate
device memory, with its working memory in one fixed per-GPU array of the library.  Its results
must equal those of vhip_knn_search_batch_device on the same engine and queries, bit for bit:
the two share every kernel and differ only in where the buffers live and in how many queries
one batch holds.  Each case runs two calls in a row, the second on fewer queries, since the
array keeps the previous call's contents.  Results are also checked against the oracle.
"""
import ctypes
import gc

import numpy as np
import pytest

from knn_check import check_knn

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    assert vector_hip.CudaDeviceContext.device_count() >= 1, "no gfx950 GPU visible"
    return vector_hip


def _free_bytes():
    """Free device memory of the current GPU (hipMemGetInfo of the HIP runtime the library uses)."""
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_first_call_loads_the_array(vh):
    """The array lives in a code object of its own with no kernels, loaded onto the GPU by the
    first allocation-free call: creating engines and searching with the allocating entry point
    reserve nothing for it.  (This is the first test of the file, and no other test file calls
    the allocation-free entry point, so in one process this call is the first.)"""
    from vector_hip import datasets as ds

    gc.collect()
    base = ds.uniform_int(20_000, 128, 31)
    eng = vh.CudaKnnEngine(base, 128)
    q = ds.uniform_int(100, 128, 32)
    dq = vh.DeviceBuffer.from_host(q)
    di = vh.DeviceBuffer(100 * 10 * 4)
    dd = vh.DeviceBuffer(100 * 10 * 4)
    eng.search_batch_device(dq.ptr, 100, 10, di.ptr, dd.ptr)
    vh.synchronize()
    f0 = _free_bytes()
    eng.search_batch_device_noalloc(dq.ptr, 100, 10, di.ptr, dd.ptr)
    vh.synchronize()
    f1 = _free_bytes()
    print(f"  free memory before {f0}, after the first allocation-free call {f1}", flush=True)
    assert f0 - f1 >= vh.NOALLOC_SCRATCH_BYTES - (4 << 20), (
        f"the first allocation-free call should load the {vh.NOALLOC_SCRATCH_BYTES}-byte array; free memory "
        f"fell by {f0 - f1} bytes")


def _both(vh, eng, q, k):
    """(ids, dist) of the allocating and the allocation-free entry point for the same queries."""
    nq = q.shape[0]
    dq = vh.DeviceBuffer.from_host(q)
    out = []
    for fn in (eng.search_batch_device, eng.search_batch_device_noalloc):
        di = vh.DeviceBuffer(nq * k * 4)
        dd = vh.DeviceBuffer(nq * k * 4)
        print(f"  {fn.__name__}: nq={nq} k={k}", flush=True)
        fn(dq.ptr, nq, k, di.ptr, dd.ptr)
        out.append((di.to_host(np.empty((nq, k), np.uint32)), dd.to_host(np.empty((nq, k), np.float32))))
    return out


def _check_pair(vh, oracle, eng, base, q, k, metric, **tol):
    (ia, da), (ib, db) = _both(vh, eng, q, k)
    assert np.array_equal(ia, ib), "ids differ between the allocating and the allocation-free search"
    assert np.array_equal(da.view(np.uint32), db.view(np.uint32)), "distances differ"
    check_knn(oracle, base, q, ib, db, k, metric, **tol)


def test_integer_l2_several_batches(vh, oracle):
    """k = 100 over integer rows: about 2,000 queries fit the array per batch, so 5,000 queries
    take three batches; then a second call on 300 queries."""
    from vector_hip import datasets as ds

    base = ds.uniform_int(60_000, 128, 21)
    eng = vh.CudaKnnEngine(base, 128)
    q = ds.uniform_int(5000, 128, 22)
    _check_pair(vh, oracle, eng, base, q[:5000], 100, "l2", rtol=0.0, atol=0.0)
    _check_pair(vh, oracle, eng, base, q[:300], 100, "l2", rtol=0.0, atol=0.0)


@pytest.mark.parametrize("metric", ["l2", "cosine", "dot", "l1"])
def test_float_metrics_two_calls(vh, oracle, metric):
    from vector_hip import datasets as ds

    names = {"l2": "L2Squared", "cosine": "CosineSimilarity", "dot": "DotProduct", "l1": "Manhattan"}
    base = ds.gaussian(30_000, 96, 23)
    eng = vh.CudaKnnEngine(base, 96, vh.DistanceMetric[names[metric]])
    q = ds.gaussian(700, 96, 24)
    _check_pair(vh, oracle, eng, base, q, 10, metric, rtol=1e-4, atol=1e-5)
    _check_pair(vh, oracle, eng, base, q[:37], 10, metric, rtol=1e-4, atol=1e-5)


def test_reruns_split_rounds(vh, oracle):
    """Tight clusters far from the origin: most queries need the direct-form re-run, which in the
    allocation-free search splits its rounds to fit the batch's candidate lists."""
    rng = np.random.default_rng(25)
    centres = rng.standard_normal((50, 64)) * 1000.0
    base = (centres[np.repeat(np.arange(50), 400)] + rng.standard_normal((20_000, 64)) * 0.01).astype(np.float32)
    q = (centres[rng.integers(0, 50, 40)] + rng.standard_normal((40, 64)) * 0.01).astype(np.float32)
    eng = vh.CudaKnnEngine(base, 64)
    _check_pair(vh, oracle, eng, base, q, 100, "l2", rtol=1e-4, atol=1e-9, min_recall=1.0)
    _check_pair(vh, oracle, eng, base, q[:9], 100, "l2", rtol=1e-4, atol=1e-9, min_recall=1.0)


def test_cut_rounds_score_alike(vh, oracle):
    """Cosine over rows far from the origin, where the similarities of most rows agree to within a
    few ulps: the queries overflow their candidate lists on the small-batch plan and are re-run,
    and the allocation-free search cuts the re-run's rounds to fit the batch's candidate buffer.
    The small-batch scan splits each score's K range by the length of the whole round, not of the
    piece, so the scores, and with them the results, come out the same bit for bit (splitting by
    the piece's length changed the results of 25 of these 100 queries)."""
    rng = np.random.default_rng(1)
    base = (rng.standard_normal((60_000, 128)) * 0.5 + 1000.0).astype(np.float32)
    q = (rng.standard_normal((100, 128)) * 0.5 + 1000.0).astype(np.float32)
    eng = vh.CudaKnnEngine(base, 128, vh.DistanceMetric.CosineSimilarity)
    _check_pair(vh, oracle, eng, base, q, 10, "cosine", rtol=1e-4, atol=1e-5)
    _check_pair(vh, oracle, eng, base, q[:31], 10, "cosine", rtol=1e-4, atol=1e-5)


def test_mid_batch_on_a_large_base(vh, oracle):
    """100 queries over 300,000 rows of 64 floats take the small-batch scan, whose per-query
    candidate counters (one cache line apart) are carved from the array like the rest; then 33."""
    from vector_hip import datasets as ds

    base = ds.uniform_int(300_000, 64, 33)
    eng = vh.CudaKnnEngine(base, 64)
    q = ds.uniform_int(100, 64, 34)
    _check_pair(vh, oracle, eng, base, q, 10, "l2", rtol=0.0, atol=0.0)
    _check_pair(vh, oracle, eng, base, q[:33], 10, "l2", rtol=0.0, atol=0.0)

def test_max_k(vh, oracle):
    """k = VHIP_MAX_K: each query's candidate list is half a megabyte, so batches are small."""
    from vector_hip import datasets as ds

    base = ds.gaussian(50_000, 32, 26)
    eng = vh.CudaKnnEngine(base, 32)
    q = ds.gaussian(300, 32, 27)
    _check_pair(vh, oracle, eng, base, q, 2048, "l2", rtol=1e-4, atol=1e-5)
    _check_pair(vh, oracle, eng, base, q[:3], 2048, "l2", rtol=1e-4, atol=1e-5)


def test_allocates_nothing(vh):
    """A fresh engine's allocation-free searches leave free device memory unchanged (the
    allocating entry point grows a workspace of tens of megabytes for the same batch)."""
    from vector_hip import datasets as ds

    gc.collect()  # engines of earlier tests left in reference cycles free their memory now
    base = ds.uniform_int(60_000, 128, 28)
    eng = vh.CudaKnnEngine(base, 128)
    q = ds.uniform_int(4000, 128, 29)
    dq = vh.DeviceBuffer.from_host(q)
    di = vh.DeviceBuffer(4000 * 100 * 4)
    dd = vh.DeviceBuffer(4000 * 100 * 4)
    eng.search_batch_device_noalloc(dq.ptr, 4000, 100, di.ptr, dd.ptr)  # first use on this GPU
    vh.synchronize()
    f0 = _free_bytes()
    for n in (4000, 1000):
        eng.search_batch_device_noalloc(dq.ptr, n, 100, di.ptr, dd.ptr)
    vh.synchronize()
    f1 = _free_bytes()
    assert f0 - f1 < (4 << 20), f"free memory fell by {f0 - f1} bytes"
    eng.search_batch_device(dq.ptr, 4000, 100, di.ptr, dd.ptr)
    vh.synchronize()
    assert f1 - _free_bytes() > (16 << 20), "the allocating search should have grown its workspace"


def test_too_large_for_the_array_is_an_error(vh):
    """Rows of 40,000 dimensions: one 128-query tile of prepared rows alone exceeds the array."""
    rng = np.random.default_rng(30)
    base = rng.standard_normal((8, 40_000)).astype(np.float32)
    eng = vh.CudaKnnEngine(base, 40_000)
    q = base[:2].copy()
    dq = vh.DeviceBuffer.from_host(q)
    di = vh.DeviceBuffer(2 * 4 * 4)
    dd = vh.DeviceBuffer(2 * 4 * 4)
    with pytest.raises(vh.CudaError, match="allocation-free"):
        eng.search_batch_device_noalloc(dq.ptr, 2, 4, di.ptr, dd.ptr)
    # the allocating entry point still serves it, and a fitting call still works afterwards
    eng.search_batch_device(dq.ptr, 2, 4, di.ptr, dd.ptr)
    ids = di.to_host(np.empty((2, 4), np.uint32))
    assert ids[0, 0] == 0 and ids[1, 0] == 1
    small = vh.CudaKnnEngine(base[:, :64].copy(), 64)
    dq2 = vh.DeviceBuffer.from_host(base[:2, :64].copy())
    small.search_batch_device_noalloc(dq2.ptr, 2, 4, di.ptr, dd.ptr)
    assert di.to_host(np.empty((2, 4), np.uint32))[:, 0].tolist() == [0, 1]
