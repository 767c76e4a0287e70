"""GPU parity on data away from the origin, where the GEMM (norm) form of squared L2 cancels.

The reference CPU engine computes squared L2 in direct form, sum (q - x)^2
(vector-simd/src/avx512.rs:87-148, scalar.rs:35-44), and so does find_nearest_centroid
(ivf/kmeans.rs:264-309).  The GPU scans score ||q'||^2 + ||x'||^2 - 2 q'.x' on operands shifted by
the column means, keep every candidate within a proven error bound of the k-th, re-rank those in
direct form, and fall back to a direct-form scan (kNN) or a direct-form fix-up (k-means assign)
where the bound cannot separate the candidates.  Each case here is one the plain fp32 norm form
gets wrong (tests/test_offset_host.py replays it on the CPU and shows the failure).
"""
import numpy as np
import pytest

from kmeans_check import check_chain, check_step
from knn_check import check_knn

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    assert vector_hip.CudaDeviceContext.device_count() >= 1, "no gfx950 GPU visible"
    return vector_hip


def offset_gaussian(n, dim, offset, seed):
    rng = np.random.default_rng(seed)
    return (offset + rng.standard_normal((n, dim))).astype(np.float32)


def far_clusters(n_clusters, per, dim, seed, spread=1000.0, noise=0.01):
    """Tight clusters (noise 0.01) around centres spread 1000 apart: the k-th neighbour distance
    is about 1e-6 of the operands' squared norms even after centring, so every member of the
    query's cluster lies within the GEMM form's error bound."""
    rng = np.random.default_rng(seed)
    centres = rng.standard_normal((n_clusters, dim)) * spread
    lab = np.repeat(np.arange(n_clusters), per)
    return (centres[lab] + rng.standard_normal((n_clusters * per, dim)) * noise).astype(np.float32), centres


@pytest.mark.parametrize("offset", [100.0, 1000.0])
@pytest.mark.parametrize("k", [10, 100])
def test_l2_offset_data(vh, oracle, offset, k):
    base = offset_gaussian(20_000, 128, offset, 1)
    q = offset_gaussian(50, 128, offset, 2)
    ids, dist, lens = vh.CudaKnnEngine(base, 128).search_batch_arrays(q, k)
    assert np.all(lens == k)
    check_knn(oracle, base, q, ids, dist, k, "l2", rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("offset", [100.0, 1000.0])
def test_cosine_offset_data_768(vh, oracle, offset):
    base = offset_gaussian(20_000, 768, offset, 3)
    q = offset_gaussian(20, 768, offset, 4)
    ids, dist, lens = vh.CudaKnnEngine(base, 768, vh.DistanceMetric.CosineSimilarity).search_batch_arrays(q, 10)
    assert np.all(lens == 10)
    check_knn(oracle, base, q, ids, dist, 10, "cosine", rtol=1e-4, atol=1e-6)


def test_dot_offset_data(vh, oracle):
    base = offset_gaussian(20_000, 128, 1000.0, 5)
    q = offset_gaussian(30, 128, 1000.0, 6)
    ids, dist, _ = vh.CudaKnnEngine(base, 128, vh.DistanceMetric.DotProduct).search_batch_arrays(q, 10)
    check_knn(oracle, base, q, ids, dist, 10, "dot", rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("k", [1, 10, 100])
def test_l2_far_tight_clusters_take_direct_form(vh, oracle, k):
    """Clusters of 400 rows: more members lie within the error bound than the kept margin holds,
    so the search re-runs these queries in direct form; results must be the exact top-k."""
    base, centres = far_clusters(50, 400, 64, 7)
    rng = np.random.default_rng(8)
    q = (centres[rng.integers(0, 50, 40)] + rng.standard_normal((40, 64)) * 0.01).astype(np.float32)
    ids, dist, lens = vh.CudaKnnEngine(base, 64).search_batch_arrays(q, k)
    assert np.all(lens == k)
    check_knn(oracle, base, q, ids, dist, k, "l2", rtol=1e-4, atol=1e-9, min_recall=1.0)


def test_l2_max_k_float_and_integer(vh, oracle):
    """k = VHIP_MAX_K (2048): the kept lists grow to k + 256 entries on float data."""
    assert vh.VHIP_MAX_K == 2048
    base = offset_gaussian(30_000, 64, 50.0, 9)
    q = offset_gaussian(6, 64, 50.0, 10)
    ids, dist, lens = vh.CudaKnnEngine(base, 64).search_batch_arrays(q, 2048)
    assert np.all(lens == 2048)
    check_knn(oracle, base, q, ids, dist, 2048, "l2", rtol=1e-4, atol=1e-5)
    from vector_hip import datasets as ds

    bi = ds.uniform_int(30_000, 64, 11)
    qi = ds.uniform_int(5, 64, 12)
    ids, dist, _ = vh.CudaKnnEngine(bi, 64).search_batch_arrays(qi, 2048)
    check_knn(oracle, bi, qi, ids, dist, 2048, "l2", rtol=0.0, atol=0.0)
    ids, dist, _ = vh.CudaKnnEngine(base, 64, vh.DistanceMetric.CosineSimilarity).search_batch_arrays(q, 2048)
    check_knn(oracle, base, q, ids, dist, 2048, "cosine", rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("offset", [100.0, 1000.0])
def test_kmeans_step_offset_data(vh, oracle, offset, assign_path):
    from vector_hip import datasets as ds

    data, _, _ = ds.gaussian_mixture(20_000, 96, 64, 13)
    data = (data + offset).astype(np.float32)
    st = vh.KMeansState(data)
    cent = data[:64].copy()
    for _ in range(2):
        st.set_centroids(cent)
        st.run(1)
        got = st.read()
        check_step(oracle, data, cent, got, "l2")
        cent = got["centroids"]


def test_kmeans_wide_range_clusters(vh, oracle, assign_path):
    """Clusters at |x| ~ 1e4 (spread 1) and at |x| ~ 1e-2 (spread 1e-3) in one dataset: the small
    ones sit 5e3 from the column means, so the assignment goes through the direct-form fix-up, and
    the update must keep 1e-4 of their norm (per-cluster fixed-point scales)."""
    rng = np.random.default_rng(14)
    dim, per = 32, 1250
    big = rng.standard_normal((8, dim))
    big = big / np.linalg.norm(big, axis=1, keepdims=True) * 1e4
    small = rng.standard_normal((8, dim))
    small = small / np.linalg.norm(small, axis=1, keepdims=True) * 1e-2
    parts = [c + rng.standard_normal((per, dim)) for c in big] + \
            [c + rng.standard_normal((per, dim)) * 1e-3 for c in small]
    data = np.concatenate(parts).astype(np.float32)
    data = data[rng.permutation(len(data))]
    st = vh.KMeansState(data)
    # one initial centroid per cluster, taken from the data
    cent = np.concatenate([data[np.argmin(np.linalg.norm(data - c, axis=1))][None] for c in
                           list(big) + list(small)]).astype(np.float32)
    for _ in range(2):
        st.set_centroids(cent)
        st.run(1)
        got = st.read()
        check_step(oracle, data, cent, got, "l2")
        cent = got["centroids"]
    small_c = got["centroids"][8:]
    assert np.all(np.linalg.norm(small_c, axis=1) < 0.02)


@pytest.mark.parametrize("metric", ["l2", "dot"])
def test_kmeans_fit_offset_vs_oracle(vh, oracle, metric, assign_path):
    from vector_hip import datasets as ds

    data, _, _ = ds.gaussian_mixture(12_000, 48, 32, 15)
    data = (data + 500.0).astype(np.float32)
    init = data[:32].copy()
    m = vh.DistanceMetric(oracle.METRICS[metric])
    r, assign = vh.CudaKMeansEngine().fit(data, 48, 32, 4, -1.0, m, init=init, return_assign=True)
    # each of the 4 iterations against the oracle's step from the GPU's previous centroids (near-tie
    # flips only, centroids within 1e-4 of the mean of the points assigned), and fit() equal to
    # those 4 steps bit for bit
    check_chain(vh, oracle, data, init, 4, metric, r.centroids, assign, r.inertia)


def test_kmeans_cosine_offset_assign_near_optimal(vh, oracle, assign_path):
    """Cosine at offset 500: every similarity lies within ~1e-6 of 1, so which of several
    centroids wins is decided by fp32 rounding, in the reference as here.  Every GPU assignment must
    be optimal up to that rounding: its direct-form similarity (the oracle's) within 1e-5 of the
    best one."""
    from vector_hip import datasets as ds

    data, _, _ = ds.gaussian_mixture(12_000, 48, 32, 15)
    data = (data + 500.0).astype(np.float32)
    cent = data[:32].copy()
    st = vh.KMeansState(data, vh.DistanceMetric.CosineSimilarity)
    st.set_centroids(cent)
    st.run(1)
    got = st.read()
    sims = np.stack([oracle.distance_rows("cosine", data, np.repeat(cent[c:c + 1], len(data), 0))
                     for c in range(32)], 1)
    mine = sims[np.arange(len(data)), got["assign"]]
    assert np.all(mine >= sims.max(1) - 1e-5)
    counts = np.bincount(got["assign"], minlength=32)
    assert np.array_equal(counts, got["counts"])


@pytest.mark.parametrize("offset", [1000.0])
def test_coarse_assign_offset(vh, oracle, offset):
    from vector_hip import datasets as ds

    data, _, _ = ds.gaussian_mixture(20_000, 48, 128, 16)
    data = np.ascontiguousarray(data + offset, np.float32)
    cent = data[:128].copy()
    cl, sc, res = vh.IvfCoarseQuantizer(cent, 48).assign(data, residuals=True)
    ref = oracle.kmeans_step(data, cent, "l2", threads=0)["assign"]
    flips = np.nonzero(cl.astype(np.int64) != ref)[0]
    assert len(flips) <= 2
    for p in flips:
        dg = oracle.distance("l2", data[p], cent[cl[p]])
        dr = oracle.distance("l2", data[p], cent[ref[p]])
        assert abs(dg - dr) <= 1e-4 * max(1.0, abs(dr))
    refv = oracle.distance_rows("l2", data, cent[cl])
    assert np.all(np.abs(sc - refv) <= 1e-4 * np.abs(refv) + 1e-5)
    assert np.array_equal(res, data - cent[cl])


def _free_bytes():
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_integer_base_keeps_one_copy(vh):
    """Integer rows with an integer column shift give back the unshifted rows exactly as shifted
    row + shift, so the engine keeps no second, unshifted copy of the base; float rows keep one
    (their shifted values lose bits)."""
    import gc

    from vector_hip import datasets as ds

    gc.collect()
    n, d = 400_000, 128
    copy = n * d * 4  # 205 MB
    rng = np.random.default_rng(71)
    used = {}
    for name, base in (("int", ds.uniform_int(n, d, 72)), ("float", (0.5 + rng.random((n, d))).astype(np.float32))):
        f0 = _free_bytes()
        eng = vh.CudaKnnEngine(base, d)
        vh.synchronize()
        used[name] = f0 - _free_bytes()
        ids, _, _ = eng.search_batch_arrays(base[:3], 1)
        assert ids[:, 0].tolist() == [0, 1, 2]
        del eng
        gc.collect()
    print(f"  device bytes held: integer base {used['int']}, float base {used['float']} (one copy {copy})",
          flush=True)
    assert used["int"] < 1.3 * copy, used
    assert used["float"] > 1.8 * copy, used


def test_integer_far_clusters_direct_form_exact(vh, oracle):
    """Integer points in tight clusters far from the origin: the GEMM form's error bound admits
    whole clusters, so most queries take the direct-form re-run, over rows rebuilt as shifted row +
    shift (the engine keeps no unshifted copy of integer data).  Distances are exact integers."""
    rng = np.random.default_rng(73)
    centres = rng.integers(-20_000, 20_000, (40, 64))
    lab = np.repeat(np.arange(40), 300)
    base = (centres[lab] + rng.integers(-2, 3, (12_000, 64))).astype(np.float32)
    q = (centres[rng.integers(0, 40, 30)] + rng.integers(-2, 3, (30, 64))).astype(np.float32)
    for k in (10, 100):
        ids, dist, lens = vh.CudaKnnEngine(base, 64).search_batch_arrays(q, k)
        assert np.all(lens == k)
        check_knn(oracle, base, q, ids, dist, k, "l2", rtol=0.0, atol=0.0, min_recall=1.0)
