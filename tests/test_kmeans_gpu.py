"""GPU parity of k-means (Lloyd) through the C ABI.

Reference tests restated (kmeans.rs:473-577, distributed_kmeans.rs:548-641,
ivf/kmeans.rs:378-417, integration_tests.rs:7-56), plus per-iteration parity with the
oracle on Gaussian-mixture data shaped like the 2M x 96 / 4096-centroid workload:
assignments may differ on <= 0.01% of points and only at near-ties; centroids must be within
1e-4 (per-centroid norm-relative) of the mean of their assigned points, and of the oracle's
update wherever the membership agrees.  Each iteration is checked from the same centroids.
"""
import numpy as np
import pytest

from kmeans_check import check_chain
from kmeans_check import check_step as _check_step

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    assert vector_hip.CudaDeviceContext.device_count() >= 1
    return vector_hip


def _three_clusters(n_per=50):
    return np.concatenate([np.tile([0.1, -0.1, 0.05, -0.05], (n_per, 1)),
                           np.tile([10.1, 9.9, 10.05, 9.95], (n_per, 1)),
                           np.tile([20.1, 19.9, 20.05, 19.95], (n_per, 1))]).astype(np.float32)


# ---- reference known-answer tests -----------------------------------------------------
def test_kmeans_rs_kats(vh):
    eng = vh.CudaKMeansEngine()
    r = eng.fit(_three_clusters(), 4, 3, 20, 1e-4, vh.DistanceMetric.L2Squared)       # kmeans.rs:474-504
    assert r.k == 3 and r.dimension == 4 and r.iterations > 0 and r.inertia < 1.0
    assert all(len(r.centroid(c)) == 4 for c in range(3))
    r = eng.fit(np.array([1, 1, 1.1, .9, .9, 1.1], np.float32), 2, 1, 10, 1e-4)        # :507-517
    assert r.k == 1 and abs(r.centroid(0)[0] - 1) < 0.1 and abs(r.centroid(0)[1] - 1) < 0.1
    assert eng.fit(np.zeros(0, np.float32), 4, 3, 10, 1e-4).k == 0                     # :520-527
    assert eng.fit(np.array([1, 2], np.float32), 2, 0, 10, 1e-4).k == 0
    assert eng.fit(np.array([1, 2, 3, 4], np.float32), 2, 5, 10, 1e-4).k == 2          # :530-537
    data = np.array([1, 0, 0, 0, 1, 0, 0, 0, 1, .9, .1, 0], np.float32)                # :540-557
    assert eng.fit(data, 3, 3, 10, 1e-4, vh.DistanceMetric.CosineSimilarity).k == 3
    assert eng.fit(data, 3, 3, 10, 1e-4, vh.DistanceMetric.DotProduct).k == 3
    hd = (np.arange(20 * 128) * 0.01).astype(np.float32)                               # :560-570
    r = eng.fit(hd, 128, 4, 5, 1e-3)
    assert r.k == 4 and r.dimension == 128
    assert eng.context().device_id() == 0 and eng.context().total_memory_bytes() > 0  # :573-577


def test_ivf_kmeans_single_cluster_mean(vh):
    """ivf/kmeans.rs:386-395: the single centroid is the exact mean."""
    data = np.array([1, 2, 3, 4, 1.1, 2.1, 3.1, 4.1], np.float32)
    r = vh.CudaKMeansEngine().fit(data, 4, 1, 10, 1e-4)
    assert abs(r.centroid(0)[0] - 1.05) < 1e-3 and abs(r.centroid(0)[1] - 2.05) < 1e-3


def test_distributed_kmeans_kats(vh):
    e = vh.DistributedKMeansEngine.emulator(4)                                          # :548-569
    r = e.fit(np.array([0, 0, .1, .1, -.1, -.1, 10, 10, 10.1, 10.1, 9.9, 9.9], np.float32), 2, 2, 25, 1e-5)
    assert r.k == 2 and r.dimension == 2 and r.iterations > 0 and r.inertia >= 0
    c0, c1 = r.centroid(0), r.centroid(1)
    near0, near10 = (c0, c1) if c0[0] < 5 else (c1, c0)
    assert np.all(np.abs(near0) < 0.5) and np.all(np.abs(near10 - 10) < 0.5)
    res = e.fit(np.zeros(0, np.float32), 2, 2, 10, 1e-4)                                # :572-584
    assert res.k == 0 and res.centroids.size == 0 and res.iterations == 0
    assert e.fit(np.array([1, 2, 3, 4], np.float32), 2, 0, 10, 1e-4).k == 0
    r = vh.DistributedKMeansEngine.emulator(8).fit(np.array([1, 1, 2, 2, 3, 3], np.float32), 2, 2, 15, 1e-4)
    assert r.k == 2 and r.centroids.size == 4                                            # :587-594
    r = vh.DistributedKMeansEngine.emulator(2).fit(np.array([1, 1, 3, 3, 5, 5, 7, 7], np.float32), 2, 1, 10, 1e-5)
    assert np.all(np.abs(r.centroid(0) - 4.0) < 1e-3)                                    # :597-606
    r = vh.DistributedKMeansEngine.emulator(2).fit(np.array([1, 0, .98, .2, 0, 1, .2, .98], np.float32), 2, 2, 20,
                                                   1e-4, vh.DistanceMetric.CosineSimilarity)
    assert r.k == 2 and r.dimension == 2                                                 # :609-616
    assert vh.DistributedKMeansEngine.emulator(6).num_gpus() == 6                         # :619-622
    assert vh.DistributedKMeansEngine.try_new(1).num_gpus() == 1


def test_integration_clustering_then_sharded_search(vh):
    """integration_tests.rs:7-56."""
    data = np.concatenate([np.tile([0.1, 0.0, -0.1, 0.05], (30, 1)), np.tile([9.9, 10.1, 10.0, 9.95], (30, 1)),
                           np.tile([20.0, 19.9, 20.1, 20.05], (30, 1))]).astype(np.float32)
    r = vh.DistributedKMeansEngine.emulator(4).fit(data, 4, 3, 30, 1e-5)
    assert r.k == 3 and r.dimension == 4
    knn = vh.DistributedKnnEngine.emulator(data, 4, 3, vh.GpuShardMode.Sharded)
    assert knn.num_vectors() == 90
    res = knn.search(np.full(4, 10.0, np.float32), 5)
    assert len(res) == 5 and all(30 <= x.id < 60 and x.distance < 1.0 for x in res)


# ---- per-iteration parity against the oracle -------------------------------------------
def test_mixture_10_iterations_parity(vh, oracle):
    from vector_hip import datasets as ds

    data, _, _ = ds.gaussian_mixture(60_000, 96, 256, ds.SEED_MIXTURE)
    st = vh.KMeansState(data)
    cent = data[:256].copy()
    st.set_centroids(cent)
    total_flips = 0
    for it in range(10):
        st.run(1)
        got = st.read()
        total_flips += _check_step(oracle, data, cent, got, "l2")
        cent = got["centroids"]
        st.set_centroids(cent)
    assert total_flips <= 10 * 6


@pytest.mark.parametrize("metric", ["dot", "cosine", "l1", "linf", "minkowski", "hellinger", "jaccard", "mahalanobis"])
def test_other_metrics_one_step(vh, oracle, metric, assign_path):
    from vector_hip import datasets as ds

    data, _, _ = ds.gaussian_mixture(8_000, 40, 32, 11)
    if metric in ("cosine", "dot"):
        data = data + 3.0  # keep clusters in one orthant so similarity argmax is well posed
    st = vh.KMeansState(data, vh.DistanceMetric(oracle.METRICS[metric]))
    cent = data[:32].copy()
    st.set_centroids(cent)
    st.run(1)
    got = st.read()
    # at most 2 flips, each a near-tie; centroids the means of the points assigned; inertia the
    # oracle's (the distance metrics) or the float64 sum of -dot / 1 - cos (kmeans.cu's convention)
    _check_step(oracle, data, cent, got, metric, max_flip_frac=2.5e-4)


def test_fit_deterministic_and_explicit_init(vh, oracle, assign_path):
    from vector_hip import datasets as ds

    data, _, _ = ds.gaussian_mixture(30_000, 96, 128, 5)
    init = data[:128]
    a, aa = vh.CudaKMeansEngine().fit(data, 96, 128, 6, -1.0, init=init, return_assign=True)
    b, ba = vh.CudaKMeansEngine().fit(data, 96, 128, 6, -1.0, init=init, return_assign=True)
    assert a.iterations == 6 and np.array_equal(a.centroids, b.centroids) and np.array_equal(aa, ba)
    assert a.inertia == b.inertia
    # the 6 iterations, each against the oracle's step from the GPU's previous centroids
    check_chain(vh, oracle, data, init, 6, "l2", a.centroids, aa, a.inertia)
    # seeded default inits are reproducible too
    c = vh.CudaKMeansEngine().fit(data, 96, 16, 3, -1.0, seed=9)
    d = vh.CudaKMeansEngine().fit(data, 96, 16, 3, -1.0, seed=9)
    assert np.array_equal(c.centroids, d.centroids)
    e = vh.DistributedKMeansEngine.emulator(1).fit(data, 96, 16, 3, -1.0, seed=9)
    f = vh.DistributedKMeansEngine.emulator(1).fit(data, 96, 16, 3, -1.0, seed=9)
    assert np.array_equal(e.centroids, f.centroids)


@pytest.mark.parametrize("init_mode", [0, 1])
def test_seeded_inits_draw_distinct_data_rows(vh, init_mode):
    """Both seeded inits pick data points as centroids, as the reference's do: k-means++
    (kmeans.rs:409-460) samples rows by D^2 weight, init_random (distributed_kmeans.rs:524-535)
    takes the first k of a shuffle.  With no iteration the state holds the drawn rows: each must
    be an exact row of the data (a wrong gather index or row stride fails this), all distinct,
    reproducible by seed and different across seeds.  The dimension (40, padded to 64 on the
    device) exercises the padded gather."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal((5_000, 40)).astype(np.float32)
    st = vh.KMeansState(x)
    rows = {r.tobytes(): i for i, r in enumerate(x)}
    c, _, (d, k, iters, _) = st.fit(100, 0, -1.0, init_mode=init_mode, seed=5)
    assert (d, k, iters) == (40, 100, 0)
    picked = [rows.get(v.tobytes()) for v in c]
    assert None not in picked and len(set(picked)) == 100
    c2, _, _ = st.fit(100, 0, -1.0, init_mode=init_mode, seed=5)
    c3, _, _ = st.fit(100, 0, -1.0, init_mode=init_mode, seed=6)
    assert np.array_equal(c, c2) and not np.array_equal(c, c3)
    # k = n draws every row exactly once
    small = vh.KMeansState(x[:64])
    cs, _, _ = small.fit(64, 0, -1.0, init_mode=init_mode, seed=1)
    assert sorted(rows[v.tobytes()] for v in cs) == list(range(64))


def test_empty_cluster_keeps_centroid(vh):
    rng = np.random.default_rng(0)
    data = rng.standard_normal((5000, 16)).astype(np.float32)
    cent = data[:8].copy()
    cent[7] = 1000.0
    st = vh.KMeansState(data)
    st.set_centroids(cent)
    st.run(1)
    got = st.read()
    assert got["counts"][7] == 0 and np.array_equal(got["centroids"][7], cent[7]) and got["shifts"][7] == 0


def test_tolerance_stops_early(vh):
    r = vh.CudaKMeansEngine().fit(_three_clusters(), 4, 3, 50, 1e-4, init=_three_clusters()[[0, 50, 100]])
    assert r.iterations == 1  # centroids already at the cluster means


@pytest.mark.parametrize("dim", [256, 200])
def test_high_dimension_one_step(vh, oracle, dim, assign_path):
    """k-means assign above 128 dimensions: the panel kernel (256) and the streaming kernel (200)."""
    from vector_hip import datasets as ds

    data, _, _ = ds.gaussian_mixture(12_000, dim, 64, 13)
    st = vh.KMeansState(data)
    cent = data[:64].copy()
    st.set_centroids(cent)
    st.run(1)
    _check_step(oracle, data, cent, st.read(), "l2")


def _splitmix64_draws(seed, count):
    m = (1 << 64) - 1
    st, out = seed, []
    for _ in range(count):
        st = (st + 0x9E3779B97F4A7C15) & m
        z = st
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
        out.append(z ^ (z >> 31))
    return out


def _kmeanspp_restated(x, k, seed):
    """kmeans.rs:409-460 with the build's seeded draws: the first centre is draw 0 mod n; each next
    one is the first point of positive weight whose running sum of D(x)^2 reaches u * total (u the
    draw's top 53 bits in [0, 1)), or draw mod n when the total is at most 1e-6.  In float64, which
    is exact here: the data are small integers."""
    draws = _splitmix64_draws(seed, k)
    xd = x.astype(np.float64)
    n = len(x)
    picks = [draws[0] % n]
    mind = np.full(n, np.finfo(np.float32).max, np.float64)
    for j in range(1, k):
        mind = np.minimum(mind, ((xd - xd[picks[-1]]) ** 2).sum(1))
        total = mind.sum()
        if total <= 1e-6:
            picks.append(draws[j] % n)
            continue
        thr = (draws[j] >> 11) * (1.0 / 9007199254740992.0) * total
        cum = np.cumsum(mind)
        picks.append(int(np.argmax((cum >= thr) & (mind > 0))))
    return picks


@pytest.mark.parametrize(
    "n,dim,k,seed,spread",
    [(3000, 40, 200, 5, 0), (1_100_000, 8, 12, 9, 0), (700, 128, 700, 3, 0), (20_000, 768, 64, 2, 0),
     (300_000, 64, 40, 7, 100), (40_000, 800, 24, 4, 60)],
)
def test_kmeanspp_matches_its_restatement(vh, n, dim, k, seed, spread):
    """The device draws (update + k_kpp_select) pick exactly the rows of the float64 restatement:
    every distance and running sum is an exact integer here.  The shapes cover both update kernels
    (point blocks of 1024 above 2^20 points, row groups of 8 to 64 lanes below), several blocks per
    step, more blocks than the select's threads (each thread then owns a run of block sums), k = n
    (the last draws find every remaining weight zero but one), a dimension that leaves some lanes
    of a 64-lane row one slice short (800), and pruning in the row-group kernel (more than 2^24
    point floats): with spread > 0 the points are 64 clusters with centres in [-spread, spread] and
    noise in [-8, 8], so that most rows are pruned once every cluster holds a centre (the squared
    distances stay below 2^24, exact in float32)."""
    rng = np.random.default_rng(seed)
    x = rng.integers(-8, 9, (n, dim))
    if spread:
        x += rng.integers(-spread, spread + 1, (64, dim))[rng.integers(0, 64, n)]
    x = x.astype(np.float32)
    st = vh.KMeansState(x)
    print(f"  k-means++ n={n} dim={dim} k={k}", flush=True)
    c, _, (_, kk, iters, _) = st.fit(k, 0, -1.0, init_mode=0, seed=seed)
    assert (kk, iters) == (k, 0)
    want = x[_kmeanspp_restated(x, k, seed)]
    assert np.array_equal(c, want)


@pytest.mark.parametrize("metric,dim", [("l2", 96), ("dot", 40), ("cosine", 768), ("l2", 200)])
def test_small_set_direct_assign_matches_mfma(vh, oracle, monkeypatch, metric, dim):
    """The direct-form assignment of small point sets and the MFMA scan with its certified
    selection give the same assignments on well-separated clusters (no near-ties), and centroids
    and inertia that agree to rounding, over 3 iterations."""
    from vector_hip import datasets as ds

    data, _, _ = ds.gaussian_mixture(6_000, dim, 24, 21)
    data = (data * 4.0 + (3.0 if metric != "l2" else 0.0)).astype(np.float32)
    m = vh.DistanceMetric(oracle.METRICS[metric])
    init = data[:24].copy()
    out = {}
    for path in ("direct", "mfma"):
        if path == "mfma":
            monkeypatch.setenv("VHIP_KMEANS_ASSIGN", "mfma")
        else:
            monkeypatch.delenv("VHIP_KMEANS_ASSIGN", raising=False)
        out[path] = vh.CudaKMeansEngine().fit(data, dim, 24, 3, -1.0, m, init=init, return_assign=True)
    (rd, ad), (rm, am) = out["direct"], out["mfma"]
    assert np.array_equal(ad, am)
    c_d, c_m = rd.centroids.reshape(24, dim), rm.centroids.reshape(24, dim)
    assert np.all(np.linalg.norm(c_d - c_m, axis=1) <= 1e-6 * np.maximum(np.linalg.norm(c_m, axis=1), 1e-6))
    assert abs(rd.inertia - rm.inertia) <= 1e-5 * abs(rm.inertia) + 1e-3


@pytest.mark.parametrize("n,dim,k,metric", [(3, 40, 1, "l2"), (5, 40, 3, "cosine"), (700, 1000, 7, "dot"),
                                            (700, 1024, 7, "l2"), (2_000, 128, 256, "l2")])
def test_small_set_edges(vh, oracle, n, dim, k, metric):
    """Edges of the direct-form assignment: k = 1, fewer points than a wave holds, 1000 and 1024
    dimensions (dpad 1024, k-means' largest: 16 slices per lane, the last partly and wholly
    filled), and 256 centroids (its largest k).  Each step against the oracle's from the same
    centroids."""
    rng = np.random.default_rng(n + dim + k)
    data = rng.standard_normal((n, dim)).astype(np.float32)
    if metric != "l2":
        data += 2.0
    st = vh.KMeansState(data, vh.DistanceMetric(oracle.METRICS[metric]))
    cent = data[:k].copy()
    st.set_centroids(cent)
    st.run(1)
    _check_step(oracle, data, cent, st.read(), metric, max_flip_frac=1.0 / n)


@pytest.mark.parametrize("metric", ["cosine", "dot"])
def test_inertia_of_points_that_are_centroids(vh, oracle, metric):
    """Integer points in [0, 255] at 1024 dimensions, 400 of the 600 of them centroids: a point's
    value against itself is 1 - cos = 0 (or -||x||^2), which a sequential float sum over the
    dimensions misses by about 6e-6 each (odd squares added to an even running sum above 2^24 all
    round down).  The reported inertia is the sum of the per-point values in direct form, within
    rounding of the float64 sum over the GPU's own assignment."""
    rng = np.random.default_rng(77)
    n, dim, k = 600, 1024, 400
    data = rng.integers(0, 256, (n, dim)).astype(np.float32)
    cent = data[rng.choice(n, size=k, replace=False)].copy()
    st = vh.KMeansState(data, vh.DistanceMetric(oracle.METRICS[metric]))
    st.set_centroids(cent)
    st.run(1)
    got = st.read()
    _check_step(oracle, data, cent, got, metric, max_flip_frac=1.0 / n)
    x, c = data.astype(np.float64), cent.astype(np.float64)[got["assign"]]
    dots = np.einsum("ij,ij->i", x, c)
    if metric == "dot":
        want = -dots.sum()
        assert abs(got["inertia"] - want) <= 1e-6 * abs(want)
    else:
        den = np.linalg.norm(x, axis=1) * np.linalg.norm(c, axis=1)
        want = np.sum(1.0 - dots / den)
        assert abs(got["inertia"] - want) <= 2e-7 * n + 2e-6 * abs(want)
