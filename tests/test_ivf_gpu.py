"""GPU parity of the IVF coarse quantizer and the offline k-means trainer.

* find_nearest_centroid over a whole build (ivf/mod.rs:119-132, ivf/kmeans.rs:262-309): every
  point's cluster equals the oracle's (the same strict, lowest-index-first scan) except at
  near-ties; the reported value is the reference engine's metric of that pair; the residual is
  x - c bit for bit.
* find_top_centroids (ivf/kmeans.rs:311-356) for query batches: tie-aware parity with the
  oracle's exact top-nprobe over the centroids, nprobe clamped to nlist.
* fit_cuda_aware / mpi_kmeans --use-cuda (vector-mpi distributed_kmeans.rs:375-415,
  mpi_kmeans.rs:284-364): shards in, centroid file out; the reference's own tests restated
  (distributed_kmeans.rs:421-550).
"""
import os
import subprocess

import numpy as np
import pytest

from knn_check import check_knn

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    assert vector_hip.CudaDeviceContext.device_count() >= 1, "no gfx950 GPU visible"
    return vector_hip


TWO = np.array([0.0, 0.1, 0.1, 0.0, -0.1, 0.0, 10.0, 10.1, 10.1, 10.0, 9.9, 10.0], np.float32)


# ---- reference known-answer tests (vector-mpi/src/distributed_kmeans.rs:421-550) -----------
def test_find_nearest_centroid_kats(vh):
    q = vh.IvfCoarseQuantizer([0.0, 0.0, 10.0, 10.0], 2)
    idx, d = q.find_nearest_centroid([1.0, 1.0])
    assert idx == 0 and abs(d - 2.0) < 1e-5 and q.nlist() == 2 and q.dimension() == 2
    q = vh.IvfCoarseQuantizer([1.0, 0.0, 0.0, 1.0], 2, vh.DistanceMetric.DotProduct)
    assert q.find_nearest_centroid([1.0, 0.0])[0] == 0
    # parallel_assign_basic: counts 1 / 1, each point its own centroid
    cl, sc, _ = vh.IvfCoarseQuantizer([0.0, 0.0, 10.0, 10.0], 2).assign([0.0, 0.0, 10.0, 10.0])
    assert list(cl) == [0, 1] and list(sc) == [0.0, 0.0]


def test_fit_cuda_aware_kats(vh):
    for g in (1, 2):
        r = vh.fit_cuda_aware(TWO, 2, 2, 30, 1e-5, vh.DistanceMetric.L2Squared, g)
        assert r.k == 2 and r.dimension == 2 and 0 < r.iterations <= 30
        lo, hi = sorted([r.centroid(0), r.centroid(1)], key=lambda c: c[0])
        assert np.all(np.abs(lo) < 0.5) and np.all(np.abs(hi - 10.0) < 0.5)
    assert vh.fit_cuda_aware(np.zeros(0, np.float32), 4, 2, 10, 1e-4).k == 0
    r = vh.fit_cuda_aware(np.array([1.0, 2.0, 3.0], np.float32), 3, 1, 10, 1e-4)
    assert r.k == 1 and np.allclose(r.centroid(0), [1.0, 2.0, 3.0], atol=1e-6)
    r = vh.fit_cuda_aware(np.array([1, 0, .9, .1, 0, 1, .1, .9], np.float32), 2, 2, 30, 1e-5,
                          vh.DistanceMetric.CosineSimilarity)
    assert r.k == 2 and r.iterations > 0


# ---- build-time assignment -----------------------------------------------------------------
METRICS = ["l2", "dot", "cosine", "l1", "linf", "minkowski", "hellinger", "jaccard", "mahalanobis", "hamming"]


@pytest.mark.parametrize("metric", METRICS)
def test_coarse_assign_parity(vh, oracle, metric):
    from vector_hip import datasets as ds

    data, _, _ = ds.gaussian_mixture(20_000, 48, 128, 21)
    if metric in ("dot", "cosine"):
        data = data + 3.0
    if metric == "hamming":  # thresholded float Hamming needs coincident values to be meaningful
        data = np.round(data * 2) / 2
    data = np.ascontiguousarray(data, np.float32)
    cent = data[:128].copy()
    q = vh.IvfCoarseQuantizer(cent, 48, vh.DistanceMetric(oracle.METRICS[metric]))
    cl, sc, res = q.assign(data, residuals=True)
    ref = oracle.kmeans_step(data, cent, metric, threads=0)["assign"]
    flips = np.nonzero(cl.astype(np.int64) != ref)[0]
    assert len(flips) <= max(2, int(1e-4 * len(data))), f"{len(flips)} assignment flips"
    for p in flips:
        dg = oracle.distance(metric, data[p], cent[cl[p]])
        dr = oracle.distance(metric, data[p], cent[ref[p]])
        assert abs(dg - dr) <= 1e-4 * max(1.0, abs(dr)), f"point {p}: {dg} vs {dr} is not a near-tie"
    refv = oracle.distance_rows(metric, data, cent[cl])
    assert np.all(np.abs(sc - refv) <= 1e-4 * np.abs(refv) + 1e-5)
    assert np.array_equal(res, data - cent[cl])


def test_coarse_assign_more_centroids_than_points(vh, oracle):
    rng = np.random.default_rng(4)
    cent = rng.standard_normal((500, 16)).astype(np.float32)
    pts = rng.standard_normal((7, 16)).astype(np.float32)
    cl, sc, _ = vh.IvfCoarseQuantizer(cent, 16).assign(pts)
    ref = oracle.kmeans_step(pts, cent, "l2", threads=0)["assign"]
    assert np.array_equal(cl.astype(np.int64), ref)
    assert np.allclose(sc, oracle.distance_rows("l2", pts, cent[cl]), rtol=1e-4)


# ---- query-time probe ------------------------------------------------------------------------
@pytest.mark.parametrize("metric", ["l2", "cosine", "dot", "l1"])
def test_coarse_probe_parity(vh, oracle, metric):
    from vector_hip import datasets as ds

    cent = ds.gaussian(1000, 64, 41)
    qs = ds.gaussian(300, 64, 42)
    q = vh.IvfCoarseQuantizer(cent, 64, vh.DistanceMetric(oracle.METRICS[metric]))
    for nprobe in (1, 16, 1500):
        ids, sc, lens = q.probe_batch(qs, nprobe)
        p = min(nprobe, 1000)
        assert np.all(lens == p)
        check_knn(oracle, cent, qs, ids[:, :p], sc[:, :p], p, metric, rtol=1e-4, atol=1e-5)
    top = q.find_top_centroids(qs[5], 16)
    ids, sc, _ = q.probe_batch(qs[5:6], 16)
    assert [t[0] for t in top] == list(ids[0]) and len(top) == 16
    assert q.find_top_centroids(qs[0], 0) == []


# ---- offline trainer ---------------------------------------------------------------------------
def test_train_from_shards_end_to_end(vh, tmp_path):
    from vector_hip import datasets as ds

    data, _, _ = ds.gaussian_mixture(30_000, 32, 64, 17)
    for i in range(3):
        vh.MmapStorage.create_from_flat(tmp_path / f"shard_{i}.bin", 32, data[10_000 * i:10_000 * (i + 1)])
    (dim, k, iters, inertia), shards = vh.train_from_shards(tmp_path, k=64, max_iters=8, tolerance=-1.0,
                                                            output="c.bin", seed=7)
    assert (shards, dim, k, iters) == (3, 32, 64, 8)
    f = vh.load_centroid_file(tmp_path / "c.bin")
    assert (f.dimension, f.k, f.metric, f.iterations) == (32, 64, vh.DistanceMetric.L2Squared, 8)
    assert f.inertia == np.float32(inertia)
    direct = vh.CudaKMeansEngine().fit(data, 32, 64, 8, -1.0, seed=7)
    assert np.array_equal(direct.centroids.reshape(-1), f.centroids) and direct.inertia == f.inertia
    # the command-line trainer writes the same file
    exe = os.path.join(os.path.dirname(vh.library_path()), "vhip_kmeans_train")
    out = subprocess.run([exe, "-d", str(tmp_path), "-k", "64", "--max-iters", "8", "--tolerance", "-1",
                          "-o", "cli.bin", "--seed", "7"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert (tmp_path / "cli.bin").read_bytes() == (tmp_path / "c.bin").read_bytes()
    empty = tmp_path / "empty"
    empty.mkdir()
    with pytest.raises(vh.CudaError, match="no shard files"):
        vh.train_from_shards(empty)
