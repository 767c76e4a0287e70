"""Engines built straight from VECRSTOR files (storage/mmap.rs:9-16) on the GPU.

The reference reads every shard into one Vec before it reaches the GPU (mpi_kmeans.rs:307-325)
and CudaKnnEngine::new copies the base again (knn.rs:111-122).  Here the files are mapped and
streamed through the pinned staging ring, and k-means takes several files as segments of one
point set.  Parity: the engines built from the files answer bit for bit what the engines built
from the same rows as arrays answer (the device data is the same, so any difference is an upload
bug: a dropped block, a shifted segment, a torn copy).  The sizes cross the 32 MiB staging block
and the 4 MiB per-thread copy split, with row counts that fit neither.
"""
import ctypes
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    assert vector_hip.CudaDeviceContext.device_count() >= 1
    return vector_hip


@pytest.mark.parametrize("n,dim,metric", [(120_001, 100, 0), (70_003, 128, 1), (5, 3, 2)])
def test_knn_from_file_matches_array(vh, tmp_path, n, dim, metric):
    print(f"knn from file n={n} dim={dim} metric={metric}", flush=True)
    rng = np.random.default_rng(n)
    x = rng.standard_normal((n, dim)).astype(np.float32)
    q = rng.standard_normal((64, dim)).astype(np.float32)
    p = tmp_path / "base.bin"
    vh.MmapStorage.create_from_flat(p, dim, x)
    m = vh.DistanceMetric(metric)
    a = vh.CudaKnnEngine(x, dim, m)
    b = vh.CudaKnnEngine.from_vecrstor(p, m)
    assert (b.num_vectors(), b.dimension(), b.metric()) == (n, dim, m)
    k = min(10, n)
    ia, da, la = a.search_batch_arrays(q, k)
    ib, db, lb = b.search_batch_arrays(q, k)
    assert np.array_equal(la, lb) and np.all(lb == k)
    assert np.array_equal(ia, ib) and np.array_equal(da.view(np.uint32), db.view(np.uint32))
    # the engine also accepts the numpy memmap view MmapStorage.open returns
    c = vh.CudaKnnEngine(vh.MmapStorage.open(p).as_raw_slice(), dim, m)
    ic, dc, _ = c.search_batch_arrays(q, k)
    assert np.array_equal(ia, ic) and np.array_equal(da.view(np.uint32), dc.view(np.uint32))


def test_knn_from_file_errors(vh, tmp_path):
    with pytest.raises(vh.CudaError):
        vh.CudaKnnEngine.from_vecrstor(tmp_path / "missing.bin")
    bad = tmp_path / "bad.bin"
    bad.write_bytes(b"\0" * 40)
    with pytest.raises(vh.CudaError, match="magic"):
        vh.CudaKnnEngine.from_vecrstor(bad)


def _shards(vh, tmp_path, x, sizes):
    paths, o = [], 0
    for i, s in enumerate(sizes):
        p = tmp_path / f"shard_{i}.bin"
        vh.MmapStorage.create_from_flat(p, x.shape[1], x[o:o + s])
        paths.append(p)
        o += s
    return paths


def test_kmeans_segments_match_single_upload(vh, tmp_path):
    from vector_hip import datasets as ds

    print("kmeans segments 3 shards 27014 x 96", flush=True)
    x, _, _ = ds.gaussian_mixture(27_014, 96, 64, 23)
    paths = _shards(vh, tmp_path, x, [7_001, 13, 20_000])
    st_a = vh.KMeansState(x)
    st_b = vh.KMeansState.from_vecrstor(paths)
    for st in (st_a, st_b):
        st.set_centroids(x[:64])
        st.run(3)
    ra, rb = st_a.read(), st_b.read()
    for key in ("centroids", "assign", "counts", "shifts"):
        assert np.array_equal(ra[key], rb[key]), key
    assert ra["inertia"] == rb["inertia"]
    # residuals and scores of the assign-only pass agree too
    aa, sa, qa = st_a.assign_only(residuals=True)
    ab, sb, qb = st_b.assign_only(residuals=True)
    assert np.array_equal(aa, ab) and np.array_equal(sa, sb) and np.array_equal(qa, qb)


@pytest.mark.parametrize("init_mode", [0, 1])
def test_fit_on_resident_points_matches_fit(vh, tmp_path, init_mode):
    """fit_state on a state built from files == the one-call fit on the concatenated rows, for
    the k-means++ init (CudaKMeansEngine) and the seeded shuffle init (DistributedKMeansEngine)."""
    from vector_hip import datasets as ds

    print(f"kmeans fit_state init_mode={init_mode}", flush=True)
    x, _, _ = ds.gaussian_mixture(20_000, 32, 48, 29)
    paths = _shards(vh, tmp_path, x, [4_000, 0, 16_000])
    st = vh.KMeansState.from_vecrstor(paths)
    c, a, (d, k, iters, inertia) = st.fit(48, 6, -1.0, init_mode=init_mode, seed=11)
    if init_mode == 0:
        ref, ra = vh.CudaKMeansEngine().fit(x, 32, 48, 6, -1.0, seed=11, return_assign=True)
    else:
        ref, ra = vh.DistributedKMeansEngine.emulator(1).fit(x, 32, 48, 6, -1.0, seed=11, return_assign=True)
    assert (d, k, iters) == (32, 48, 6)
    assert np.array_equal(c, ref.centroids) and np.array_equal(a, ra) and inertia == ref.inertia
    # a second fit on the same state starts over from the same init
    c2, a2, r2 = st.fit(48, 6, -1.0, init_mode=init_mode, seed=11)
    assert np.array_equal(c, c2) and np.array_equal(a, a2) and r2[3] == inertia
    # explicit init centroids: the seeded init is skipped
    ci, ai, ri = st.fit(8, 4, -1.0, init=x[100:108])
    ref_i, ra_i = vh.CudaKMeansEngine().fit(x, 32, 8, 4, -1.0, init=x[100:108], return_assign=True)
    assert np.array_equal(ci, ref_i.centroids) and np.array_equal(ai, ra_i)
    # more clusters than points: k is clamped to n (kmeans.rs:78)
    small = vh.KMeansState(x[:5])
    cs, _, rs = small.fit(16, 2, -1.0)
    assert rs[1] == 5 and cs.shape == (5, 32)


def test_kmeans_from_files_errors(vh, tmp_path):
    rng = np.random.default_rng(5)
    vh.MmapStorage.create_from_flat(tmp_path / "a.bin", 8, rng.standard_normal((10, 8)).astype(np.float32))
    vh.MmapStorage.create_from_flat(tmp_path / "b.bin", 4, rng.standard_normal((10, 4)).astype(np.float32))
    with pytest.raises(vh.CudaError, match="dimension mismatch"):
        vh.KMeansState.from_vecrstor([tmp_path / "a.bin", tmp_path / "b.bin"])
    vh.MmapStorage.create_from_flat(tmp_path / "e.bin", 8, np.zeros(0, np.float32))
    with pytest.raises(vh.CudaError, match="at least one point"):
        vh.KMeansState.from_vecrstor([tmp_path / "e.bin"])


def test_kmeans_create_segments_c_abi(vh):
    """vhip_kmeans_create_segments with host arrays: an empty segment in the middle, ragged
    counts; a null pointer for a non-empty segment is rejected."""
    lib = vh._lib
    rng = np.random.default_rng(6)
    x = rng.standard_normal((3_001, 20)).astype(np.float32)
    parts = [x[:1_000], x[1_000:1_000], x[1_000:]]
    fp = ctypes.POINTER(ctypes.c_float)
    segs = (fp * 3)(*[p.ctypes.data_as(fp) for p in parts])
    counts = (ctypes.c_size_t * 3)(*[p.shape[0] for p in parts])
    h = ctypes.c_void_p()
    assert lib.vhip_kmeans_create_segments(0, segs, counts, 3, 20, 0, ctypes.byref(h)) == 0
    st = vh.KMeansState.__new__(vh.KMeansState)
    st._h, st._n, st._d, st._k = h, 3_001, 20, 0
    ref = vh.KMeansState(x)
    for s in (st, ref):
        s.set_centroids(x[:16])
        s.run(2)
    assert np.array_equal(st.read()["centroids"], ref.read()["centroids"])
    assert np.array_equal(st.read()["assign"], ref.read()["assign"])
    segs[0] = fp()
    h2 = ctypes.c_void_p()
    assert lib.vhip_kmeans_create_segments(0, segs, counts, 3, 20, 0, ctypes.byref(h2)) != 0
    assert not h2.value and b"null" in lib.vhip_last_error()
