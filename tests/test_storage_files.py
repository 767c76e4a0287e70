"""The trainer's file formats through the C ABI (host code, no GPU needed).

Restates the reference's own tests of MmapStorage (vector-index/src/storage/mmap.rs:276-430)
and of the centroid file (ivf/serializer.rs:551-606), and pins both formats byte for byte
against layouts built here with struct from the format tables (mmap.rs:9-16,
ivf/serializer.rs:264-280): a swapped field, a wrong width or a missing byte fails them.
"""
import os
import struct

import numpy as np
import pytest


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    return vector_hip


VEC_MAGIC = 0x5645435253544F52
CENT_MAGIC = 0x5652534B4D45414E


# ---- VECRSTOR (mmap.rs) ----------------------------------------------------------------
def test_create_and_open_round_trip(vh, tmp_path):
    p = tmp_path / "test_vectors.bin"
    vh.MmapStorage.create(p, 4, [[1.0, 2.0, 3.0, 4.0], [5.0, 6.0, 7.0, 8.0], [9.0, 10.0, 11.0, 12.0]])
    s = vh.MmapStorage.open(p)
    assert s.dimension() == 4 and len(s) == 3 and not s.is_empty()
    assert list(s.get(0)) == [1, 2, 3, 4] and list(s.get(1)) == [5, 6, 7, 8] and list(s.get(2)) == [9, 10, 11, 12]


def test_create_from_flat_round_trip_and_raw_slice(vh, tmp_path):
    p = tmp_path / "flat_vectors.bin"
    vh.MmapStorage.create_from_flat(p, 3, [1.0, 2.0, 3.0, 4.0, 5.0, 6.0])
    s = vh.MmapStorage.open(p)
    assert (len(s), s.dimension()) == (2, 3)
    assert list(s.get(0)) == [1, 2, 3] and list(s.get(1)) == [4, 5, 6]
    p2 = tmp_path / "raw_slice.bin"
    vh.MmapStorage.create_from_flat(p2, 2, [10.0, 20.0, 30.0, 40.0])
    assert list(vh.MmapStorage.open(p2).as_raw_slice()) == [10, 20, 30, 40]


def test_empty_storage(vh, tmp_path):
    p = tmp_path / "empty.bin"
    vh.MmapStorage.create(p, 128, [])
    s = vh.MmapStorage.open(p)
    assert len(s) == 0 and s.is_empty() and s.dimension() == 128 and s.as_raw_slice().size == 0


def test_invalid_magic_truncated_and_too_small(vh, tmp_path):
    p = tmp_path / "bad_magic.bin"
    p.write_bytes(bytes(24))
    with pytest.raises(vh.CudaError, match="invalid magic number"):
        vh.MmapStorage.open(p)
    p = tmp_path / "truncated.bin"
    p.write_bytes(struct.pack("<QQQ", VEC_MAGIC, 10, 4))
    with pytest.raises(vh.CudaError, match="size mismatch"):
        vh.MmapStorage.open(p)
    p = tmp_path / "small.bin"
    p.write_bytes(b"tiny")
    with pytest.raises(vh.CudaError, match="too small"):
        vh.MmapStorage.open(p)
    with pytest.raises(vh.CudaError):
        vh.MmapStorage.open(tmp_path / "missing.bin")


def test_dimension_mismatch_and_out_of_bounds(vh, tmp_path):
    with pytest.raises(vh.CudaError):
        vh.MmapStorage.create(tmp_path / "mismatch.bin", 3, [[1.0, 2.0, 3.0], [4.0, 5.0]])
    p = tmp_path / "oob.bin"
    vh.MmapStorage.create_from_flat(p, 2, [1.0, 2.0])
    with pytest.raises(IndexError):
        vh.MmapStorage.open(p).get(1)


def test_high_dimensional_round_trip(vh, tmp_path):
    dim = 1536
    v1 = np.arange(dim, dtype=np.float32) * np.float32(0.001)
    v2 = (dim - np.arange(dim)).astype(np.float32) * np.float32(0.001)
    p = tmp_path / "high_dim.bin"
    vh.MmapStorage.create(p, dim, [v1, v2])
    s = vh.MmapStorage.open(p)
    assert np.array_equal(s.get(0), v1) and np.array_equal(s.get(1), v2)


def test_vecrstor_bytes(vh, tmp_path):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 7)).astype(np.float32)
    p = tmp_path / "bytes.bin"
    vh.MmapStorage.create_from_flat(p, 7, x)
    want = struct.pack("<QQQ", VEC_MAGIC, 5, 7) + b"".join(struct.pack("<f", float(v)) for v in x.reshape(-1))
    assert p.read_bytes() == want
    assert p.read_bytes()[:8] == b"ROTSRCEV"  # "VECRSTOR" as a little-endian u64


def test_vecrstor_map_view(vh, tmp_path):
    """The zero-copy view: the pointer reads the file's floats in place, 24 bytes past its start,
    and the same header checks as open() reject bad files."""
    import ctypes

    lib = vh._lib
    rng = np.random.default_rng(4)
    x = rng.standard_normal((37, 11)).astype(np.float32)
    p = tmp_path / "m.bin"
    vh.MmapStorage.create_from_flat(p, 11, x)
    data, n, d, view = ctypes.POINTER(ctypes.c_float)(), ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_void_p()
    assert lib.vhip_vecrstor_map(os.fsencode(p), ctypes.byref(data), ctypes.byref(n), ctypes.byref(d),
                                 ctypes.byref(view)) == 0
    try:
        assert (n.value, d.value) == (37, 11)
        got = np.ctypeslib.as_array(data, shape=(37 * 11,)).copy()
        assert np.array_equal(got.reshape(37, 11), x)
        # the view maps the file itself: the pointer sits at the mapping's start plus the header
        assert ctypes.addressof(data.contents) % 4096 == 24
    finally:
        lib.vhip_vecrstor_unmap(view)
    e = tmp_path / "e.bin"
    vh.MmapStorage.create_from_flat(e, 3, np.zeros(0, np.float32))
    assert lib.vhip_vecrstor_map(os.fsencode(e), ctypes.byref(data), ctypes.byref(n), ctypes.byref(d),
                                 ctypes.byref(view)) == 0
    assert (n.value, d.value) == (0, 3)
    lib.vhip_vecrstor_unmap(view)
    bad = tmp_path / "bad.bin"
    bad.write_bytes(struct.pack("<QQQ", VEC_MAGIC, 10, 4) + b"\0" * 16)  # 10 x 4 floats promised, 4 present
    rc = lib.vhip_vecrstor_map(os.fsencode(bad), ctypes.byref(data), ctypes.byref(n), ctypes.byref(d),
                               ctypes.byref(view))
    assert rc != 0 and not view.value and b"size mismatch" in lib.vhip_last_error()
    rc = lib.vhip_vecrstor_map(os.fsencode(tmp_path / "missing.bin"), ctypes.byref(data), ctypes.byref(n),
                               ctypes.byref(d), ctypes.byref(view))
    assert rc != 0 and not view.value


# ---- VRSKMEAN (ivf/serializer.rs) -----------------------------------------------------------
def test_centroid_file_roundtrip(vh, tmp_path):
    p = tmp_path / "c.bin"
    vh.save_centroid_file(p, [1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0, 8.0], 4, 2, vh.DistanceMetric.L2Squared, 15, 42.5)
    got = vh.load_centroid_file(p)
    assert list(got.centroids) == [1, 2, 3, 4, 5, 6, 7, 8]
    assert (got.dimension, got.k, got.metric, got.iterations) == (4, 2, vh.DistanceMetric.L2Squared, 15)
    assert abs(got.inertia - 42.5) < 1e-6


def test_centroid_file_all_metrics(vh, tmp_path):
    p = tmp_path / "m.bin"
    for m in vh.DistanceMetric:
        vh.save_centroid_file(p, [1.0, 2.0], 2, 1, m, 1, 0.0)
        assert vh.load_centroid_file(p).metric == m


def test_centroid_file_bytes_and_bad_headers(vh, tmp_path):
    p = tmp_path / "b.bin"
    c = np.array([[0.5, -1.25, 3.0], [7.0, 8.5, -0.0]], np.float32)
    vh.save_centroid_file(p, c, 3, 2, vh.DistanceMetric.Jaccard, 9, 123.25)
    want = (struct.pack("<QIBIIIf", CENT_MAGIC, 1, 8, 3, 2, 9, 123.25)
            + b"".join(struct.pack("<f", float(v)) for v in c.reshape(-1)))
    assert len(want) == 29 + 24 and p.read_bytes() == want
    bad = tmp_path / "bad.bin"
    bad.write_bytes(b"NOTCENTR12345678")
    with pytest.raises(vh.CudaError):
        vh.load_centroid_file(bad)
    bad.write_bytes(struct.pack("<QIBIIIf", CENT_MAGIC, 2, 0, 1, 1, 1, 0.0) + struct.pack("<f", 1.0))
    with pytest.raises(vh.CudaError, match="version"):
        vh.load_centroid_file(bad)
    bad.write_bytes(struct.pack("<QIBIIIf", CENT_MAGIC, 1, 10, 1, 1, 1, 0.0) + struct.pack("<f", 1.0))
    with pytest.raises(vh.CudaError, match="metric"):
        vh.load_centroid_file(bad)
    bad.write_bytes(struct.pack("<QIBIIIf", CENT_MAGIC, 1, 0, 4, 2, 1, 0.0) + struct.pack("<f", 1.0))
    with pytest.raises(vh.CudaError, match="truncated"):
        vh.load_centroid_file(bad)


def test_trainer_cli_usage(vh):
    """The trainer binary is built next to the library and answers --help without a GPU."""
    import subprocess

    exe = os.path.join(os.path.dirname(vh.library_path()), "vhip_kmeans_train")
    out = subprocess.run([exe, "--help"], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0 and "--data-dir" in out.stdout and "--num-clusters" in out.stdout
