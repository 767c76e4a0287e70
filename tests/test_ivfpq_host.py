"""Host-side parts of the IVF-PQ index (no GPU): IvfPqConfig (ivf/config.rs:156-240),
IvfPqSerializer files (ivf/serializer.rs:438-550), InvertedIndex (ivf/inverted_list.rs) and the
ProductQuantizer host helpers (ivf/pq.rs:349-426).  The file layout is also checked byte for
byte against a golden encoding written here with `struct`."""
import struct

import numpy as np
import pytest

import vector_hip as vh

M = vh.DistanceMetric


# ---- config.rs:156-240 ---------------------------------------------------------------------
def test_default_config():
    c = vh.IvfPqConfig()
    assert (c.nlist, c.nprobe, c.num_subvectors, c.sub_clusters, c.max_kmeans_iters) == (64, 8, 8, 256, 25)
    c.validate(128)


def test_custom_builders():
    c = (vh.IvfPqConfig.new(32, 4, 4).with_sub_clusters(64).with_max_kmeans_iters(15)
         .with_kmeans_tolerance(1e-5).with_max_train_points(5000))
    assert (c.nlist, c.nprobe, c.num_subvectors, c.sub_clusters, c.max_kmeans_iters) == (32, 4, 4, 64, 15)
    assert c.kmeans_tolerance == float(np.float32(1e-5)) and c.max_train_points == 5000
    assert c.sub_dimension(128) == 32
    c.validate(128)


@pytest.mark.parametrize("cfg,reason", [
    (vh.IvfPqConfig.new(0, 1, 4), "nlist must be greater than 0"),
    (vh.IvfPqConfig.new(10, 0, 4), "nprobe must be greater than 0"),
    (vh.IvfPqConfig.new(10, 11, 4), "nprobe (11) cannot be greater than nlist (10)"),
    (vh.IvfPqConfig.new(10, 5, 0), "num_subvectors must be greater than 0"),
    (vh.IvfPqConfig.new(10, 5, 5), "vector dimension (128) must be divisible by num_subvectors (5)"),
    (vh.IvfPqConfig.new(10, 5, 4).with_sub_clusters(0), "sub_clusters must be between 1 and 256, got 0"),
    (vh.IvfPqConfig.new(10, 5, 4).with_sub_clusters(300), "sub_clusters must be between 1 and 256, got 300"),
    (vh.IvfPqConfig.new(10, 5, 4).with_max_kmeans_iters(0), "max_kmeans_iters must be greater than 0"),
    (vh.IvfPqConfig.new(10, 5, 4).with_kmeans_tolerance(-1.0), "kmeans_tolerance must be non-negative"),
])
def test_validation_errors(cfg, reason):
    with pytest.raises(vh.InvalidConfig) as e:
        cfg.validate(128)
    assert reason in str(e.value)


def test_config_traits_and_high_dim():
    c1 = vh.IvfPqConfig.new(16, 2, 4)
    assert c1 == vh.IvfPqConfig.new(16, 2, 4)
    assert "IvfPqConfig" in repr(c1) and "nlist=16" in repr(c1)
    c = vh.IvfPqConfig.new(64, 8, 16)
    assert c.sub_dimension(1536) == 96
    c.validate(1536)


# ---- ProductQuantizer host helpers (pq.rs:388-426) -------------------------------------------
def test_get_sub_centroid_accessor():
    pq = vh.ProductQuantizer(4, 2, 2, [1, 2, 3, 4, 5, 6, 7, 8])
    assert pq.get_sub_centroid(0, 0).tolist() == [1, 2]
    assert pq.get_sub_centroid(0, 1).tolist() == [3, 4]
    assert pq.get_sub_centroid(1, 0).tolist() == [5, 6]
    assert pq.get_sub_centroid(1, 1).tolist() == [7, 8]
    assert pq.decode([1, 0]).tolist() == [3, 4, 5, 6]


def test_distance_with_lut_host_helper():
    pq = vh.ProductQuantizer(4, 2, 2, [0, 0, 1, 1, 0, 0, 2, 2])
    lut = np.array([2.0, 0.0, 8.0, 0.0], np.float32)  # pq.rs:369-379
    assert pq.compute_distance_with_lut([1, 1], lut) == 0.0
    assert pq.compute_distance_with_lut([0, 0], lut) == 10.0
    pq4 = vh.ProductQuantizer(4, 4, 2, np.zeros(8))
    assert pq4.compute_distance_with_lut([0] * 4, np.array([1e8, 0, 1, 0, -1e8, 0, 1, 0], np.float32)) == 0.0


def test_product_quantizer_shape_errors():
    with pytest.raises(vh.InvalidConfig):
        vh.ProductQuantizer(5, 2, 2, np.zeros(10))
    with pytest.raises(vh.InvalidConfig):
        vh.ProductQuantizer(4, 2, 2, np.zeros(7))


# ---- inverted_list.rs ------------------------------------------------------------------------
def test_inverted_index_add_and_get():
    inv = vh.InvertedIndex(3, 2)
    inv.add(0, 10, [0, 1])
    inv.add(2, 20, [1, 0])
    inv.add(0, 11, [3, 3])
    assert inv.nlist() == 3 and inv.total_vectors() == 3
    assert inv.get_list(0).ids.tolist() == [10, 11] and inv.get_list(0).get_code(1, 2).tolist() == [3, 3]
    assert inv.get_list(1).is_empty() and len(inv.get_list(2)) == 1


# ---- serializer.rs:438-550 -------------------------------------------------------------------
def _roundtrip_parts():
    cfg = vh.IvfPqConfig.new(2, 1, 2).with_sub_clusters(2).with_max_kmeans_iters(10)
    coarse = np.array([0, 0, 0, 0, 1, 1, 1, 1], np.float32)
    pq = vh.ProductQuantizer(4, 2, 2, [0.0, 0.0, 0.5, 0.5, 0.0, 0.0, 0.5, 0.5])
    inv = vh.InvertedIndex(2, 2)
    inv.add(0, 10, [0, 1])
    inv.add(1, 20, [1, 0])
    return cfg, coarse, pq, inv


def test_serializer_roundtrip(tmp_path):
    cfg, coarse, pq, inv = _roundtrip_parts()
    p = tmp_path / "ix.bin"
    vh.IvfPqSerializer.save_to_file(p, cfg, coarse, pq, inv, 4, M.L2Squared)
    lc, lcc, lpq, linv, ld, lm = vh.IvfPqSerializer.load_from_file(p)
    assert lc == cfg and np.array_equal(lcc, coarse) and lpq == pq and linv == inv
    assert ld == 4 and lm == M.L2Squared


def test_serializer_golden_bytes(tmp_path):
    cfg, coarse, pq, inv = _roundtrip_parts()
    p = tmp_path / "ix.bin"
    vh.IvfPqSerializer.save_to_file(p, cfg, coarse, pq, inv, 4, M.L2Squared)
    want = struct.pack("<QIBI", 0x4956465051564543, 1, 0, 4)
    want += struct.pack("<5If", 2, 1, 2, 2, 10, np.float32(1e-4))
    want += struct.pack("<I8f", 2, *coarse)
    want += struct.pack("<I8f", 8, 0.0, 0.0, 0.5, 0.5, 0.0, 0.0, 0.5, 0.5)
    want += struct.pack("<I", 2)
    want += struct.pack("<II", 1, 10) + bytes([0, 1])
    want += struct.pack("<II", 1, 20) + bytes([1, 0])
    assert p.read_bytes() == want


def test_serializer_metrics_roundtrip(tmp_path):
    cfg = vh.IvfPqConfig.new(1, 1, 1).with_sub_clusters(1)
    pq = vh.ProductQuantizer(2, 1, 1, [1.0, 2.0])
    inv = vh.InvertedIndex(1, 1)
    inv.add(0, 1, [0])
    p = tmp_path / "m.bin"
    for metric in M:
        vh.IvfPqSerializer.save_to_file(p, cfg, [1.0, 2.0], pq, inv, 2, metric)
        assert vh.IvfPqSerializer.load_from_file(p)[5] == metric


def test_serializer_invalid_files(tmp_path):
    p = tmp_path / "bad.bin"
    p.write_bytes(b"BADMAGIC12345678")
    with pytest.raises(vh.InvalidConfig, match="magic"):
        vh.IvfPqSerializer.load_from_file(p)
    p.write_bytes(struct.pack("<QI", 0x4956465051564543, 999))
    with pytest.raises(vh.InvalidConfig, match="version"):
        vh.IvfPqSerializer.load_from_file(p)
    p.write_bytes(struct.pack("<QIB", 0x4956465051564543, 1, 99))
    with pytest.raises(vh.InvalidConfig, match="metric"):
        vh.IvfPqSerializer.load_from_file(p)
    with pytest.raises(vh.InvalidConfig):
        vh.IvfPqSerializer.load_from_file(tmp_path / "non_existent_file_path_12345.bin")


def test_serializer_truncated_and_bad_codebook(tmp_path):
    cfg, coarse, pq, inv = _roundtrip_parts()
    p = tmp_path / "ix.bin"
    vh.IvfPqSerializer.save_to_file(p, cfg, coarse, pq, inv, 4, M.L2Squared)
    full = p.read_bytes()
    for cut in (10, 40, len(full) - 1):
        p.write_bytes(full[:cut])
        with pytest.raises(vh.InvalidConfig):
            vh.IvfPqSerializer.load_from_file(p)
    # a codebook length that ProductQuantizer::new would reject (pq.rs:38-41)
    bad = bytearray(full)
    off = 8 + 4 + 1 + 4 + 24 + 4 + 32
    bad[off:off + 4] = struct.pack("<I", 7)
    p.write_bytes(bytes(bad))
    with pytest.raises(vh.InvalidConfig, match="codebook"):
        vh.IvfPqSerializer.load_from_file(p)
