"""GPU parity of product quantization and the IVF-PQ index (vector-index/src/ivf).

* compute_adc_lut (pq.rs:233-266) and encode_batch (pq.rs:178-214) against the oracle for all 10
  metrics: tables within 1e-5, codes equal except where the oracle's own values tie within
  float rounding.
* ProductQuantizer::train (pq.rs:53-107): the reference's tests, and one Lloyd step per sub-space
  from explicit initial codebooks against the oracle's KMeans::fit.
* IvfPqIndex::search_with_nprobe (ivf/mod.rs:256-345) against the oracle's restatement on the
  probe lists the index uses.  On integer-valued parts every table entry and every ADC sum is
  an exact integer, so distances must match bit for bit and ids up to ties; float parts are
  checked within 1e-4.  Shapes cover both table paths (register-held and cached codebooks),
  the 16-, 4- and 1-byte code paths, empty lists, k above the candidate count, k = 1024, and
  more queries than workgroups.
* IvfPqIndex build / save / load: the reference's tests (ivf/mod.rs:456-647) and a pipeline
  check of a built index's lists and codes against the oracle on the index's own parameters.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

METRICS = ["l2", "dot", "cosine", "l1", "minkowski", "linf", "hamming", "mahalanobis", "jaccard", "hellinger"]


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    assert vector_hip.CudaDeviceContext.device_count() >= 1, "no gfx950 GPU visible"
    return vector_hip


def _m(vh, name):
    return vh.DistanceMetric(["l2", "dot", "cosine", "l1", "minkowski", "linf", "hamming", "mahalanobis",
                              "jaccard", "hellinger"].index(name))


# ---- ProductQuantizer -------------------------------------------------------------------------
def test_adc_lut_kats(vh):
    pq = vh.ProductQuantizer(4, 2, 2, [0, 0, 1, 1, 0, 0, 2, 2])  # pq.rs:349-386
    lut = pq.compute_adc_lut([1, 1, 2, 2])
    assert lut.tolist() == [2.0, 0.0, 8.0, 0.0]
    assert pq.compute_distance_with_lut([1, 1], lut) == 0.0 and pq.compute_distance_with_lut([0, 0], lut) == 10.0
    pq5 = vh.ProductQuantizer(5, 5, 2, np.tile([0.0, 1.0], 5))  # pq.rs:403-426
    lut = pq5.compute_adc_lut(np.ones(5))
    assert abs(pq5.compute_distance_with_lut([1] * 5, lut)) < 1e-5
    assert abs(pq5.compute_distance_with_lut([0] * 5, lut) - 5.0) < 1e-5


@pytest.mark.parametrize("metric", METRICS)
def test_adc_lut_parity(vh, oracle, metric):
    rng = np.random.default_rng(METRICS.index(metric))
    pq = vh.ProductQuantizer(32, 4, 16, rng.standard_normal(4 * 16 * 8).astype(np.float32))
    q = rng.standard_normal((7, 32)).astype(np.float32)
    got = pq.compute_adc_lut_batch(q, _m(vh, metric))
    for i in range(7):
        want = oracle.pq_adc_lut(q[i], pq.codebooks, 4, 16, metric)
        np.testing.assert_allclose(got[i], want, rtol=1e-5, atol=1e-5)


def _check_codes(oracle, x, cb, m_sub, ks, got, metric, max_flip=0.01):
    want = oracle.pq_encode(x, cb, m_sub, ks, metric)
    diff = np.argwhere(got != want)
    assert len(diff) <= max_flip * got.size, f"{len(diff)} of {got.size} codes differ"
    ds = x.shape[1] // m_sub
    hib = metric in ("dot", "cosine")
    for i, m in diff:  # each differing code must be a near-tie of the oracle's own values
        sub = x[i, m * ds:(m + 1) * ds]
        a = oracle.distance(metric, sub, cb[(m * ks + got[i, m]) * ds:(m * ks + got[i, m] + 1) * ds])
        b = oracle.distance(metric, sub, cb[(m * ks + want[i, m]) * ds:(m * ks + want[i, m] + 1) * ds])
        assert abs(a - b) <= 1e-5 * max(1.0, abs(b)), (i, m, a, b, hib)


@pytest.mark.parametrize("metric", METRICS)
def test_encode_parity(vh, oracle, metric):
    rng = np.random.default_rng(100 + METRICS.index(metric))
    dim, m_sub, ks = 32, 4, 64
    cb = rng.standard_normal(m_sub * ks * 8).astype(np.float32)
    x = rng.standard_normal((700, dim)).astype(np.float32)
    pq = vh.ProductQuantizer(dim, m_sub, ks, cb)
    _check_codes(oracle, x, cb, m_sub, ks, pq.encode_batch(x, _m(vh, metric)), metric)


@pytest.mark.parametrize("dim,m_sub,ks", [(12, 4, 5), (256, 2, 256), (80, 2, 256), (8, 8, 256)])
def test_encode_shapes_integer_exact(vh, oracle, dim, m_sub, ks):
    # integer data: the direct form is exact, so codes equal the oracle's, ties to the lowest index
    # (256 x 128 floats is a codebook read through the caches; sub-dimension 40 is past the
    # register-held sub-vector)
    rng = np.random.default_rng(dim + ks)
    cb = rng.integers(-3, 4, m_sub * ks * (dim // m_sub)).astype(np.float32)
    x = rng.integers(-3, 4, (333, dim)).astype(np.float32)
    pq = vh.ProductQuantizer(dim, m_sub, ks, cb)
    for metric in ("l2", "l1", "dot"):
        got = pq.encode_batch(x, _m(vh, metric))
        np.testing.assert_array_equal(got, oracle.pq_encode(x, cb, m_sub, ks, metric))
    assert pq.encode_batch(np.zeros((0, dim), np.float32)).shape == (0, m_sub)


def test_train_kats(vh):
    # pq.rs:302-346
    data = np.array([[i, i + 1, i + 2, i + 3, i, i, i, i] for i in range(20)], np.float32)
    pq = vh.ProductQuantizer.train(data, 8, 2, 4, 15, 1e-4, vh.DistanceMetric.L2Squared)
    assert (pq.dimension, pq.num_subvectors, pq.sub_dimension, pq.sub_clusters) == (8, 2, 4, 4)
    assert pq.codebooks.size == 32
    code = pq.encode(data[0])
    assert code[0] < 4 and code[1] < 4 and pq.decode(code).size == 8
    assert np.array_equal(pq.encode_batch(data)[0], code)
    # pq.rs:428-469: cosine and dot training on identical rows
    same = np.tile(np.array([1.0, 0.0, 0.0, 1.0], np.float32), (10, 1))
    for m in (vh.DistanceMetric.CosineSimilarity, vh.DistanceMetric.DotProduct):
        p = vh.ProductQuantizer.train(same, 4, 2, 2, 10, 1e-4, m)
        assert p.encode([1.0, 0.0, 0.0, 1.0], m).size == 2


def test_train_pads_when_fewer_points_than_sub_clusters(vh):
    x = np.arange(5 * 4, dtype=np.float32).reshape(5, 4)
    pq = vh.ProductQuantizer.train(x, 4, 2, 8, 10, 1e-4)
    cb = pq.codebooks.reshape(2, 8, 2)
    assert np.all(cb[:, 5:] == 0.0)  # pq.rs:84-88
    assert sorted(map(tuple, cb[0, :5].tolist())) == sorted(map(tuple, x[:, :2].tolist()))


@pytest.mark.parametrize("metric", ["l2", "dot", "l1"])
def test_train_one_step_parity(vh, oracle, metric):
    rng = np.random.default_rng(7)
    dim, m_sub, ks, n = 16, 4, 32, 3000
    x = rng.standard_normal((n, dim)).astype(np.float32)
    ds = dim // m_sub
    init = np.concatenate([x[:ks, m * ds:(m + 1) * ds].reshape(-1) for m in range(m_sub)])
    pq = vh.ProductQuantizer.train(x, dim, m_sub, ks, 1, -1.0, _m(vh, metric), init_codebooks=init)
    got = pq.codebooks.reshape(m_sub, ks, ds)
    bad = 0
    for m in range(m_sub):
        sub = np.ascontiguousarray(x[:, m * ds:(m + 1) * ds])
        c = oracle.kmeans_fit(sub, x[:ks, m * ds:(m + 1) * ds], 1, tol=-1.0, metric=metric)["centroids"]
        err = np.linalg.norm(got[m] - c, axis=1) / np.maximum(np.linalg.norm(c, axis=1), 1e-6)
        bad += int(np.sum(err > 1e-4))
    assert bad <= 2, f"{bad} sub-centroids differ"


# ---- IVF-PQ search ----------------------------------------------------------------------------
def _parts(rng, dim, m_sub, ks, nlist, n, integer=True, empty=()):
    ds = dim // m_sub
    if integer:
        coarse = rng.integers(-4, 5, (nlist, dim)).astype(np.float32)
        cb = rng.integers(-2, 3, m_sub * ks * ds).astype(np.float32)
    else:
        coarse = rng.standard_normal((nlist, dim)).astype(np.float32)
        cb = (0.5 * rng.standard_normal(m_sub * ks * ds)).astype(np.float32)
    choices = np.array([c for c in range(nlist) if c not in empty])
    assign = choices[rng.integers(0, choices.size, n)]
    order = np.argsort(assign, kind="stable")
    sizes = np.bincount(assign, minlength=nlist).astype(np.uint32)
    codes = rng.integers(0, ks, (n, m_sub)).astype(np.uint8)
    return coarse, cb, sizes, order.astype(np.uint32), codes[order]


def _index(vh, parts, dim, m_sub, ks, metric):
    coarse, cb, sizes, ids, codes = parts
    cfg = vh.IvfPqConfig.new(len(sizes), 1, m_sub).with_sub_clusters(ks)
    inv = vh.InvertedIndex.from_csr(sizes, ids, codes, m_sub)
    pq = vh.ProductQuantizer(dim, m_sub, ks, cb)
    return vh.IvfPqIndex.from_parts(np.zeros((0, dim), np.float32), cfg, coarse, pq, inv, dim, metric)


def _oracle_all(oracle, q, parts, m_sub, ks, probes, metric):
    coarse, cb, sizes, ids, codes = parts
    off = np.concatenate([[0], np.cumsum(sizes)]).astype(np.uint64)
    total = int(sum(sizes[p] for p in probes))
    return oracle.ivfpq_search(q, coarse, cb, m_sub, ks, off, ids, codes, probes, max(total, 1), metric)


def _check_search(vh, oracle, ix, parts, queries, k, nprobe, metric, m_sub, ks, exact):
    ids, dist, lens = ix.search_batch_arrays(queries, k, nprobe)
    probes = ix.probe(queries, nprobe)
    hib = metric in ("dot", "cosine")
    for q in range(queries.shape[0]):
        oi, od = _oracle_all(oracle, queries[q], parts, m_sub, ks, probes[q], metric)
        want_len = min(k, oi.size)
        assert lens[q] == want_len, (q, lens[q], want_len)
        gi, gd = ids[q, :want_len], dist[q, :want_len]
        assert np.all(ids[q, want_len:] == 0xFFFFFFFF) and np.all(np.isnan(dist[q, want_len:]))
        if want_len == 0:
            continue
        of = dict(zip(oi.tolist(), od.tolist()))
        assert len(set(gi.tolist())) == want_len and all(int(v) in of for v in gi)
        mine = np.array([of[int(v)] for v in gi], np.float32)
        if exact:
            np.testing.assert_array_equal(gd, od[:want_len])
            np.testing.assert_array_equal(gd, mine)
        else:
            tol = 1e-4 * max(1.0, float(np.max(np.abs(od[:want_len]))))
            np.testing.assert_allclose(gd, od[:want_len], atol=tol, rtol=0)
            np.testing.assert_allclose(gd, mine, atol=tol, rtol=0)
            kth = od[want_len - 1]
            assert np.all(mine >= kth - tol) if hib else np.all(mine <= kth + tol)
        # best first
        assert np.all(np.diff(gd) <= 0) if hib else np.all(np.diff(gd) >= 0)


SHAPES = [  # dim, M, Ks: register-held codebooks (ds 4 / 8 / 32 with Ks 256), cached codebooks
    # (ds 2 / 6 / 32, Ks <= 128), code rows through the DMA rings (M 16 / 32) and through
    # registers (16-, 4- and 1-byte pieces); (128, 16, 256) is the benchmark's shape
    (16, 4, 16), (64, 8, 256), (128, 4, 64), (96, 3, 100), (32, 16, 256), (30, 5, 7), (24, 4, 256),
    (128, 32, 256), (64, 32, 256), (256, 16, 128), (64, 16, 256), (128, 16, 256), (64, 4, 256),
    (128, 4, 256)]


@pytest.mark.parametrize("dim,m_sub,ks", SHAPES)
@pytest.mark.parametrize("metric", ["l2", "dot"])
def test_search_integer_exact(vh, oracle, dim, m_sub, ks, metric):
    rng = np.random.default_rng(dim * 7 + m_sub + ks)
    parts = _parts(rng, dim, m_sub, ks, 12, 2500, empty=(3, 7))
    ix = _index(vh, parts, dim, m_sub, ks, _m(vh, metric))
    assert len(ix) == 2500 and ix.nlist() == 12
    qs = rng.integers(-4, 5, (40, dim)).astype(np.float32)
    for k, nprobe in ((10, 4), (1, 1), (100, 12)):
        _check_search(vh, oracle, ix, parts, qs, k, nprobe, metric, m_sub, ks, exact=True)


@pytest.mark.parametrize("metric", METRICS)
def test_search_float_all_metrics(vh, oracle, metric):
    rng = np.random.default_rng(500 + METRICS.index(metric))
    dim, m_sub, ks = 32, 8, 64
    parts = _parts(rng, dim, m_sub, ks, 10, 3000, integer=False)
    if metric in ("hellinger", "jaccard"):
        parts = (np.abs(parts[0]), np.abs(parts[1])) + parts[2:]
    ix = _index(vh, parts, dim, m_sub, ks, _m(vh, metric))
    qs = rng.standard_normal((25, dim)).astype(np.float32)
    if metric in ("hellinger", "jaccard"):
        qs = np.abs(qs)
    _check_search(vh, oracle, ix, parts, qs, 20, 3, metric, m_sub, ks, exact=False)


@pytest.mark.parametrize("dim,m_sub", [(128, 16), (64, 8), (64, 4), (128, 4)])
def test_search_float_l2_register_codebooks(vh, oracle, dim, m_sub):
    """Squared L2 on float parts with register-held codebooks of 8-, 16- and 32-float sub-spaces
    (the first is the benchmark's shape, code rows through the DMA ring)."""
    rng = np.random.default_rng(900 + dim + m_sub)
    ks = 256
    parts = _parts(rng, dim, m_sub, ks, 12, 4000, integer=False)
    ix = _index(vh, parts, dim, m_sub, ks, vh.DistanceMetric.L2Squared)
    qs = rng.standard_normal((30, dim)).astype(np.float32)
    _check_search(vh, oracle, ix, parts, qs, 25, 4, "l2", m_sub, ks, exact=False)


def test_search_large_k_and_short_lists(vh, oracle):
    rng = np.random.default_rng(11)
    dim, m_sub, ks = 64, 16, 256
    parts = _parts(rng, dim, m_sub, ks, 8, 1500)
    ix = _index(vh, parts, dim, m_sub, ks, vh.DistanceMetric.L2Squared)
    qs = rng.integers(-4, 5, (6, dim)).astype(np.float32)
    _check_search(vh, oracle, ix, parts, qs, 1024, 8, "l2", m_sub, ks, exact=True)   # k = VHIP_IVFPQ_MAX_K
    _check_search(vh, oracle, ix, parts, qs, 900, 2, "l2", m_sub, ks, exact=True)    # k above the candidates
    with pytest.raises(vh.InvalidConfig):
        ix.search_batch_arrays(qs, 1025, 8)


def test_search_many_queries(vh, oracle):
    # more queries than workgroups: each workgroup serves several queries in turn
    rng = np.random.default_rng(12)
    dim, m_sub, ks = 32, 8, 256
    parts = _parts(rng, dim, m_sub, ks, 16, 4000)
    ix = _index(vh, parts, dim, m_sub, ks, vh.DistanceMetric.L2Squared)
    qs = rng.integers(-4, 5, (2000, dim)).astype(np.float32)
    ids, dist, lens = ix.search_batch_arrays(qs, 10, 3)
    sel = rng.choice(2000, 60, replace=False)
    _check_search(vh, oracle, ix, parts, qs[sel], 10, 3, "l2", m_sub, ks, exact=True)
    ids2, dist2, _ = ix.search_batch_arrays(qs[sel], 10, 3)
    assert np.array_equal(ids[sel], ids2) and np.array_equal(dist[sel], dist2)  # batch independent


def test_search_edges(vh, oracle):
    rng = np.random.default_rng(13)
    parts = _parts(rng, 16, 4, 16, 5, 300)
    ix = _index(vh, parts, 16, 4, 16, vh.DistanceMetric.L2Squared)
    q = rng.integers(-4, 5, 16).astype(np.float32)
    assert ix.search_with_nprobe(q, 0, 3) == []                    # ivf/mod.rs:272-274
    assert len(ix.search_with_nprobe(q, 5, 0)) == 5                # nprobe clamped to >= 1 (:276)
    a = ix.search_with_nprobe(q, 7, 99)                            # and to <= nlist
    b = ix.search_with_nprobe(q, 7, 5)
    assert a == b
    assert ix.probe(q.reshape(1, -1), 99).shape == (1, 5)
    with pytest.raises(vh.DimensionMismatch):
        ix.search(np.zeros(8, np.float32), 3)
    assert ix.search_batch(np.zeros((0, 16), np.float32), 3) == []


def test_probe_matches_find_top_centroids(vh, oracle):
    rng = np.random.default_rng(14)
    parts = _parts(rng, 32, 4, 16, 40, 500, integer=False)
    ix = _index(vh, parts, 32, 4, 16, vh.DistanceMetric.L2Squared)
    qs = rng.standard_normal((30, 32)).astype(np.float32)
    pr = ix.probe(qs, 7)
    for q in range(30):
        oi, osc = oracle.find_top_centroids(qs[q], parts[0], 7, "l2")
        s = np.array([oracle.distance("l2", qs[q], parts[0][c]) for c in pr[q]])
        assert np.all(s <= osc[-1] * (1 + 1e-5) + 1e-5) and np.all(np.diff(s) >= -1e-4)


# ---- IvfPqIndex build (ivf/mod.rs:456-647) ------------------------------------------------------
def _storage(rows):
    return np.asarray(rows, np.float32)


def test_ivf_pq_end_to_end_search(vh):
    st = _storage([[(i * 10 + d) * 0.1 for d in range(8)] for i in range(50)])
    cfg = vh.IvfPqConfig.new(4, 2, 2).with_sub_clusters(8).with_max_kmeans_iters(15)
    ix = vh.IvfPqIndex.build_with_config(st, cfg, vh.DistanceMetric.L2Squared)
    assert len(ix) == 50
    res = ix.search(st[10], 5)
    assert len(res) == 5 and 10 in [r.id for r in res]


def test_ivf_pq_recall_vs_flat(vh, oracle):
    st = _storage([[((i * 7 + d) % 30) for d in range(16)] for i in range(100)])
    cfg = vh.IvfPqConfig.new(8, 4, 4).with_sub_clusters(16).with_max_kmeans_iters(20)
    ix = vh.IvfPqIndex.build_with_config(st, cfg, vh.DistanceMetric.L2Squared)
    gi, gd = oracle.flat_search(st, st[42], 10, "l2")
    gt = [vh.SearchResult(int(i), float(d)) for i, d in zip(gi, gd)]
    assert vh.IvfPqIndex.evaluate_recall(gt, ix.search(st[42], 10)) >= 0.5


def test_ivf_pq_save_and_load(vh, tmp_path):
    st = _storage([[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12]])
    ix = vh.IvfPqIndex.build_with_config(st, vh.IvfPqConfig.new(2, 2, 2).with_sub_clusters(4),
                                         vh.DistanceMetric.L2Squared)
    p = tmp_path / "ix.bin"
    ix.save_to_file(p)
    lo = vh.IvfPqIndex.load_from_file(st, p)
    assert len(lo) == 3 and lo.inverted_index().nlist() == 2
    assert lo.search(st[1], 3) == ix.search(st[1], 3)
    with pytest.raises(vh.DimensionMismatch):
        vh.IvfPqIndex.load_from_file(np.zeros((1, 5), np.float32), p)


def test_ivf_pq_cosine_and_dot(vh):
    cos = _storage([[f, f + 1, f + 2, f + 3] for f in range(1, 21)])
    dot = _storage([[f, f * 2, f * 0.5, f + 1] for f in range(1, 21)])
    cfg = vh.IvfPqConfig.new(2, 2, 2).with_sub_clusters(4)
    assert len(vh.IvfPqIndex.build_with_config(cos, cfg, vh.DistanceMetric.CosineSimilarity)
               .search([1, 2, 3, 4], 2)) == 2
    assert len(vh.IvfPqIndex.build_with_config(dot, cfg, vh.DistanceMetric.DotProduct)
               .search([1, 2, 0.5, 2], 2)) == 2


def test_ivf_pq_k_zero_and_empty_storage(vh):
    cfg = vh.IvfPqConfig.new(1, 1, 1).with_sub_clusters(1)
    with pytest.raises(vh.EmptyIndex):
        vh.IvfPqIndex.build_with_config(np.zeros((0, 2), np.float32), cfg, vh.DistanceMetric.L2Squared)
    ix = vh.IvfPqIndex.build_with_config(_storage([[1, 2]]), cfg, vh.DistanceMetric.L2Squared)
    assert ix.search([1, 2], 0) == []


def test_ivf_pq_custom_nprobe_and_dimension_mismatch(vh):
    st = _storage([[i, i + 1, i + 2, i + 3] for i in range(30)])
    ix = vh.IvfPqIndex.build_with_config(st, vh.IvfPqConfig.new(4, 1, 2).with_sub_clusters(4),
                                         vh.DistanceMetric.L2Squared)
    assert ix.search_with_nprobe([0, 1, 2, 3], 3, 1) and ix.search_with_nprobe([0, 1, 2, 3], 3, 4)
    one = vh.IvfPqIndex.build_with_config(_storage([[1, 2, 3, 4]]), vh.IvfPqConfig.new(1, 1, 2).with_sub_clusters(2),
                                          vh.DistanceMetric.L2Squared)
    with pytest.raises(vh.DimensionMismatch):
        one.search([1, 2], 1)
    with pytest.raises(vh.InvalidConfig):
        vh.IvfPqIndex.build_with_config(st, vh.IvfPqConfig.new(4, 5, 2), vh.DistanceMetric.L2Squared)


def test_ivf_pq_getters(vh):
    st = _storage([[1, 2]])
    cfg = vh.IvfPqConfig.new(1, 1, 1).with_sub_clusters(2)
    ix = vh.IvfPqIndex.build_with_config(st, cfg, vh.DistanceMetric.L2Squared)
    assert ix.storage().shape[1] == 2 and ix.config().nlist == 1 and ix.metric() == vh.DistanceMetric.L2Squared
    assert ix.coarse_centroids().size == 2 and ix.pq().num_subvectors == 1 and ix.inverted_index().nlist() == 1
    assert not ix.is_empty()


@pytest.mark.parametrize("metric", ["l2", "cosine"])
def test_build_pipeline_parity(vh, oracle, metric):
    # the index's lists and codes follow from its own coarse centroids and codebooks
    rng = np.random.default_rng(21)
    n, dim = 4000, 32
    x = rng.standard_normal((n, dim)).astype(np.float32)
    cfg = vh.IvfPqConfig.new(16, 4, 8).with_sub_clusters(32).with_max_kmeans_iters(8)
    ix = vh.IvfPqIndex.build_with_config(x, cfg, _m(vh, metric))
    cc = ix.coarse_centroids().reshape(-1, dim)
    pq = ix.pq()
    inv = ix.inverted_index()
    assert inv.total_vectors() == n and ix.nlist() == 16
    lst = np.zeros(n, np.int64)
    for c, L in enumerate(inv.lists):
        assert np.all(np.diff(L.ids.astype(np.int64)) > 0)  # insertion (ascending id) order
        lst[L.ids] = c
    hib = metric == "cosine"
    flips = 0
    for i in range(n):
        s = np.array([oracle.distance(metric, x[i], c) for c in cc])
        best = int(np.argmax(s) if hib else np.argmin(s))
        if best != lst[i]:
            flips += 1
            assert abs(s[best] - s[lst[i]]) <= 1e-5 * max(1.0, abs(s[best]))
    assert flips <= n * 1e-3
    codes = np.zeros((n, 8), np.uint8)
    for L in inv.lists:
        codes[L.ids] = L.codes
    resid = x - cc[lst]
    _check_codes(oracle, resid, pq.codebooks, 8, 32, codes, metric, max_flip=0.002)


def test_build_search_float_parity(vh, oracle):
    # an end-to-end build of 20k vectors, searched against the oracle on the built parts
    rng = np.random.default_rng(22)
    n, dim = 20000, 64
    x = rng.uniform(-1, 1, (n, dim)).astype(np.float32)
    cfg = vh.IvfPqConfig.new(64, 8, 16).with_max_kmeans_iters(10)
    ix = vh.IvfPqIndex.build_with_config(x, cfg, vh.DistanceMetric.L2Squared)
    inv = ix.inverted_index()
    sizes, ids, codes = inv._csr()
    parts = (ix.coarse_centroids().reshape(-1, dim), ix.pq().codebooks, sizes, ids, codes)
    qs = rng.uniform(-1, 1, (40, dim)).astype(np.float32)
    _check_search(vh, oracle, ix, parts, qs, 10, 8, "l2", 16, 256, exact=False)
