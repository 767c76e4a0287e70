"""Pins the oracle's product-quantization and IVF-PQ functions before they are trusted.

Reference known-answer tests (vector-index/src/ivf/pq.rs:349-427) are restated with
their inputs and expected values; everything else is checked against what the
mathematics fixes: brute-force argmin / sort in float64, integer-valued tables whose
sums are exact in any order, and a hand-derived IVF-PQ search result.  One check is
built so that a wrong summation order of compute_distance_with_lut fails it.
"""
import numpy as np
import pytest

import oracle as O


def test_adc_lut_kat():
    # pq.rs:349-386: two sub-spaces of dimension 2, two sub-centroids each
    cb = np.array([0, 0, 1, 1, 0, 0, 2, 2], np.float32)
    lut = O.pq_adc_lut([1, 1, 2, 2], cb, 2, 2, "l2")
    assert lut.tolist() == [2.0, 0.0, 8.0, 0.0]
    assert O.pq_distance_with_lut([1, 1], lut, 2) == 0.0
    assert O.pq_distance_with_lut([0, 0], lut, 2) == 10.0


def test_distance_with_lut_remainder_kat():
    # pq.rs:403-426: M = 5 (one quad + one remainder), sub-dimension 1
    cb = np.tile(np.array([0.0, 1.0], np.float32), 5)
    lut = O.pq_adc_lut(np.ones(5, np.float32), cb, 5, 2, "l2")
    assert abs(O.pq_distance_with_lut([1] * 5, lut, 2)) < 1e-5
    assert abs(O.pq_distance_with_lut([0] * 5, lut, 2) - 5.0) < 1e-5


def test_distance_with_lut_summation_order():
    # The reference adds each quad as (d0 + d1) + (d2 + d3).  In f32, 1e8 + 1 == 1e8, so
    # the pairwise order gives exactly 0 here while a left-to-right sum gives 1 and an
    # exact sum 2: a changed order fails this test.
    lut = np.array([1e8, 0, 1, 0, -1e8, 0, 1, 0], np.float32)  # M = 4, Ks = 2
    assert O.pq_distance_with_lut([0, 0, 0, 0], lut, 2) == 0.0
    seq = np.float32(0)
    for v in (np.float32(1e8), np.float32(1), np.float32(-1e8), np.float32(1)):
        seq = np.float32(seq + v)
    assert seq == 1.0  # the planted order really differs


@pytest.mark.parametrize("m_sub,ks", [(4, 16), (3, 7), (8, 256)])
def test_distance_with_lut_integer_tables_exact(m_sub, ks):
    rng = np.random.default_rng(5)
    lut = rng.integers(-1000, 1000, m_sub * ks).astype(np.float32)
    for _ in range(20):
        code = rng.integers(0, ks, m_sub).astype(np.uint8)
        want = sum(int(lut[m * ks + int(code[m])]) for m in range(m_sub))
        assert O.pq_distance_with_lut(code, lut, ks) == float(want)


def _brute_lut(q, cb, m_sub, ks, metric):
    ds = q.size // m_sub
    out = np.zeros(m_sub * ks)
    from tests.test_oracle import ref64  # closed forms in float64
    for m in range(m_sub):
        for j in range(ks):
            out[m * ks + j] = ref64(metric, q[m * ds:(m + 1) * ds], cb[(m * ks + j) * ds:(m * ks + j + 1) * ds])
    return out


@pytest.mark.parametrize("metric", ["l2", "dot", "cosine", "l1", "linf", "minkowski", "hamming", "mahalanobis",
                                    "jaccard", "hellinger"])
def test_adc_lut_matches_closed_forms(metric):
    rng = np.random.default_rng(7)
    m_sub, ks, ds = 4, 9, 5
    cb = rng.standard_normal(m_sub * ks * ds).astype(np.float32)
    q = rng.standard_normal(m_sub * ds).astype(np.float32)
    got = O.pq_adc_lut(q, cb, m_sub, ks, metric)
    want = _brute_lut(q, cb, m_sub, ks, metric)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("metric", ["l2", "l1", "linf", "dot"])
def test_encode_integer_data_exact(metric):
    # integer data and codebooks: every metric value is an exact integer, so the argmin is
    # fixed; ties (frequent with small integers) must go to the lowest index
    rng = np.random.default_rng(11)
    m_sub, ks, ds, n = 4, 12, 3, 300
    cb = rng.integers(-3, 4, m_sub * ks * ds).astype(np.float32)
    x = rng.integers(-3, 4, (n, m_sub * ds)).astype(np.float32)
    codes = O.pq_encode(x, cb, m_sub, ks, metric)
    hib = metric == "dot"
    for i in range(n):
        for m in range(m_sub):
            sub = x[i, m * ds:(m + 1) * ds].astype(np.int64)
            c = cb[m * ks * ds:(m + 1) * ks * ds].reshape(ks, ds).astype(np.int64)
            if metric == "l2":
                s = ((c - sub) ** 2).sum(1)
            elif metric == "l1":
                s = np.abs(c - sub).sum(1)
            elif metric == "linf":
                s = np.abs(c - sub).max(1)
            else:
                s = -(c * sub).sum(1)
            best = int(np.flatnonzero(s == s.min())[0])
            assert codes[i, m] == best, (i, m, s)
    del hib


def test_encode_random_cosine_is_argmax():
    rng = np.random.default_rng(3)
    m_sub, ks, ds, n = 2, 16, 6, 200
    cb = rng.standard_normal(m_sub * ks * ds).astype(np.float32)
    x = rng.standard_normal((n, m_sub * ds)).astype(np.float32)
    codes = O.pq_encode(x, cb, m_sub, ks, "cosine")
    for i in range(n):
        for m in range(m_sub):
            lut = _brute_lut(x[i, m * ds:(m + 1) * ds], cb[m * ks * ds:(m + 1) * ks * ds], 1, ks, "cosine")
            assert lut[codes[i, m]] >= lut.max() - 1e-6


@pytest.mark.parametrize("metric", ["l2", "dot", "l1"])
def test_find_top_centroids_sorted_with_index_ties(metric):
    rng = np.random.default_rng(2)
    cent = rng.integers(-2, 3, (40, 3)).astype(np.float32)  # many exact ties
    q = rng.integers(-2, 3, 3).astype(np.float32)
    idx, sc = O.find_top_centroids(q, cent, 17, metric)
    from tests.test_oracle import ref64
    s = np.array([ref64(metric, q, c) for c in cent])
    order = sorted(range(40), key=(lambda i: (-s[i], i)) if metric == "dot" else (lambda i: (s[i], i)))
    assert idx.tolist() == order[:17]
    np.testing.assert_array_equal(sc, s[order[:17]].astype(np.float32))
    assert O.find_top_centroids(q, cent, 0, metric)[0].size == 0
    assert O.find_top_centroids(q, cent, 100, metric)[0].size == 40


def _csr(assign, nlist):
    order = np.argsort(assign, kind="stable")
    off = np.zeros(nlist + 1, np.uint64)
    np.add.at(off, assign + 1, 1)
    return np.cumsum(off).astype(np.uint64), order.astype(np.uint32)


def test_ivfpq_search_hand_derived():
    # The serializer round-trip index (serializer.rs:438-480): coarse (0,0,0,0) and (1,1,1,1),
    # both sub-codebooks {(0,0), (0.5,0.5)}, list 0 = {id 10: code [0,1]}, list 1 = {id 20: [1,0]}.
    # Query 0: residual 0 in list 0 -> 0 + 0.5; residual -1 in list 1 -> 4.5 + 2.
    coarse = np.array([[0, 0, 0, 0], [1, 1, 1, 1]], np.float32)
    cb = np.array([0, 0, 0.5, 0.5, 0, 0, 0.5, 0.5], np.float32)
    off = np.array([0, 1, 2], np.uint64)
    ids = np.array([10, 20], np.uint32)
    codes = np.array([[0, 1], [1, 0]], np.uint8)
    q = np.zeros(4, np.float32)
    i, d = O.ivfpq_search(q, coarse, cb, 2, 2, off, ids, codes, [0, 1], 5, "l2")
    assert i.tolist() == [10, 20] and d.tolist() == [0.5, 6.5]
    i, d = O.ivfpq_search(q, coarse, cb, 2, 2, off, ids, codes, [1], 5, "l2")
    assert i.tolist() == [20] and d.tolist() == [6.5]
    i, d = O.ivfpq_search(q, coarse, cb, 2, 2, off, ids, codes, [0, 1], 1, "l2")
    assert i.tolist() == [10]
    assert O.ivfpq_search(q, coarse, cb, 2, 2, off, ids, codes, [0, 1], 0, "l2")[0].size == 0


@pytest.mark.parametrize("metric", ["l2", "dot"])
def test_ivfpq_search_brute_force_integer(metric):
    # integer coarse centroids, codebooks and queries: every table entry and every sum is an
    # exact integer, so the float64 brute force fixes the distances exactly
    rng = np.random.default_rng(9)
    dim, m_sub, ks, nlist, n, k = 8, 4, 8, 6, 400, 15
    coarse = rng.integers(-4, 5, (nlist, dim)).astype(np.float32)
    cb = rng.integers(-2, 3, m_sub * ks * (dim // m_sub)).astype(np.float32)
    assign = rng.integers(0, nlist, n)
    off, ids = _csr(assign, nlist)
    codes = rng.integers(0, ks, (n, m_sub)).astype(np.uint8)
    hib = metric == "dot"
    for t in range(5):
        q = rng.integers(-4, 5, dim).astype(np.float32)
        probes = rng.permutation(nlist)[:3].astype(np.uint32)
        gi, gd = O.ivfpq_search(q, coarse, cb, m_sub, ks, off, ids, codes[np.argsort(assign, kind="stable")],
                                probes, k, metric)
        cand = []
        for c in probes:
            lut = _brute_lut(q - coarse[c], cb, m_sub, ks, metric)
            for j in range(int(off[c]), int(off[c + 1])):
                v = int(ids[j])
                cand.append((sum(lut[m * ks + int(codes[v, m])] for m in range(m_sub)), v))
        cand.sort(key=lambda e: (-e[0] if hib else e[0], e[1]))
        want = [e[0] for e in cand[:k]]
        assert gd.tolist() == want
        kth = want[-1]
        dist_of = {v: s for s, v in cand}
        for v, s in zip(gi.tolist(), gd.tolist()):  # tie-aware ids
            assert dist_of[v] == s and ((s >= kth) if hib else (s <= kth))
