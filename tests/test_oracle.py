"""Pins the CPU oracle before the GPU results are checked against it.

Every oracle function is checked against (a) the reference's own known-answer
tests, restated with their inputs and expected values, and (b) what the
mathematics fixes: closed forms evaluated in float64 by numpy, brute-force
sorted top-k, exact integer identities.  The checks are chosen so that a
plausible slip (dropped term, wrong sign, swapped operand, off-by-one tail)
fails at least one of them; ``test_checks_catch_planted_mistakes`` verifies
that for a few planted slips.
"""
import math

import numpy as np
import pytest

BACKENDS = [0, 1, 2]  # scalar, AVX2+FMA, AVX-512F


def _backends(oracle):
    best = oracle.detect_backend()
    return [b for b in BACKENDS if b <= best]


# ---- closed forms in float64 (the mathematics, not the oracle's code) -------
def ref64(metric, a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    if metric == "l2":
        return float(np.sum((a - b) ** 2))
    if metric == "dot":
        return float(np.dot(a, b))
    if metric == "cosine":
        den = math.sqrt(np.dot(a, a)) * math.sqrt(np.dot(b, b))
        return 0.0 if den <= 1e-9 else float(np.dot(a, b) / den)
    if metric == "l1":
        return float(np.sum(np.abs(a - b)))
    if metric == "minkowski":
        return float(np.sum(np.abs(a - b) ** 3) ** (1.0 / 3.0))
    if metric == "linf":
        return float(np.max(np.abs(a - b))) if a.size else 0.0
    if metric == "hamming":
        return float(np.sum(np.abs(a.astype(np.float32) - b.astype(np.float32)) > np.float32(1e-6)))
    if metric == "mahalanobis":
        return math.sqrt(float(np.sum((a - b) ** 2)))
    if metric == "jaccard":
        mn = np.sum(np.minimum(np.abs(a), np.abs(b)))
        mx = np.sum(np.maximum(np.abs(a), np.abs(b)))
        return 0.0 if mx <= 1e-9 else float(1.0 - mn / mx)
    if metric == "hellinger":
        return math.sqrt(0.5 * float(np.sum((np.sqrt(np.abs(a)) - np.sqrt(np.abs(b))) ** 2)))
    raise KeyError(metric)


# ---- scalar.rs:271-362 known-answer tests, on every backend -----------------
KATS = [
    ("dot", [1, 2, 3], [4, 5, 6], 32.0),                       # scalar.rs:272-277
    ("l2", [1, 2, 3], [4, 6, 3], 25.0),                        # scalar.rs:280-285
    ("cosine", [1, 2, 3], [1, 2, 3], 1.0),                     # scalar.rs:288-290
    ("cosine", [0, 0], [1, 2], 0.0),                           # scalar.rs:291 (zero norm)
    ("l1", [1, 5, 2], [4, 1, 6], 11.0),                        # scalar.rs:295-298
    ("l1", [1, 5, 2], [1, 5, 2], 0.0),                         # scalar.rs:299
    ("minkowski", [1, 2, 3], [4, 2, 7], (27.0 + 64.0) ** (1 / 3)),  # scalar.rs:303-308
    ("linf", [1, 10, 3], [5, 2, 4], 8.0),                      # scalar.rs:316-319
    ("hamming", [1, 2, 3, 4], [1, 9, 3, 8], 2.0),              # scalar.rs:324-327
    ("hamming", [1, 2, 3, 4], [1, 2, 3, 4], 0.0),              # scalar.rs:328
    ("mahalanobis", [0, 0], [3, 4], 5.0),                      # scalar.rs:332-336
    ("jaccard", [1, 2, 0], [1, 0, 0], 2.0 / 3.0),              # scalar.rs:350-353
    ("jaccard", [1, 2, 0], [1, 2, 0], 0.0),                    # scalar.rs:354
    ("hellinger", [0.25, 0.25], [0.25, 0.25], 0.0),            # scalar.rs:358-361
]


@pytest.mark.parametrize("metric,a,b,want", KATS)
def test_reference_kats(oracle, metric, a, b, want):
    for be in _backends(oracle):
        got = oracle.distance(metric, np.array(a, np.float32), np.array(b, np.float32), backend=be)
        assert abs(got - want) < 1e-5, (metric, be, got, want)


def test_engine_matches_scalar_lib_rs(oracle):
    """vector-simd lib.rs:335-438: dispatched engine vs scalar within 1e-4."""
    cases = [
        ("dot", np.arange(1, 9), np.arange(8, 0, -1)),
        ("l2", np.arange(1, 9), np.arange(8, 0, -1)),
        ("cosine", np.arange(1, 33), np.arange(1, 33) * 2.0),
        ("l1", [1, 2, 3, 4], [4, 3, 2, 1]),
        ("linf", [1, 10, 3, 4], [4, 2, 2, 1]),
        ("jaccard", [1, 2, 0, 4], [1, 0, 0, 2]),
        ("hellinger", [0.5, 0.5], [0.5, 0.5]),
        ("mahalanobis", [1, 2], [4, 6]),
    ]
    for m, a, b in cases:
        a = np.asarray(a, np.float32)
        b = np.asarray(b, np.float32)
        s = oracle.distance(m, a, b, backend=0)
        for be in _backends(oracle):
            assert abs(oracle.distance(m, a, b, backend=be) - s) < 1e-4, (m, be)
    # lib.rs:421-437 (1536-d, relative 1e-3)
    i = np.arange(1536)
    a = (((i * 7 + 3) % 100) * 0.01).astype(np.float32)
    b = (((i * 13 + 5) % 100) * 0.01).astype(np.float32)
    for m in ("dot", "l1"):
        s = oracle.distance(m, a, b, backend=0)
        for be in _backends(oracle):
            assert abs(oracle.distance(m, a, b, backend=be) - s) / abs(s) < 1e-3


@pytest.mark.parametrize("dim", [1, 7, 8, 15, 16, 31, 32, 63, 64, 96, 128, 768])
def test_simd_sweep_vs_float64(oracle, dim):
    """avx512.rs:624-677 sweep (same inputs), checked against float64 closed forms
    and scalar; every tail length of every backend is exercised."""
    i = np.arange(dim)
    a = (((i * 7 + 3) % 100) * 0.1).astype(np.float32)
    b = (((i * 13 + 5) % 100) * 0.1).astype(np.float32)
    for m in oracle.METRICS:
        want = ref64(m, a, b)
        for be in _backends(oracle):
            got = oracle.distance(m, a, b, backend=be)
            tol = 1e-4 if m in ("linf", "hamming", "jaccard") else 1e-3 * max(1.0, abs(want))
            assert abs(got - want) <= tol, (m, dim, be, got, want)


def test_random_vs_float64(oracle):
    rng = np.random.default_rng(7)
    for dim in (3, 17, 100, 129):
        for _ in range(5):
            a = rng.standard_normal(dim).astype(np.float32)
            b = rng.standard_normal(dim).astype(np.float32)
            for m in oracle.METRICS:
                want = ref64(m, a, b)
                for be in _backends(oracle):
                    got = oracle.distance(m, a, b, backend=be)
                    assert abs(got - want) <= 1e-4 * max(1.0, abs(want)), (m, dim, be)


def test_l2_integer_data_is_exact(oracle):
    """C2-style data: integers in [0,255], D=128 -- every partial sum is an integer
    < 2^24, so the f32 result equals the int64 result bit for bit."""
    rng = np.random.default_rng(3)
    a = rng.integers(0, 256, (64, 128)).astype(np.float32)
    b = rng.integers(0, 256, (64, 128)).astype(np.float32)
    exact = ((a.astype(np.int64) - b.astype(np.int64)) ** 2).sum(1)
    for be in _backends(oracle):
        got = oracle.distance_rows("l2", a, b, backend=be)
        assert np.array_equal(got.astype(np.int64), exact)


# ---- top-k: flat.rs, knn.rs, collective.rs known answers -------------------
def _storage_3d():
    return np.array([[1, 0, 0], [0, 1, 0], [0, 0, 1], [1, 1, 0], [1, 1, 1]], np.float32)


def test_flat_kats(oracle):
    s = _storage_3d()
    ids, d = oracle.flat_search(s, [1, 0, 0], 3, "l2")                 # flat.rs:380-391
    assert len(ids) == 3 and ids[0] == 0 and abs(d[0]) < 1e-5 and ids[1] == 3 and abs(d[1] - 1) < 1e-5
    ids, d = oracle.flat_search(s, [0, 0, 1], 1, "l2")                 # flat.rs:394-400
    assert list(ids) == [2] and abs(d[0]) < 1e-5
    assert len(oracle.flat_search(s, [0, 0, 0], 100, "l2")[0]) == 5    # flat.rs:403-407
    assert len(oracle.flat_search(s, [0, 0, 0], 0, "l2")[0]) == 0      # flat.rs:410-414
    ids, d = oracle.flat_search(s, [1, 1, 1], 2, "dot")                # flat.rs:435-441
    assert ids[0] == 4 and abs(d[0] - 3.0) < 1e-5
    ids, d = oracle.flat_search(s, [1, 0, 0], 1, "cosine")             # flat.rs:462-467
    assert ids[0] == 0 and abs(d[0] - 1.0) < 1e-5
    for m, q in (("l2", [0.5, 0.5, 0.5]), ("dot", [1, 1, 1]), ("cosine", [1, 0.5, 0])):
        _, d = oracle.flat_search(s, q, 5, m)                          # flat.rs:417-481
        if m == "l2":
            assert np.all(np.diff(d) >= -1e-5)
        else:
            assert np.all(np.diff(d) <= 1e-5)
    with pytest.raises(ValueError):
        oracle.flat_search(np.zeros((0, 3), np.float32), [1, 2, 3], 5)  # flat.rs:488-493


def test_flat_high_dim_accuracy(oracle):
    """flat.rs:573-613 and :616-655 inputs, checked against float64."""
    dim, n = 768, 100
    i = np.arange(n)[:, None]
    d = np.arange(dim)[None, :]
    base = (((i * 7 + d * 13 + 3) % 97) * 0.01).astype(np.float32)
    q = (((np.arange(dim) * 11 + 5) % 89) * 0.01).astype(np.float32)
    ids, dist = oracle.flat_search(base, q, 10, "l2")
    for r, v in zip(ids, dist):
        want = ref64("l2", q, base[r])
        assert abs(v - want) / want < 1e-3
    dim, n = 1536, 50
    i = np.arange(n)[:, None]
    d = np.arange(dim)[None, :]
    base = (((i * 3 + d * 17 + 7) % 101) * 0.01).astype(np.float32)
    q = (((np.arange(dim) * 19 + 11) % 83) * 0.01).astype(np.float32)
    ids, dist = oracle.flat_search(base, q, 5, "cosine")
    assert np.all(np.diff(dist) <= 1e-5)
    for r, v in zip(ids, dist):
        assert abs(v - ref64("cosine", q, base[r])) < 1e-3


def _knn_rs_data(n=50):
    i = np.arange(n, dtype=np.float32)
    return np.stack([i * i * 0.1, i * 2.0, i + 5.0, i * 3.0], 1).astype(np.float32)


def test_knn_cpu_batch_kats(oracle):
    data = _knn_rs_data()
    ids, d, _ = oracle.knn_search_batch(data, data[10:11], 5, "l2")    # knn.rs:410-441
    fids, fd = oracle.flat_search(data, data[10], 5, "l2")
    assert list(ids[0]) == list(fids) and np.all(np.abs(d[0] - fd) < 1e-4)
    data = np.array([[0, 0], [1, 1], [2, 2]], np.float32)
    ids, _, _ = oracle.knn_search_batch(data, np.array([[0.1, 0.1], [1.9, 1.9]], np.float32), 1)  # :444-455
    assert ids[0, 0] == 0 and ids[1, 0] == 2
    ids, _, lens = oracle.knn_search_batch(data, np.array([[0.5, 0.5]], np.float32), 100)         # :475-482
    assert lens[0] == 3
    data = np.array([[1, 0], [0, 1], [-1, 0]], np.float32)
    ids, _, _ = oracle.knn_search_batch(data, np.array([[0.95, 0.05]], np.float32), 3, "cosine")  # :485-499
    assert ids[0, 0] == 0 and ids[0, 2] == 2
    data = np.array([[1, 1], [2, 2], [3, 3]], np.float32)
    ids, _, _ = oracle.knn_search_batch(data, np.array([[2, 3]], np.float32), 2, "dot")          # :502-516
    assert list(ids[0]) == [2, 1]
    data = np.array([[10, 20], [30, 40], [50, 60]], np.float32)
    ids, d, _ = oracle.knn_search_batch(data, data, 1)                                           # :531-542
    assert list(ids[:, 0]) == [0, 1, 2] and np.all(np.abs(d) < 1e-4)


def test_top_k_reduce_kats(oracle):
    ids, _ = oracle.top_k_reduce([([0, 1], [1.0, 5.0]), ([10, 11], [0.5, 4.0])], 2, "l2")      # collective.rs:239-247
    assert list(ids) == [10, 0]
    assert len(oracle.top_k_reduce([], 5)[0]) == 0                                                # :250-252
    assert len(oracle.top_k_reduce([([0], [1.0])], 0)[0]) == 0                                    # :254-256
    ids, _ = oracle.top_k_reduce([([0, 1], [0.85, 0.40]), ([2, 3], [0.95, 0.70])], 3, "cosine")  # :260-271
    assert list(ids) == [2, 0, 3]
    ids, _ = oracle.top_k_reduce([([0], [2.0]), ([1], [1.0])], 10, "l2")                         # :274-282
    assert list(ids) == [1, 0]


def _brute_topk(base, queries, k, metric):
    """Sorted brute force in float64 with (distance, id) order."""
    out = []
    for q in queries:
        d = np.array([ref64(metric, q, x) for x in base])
        s = -d if metric in ("dot", "cosine") else d
        order = np.lexsort((np.arange(len(d)), s))[:k]
        out.append((order, d[order]))
    return out


@pytest.mark.parametrize("metric", ["l2", "dot", "cosine", "l1", "linf", "minkowski", "jaccard", "hellinger",
                                    "mahalanobis"])
def test_knn_batch_vs_sorted_brute_force(oracle, metric):
    rng = np.random.default_rng(11)
    base = rng.standard_normal((300, 19)).astype(np.float32)
    qs = rng.standard_normal((8, 19)).astype(np.float32)
    ids, dist, lens = oracle.knn_search_batch(base, qs, 7, metric)
    for qi, (bi, bd) in enumerate(_brute_topk(base, qs, 7, metric)):
        assert lens[qi] == 7
        assert list(ids[qi]) == list(bi), (metric, qi)
        assert np.allclose(dist[qi], bd, rtol=1e-4, atol=1e-5)


def test_knn_ties_keep_first_seen(oracle):
    """Reference tie rule (strict `<` eviction, knn.rs:357-366): with all
    distances equal, the k first-seen (lowest) ids survive."""
    base = np.ones((20, 4), np.float32)
    ids, _, _ = oracle.knn_search_batch(base, np.zeros((1, 4), np.float32), 5)
    assert sorted(ids[0]) == [0, 1, 2, 3, 4]


# ---- k-means ----------------------------------------------------------------
def test_kmeans_kats(oracle):
    data = np.array([[1, 2, 3, 4], [1.1, 2.1, 3.1, 4.1]], np.float32)             # ivf/kmeans.rs:386-395
    r = oracle.kmeans_fit(data, data[:1], 10, 1e-4)
    assert abs(r["centroids"][0, 0] - 1.05) < 1e-3 and abs(r["centroids"][0, 1] - 2.05) < 1e-3
    data = np.array([[1, 1], [3, 3], [5, 5], [7, 7]], np.float32)                  # distributed_kmeans.rs:597-606
    r = oracle.kmeans_fit(data, data[2:3], 10, 1e-5)
    assert np.all(np.abs(r["centroids"][0] - 4.0) < 1e-3)
    data = np.array([[0, 0.1], [0.1, 0], [-0.1, 0], [10, 10.1], [10.1, 10], [9.9, 10]], np.float32)  # :398-417
    r = oracle.kmeans_fit(data, data[[0, 3]], 20, 1e-5)
    c = r["centroids"]
    near0, near10 = (c[0], c[1]) if c[0, 0] < 5 else (c[1], c[0])
    assert np.all(np.abs(near0) < 0.5) and np.all(np.abs(near10 - 10) < 0.5)


def test_kmeans_step_vs_float64(oracle):
    """Assignment = argmin in float64 with lowest-index tie-break; update = per-cluster
    mean in float64; empty cluster keeps its centroid (shift 0)."""
    rng = np.random.default_rng(5)
    data = rng.standard_normal((2000, 12)).astype(np.float32)
    cent = rng.standard_normal((16, 12)).astype(np.float32)
    cent[15] = 100.0  # far away: stays empty
    r = oracle.kmeans_step(data, cent)
    d64 = ((data[:, None, :].astype(np.float64) - cent[None].astype(np.float64)) ** 2).sum(-1)
    a64 = np.argmin(d64, 1)
    gap = np.sort(d64, 1)[:, 1] - np.sort(d64, 1)[:, 0]
    flips = (a64 != r["assign"])
    assert np.all(gap[flips] < 1e-3)
    for c in range(16):
        m = r["assign"] == c
        assert r["counts"][c] == m.sum()
        if m.sum():
            want = data[m].astype(np.float64).mean(0)
            assert np.linalg.norm(r["centroids"][c] - want) <= 1e-5 * max(1.0, np.linalg.norm(want))
        else:
            assert np.array_equal(r["centroids"][c], cent[c]) and r["shifts"][c] == 0.0
    inertia = d64[np.arange(len(data)), r["assign"]].sum()
    assert abs(r["inertia"] - inertia) / inertia < 1e-4


def test_kmeans_parallel_equals_sequential_assign(oracle):
    rng = np.random.default_rng(9)
    data = rng.standard_normal((3000, 8)).astype(np.float32)
    cent = data[:10].copy()
    a = oracle.kmeans_step(data, cent, threads=1)
    b = oracle.kmeans_step(data, cent, threads=4)
    assert np.array_equal(a["assign"], b["assign"])
    assert np.allclose(a["centroids"], b["centroids"], rtol=1e-5, atol=1e-6)


# ---- packed Hamming -----------------------------------------------------------
def test_hamming_packed_identity(oracle):
    """popcount(a xor b) == reference float-Hamming (scalar.rs:143-153) over the
    codes unpacked to 0.0/1.0 floats, on every backend."""
    rng = np.random.default_rng(2)
    codes = rng.integers(0, 1 << 32, (64, 8), dtype=np.uint64).astype(np.uint32)
    un = oracle.unpack_bits(codes)
    assert un.shape == (64, 256)
    # unpack is bit j of word w -> element 32w + j
    assert un[0, 5] == float((codes[0, 0] >> 5) & 1) and un[0, 32 + 7] == float((codes[0, 1] >> 7) & 1)
    for i in range(1, 64):
        want = sum(bin(int(x) ^ int(y)).count("1") for x, y in zip(codes[0], codes[i]))
        assert oracle.hamming_packed(codes[0], codes[i]) == want
        for be in _backends(oracle):
            assert oracle.distance("hamming", un[0], un[i], backend=be) == float(want)


def test_hamming_packed_knn_vs_brute_force(oracle):
    rng = np.random.default_rng(4)
    codes = rng.integers(0, 1 << 32, (500, 2), dtype=np.uint64).astype(np.uint32)
    qs = rng.integers(0, 1 << 32, (6, 2), dtype=np.uint64).astype(np.uint32)
    ids, dist, _ = oracle.hamming_packed_knn(codes, qs, 9)
    for qi in range(6):
        d = np.array([bin(int(a) ^ int(b)).count("1") + bin(int(c) ^ int(e)).count("1")
                      for (a, c), (b, e) in zip([qs[qi]] * 500, codes)])
        order = np.lexsort((np.arange(500), d))[:9]
        assert list(ids[qi]) == list(order) and list(dist[qi]) == list(d[order])


# ---- the checks above are discriminative -----------------------------------
def test_checks_catch_planted_mistakes(oracle):
    """Plants typical slips in a copy of the oracle's arithmetic (on the CPU) and
    confirms the same checks reject them."""
    a = np.array([1, 2, 3], np.float32)
    b = np.array([4, 6, 3], np.float32)
    wrong_sign = float(np.sum(a * a) + np.sum(b * b) + 2 * np.dot(a, b))   # + instead of -
    assert abs(wrong_sign - 25.0) > 1e-3
    dropped = float(np.sum(a * a) - 2 * np.dot(a, b))                      # dropped ||b||^2
    assert abs(dropped - 25.0) > 1e-3
    tail = np.arange(17, dtype=np.float32)                                 # last tail element dropped
    assert abs(float(np.sum(np.abs(tail[:16] - 0))) - ref64("l1", tail, np.zeros(17))) > 1e-3
    # swapped tie-break (highest id first) is caught by the tie test's expectation
    base = np.ones((20, 4), np.float32)
    ids, _, _ = oracle.knn_search_batch(base, np.zeros((1, 4), np.float32), 5)
    assert sorted(ids[0]) != [15, 16, 17, 18, 19]
