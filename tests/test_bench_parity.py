"""CPU checks of the benchmark's parity checks (bench.knn_parity, bench.kmeans_parity,
bench.ivfpq_parity).

The oracle's own results pass; results with a planted mistake (a wrong neighbour, a perturbed
distance, a flipped assignment that is not a near-tie, a shifted centroid, an IVF-PQ id that does
not tie with the k-th) fail.
"""
import numpy as np

import bench


def _knn_case(oracle, metric, seed=0, n=3000, d=32, nq=40, k=10):
    rng = np.random.default_rng(seed)
    if metric == "hamming":
        base = rng.integers(0, 2**32, size=(n, 8), dtype=np.uint64).astype(np.uint32)
        q = rng.integers(0, 2**32, size=(nq, 8), dtype=np.uint64).astype(np.uint32)
        ref = oracle.hamming_packed_knn(base, q, k)
    else:
        base = rng.integers(0, 256, size=(n, d)).astype(np.float32)
        q = rng.integers(0, 256, size=(nq, d)).astype(np.float32)
        ref = oracle.knn_search_batch(base, q, k, metric)
    return base, q, (ref, np.arange(nq))


def test_parity_sample_takes_a_stride_and_the_last_queries():
    assert np.array_equal(bench.parity_sample(10_000, 20_000), np.arange(10_000))
    idx = bench.parity_sample(10_000, 1_000)
    assert np.all(np.isin(np.arange(10_000 - 128, 10_000), idx)) and idx[0] == 0
    assert 900 <= len(idx) <= 1_000 and np.all(np.diff(idx) > 0)
    assert len(set(np.diff(idx[idx < 10_000 - 128]).tolist())) == 1


def test_knn_parity_on_a_sample_checks_the_sampled_queries(oracle):
    """The reference holds the oracle's results of a strided sample with the last queries: the GPU
    rows of exactly those queries are compared, so a mistake in the last query is caught."""
    base, q, ((ids, dist, lens), _) = _knn_case(oracle, "l2", seed=4, nq=300)
    idx = bench.parity_sample(300, 160)
    ref = ((ids[idx].copy(), dist[idx].copy(), lens[idx].copy()), idx)
    r = bench.knn_parity(base, q, ids.copy(), dist.copy(), ref, 10, "l2", 0.0, 0.0)
    assert r["ok"] and r["last_query"] == 299 and r["last_tile_checked"], r
    bad = dist.copy()
    bad[299, 0] += 1.0
    assert not bench.knn_parity(base, q, ids.copy(), bad, ref, 10, "l2", 0.0, 0.0)["ok"]
    # the GPU rows must be those of the sampled queries, not the first len(idx) rows
    shifted = np.roll(ids, 1, axis=0)
    assert not bench.knn_parity(base, q, shifted, dist.copy(), ref, 10, "l2", 0.0, 0.0)["ok"]


def test_knn_parity_accepts_oracle_results(oracle):
    for metric in ("l2", "cosine", "l1"):
        base, q, ref = _knn_case(oracle, metric)
        r = bench.knn_parity(base, q, ref[0][0].copy(), ref[0][1].copy(), ref, 10, metric, 1e-4, 1e-6)
        assert r["ok"] and r["recall_tie_aware"] == 1.0, (metric, r)
    base, q, ref = _knn_case(oracle, "hamming")
    r = bench.knn_parity(base, q, ref[0][0].copy(), ref[0][1].copy(), ref, 10, "hamming", 0.0, 0.0, min_recall=1.0)
    assert r["ok"], r


def test_knn_parity_rejects_planted_mistakes(oracle):
    base, q, ref = _knn_case(oracle, "l2", seed=1)
    ids, dist = ref[0][0].copy(), ref[0][1].copy()
    # a far neighbour in place of a true one: recall drops below 1 (0.999 of 400 entries)
    far = int(np.argmax(((base - q[0]) ** 2).sum(1)))
    ids[0, 3] = far
    r = bench.knn_parity(base, q, ids, dist, ref, 10, "l2", 0.0, 0.0, min_recall=1.0)
    assert not r["ok"]
    ids, dist = ref[0][0].copy(), ref[0][1].copy()
    dist[5, 2] += 1.0  # a distance that is not the pair's value
    r = bench.knn_parity(base, q, ids, dist, ref, 10, "l2", 0.0, 0.0)
    assert not r["ok"] and not r["distances_ok"]
    ids, dist = ref[0][0].copy(), ref[0][1].copy()
    ids[7, 1] = ids[7, 0]  # a duplicated id
    r = bench.knn_parity(base, q, ids, dist, ref, 10, "l2", 0.0, 0.0)
    assert not r["ok"]
    base, q, ref = _knn_case(oracle, "hamming", seed=2)
    dist = ref[0][1].copy()
    dist[0, 0] += 1
    r = bench.knn_parity(base, q, ref[0][0].copy(), dist, ref, 10, "hamming", 0.0, 0.0, min_recall=1.0)
    assert not r["ok"]


def test_kmeans_parity(oracle):
    from vector_hip import datasets as ds

    data, _, _ = ds.gaussian_mixture(20_000, 16, 32, 3)
    cent = data[:32].copy()
    ref = oracle.kmeans_step(data, cent, "l2", threads=0)
    got = {"assign": ref["assign"].copy(), "centroids": ref["centroids"].copy(),
           "counts": np.bincount(ref["assign"], minlength=32), "inertia": ref["inertia"]}
    r = bench.kmeans_parity(data, cent, got, ref)
    assert r["ok"] and r["assignment_flips"] == 0, r
    # a flip that is not a near-tie: move a point to its farthest centroid
    bad = dict(got, assign=got["assign"].copy())
    p = 0
    bad["assign"][p] = int(np.argmax(((cent - data[p]) ** 2).sum(1)))
    bad["counts"] = np.bincount(bad["assign"], minlength=32)
    r = bench.kmeans_parity(data, cent, bad, ref)
    assert not r["ok"] and not r["flips_all_near_ties"]
    # a centroid moved by 1e-3 of its norm
    bad = dict(got, centroids=got["centroids"].copy())
    bad["centroids"][4] *= 1.001
    r = bench.kmeans_parity(data, cent, bad, ref)
    assert not r["ok"]


def _ivfpq_case(oracle, seed=3, nlist=6, m_sub=4, ks=16, dim=16, n=600, nq=12, k=5, nprobe=3):
    """A small IVF-PQ index from random parts, and the oracle's search of each query."""
    rng = np.random.default_rng(seed)
    coarse = rng.standard_normal((nlist, dim)).astype(np.float32)
    cb = rng.standard_normal(m_sub * ks * (dim // m_sub)).astype(np.float32)
    sizes = np.bincount(rng.integers(0, nlist, n), minlength=nlist)
    off = np.concatenate([[0], np.cumsum(sizes)]).astype(np.uint64)
    lids = rng.permutation(n).astype(np.uint32)
    codes = rng.integers(0, ks, (n, m_sub)).astype(np.uint8)
    q = rng.standard_normal((nq, dim)).astype(np.float32)
    probes, ref = [], []
    for i in range(nq):
        pr, _ = oracle.find_top_centroids(q[i], coarse, nprobe, "l2")
        ri, rd = oracle.ivfpq_search(q[i], coarse, cb, m_sub, ks, off, lids, codes, pr, k, "l2")
        probes.append(np.asarray(pr, np.uint32))
        ref.append((i, pr, ri, rd))
    ids = np.full((nq, k), 0xFFFFFFFF, np.uint32)
    dist = np.full((nq, k), np.nan, np.float32)
    for i, _, ri, rd in ref:
        ids[i, :len(ri)], dist[i, :len(rd)] = ri, rd
    return ids, dist, np.stack(probes), ref, k


def test_ivfpq_parity_accepts_oracle_results_and_rejects_mistakes(oracle):
    ids, dist, probes, ref, k = _ivfpq_case(oracle)
    r = bench.ivfpq_parity(ids, dist, probes, ref, k)
    assert r["ok"] and r["queries_checked"] == len(ref) and r["probe_ties_skipped"] == 0, r
    # a perturbed distance fails
    bad = dist.copy()
    bad[2, 1] += 0.5
    assert not bench.ivfpq_parity(ids, bad, probes, ref, k)["distances_ok"]
    # an id outside the oracle's k best that does not tie with the k-th fails
    bad_ids = ids.copy()
    others = set(range(600)) - set(ids[4].tolist())
    bad_ids[4, 0] = min(others)
    assert not bench.ivfpq_parity(bad_ids, dist, probes, ref, k)["ids_ok_up_to_ties"]
    # a query whose probes differ is skipped, not failed; too many skipped fails
    alt = probes.copy()
    alt[0] = (alt[0] + 1) % 6
    r = bench.ivfpq_parity(ids, dist, alt, ref, k)
    assert r["probe_ties_skipped"] == 1 and not r["ok"]
