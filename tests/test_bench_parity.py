"""CPU checks of the benchmark's parity checks (bench.knn_parity, bench.kmeans_parity).

The oracle's own results pass; results with a planted mistake (a wrong neighbour, a perturbed
distance, a flipped assignment that is not a near-tie, a shifted centroid) fail.
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
    return base, q, ref


def test_knn_parity_accepts_oracle_results(oracle):
    for metric in ("l2", "cosine", "l1"):
        base, q, ref = _knn_case(oracle, metric)
        r = bench.knn_parity(base, q, ref[0].copy(), ref[1].copy(), ref, 10, metric, 1e-4, 1e-6)
        assert r["ok"] and r["recall_tie_aware"] == 1.0, (metric, r)
    base, q, ref = _knn_case(oracle, "hamming")
    r = bench.knn_parity(base, q, ref[0].copy(), ref[1].copy(), ref, 10, "hamming", 0.0, 0.0, min_recall=1.0)
    assert r["ok"], r


def test_knn_parity_rejects_planted_mistakes(oracle):
    base, q, ref = _knn_case(oracle, "l2", seed=1)
    ids, dist = ref[0].copy(), ref[1].copy()
    # a far neighbour in place of a true one: recall drops below 1 (0.999 of 400 entries)
    far = int(np.argmax(((base - q[0]) ** 2).sum(1)))
    ids[0, 3] = far
    r = bench.knn_parity(base, q, ids, dist, ref, 10, "l2", 0.0, 0.0, min_recall=1.0)
    assert not r["ok"]
    ids, dist = ref[0].copy(), ref[1].copy()
    dist[5, 2] += 1.0  # a distance that is not the pair's value
    r = bench.knn_parity(base, q, ids, dist, ref, 10, "l2", 0.0, 0.0)
    assert not r["ok"] and not r["distances_ok"]
    ids, dist = ref[0].copy(), ref[1].copy()
    ids[7, 1] = ids[7, 0]  # a duplicated id
    r = bench.knn_parity(base, q, ids, dist, ref, 10, "l2", 0.0, 0.0)
    assert not r["ok"]
    base, q, ref = _knn_case(oracle, "hamming", seed=2)
    dist = ref[1].copy()
    dist[0, 0] += 1
    r = bench.knn_parity(base, q, ref[0].copy(), dist, ref, 10, "hamming", 0.0, 0.0, min_recall=1.0)
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
