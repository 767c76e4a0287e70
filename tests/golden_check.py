"""Checks against the golden fixtures of tests/golden/ (helpers, not collected by pytest).

The fixtures hold float64 expected values computed from the metric definitions
(tests/golden/make_golden.py); both the CPU oracle and the HIP library are held to them.
"""
import hashlib
import importlib.util
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
ROOT = os.path.dirname(HERE)
HIGHER = {"dot", "cosine"}


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def datasets():
    path = os.path.join(ROOT, "vector-rs_amd", "vector_hip", "datasets.py")
    spec = importlib.util.spec_from_file_location("vh_datasets_golden", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def dist64(metric, q, X):
    import importlib.util as iu

    spec = iu.spec_from_file_location("vh_make_golden", os.path.join(GOLDEN, "make_golden.py"))
    mod = iu.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.dist64(metric, q.astype(np.float64), X.astype(np.float64))


def check_topk(metric, base, queries, ids, dist, exp_ids, exp_dist, exp_kth, rtol=1e-4, atol=1e-5):
    """ids/dist: [nq, k] results under test.  Distances must match the float64 values within
    rtol/atol; ids must be exact up to ties at the k-th distance (tie-aware: every returned id's
    float64 distance is within tolerance of the expected k-th or better), with no duplicates."""
    nq, k = exp_ids.shape
    assert ids.shape[0] == nq and ids.shape[1] >= k
    hib = metric in HIGHER
    for q in range(nq):
        got = ids[q, :k].astype(np.int64)
        assert len(set(got.tolist())) == k, f"query {q}: duplicate ids"
        tol = rtol * abs(exp_kth[q]) + atol
        d64 = dist64(metric, queries[q], base[got])
        ok = d64 >= exp_kth[q] - tol if hib else d64 <= exp_kth[q] + tol
        assert ok.all(), f"query {q}: ids {got[~ok]} are not among the true top-{k}"
        # values: sorted multiset equality with the exact top-k
        a = np.sort(np.asarray(dist[q, :k], np.float64))
        b = np.sort(exp_dist[q])
        assert np.all(np.abs(a - b) <= rtol * np.abs(b) + atol), (
            f"query {q}: distances {a} vs expected {b}")
        # order: best first
        d = np.asarray(dist[q, :k], np.float64)
        step = np.diff(d)
        assert np.all(step <= atol + rtol * np.abs(d[1:])) if hib else np.all(step >= -(atol + rtol * np.abs(d[1:])))
        # exact id agreement where the k-th distance has no tie within tolerance
        full = dist64(metric, queries[q], base)
        tied = np.abs(full - exp_kth[q]) <= tol
        if tied.sum() == 1:
            assert set(got.tolist()) == set(exp_ids[q].tolist()), f"query {q}: untied top-{k} differs"


def c1_inputs():
    ds = datasets()
    f = load("c1_l2_gauss_10000x128_q100_k10.npz")
    base = ds.gaussian(10_000, 128, int(f["base_seed"]))
    q = ds.gaussian(100, 128, int(f["query_seed"]))
    assert sha(base) == str(f["base_sha256"]) and sha(q) == str(f["queries_sha256"]), "generator drifted"
    return base, q, f


def kmeans_inputs():
    ds = datasets()
    f = load("kmeans_mixture.npz")
    X, _, _ = ds.gaussian_mixture(3000, 16, 12, 7, centre_sigma=3.0)
    assert sha(X) == str(f["data_sha256"]), "generator drifted"
    return X, X[:12].copy(), f


def check_kmeans(it, assign, centroids, f, X, max_flip_frac=1e-4):
    """After `it` Lloyd iterations from the fixture's init: assignments may differ only on
    near-ties (best-vs-second gap within an fp32 rounding bound), and every centroid must be
    within 1e-4 of the float64 one relative to its norm."""
    exp_a = f["assign"][it - 1].astype(np.int64)
    gap = f["gap"][it - 1].astype(np.float64)
    diff = np.nonzero(np.asarray(assign, np.int64) != exp_a)[0]
    scale = np.mean(np.sum(X.astype(np.float64) ** 2, 1))
    assert len(diff) <= max(0, int(max_flip_frac * len(exp_a))), f"{len(diff)} assignment flips"
    assert np.all(gap[diff] <= 1e-5 * scale), "an assignment flipped on a non-tie"
    exp_c = f["centroids"][it - 1]
    err = np.linalg.norm(np.asarray(centroids, np.float64) - exp_c, axis=1)
    nrm = np.maximum(np.linalg.norm(exp_c, axis=1), 1e-12)
    assert np.all(err <= 1e-4 * nrm), f"centroid error {np.max(err / nrm)}"
