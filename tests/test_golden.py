"""The CPU oracle against the golden fixtures (float64 expected values independent of it)."""
import numpy as np
import pytest

import golden_check as gc

METRICS = ["l2", "dot", "cosine", "l1", "minkowski", "linf", "hamming", "mahalanobis", "jaccard", "hellinger"]


def test_c1_gauss_10k_x128_top10(oracle):
    base, q, f = gc.c1_inputs()
    ids, dist, lens = oracle.knn_search_batch(base, q, 10, "l2")
    assert np.all(lens == 10)
    gc.check_topk("l2", base, q, ids, dist, f["ids"], f["dist"], f["kth"])


@pytest.mark.parametrize("metric", METRICS)
def test_tiny_all_metrics(oracle, metric):
    f = gc.load("metrics_tiny.npz")
    ids, dist, _ = oracle.knn_search_batch(f["base"], f["queries"], 7, metric)
    gc.check_topk(metric, f["base"], f["queries"], ids, dist, f[f"{metric}_ids"], f[f"{metric}_dist"],
                  f[f"{metric}_kth"])


def test_reference_inline_datasets(oracle):
    f = gc.load("reference_inline.npz")
    ids, dist = oracle.flat_search(f["knn_rs"], f["knn_rs"][10], 5, "l2")
    assert list(ids) == list(f["knn_rs_ids"][0])
    assert np.allclose(dist, f["knn_rs_dist"][0], rtol=1e-5, atol=1e-4)
    for metric, key in (("l2", "flat_l2"), ("cosine", "flat_cos")):
        ids, dist, _ = oracle.knn_search_batch(f["flat_rs"], f["flat_rs_queries"], 10, metric)
        exp = f[f"{key}_dist"]
        gc.check_topk(metric, f["flat_rs"], f["flat_rs_queries"], ids, dist, f[f"{key}_ids"], exp,
                      exp[:, -1])


@pytest.mark.parametrize("iters", [1, 3, 6])
def test_kmeans_mixture(oracle, iters):
    X, init, f = gc.kmeans_inputs()
    r = oracle.kmeans_fit(X, init, iters, -1.0, "l2", threads=4)
    assert r["iterations"] == iters
    gc.check_kmeans(iters, r["assign"], r["centroids"], f, X)


def test_hamming_packed(oracle):
    f = gc.load("hamming_packed.npz")
    ids, dist, _ = oracle.hamming_packed_knn(f["codes"], f["queries"], 10)
    assert np.array_equal(dist, f["dist"])
    for q in range(f["ids"].shape[0]):
        # ids equal up to ties at the 10th distance
        kth = f["dist"][q, -1]
        strict = set(f["ids"][q][f["dist"][q] < kth].tolist())
        assert strict <= set(ids[q].tolist())


def test_fixture_checks_reject_planted_mistakes(oracle):
    """The same checks fail on results with a planted slip (done on the CPU)."""
    base, q, f = gc.c1_inputs()
    ids, dist, _ = oracle.knn_search_batch(base, q, 10, "l2")
    bad = ids.copy()
    bad[0, 3] = (bad[0, 3] + 1) % base.shape[0]   # a wrong neighbour
    with pytest.raises(AssertionError):
        gc.check_topk("l2", base, q, bad, dist, f["ids"], f["dist"], f["kth"])
    with pytest.raises(AssertionError):            # distances off by a dropped term
        gc.check_topk("l2", base, q, ids, dist - 0.5, f["ids"], f["dist"], f["kth"])
    X, init, fk = gc.kmeans_inputs()
    r = oracle.kmeans_fit(X, init, 3, -1.0, "l2", threads=4)
    with pytest.raises(AssertionError):
        gc.check_kmeans(3, r["assign"], r["centroids"] * 1.001, fk, X)
