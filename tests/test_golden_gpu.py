"""The HIP library (through the C ABI) against the golden fixtures."""
import numpy as np
import pytest

import golden_check as gc

pytestmark = pytest.mark.gpu
METRICS = ["l2", "dot", "cosine", "l1", "minkowski", "linf", "hamming", "mahalanobis", "jaccard", "hellinger"]
CODES = {m: i for i, m in enumerate(METRICS)}


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    assert vector_hip.CudaDeviceContext.device_count() >= 1, "no gfx950 GPU visible"
    return vector_hip


def test_c1_gauss_10k_x128_top10(vh):
    base, q, f = gc.c1_inputs()
    ids, dist, lens = vh.CudaKnnEngine(base, 128).search_batch_arrays(q, 10)
    assert np.all(lens == 10)
    gc.check_topk("l2", base, q, ids, dist, f["ids"], f["dist"], f["kth"])


@pytest.mark.parametrize("metric", METRICS)
def test_tiny_all_metrics(vh, metric):
    f = gc.load("metrics_tiny.npz")
    eng = vh.CudaKnnEngine(f["base"], 37, vh.DistanceMetric(CODES[metric]))
    ids, dist, _ = eng.search_batch_arrays(f["queries"], 7)
    gc.check_topk(metric, f["base"], f["queries"], ids, dist, f[f"{metric}_ids"], f[f"{metric}_dist"],
                  f[f"{metric}_kth"])


def test_reference_inline_datasets(vh):
    f = gc.load("reference_inline.npz")
    r = vh.CudaKnnEngine(f["knn_rs"], 4).search(f["knn_rs"][10], 5)
    assert [x.id for x in r] == list(f["knn_rs_ids"][0])
    assert np.allclose([x.distance for x in r], f["knn_rs_dist"][0], rtol=1e-5, atol=1e-4)
    for metric, key in (("l2", "flat_l2"), ("cosine", "flat_cos")):
        eng = vh.CudaKnnEngine(f["flat_rs"], 64, vh.DistanceMetric(CODES[metric]))
        ids, dist, _ = eng.search_batch_arrays(f["flat_rs_queries"], 10)
        exp = f[f"{key}_dist"]
        gc.check_topk(metric, f["flat_rs"], f["flat_rs_queries"], ids, dist, f[f"{key}_ids"], exp, exp[:, -1])


@pytest.mark.parametrize("iters", [1, 3, 6])
def test_kmeans_mixture(vh, iters):
    X, init, f = gc.kmeans_inputs()
    st = vh.KMeansState(X)
    st.set_centroids(init)
    st.run(iters)
    out = st.read()
    gc.check_kmeans(iters, out["assign"], out["centroids"], f, X)


def test_hamming_packed(vh):
    f = gc.load("hamming_packed.npz")
    ids, dist, _ = vh.HammingKnnEngine(f["codes"]).search_batch_arrays(f["queries"], 10)
    assert np.array_equal(dist, f["dist"])
    for q in range(f["ids"].shape[0]):
        kth = f["dist"][q, -1]
        strict = set(f["ids"][q][f["dist"][q] < kth].tolist())
        assert strict <= set(ids[q].tolist())
