"""Per-iteration k-means parity helper shared by the GPU tests (not collected by pytest).

One Lloyd step of the GPU state from centroids `cent` is checked against the oracle's step
from the same centroids: assignments may differ on at most max_flip_frac of the points and
only at near-ties; every centroid must be within 1e-4 (norm-relative) of the float64 mean of
the points the GPU assigned to it, and of the oracle's own f32 update wherever membership
agrees; empty clusters keep their centroid with shift 0; inertia within 1e-4 relative.
"""
import numpy as np


def check_step(oracle, data, cent, got, metric, max_flip_frac=1e-4):
    """got: GPU state after one iteration from `cent`."""
    ref = oracle.kmeans_step(data, cent, metric, threads=0)
    ga, ra = got["assign"], ref["assign"]
    flips = np.nonzero(ga != ra)[0]
    assert len(flips) <= max(1, int(max_flip_frac * len(data))), f"{len(flips)} assignment flips"
    for p in flips:  # only near-ties may flip
        dg = oracle.distance(metric, data[p], cent[ga[p]])
        dr = oracle.distance(metric, data[p], cent[ra[p]])
        assert abs(dg - dr) <= 1e-4 * max(1.0, abs(dr)), f"point {p}: {dg} vs {dr} is not a near-tie"
    k, d = cent.shape
    # update = mean of the assigned points (float64), empty clusters keep their centroid
    counts = np.bincount(ga, minlength=k)
    assert np.array_equal(counts, got["counts"])
    sums = np.zeros((k, d))
    np.add.at(sums, ga, data.astype(np.float64))
    for c in range(k):
        if counts[c] == 0:
            assert np.array_equal(got["centroids"][c], cent[c]) and got["shifts"][c] == 0
            continue
        want = sums[c] / counts[c]
        err = np.linalg.norm(got["centroids"][c] - want)
        assert err <= 1e-4 * max(np.linalg.norm(want), 1e-6), f"centroid {c} off by {err}"
    # and the oracle's own f32 update wherever membership agrees
    same = np.ones(k, bool)
    same[np.unique(np.concatenate([ga[flips], ra[flips]]))] = False
    for c in np.nonzero(same)[0]:
        want = ref["centroids"][c]
        assert np.linalg.norm(got["centroids"][c] - want) <= 1e-4 * max(np.linalg.norm(want), 1e-6)
    if metric in ("dot", "cosine"):
        # The GPU reports kmeans.cu:110-170's per-point values, -dot and 1 - cos (the oracle's
        # KMeans::fit step sums the similarities themselves): the sum over the GPU's own
        # assignment, in float64.
        x = data.astype(np.float64)
        c = cent.astype(np.float64)[ga]
        dots = np.einsum("ij,ij->i", x, c)
        if metric == "dot":
            want = -dots.sum()
        else:
            den = np.sqrt(np.einsum("ij,ij->i", x, x)) * np.sqrt(np.einsum("ij,ij->i", c, c))
            want = np.sum(1.0 - np.where(den > 1e-9, dots / np.where(den > 1e-9, den, 1.0), 0.0))
        assert abs(got["inertia"] - want) <= 1e-5 * abs(want) + 1e-3 * max(1.0, len(data) * 1e-4), \
            f"inertia {got['inertia']} against {want}"
    else:
        assert abs(got["inertia"] - ref["inertia"]) <= 1e-4 * abs(ref["inertia"]) + 1e-3
    return len(flips)


def check_chain(vh, oracle, data, init, iters, metric, fit_centroids, fit_assign, fit_inertia,
                max_flip_frac=1e-4):
    """A chained fit, pinned step by step: fit()'s centroids, assignment and inertia after `iters`
    iterations from `init` equal those of a GPU state stepped `iters` times from `init` (bit for
    bit: the same kernels in the same order), and every one of those steps passes check_step
    against the oracle's step from the GPU's previous centroids.  Returns the flips per step."""
    st = vh.KMeansState(data, metric=vh.DistanceMetric(oracle.METRICS[metric]))
    cent = np.array(init, np.float32)
    st.set_centroids(cent)
    flips = []
    for _ in range(iters):
        st.run(1)
        got = st.read()
        flips.append(check_step(oracle, data, cent, got, metric, max_flip_frac))
        cent = got["centroids"]
    assert np.array_equal(fit_centroids.reshape(cent.shape), cent)
    assert np.array_equal(fit_assign, got["assign"])
    assert fit_inertia == got["inertia"]
    return flips
