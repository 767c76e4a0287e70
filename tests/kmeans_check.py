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
    assert abs(got["inertia"] - ref["inertia"]) <= 1e-4 * abs(ref["inertia"]) + 1e-3
    return len(flips)
