"""Parity helpers shared by the GPU tests (not collected by pytest).

Tie-aware recall: a returned id counts as correct when its reference distance is at
least as good as the reference's k-th distance (ties at the boundary may resolve to
different ids).  Reported distances must match the reference CPU engine's value for the
same (query, id) within the stated tolerance.
"""
import numpy as np


def check_knn(oracle, base, queries, ids, dist, k, metric, rtol=1e-4, atol=1e-6, min_recall=0.999, ref=None,
              oracle_metric=None):
    """Checks GPU (ids, dist) [nq, k] against the oracle.  Returns measured recall."""
    om = oracle_metric or metric
    if ref is None:
        ref = oracle.knn_search_batch(base, queries, k, om)
    rids, rdist, rlens = ref
    hib = om in ("dot", "cosine")
    nq = queries.shape[0]
    ok = 0
    total = 0
    for q in range(nq):
        kk = int(rlens[q])
        assert kk == min(k, base.shape[0])
        got = ids[q, :kk].astype(np.int64)
        assert len(set(got.tolist())) == kk, f"duplicate ids for query {q}"
        assert np.all(got < base.shape[0]), f"id out of range for query {q}"
        # reference values of the returned ids
        refv = oracle.distance_rows(om, np.repeat(queries[q:q + 1], kk, 0), base[got])
        kth = rdist[q, kk - 1]
        if hib:
            good = refv >= kth - (rtol * abs(kth) + atol)
        else:
            good = refv <= kth + (rtol * abs(kth) + atol)
        ok += int(good.sum())
        total += kk
        err = np.abs(dist[q, :kk] - refv)
        assert np.all(err <= rtol * np.abs(refv) + atol), (
            f"query {q}: distance mismatch max {err.max()} (ours {dist[q, :kk][np.argmax(err)]}, "
            f"ref {refv[np.argmax(err)]})")
        # best-first order
        d = dist[q, :kk]
        if hib:
            assert np.all(np.diff(d) <= rtol * np.abs(d[1:]) + atol), f"query {q} not sorted descending"
        else:
            assert np.all(np.diff(d) >= -(rtol * np.abs(d[1:]) + atol)), f"query {q} not sorted ascending"
        # distances as a multiset equal the reference's k best (tie-aware value check)
        rs = np.sort(rdist[q, :kk])
        os_ = np.sort(refv)
        assert np.all(np.abs(rs - os_) <= rtol * np.abs(rs) + atol + (0 if not hib else 0)), f"query {q} k-best values"
    recall = ok / max(total, 1)
    assert recall >= min_recall, f"tie-aware recall {recall} < {min_recall}"
    return recall
