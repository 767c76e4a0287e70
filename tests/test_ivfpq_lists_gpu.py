"""GPU tests of the list-major IVF-PQ scan (16-byte code rows, 256 sub-centroids, k <= 48).

The list-major search groups the (query, probe) pairs by list and scores each list's codes once
per batch of the queries probing it; the query-major kernel (forced with VHIP_IVFPQ_SCAN=query)
scores them once per probing query.  Both keep the k best (score, id) keys with the same tables
and the same summation order, so their ids and distances must be equal bit for bit.  Shapes
cover skewed and empty lists, lists longer than many ring chunks, more work items than
workgroups, partial items, k from 1 to 48 (the list path's limit; larger k runs query-major,
checked here too), nprobe from 1 to all lists, and the dot-product and cosine table builds.  One
case is also checked against the oracle directly.
"""
import os

import numpy as np
import pytest

from test_ivfpq_gpu import _check_search, _index, _m

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    assert vector_hip.CudaDeviceContext.device_count() >= 1, "no gfx950 GPU visible"
    return vector_hip


def _skewed_parts(rng, dim, nlist, n, empty=(), integer=False):
    """Lists of very different sizes (a few hold most rows), some empty."""
    m_sub, ks, ds = 16, 256, dim // 16
    if integer:
        coarse = rng.integers(-4, 5, (nlist, dim)).astype(np.float32)
        cb = rng.integers(-2, 3, m_sub * ks * ds).astype(np.float32)
    else:
        coarse = rng.standard_normal((nlist, dim)).astype(np.float32)
        cb = (0.5 * rng.standard_normal(m_sub * ks * ds)).astype(np.float32)
    weights = rng.exponential(1.0, nlist) ** 3
    weights[list(empty)] = 0.0
    assign = rng.choice(nlist, n, p=weights / weights.sum())
    order = np.argsort(assign, kind="stable")
    sizes = np.bincount(assign, minlength=nlist).astype(np.uint32)
    codes = rng.integers(0, ks, (n, m_sub)).astype(np.uint8)
    return coarse, cb, sizes, order.astype(np.uint32), codes[order]


def _both_paths(ix, qs, k, nprobe):
    old = os.environ.get("VHIP_IVFPQ_SCAN")
    try:
        os.environ.pop("VHIP_IVFPQ_SCAN", None)
        a = ix.search_batch_arrays(qs, k, nprobe)
        os.environ["VHIP_IVFPQ_SCAN"] = "query"
        b = ix.search_batch_arrays(qs, k, nprobe)
    finally:
        if old is None:
            os.environ.pop("VHIP_IVFPQ_SCAN", None)
        else:
            os.environ["VHIP_IVFPQ_SCAN"] = old
    return a, b


def _assert_same(a, b):
    assert np.array_equal(a[2], b[2]), "result counts differ"
    assert np.array_equal(a[0], b[0]), "ids differ"
    assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32)), "distances differ"


@pytest.mark.parametrize("dim", [128, 64])
@pytest.mark.parametrize("k,nprobe", [(10, 8), (1, 1), (48, 16), (40, 64), (37, 3), (64, 16), (100, 16)])
def test_lists_match_query_major_l2(vh, dim, k, nprobe):
    rng = np.random.default_rng(dim + 31 * k + nprobe)
    nlist = 64
    parts = _skewed_parts(rng, dim, nlist, 60_000, empty=(5, 17, 40))
    ix = _index(vh, parts, dim, 16, 256, vh.DistanceMetric.L2Squared)
    qs = rng.standard_normal((1500, dim)).astype(np.float32)
    a, b = _both_paths(ix, qs, k, nprobe)
    _assert_same(a, b)
    assert np.all(a[2] <= k)


@pytest.mark.parametrize("metric", ["dot", "cosine"])
def test_lists_match_query_major_inner_product(vh, metric):
    rng = np.random.default_rng(77 if metric == "dot" else 78)
    parts = _skewed_parts(rng, 64, 32, 30_000, empty=(2,))
    ix = _index(vh, parts, 64, 16, 256, _m(vh, metric))
    qs = rng.standard_normal((700, 64)).astype(np.float32)
    for k, nprobe in ((10, 4), (48, 32)):
        a, b = _both_paths(ix, qs, k, nprobe)
        _assert_same(a, b)


def test_lists_integer_exact_against_oracle(vh, oracle):
    """The list-major path on its own against the oracle: integer parts, exact distances."""
    rng = np.random.default_rng(91)
    parts = _skewed_parts(rng, 128, 24, 20_000, empty=(0, 9), integer=True)
    ix = _index(vh, parts, 128, 16, 256, vh.DistanceMetric.L2Squared)
    qs = rng.integers(-4, 5, (40, 128)).astype(np.float32)
    for k, nprobe in ((10, 6), (48, 24), (1, 2), (64, 24), (128, 24)):
        _check_search(vh, oracle, ix, parts, qs, k, nprobe, "l2", 16, 256, exact=True)


def test_lists_repeatable_and_batch_independent(vh):
    rng = np.random.default_rng(92)
    parts = _skewed_parts(rng, 128, 48, 40_000)
    ix = _index(vh, parts, 128, 16, 256, vh.DistanceMetric.L2Squared)
    qs = rng.standard_normal((3000, 128)).astype(np.float32)
    r1 = ix.search_batch_arrays(qs, 10, 12)
    r2 = ix.search_batch_arrays(qs, 10, 12)
    _assert_same(r1, r2)
    sel = rng.choice(3000, 100, replace=False)
    r3 = ix.search_batch_arrays(qs[sel], 10, 12)
    _assert_same((r1[0][sel], r1[1][sel], r1[2][sel]), r3)


def test_lists_many_lists_plan_without_lds_histogram(vh, oracle):
    """More lists (8,200) than the plan's LDS histogram holds (8,192 bins): the pair counting and
    scattering take their global-atomic path.  Checked against the query-major kernel and, exactly
    on integer parts, against the oracle."""
    rng = np.random.default_rng(93)
    parts = _skewed_parts(rng, 64, 8200, 30_000, integer=True)
    ix = _index(vh, parts, 64, 16, 256, vh.DistanceMetric.L2Squared)
    qs = rng.integers(-4, 5, (200, 64)).astype(np.float32)
    a, b = _both_paths(ix, qs, 10, 24)
    _assert_same(a, b)
    _check_search(vh, oracle, ix, parts, qs[:20], 10, 24, "l2", 16, 256, exact=True)


def test_batch_of_several_chunks(vh):
    """A batch whose (query, probe) pairs exceed one search chunk (2^22 pairs: 65,536 queries at
    nprobe 64) runs as several chunks; its results equal those of the same queries searched in
    batches of one chunk or less, bit for bit."""
    rng = np.random.default_rng(77)
    dim, nlist = 64, 64
    parts = _skewed_parts(rng, dim, nlist, 20_000)
    ix = _index(vh, parts, dim, 16, 256, vh.DistanceMetric.L2Squared)
    qs = rng.standard_normal((70_000, dim)).astype(np.float32)
    print("  70,000 queries at nprobe 64 (two chunks)", flush=True)
    whole = ix.search_batch_arrays(qs, 10, 64)
    head = ix.search_batch_arrays(qs[:40_000], 10, 64)
    tail = ix.search_batch_arrays(qs[40_000:], 10, 64)
    _assert_same(whole, tuple(np.concatenate([h, t]) for h, t in zip(head, tail)))
