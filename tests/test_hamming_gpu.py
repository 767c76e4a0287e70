"""GPU parity of packed-bit Hamming kNN (popcount of XOR) against the oracle: exact
integer distances, and with (distance, id) ordering the ids are identical too."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def vh():
    import vector_hip

    assert vector_hip.CudaDeviceContext.device_count() >= 1
    return vector_hip


# Every width runs on the fp4 matrix cores by default (32..1024 bits: every expanded width).
@pytest.mark.parametrize("n,bits,nq,k", [(100_000, 256, 50, 10), (5000, 64, 17, 33), (777, 96, 3, 777),
                                         (300_000, 256, 8, 100), (20_000, 32, 40, 10), (3000, 160, 11, 64),
                                         (50_000, 512, 20, 50), (10_000, 1024, 9, 20), (300, 256, 130, 7)])
def test_hamming_bit_exact(vh, oracle, n, bits, nq, k):
    from vector_hip import datasets as ds

    codes = ds.packed_bits(n, bits, ds.SEED_BASE)
    q = ds.packed_bits(nq, bits, ds.SEED_QUERIES)
    ids, dist, lens = vh.HammingKnnEngine(codes).search_batch_arrays(q, k)
    rids, rdist, _ = oracle.hamming_packed_knn(codes, q, k)
    assert np.all(lens == min(k, n))
    assert np.array_equal(dist, rdist), "distances must be bit-exact"
    assert np.array_equal(ids, rids), "(distance, id) order makes ids identical"


@pytest.mark.parametrize("kernel", ["popcount", "fp4"])
@pytest.mark.parametrize("n,bits,nq,k", [(20_000, 32, 33, 10), (4000, 96, 130, 40), (60_000, 256, 17, 100),
                                         (9000, 512, 5, 9), (3000, 1024, 64, 300)])
def test_hamming_kernels_bit_exact(vh, oracle, monkeypatch, kernel, n, bits, nq, k):
    """Both scan kernels, chosen with VHIP_HAMMING_KERNEL at engine creation: the popcount kernel
    over the packed words (the engine's path when the fp4 copy does not fit) and the fp4
    matrix-core kernel.  The profiler's work count shows which one ran: words per (query, row)
    for popcount, 2 K for fp4 (K = the padded bits, at least 64)."""
    from vector_hip import datasets as ds

    print(f"hamming kernel={kernel} n={n} bits={bits} nq={nq} k={k}", flush=True)
    monkeypatch.setenv("VHIP_HAMMING_KERNEL", kernel)
    codes = ds.packed_bits(n, bits, 31)
    q = ds.packed_bits(nq, bits, 32)
    eng = vh.HammingKnnEngine(codes)
    monkeypatch.delenv("VHIP_HAMMING_KERNEL")
    eng.profile(True)
    ids, dist, lens = eng.search_batch_arrays(q, k)
    per = eng.profile_read()["work"] / (nq * n)
    words = bits // 32
    padded = 1 << (words - 1).bit_length()
    assert per == (words if kernel == "popcount" else 2 * 32 * max(2, padded))
    rids, rdist, _ = oracle.hamming_packed_knn(codes, q, k)
    kk = min(k, n)
    assert np.all(lens == kk)
    assert np.array_equal(dist[:, :kk], rdist[:, :kk]) and np.array_equal(ids[:, :kk], rids[:, :kk])


def test_hamming_equals_reference_float_hamming(vh, oracle):
    """popcount distance == the reference's thresholded float Hamming on unpacked codes."""
    from vector_hip import datasets as ds

    codes = ds.packed_bits(2000, 256, 1)
    q = ds.packed_bits(4, 256, 2)
    ids, dist, _ = vh.HammingKnnEngine(codes).search_batch_arrays(q, 10)
    un_c = oracle.unpack_bits(codes)
    un_q = oracle.unpack_bits(q)
    for r in range(4):
        ref = oracle.distance_rows("hamming", np.repeat(un_q[r:r + 1], 10, 0), un_c[ids[r]])
        assert np.array_equal(ref, dist[r].astype(np.float32))


@pytest.mark.parametrize("bits", [256, 1024])
def test_hamming_massive_ties(vh, oracle, bits):
    """Every base code identical: every row ties, the per-query candidate slots overflow into
    the global lists and the overflow re-run, and the k lowest ids must come back."""
    from vector_hip import datasets as ds

    one = ds.packed_bits(1, bits, 3)
    codes = np.repeat(one, 40_000, axis=0)
    q = ds.packed_bits(5, bits, 4)
    ids, dist, lens = vh.HammingKnnEngine(codes).search_batch_arrays(q, 12)
    rids, rdist, _ = oracle.hamming_packed_knn(codes, q, 12)
    assert np.all(lens == 12)
    assert np.array_equal(dist, rdist) and np.array_equal(ids, rids)
    assert np.array_equal(ids, np.tile(np.arange(12, dtype=ids.dtype), (5, 1)))


# The 1024-column kernel serves filter rounds of codes up to 256 bits once a batch has at least
# 2048 queries and the round starts past 2048 * 3 k / 8 rows seen; the rest of a search runs on
# the 128-column kernel.  nq = 2500 leaves the last column block with 4 of its 8 waves active.
@pytest.mark.parametrize("n,bits,nq,k", [(150_000, 256, 2048, 10), (150_000, 256, 2500, 100),
                                         (120_000, 128, 2100, 10), (120_000, 32, 2048, 25),
                                         (140_000, 64, 3000, 1)])
def test_hamming_wide_kernel_bit_exact(vh, oracle, n, bits, nq, k):
    from vector_hip import datasets as ds

    print(f"hamming wide n={n} bits={bits} nq={nq} k={k}", flush=True)
    codes = ds.packed_bits(n, bits, 41)
    q = ds.packed_bits(nq, bits, 42)
    ids, dist, lens = vh.HammingKnnEngine(codes).search_batch_arrays(q, k)
    rids, rdist, _ = oracle.hamming_packed_knn(codes, q, k)
    assert np.all(lens == k)
    assert np.array_equal(dist, rdist), "distances must be bit-exact"
    assert np.array_equal(ids, rids), "(distance, id) order makes ids identical"


def test_hamming_wide_kernel_ties(vh, oracle):
    """Few distinct codes: whole items tie, so the 8 LDS slots per query overflow into the
    global lists and the capacity re-run, and the (distance, id) order must still hold."""
    from vector_hip import datasets as ds

    print("hamming wide ties", flush=True)
    distinct = ds.packed_bits(16, 256, 5)
    rng = np.random.default_rng(6)
    codes = distinct[rng.integers(0, 16, 90_000)]
    q = ds.packed_bits(2048, 256, 7)
    ids, dist, lens = vh.HammingKnnEngine(codes).search_batch_arrays(q, 10)
    rids, rdist, _ = oracle.hamming_packed_knn(codes, q, 10)
    assert np.all(lens == 10)
    assert np.array_equal(dist, rdist) and np.array_equal(ids, rids)


def test_hamming_wide_matches_tile_kernel(vh, monkeypatch):
    """The 1024-column kernel and the 128-column kernel (VHIP_HAMMING_KERNEL=fp4-tile) return
    identical results on the same engine data."""
    from vector_hip import datasets as ds

    print("hamming wide vs tile", flush=True)
    codes = ds.packed_bits(200_000, 256, 8)
    q = ds.packed_bits(4096, 256, 9)
    wide = vh.HammingKnnEngine(codes).search_batch_arrays(q, 20)
    monkeypatch.setenv("VHIP_HAMMING_KERNEL", "fp4-tile")
    tile_eng = vh.HammingKnnEngine(codes)
    monkeypatch.delenv("VHIP_HAMMING_KERNEL")
    tile = tile_eng.search_batch_arrays(q, 20)
    for a, b in zip(wide, tile):
        assert np.array_equal(a, b)
