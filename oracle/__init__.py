"""CPU oracle for the vector-hip hot path -- TEST INFRASTRUCTURE ONLY.

ctypes bindings over ``oracle/libvh_oracle.so`` (built from ``vh_oracle.c`` by
``oracle/Makefile``).  The C code restates the reference's CPU path:

* ``distance``           vector-simd ``DistanceEngine`` (lib.rs:54-310, scalar.rs,
                         avx2.rs, avx512.rs), all 10 metrics, same backend dispatch.
* ``knn_search_batch``   ``CudaKnnEngine::search_batch_cpu`` (vector-cuda/src/knn.rs:312-377).
* ``flat_search``        ``FlatIndex::search`` (vector-index/src/flat.rs:131-189).
* ``top_k_reduce``       ``CollectiveOps::top_k_reduce`` (vector-cuda/src/ddp/collective.rs:115-159).
* ``kmeans_step/fit``    ``KMeans::fit`` loop body (vector-index/src/ivf/kmeans.rs:70-155),
                         explicit init, empty clusters keep the old centroid.
* ``hamming_packed_knn`` packed-bit Hamming (an extension; equals scalar.rs:143-153 on
                         unpacked 0/1 codes).
* ``pq_encode`` / ``pq_adc_lut`` / ``pq_distance_with_lut``  ``ProductQuantizer`` (vector-index/src/ivf/pq.rs:178-293).
* ``find_top_centroids`` ``KMeans::find_top_centroids`` (ivf/kmeans.rs:311-356).
* ``ivfpq_search``       ``IvfPqIndex::search_with_nprobe`` (ivf/mod.rs:256-345) with given probes.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` and parity
legs may import this package, and only to check the GPU results or to time the CPU baseline.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libvh_oracle.so")
_lib = None

METRICS = {
    "l2": 0, "dot": 1, "cosine": 2, "l1": 3, "minkowski": 4,
    "linf": 5, "hamming": 6, "mahalanobis": 7, "jaccard": 8, "hellinger": 9,
}
HIGHER_IS_BETTER = {1, 2}

_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_szp = ctypes.POINTER(ctypes.c_size_t)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_sz = ctypes.c_size_t


def build() -> str:
    """Compile the oracle with its Makefile; returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.vho_detect_backend.restype = ctypes.c_int
        L.vho_distance.restype = ctypes.c_float
        L.vho_distance.argtypes = [ctypes.c_int, _f32p, _f32p, _sz, ctypes.c_int]
        L.vho_distance_rows.restype = None
        L.vho_distance_rows.argtypes = [ctypes.c_int, _f32p, _f32p, _sz, _sz, ctypes.c_int, _f32p]
        L.vho_knn_search_batch.restype = ctypes.c_int
        L.vho_knn_search_batch.argtypes = [_f32p, _sz, _sz, ctypes.c_int, _f32p, _sz, _sz, ctypes.c_int,
                                           ctypes.c_int, _u32p, _f32p, _szp]
        L.vho_flat_search.restype = ctypes.c_long
        L.vho_flat_search.argtypes = [_f32p, _sz, _sz, ctypes.c_int, _f32p, _sz, ctypes.c_int, _u32p, _f32p]
        L.vho_top_k_reduce.restype = ctypes.c_size_t
        L.vho_top_k_reduce.argtypes = [_u32p, _f32p, _sz, _sz, ctypes.c_int, _u32p, _f32p]
        L.vho_kmeans_step.restype = ctypes.c_int
        L.vho_kmeans_step.argtypes = [_f32p, _sz, _sz, _f32p, _sz, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      _i32p, _i64p, _f32p, _f32p, _f32p]
        L.vho_kmeans_fit.restype = ctypes.c_long
        L.vho_kmeans_fit.argtypes = [_f32p, _sz, _sz, _f32p, _sz, ctypes.c_int, _sz, ctypes.c_float,
                                     ctypes.c_int, ctypes.c_int, _i32p, _f32p]
        L.vho_hamming_packed.restype = ctypes.c_uint32
        L.vho_hamming_packed.argtypes = [_u32p, _u32p, _sz]
        L.vho_hamming_packed_knn.restype = ctypes.c_int
        L.vho_hamming_packed_knn.argtypes = [_u32p, _sz, _sz, _u32p, _sz, _sz, ctypes.c_int, _u32p, _u32p, _szp]
        L.vho_unpack_bits.restype = None
        L.vho_unpack_bits.argtypes = [_u32p, _sz, _sz, _f32p]
        L.vho_pq_encode.restype = ctypes.c_int
        L.vho_pq_encode.argtypes = [_f32p, _sz, _sz, _sz, _sz, _f32p, ctypes.c_int, ctypes.c_int, _u8p]
        L.vho_pq_adc_lut.restype = ctypes.c_int
        L.vho_pq_adc_lut.argtypes = [_f32p, _sz, _sz, _sz, _f32p, ctypes.c_int, ctypes.c_int, _f32p]
        L.vho_pq_distance_with_lut.restype = ctypes.c_float
        L.vho_pq_distance_with_lut.argtypes = [_u8p, _sz, _sz, _f32p]
        L.vho_find_top_centroids.restype = ctypes.c_size_t
        L.vho_find_top_centroids.argtypes = [_f32p, _f32p, _sz, _sz, _sz, ctypes.c_int, ctypes.c_int, _u32p, _f32p]
        L.vho_ivfpq_search.restype = ctypes.c_size_t
        L.vho_ivfpq_search.argtypes = [_f32p, _sz, ctypes.c_int, ctypes.c_int, _f32p, _sz, _sz, _sz, _f32p,
                                       _u64p, _u32p, _u8p, _u32p, _sz, _sz, _u32p, _f32p]
        _lib = L
    return _lib


def _p(a, t):
    return a.ctypes.data_as(t)


def _metric(m) -> int:
    return METRICS[m] if isinstance(m, str) else int(m)


def detect_backend() -> int:
    """0 scalar, 1 AVX2+FMA, 2 AVX-512F (vector-simd lib.rs:292-310)."""
    return lib().vho_detect_backend()


def distance(metric, a, b, backend: int = -1) -> float:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    assert a.shape == b.shape
    return float(lib().vho_distance(_metric(metric), _p(a, _f32p), _p(b, _f32p), a.size, backend))


def distance_rows(metric, a, b, backend: int = -1) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    rows, dim = a.shape
    out = np.empty(rows, np.float32)
    lib().vho_distance_rows(_metric(metric), _p(a, _f32p), _p(b, _f32p), rows, dim, backend, _p(out, _f32p))
    return out


def knn_search_batch(base, queries, k, metric="l2", backend: int = -1, threads: int = 0):
    """Returns (ids[nq, k] uint32, dist[nq, k] float32, lens[nq]) best-first."""
    base = np.ascontiguousarray(base, dtype=np.float32)
    queries = np.ascontiguousarray(queries, dtype=np.float32)
    n, dim = base.shape
    nq = queries.shape[0]
    ids = np.zeros((nq, max(k, 1)), np.uint32)
    dist = np.zeros((nq, max(k, 1)), np.float32)
    lens = np.zeros(nq, np.uintp)
    rc = lib().vho_knn_search_batch(_p(base, _f32p), n, dim, _metric(metric), _p(queries, _f32p), nq, k,
                                   backend, threads, _p(ids, _u32p), _p(dist, _f32p), _p(lens, _szp))
    assert rc == 0
    return ids[:, :k], dist[:, :k], lens


def flat_search(base, query, k, metric="l2", backend: int = -1):
    base = np.ascontiguousarray(base, dtype=np.float32)
    query = np.ascontiguousarray(query, dtype=np.float32)
    n, dim = base.shape if base.ndim == 2 else (0, query.size)
    ids = np.zeros(max(k, 1), np.uint32)
    dist = np.zeros(max(k, 1), np.float32)
    r = lib().vho_flat_search(_p(base, _f32p), n, dim, _metric(metric), _p(query, _f32p), k, backend,
                              _p(ids, _u32p), _p(dist, _f32p))
    if r < 0:
        raise ValueError("EmptyIndex")
    return ids[:r], dist[:r]


def top_k_reduce(lists, k, metric="l2"):
    """lists: sequence of (ids, dists) per rank; returns merged (ids, dists)."""
    if not lists:
        return np.zeros(0, np.uint32), np.zeros(0, np.float32)
    ids = np.ascontiguousarray(np.concatenate([np.asarray(l[0], np.uint32) for l in lists]), np.uint32)
    dist = np.ascontiguousarray(np.concatenate([np.asarray(l[1], np.float32) for l in lists]), np.float32)
    oi = np.zeros(max(k, 1), np.uint32)
    od = np.zeros(max(k, 1), np.float32)
    m = lib().vho_top_k_reduce(_p(ids, _u32p), _p(dist, _f32p), ids.size, k, _metric(metric),
                               _p(oi, _u32p), _p(od, _f32p))
    return oi[:m], od[:m]


def kmeans_step(data, centroids, metric="l2", backend: int = -1, threads: int = 1):
    """One Lloyd iteration from `centroids`.  Returns dict with new centroids,
    assign, counts, shifts, max_shift, inertia."""
    data = np.ascontiguousarray(data, dtype=np.float32)
    cent = np.array(centroids, dtype=np.float32, copy=True, order="C")
    n, dim = data.shape
    k = cent.shape[0]
    assign = np.zeros(n, np.int32)
    counts = np.zeros(k, np.int64)
    shifts = np.zeros(k, np.float32)
    ms = np.zeros(1, np.float32)
    inertia = np.zeros(1, np.float32)
    rc = lib().vho_kmeans_step(_p(data, _f32p), n, dim, _p(cent, _f32p), k, _metric(metric), backend, threads,
                               _p(assign, _i32p), _p(counts, _i64p), _p(shifts, _f32p), _p(ms, _f32p),
                               _p(inertia, _f32p))
    assert rc == 0
    return {"centroids": cent, "assign": assign, "counts": counts, "shifts": shifts,
            "max_shift": float(ms[0]), "inertia": float(inertia[0])}


def kmeans_fit(data, init_centroids, max_iters, tol=-1.0, metric="l2", backend: int = -1, threads: int = 1):
    data = np.ascontiguousarray(data, dtype=np.float32)
    cent = np.array(init_centroids, dtype=np.float32, copy=True, order="C")
    n, dim = data.shape
    assign = np.zeros(n, np.int32)
    inertia = np.zeros(1, np.float32)
    it = lib().vho_kmeans_fit(_p(data, _f32p), n, dim, _p(cent, _f32p), cent.shape[0], _metric(metric),
                              max_iters, tol, backend, threads, _p(assign, _i32p), _p(inertia, _f32p))
    return {"centroids": cent, "assign": assign, "iterations": int(it), "inertia": float(inertia[0])}


def hamming_packed(a, b) -> int:
    a = np.ascontiguousarray(a, dtype=np.uint32)
    b = np.ascontiguousarray(b, dtype=np.uint32)
    return int(lib().vho_hamming_packed(_p(a, _u32p), _p(b, _u32p), a.size))


def hamming_packed_knn(codes, queries, k, threads: int = 0):
    codes = np.ascontiguousarray(codes, dtype=np.uint32)
    queries = np.ascontiguousarray(queries, dtype=np.uint32)
    n, words = codes.shape
    nq = queries.shape[0]
    ids = np.zeros((nq, max(k, 1)), np.uint32)
    dist = np.zeros((nq, max(k, 1)), np.uint32)
    lens = np.zeros(nq, np.uintp)
    lib().vho_hamming_packed_knn(_p(codes, _u32p), n, words, _p(queries, _u32p), nq, k, threads,
                                 _p(ids, _u32p), _p(dist, _u32p), _p(lens, _szp))
    return ids[:, :k], dist[:, :k], lens


def unpack_bits(codes) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint32)
    n, words = codes.shape
    out = np.empty((n, words * 32), np.float32)
    lib().vho_unpack_bits(_p(codes, _u32p), n, words, _p(out, _f32p))
    return out


# ---- product quantization and IVF-PQ (vector-index/src/ivf) -------------------------------
def pq_encode(data, codebooks, num_subvectors, sub_clusters, metric="l2", backend: int = -1):
    """ProductQuantizer::encode_batch: codes[n, M] uint8."""
    data = np.ascontiguousarray(data, dtype=np.float32)
    codebooks = np.ascontiguousarray(codebooks, dtype=np.float32).ravel()
    n, dim = data.shape
    out = np.zeros((n, num_subvectors), np.uint8)
    rc = lib().vho_pq_encode(_p(data, _f32p), n, dim, num_subvectors, sub_clusters, _p(codebooks, _f32p),
                             _metric(metric), backend, _p(out, _u8p))
    assert rc == 0
    return out


def pq_adc_lut(query, codebooks, num_subvectors, sub_clusters, metric="l2", backend: int = -1):
    """ProductQuantizer::compute_adc_lut: lut[M * Ks] float32."""
    query = np.ascontiguousarray(query, dtype=np.float32).ravel()
    codebooks = np.ascontiguousarray(codebooks, dtype=np.float32).ravel()
    lut = np.zeros(num_subvectors * sub_clusters, np.float32)
    rc = lib().vho_pq_adc_lut(_p(query, _f32p), query.size, num_subvectors, sub_clusters, _p(codebooks, _f32p),
                              _metric(metric), backend, _p(lut, _f32p))
    assert rc == 0
    return lut


def pq_distance_with_lut(code, lut, sub_clusters) -> float:
    code = np.ascontiguousarray(code, dtype=np.uint8).ravel()
    lut = np.ascontiguousarray(lut, dtype=np.float32).ravel()
    return float(lib().vho_pq_distance_with_lut(_p(code, _u8p), code.size, sub_clusters, _p(lut, _f32p)))


def find_top_centroids(query, centroids, nprobe, metric="l2", backend: int = -1):
    """KMeans::find_top_centroids: (indices uint32, scores float32), best first."""
    query = np.ascontiguousarray(query, dtype=np.float32).ravel()
    centroids = np.ascontiguousarray(centroids, dtype=np.float32)
    k, dim = centroids.shape
    idx = np.zeros(max(1, min(nprobe, k)), np.uint32)
    sc = np.zeros(idx.size, np.float32)
    r = lib().vho_find_top_centroids(_p(query, _f32p), _p(centroids, _f32p), k, dim, nprobe, _metric(metric),
                                     backend, _p(idx, _u32p), _p(sc, _f32p))
    return idx[:r], sc[:r]


def ivfpq_search(query, coarse, codebooks, num_subvectors, sub_clusters, list_off, ids, codes, probes, k,
                 metric="l2", backend: int = -1):
    """IvfPqIndex::search_with_nprobe for one query with the probe list given (CSR lists)."""
    query = np.ascontiguousarray(query, dtype=np.float32).ravel()
    coarse = np.ascontiguousarray(coarse, dtype=np.float32)
    codebooks = np.ascontiguousarray(codebooks, dtype=np.float32).ravel()
    list_off = np.ascontiguousarray(list_off, dtype=np.uint64)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    codes = np.ascontiguousarray(codes, dtype=np.uint8).ravel()
    probes = np.ascontiguousarray(probes, dtype=np.uint32).ravel()
    out_i = np.zeros(max(k, 1), np.uint32)
    out_d = np.zeros(max(k, 1), np.float32)
    r = lib().vho_ivfpq_search(_p(query, _f32p), query.size, _metric(metric), backend, _p(coarse, _f32p),
                               coarse.shape[0], num_subvectors, sub_clusters, _p(codebooks, _f32p),
                               _p(list_off, _u64p), _p(ids, _u32p), _p(codes, _u8p), _p(probes, _u32p),
                               probes.size, k, _p(out_i, _u32p), _p(out_d, _f32p))
    return out_i[:r], out_d[:r]
