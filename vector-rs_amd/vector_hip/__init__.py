"""vector_hip -- Python view of the MI355X kNN / k-means library (libvector_hip.so).

The classes mirror the reference's Rust API of the GPU hot path (crate vector-cuda), so
code written against it reads the same:

* ``CudaDeviceContext.device_count()``                 device.rs:112-117
* ``CudaKnnEngine(dataset, dimension, metric)``          knn.rs:85-401
* ``DistributedKnnEngine.try_new / emulator / new``    ddp/distributed_knn.rs:40-262
* ``CollectiveOps.top_k_reduce``                       ddp/collective.rs:115-159
* ``CudaKMeansEngine().fit(...)``                      kmeans.rs:43-467
* ``DistributedKMeansEngine.try_new / emulator``       ddp/distributed_kmeans.rs:25-541
* ``CudaError`` and its variants                      error.rs:7-29
* ``HammingKnnEngine``                                 packed-bit extension (no counterpart)

Everything runs in the HIP library; there is no CPU fallback.  If the library is not
built, importing this package raises ImportError.
"""
from __future__ import annotations

import ctypes
import dataclasses
import enum
import os
from typing import List, NamedTuple, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvector_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() (make -C vector-rs_amd)")

_lib = ctypes.CDLL(LIB_PATH)

_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_szp = ctypes.POINTER(ctypes.c_size_t)
_dblp = ctypes.POINTER(ctypes.c_double)
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_int = ctypes.c_int


class _KMeansResultC(ctypes.Structure):
    _fields_ = [("dimension", ctypes.c_size_t), ("k", ctypes.c_size_t), ("iterations", ctypes.c_size_t),
                ("inertia", ctypes.c_float)]


def _sig(name, restype, *argtypes):
    f = getattr(_lib, name)
    f.restype = restype
    f.argtypes = list(argtypes)
    return f


_sig("vhip_last_error", ctypes.c_char_p)
_sig("vhip_last_error_devices", None, _szp, _szp)
_sig("vhip_last_error_ordinal", _int)
_sig("vhip_device_count", _int)
_sig("vhip_device_info", _int, _int, ctypes.c_char_p, _sz, _szp)
_sig("vhip_knn_create", _int, _f32p, _sz, _sz, _int, _int, ctypes.POINTER(_vp))
_sig("vhip_knn_search_batch", _int, _vp, _f32p, _sz, _sz, _u32p, _f32p, _szp)
_sig("vhip_knn_search_batch_device", _int, _vp, _vp, _sz, _sz, _vp, _vp)
_sig("vhip_knn_search_batch_device_noalloc", _int, _vp, _vp, _sz, _sz, _vp, _vp)
_sig("vhip_knn_dimension", _sz, _vp)
_sig("vhip_knn_num_vectors", _sz, _vp)
_sig("vhip_knn_metric", _int, _vp)
_sig("vhip_knn_device_id", _int, _vp)
_sig("vhip_knn_destroy", None, _vp)
_sig("vhip_knn_profile", _int, _vp, _int)
_sig("vhip_knn_profile_read", _int, _vp, _dblp, _u64p, _dblp, _dblp)
_sig("vhip_dknn_try_new", _int, _f32p, _sz, _sz, _sz, _int, _int, ctypes.POINTER(_vp))
_sig("vhip_dknn_emulator", _int, _f32p, _sz, _sz, _sz, _int, _int, ctypes.POINTER(_vp))
_sig("vhip_dknn_search_batch", _int, _vp, _f32p, _sz, _sz, _u32p, _f32p, _szp)
_sig("vhip_dknn_num_gpus", _sz, _vp)
_sig("vhip_dknn_mode", _int, _vp)
_sig("vhip_dknn_dimension", _sz, _vp)
_sig("vhip_dknn_num_vectors", _sz, _vp)
_sig("vhip_dknn_metric", _int, _vp)
_sig("vhip_dknn_destroy", None, _vp)
_sig("vhip_top_k_reduce", _sz, _u32p, _f32p, _sz, _sz, _int, _u32p, _f32p)
_sig("vhip_hamming_create", _int, _u32p, _sz, _sz, _int, ctypes.POINTER(_vp))
_sig("vhip_hamming_search_batch", _int, _vp, _u32p, _sz, _sz, _u32p, _u32p, _szp)
_sig("vhip_hamming_search_batch_device", _int, _vp, _vp, _sz, _sz, _vp, _vp)
_sig("vhip_hamming_profile", _int, _vp, _int)
_sig("vhip_hamming_profile_read", _int, _vp, _dblp, _u64p, _dblp, _dblp)
_sig("vhip_hamming_destroy", None, _vp)
_sig("vhip_malloc", _int, _int, _sz, ctypes.POINTER(_vp))
_sig("vhip_free", _int, _int, _vp)
_sig("vhip_memcpy_htod", _int, _int, _vp, _vp, _sz)
_sig("vhip_memcpy_dtoh", _int, _int, _vp, _vp, _sz)
_sig("vhip_memcpy_dtod", _int, _int, _vp, _vp, _sz)
_sig("vhip_synchronize", _int, _int)
_HAS_KMEANS = hasattr(_lib, "vhip_kmeans_fit")
if _HAS_KMEANS:
    _sig("vhip_kmeans_fit", _int, _int, _f32p, _sz, _sz, _sz, _sz, ctypes.c_float, _int, _f32p, _int,
         ctypes.c_uint64, _f32p, _i32p, ctypes.POINTER(_KMeansResultC))
    _sig("vhip_dkmeans_check", _int, _sz)
    _sig("vhip_kmeans_create", _int, _int, _f32p, _sz, _sz, _int, ctypes.POINTER(_vp))
    _sig("vhip_kmeans_set_centroids", _int, _vp, _f32p, _sz)
    _sig("vhip_kmeans_run", _int, _vp, _sz)
    _sig("vhip_kmeans_read", _int, _vp, _f32p, _i32p, _i64p, _f32p, _f32p, _f32p)
    _sig("vhip_kmeans_profile", _int, _vp, _int)
    _sig("vhip_kmeans_profile_read", _int, _vp, _dblp, _u64p, _dblp, _dblp)
    _sig("vhip_kmeans_destroy", None, _vp)
    _sig("vhip_kmeans_assign_only", _int, _vp, _i32p, _f32p, _f32p)
    _sig("vhip_coarse_create", _int, _f32p, _sz, _sz, _int, _int, ctypes.POINTER(_vp))
    _sig("vhip_coarse_assign", _int, _vp, _f32p, _sz, _u32p, _f32p, _f32p)
    _sig("vhip_coarse_probe", _int, _vp, _f32p, _sz, _sz, _u32p, _f32p, _szp)
    _sig("vhip_coarse_nlist", _sz, _vp)
    _sig("vhip_coarse_dimension", _sz, _vp)
    _sig("vhip_coarse_destroy", None, _vp)
    _sig("vhip_train_from_shards", _int, ctypes.c_char_p, _sz, _sz, ctypes.c_float, _int, _sz, ctypes.c_char_p,
         ctypes.c_uint64, ctypes.POINTER(_KMeansResultC), _szp)
class _IvfPqConfigC(ctypes.Structure):
    _fields_ = [("nlist", _sz), ("nprobe", _sz), ("num_subvectors", _sz), ("sub_clusters", _sz),
                ("max_kmeans_iters", _sz), ("kmeans_tolerance", ctypes.c_float), ("max_train_points", _sz)]


class _IvfPqDescC(ctypes.Structure):
    _fields_ = [("dimension", _sz), ("metric", _int), ("nlist", _sz), ("num_subvectors", _sz),
                ("sub_clusters", _sz), ("num_vectors", _sz), ("config", _IvfPqConfigC)]


_HAS_IVFPQ = hasattr(_lib, "vhip_ivfpq_build")
if _HAS_IVFPQ:
    _u8p = ctypes.POINTER(ctypes.c_uint8)
    _cfgp = ctypes.POINTER(_IvfPqConfigC)
    _sig("vhip_ivfpq_config_default", None, _cfgp)
    _sig("vhip_ivfpq_config_validate", _int, _cfgp, _sz)
    _sig("vhip_pq_train", _int, _int, _f32p, _sz, _sz, _sz, _sz, _sz, ctypes.c_float, _int, _f32p, ctypes.c_uint64,
         _f32p)
    _sig("vhip_pq_encode", _int, _int, _f32p, _sz, _sz, _sz, _int, _f32p, _sz, _u8p)
    _sig("vhip_pq_adc_lut", _int, _int, _f32p, _sz, _sz, _sz, _int, _f32p, _sz, _f32p)
    _sig("vhip_ivfpq_build", _int, _int, _f32p, _sz, _sz, _cfgp, _int, ctypes.c_uint64, ctypes.POINTER(_vp))
    _sig("vhip_ivfpq_create", _int, _int, _sz, _int, _cfgp, _f32p, _sz, _f32p, _u32p, _u32p, _u8p,
         ctypes.POINTER(_vp))
    _sig("vhip_ivfpq_search_batch", _int, _vp, _f32p, _sz, _sz, _sz, _u32p, _f32p, _szp)
    _sig("vhip_ivfpq_search_batch_device", _int, _vp, _vp, _sz, _sz, _sz, _vp, _vp, _vp)
    _sig("vhip_ivfpq_probe", _int, _vp, _f32p, _sz, _sz, _u32p)
    _sig("vhip_ivfpq_info", _int, _vp, ctypes.POINTER(_IvfPqDescC))
    _sig("vhip_ivfpq_export", _int, _vp, _f32p, _f32p, _u32p, _u32p, _u8p)
    _sig("vhip_ivfpq_profile", _int, _vp, _int)
    _sig("vhip_ivfpq_profile_read", _int, _vp, _dblp, _u64p)
    _sig("vhip_ivfpq_destroy", None, _vp)
    _sig("vhip_ivfpq_file_save", _int, ctypes.c_char_p, _cfgp, _sz, _int, _f32p, _sz, _f32p, _sz, _u32p, _sz, _u32p,
         _u8p)
    _sig("vhip_ivfpq_file_info", _int, ctypes.c_char_p, _cfgp, _szp, ctypes.POINTER(_int), _szp, _szp, _szp, _szp)
    _sig("vhip_ivfpq_file_load", _int, ctypes.c_char_p, _f32p, _f32p, _u32p, _u32p, _u8p)
_sig("vhip_vecrstor_write", _int, ctypes.c_char_p, _f32p, _sz, _sz)
_sig("vhip_vecrstor_open", _int, ctypes.c_char_p, _szp, _szp)
_sig("vhip_vecrstor_read", _int, ctypes.c_char_p, _f32p, _sz, _sz)
_sig("vhip_knn_create_from_vecrstor", _int, ctypes.c_char_p, _int, _int, ctypes.POINTER(_vp))
_sig("vhip_vecrstor_map", _int, ctypes.c_char_p, ctypes.POINTER(_f32p), _szp, _szp, ctypes.POINTER(_vp))
_sig("vhip_vecrstor_unmap", None, _vp)
if _HAS_KMEANS:
    _sig("vhip_kmeans_create_from_vecrstor", _int, _int, ctypes.POINTER(ctypes.c_char_p), _sz, _int,
         ctypes.POINTER(_vp))
    _sig("vhip_kmeans_create_segments", _int, _int, ctypes.POINTER(_f32p), _szp, _sz, _sz, _int, ctypes.POINTER(_vp))
    _sig("vhip_kmeans_fit_state", _int, _vp, _sz, _sz, ctypes.c_float, _f32p, _int, ctypes.c_uint64, _f32p, _i32p,
         ctypes.POINTER(_KMeansResultC))
_sig("vhip_centroid_file_save", _int, ctypes.c_char_p, _f32p, _sz, _sz, _int, _sz, ctypes.c_float)
_sig("vhip_centroid_file_info", _int, ctypes.c_char_p, _szp, _szp, ctypes.POINTER(_int), _szp, _f32p)
_sig("vhip_centroid_file_load", _int, ctypes.c_char_p, _f32p, _sz, _sz)


# ---- errors: CudaError (error.rs:7-29) ---------------------------------------------------
class CudaError(Exception):
    """Base of the error variants; ``code`` is the C status."""

    code = 0


class InsufficientDevices(CudaError):
    code = -1

    def __init__(self, requested: int, available: int, msg: str = ""):
        super().__init__(msg or f"requested {requested} device(s), but only {available} found")
        self.requested = requested
        self.available = available

    def __eq__(self, other):
        return isinstance(other, InsufficientDevices) and (self.requested, self.available) == (
            other.requested, other.available)


class DeviceNotFound(CudaError):
    code = -2

    def __init__(self, ordinal: int = -1, msg: str = ""):
        super().__init__(msg or f"HIP device with ordinal {ordinal} was not found")
        self.ordinal = ordinal


class DriverError(CudaError):
    code = -3


class HardwareNotAvailable(CudaError):
    code = -4


class InvalidConfig(CudaError):
    code = -5


class EmptyIndex(CudaError):
    """vector-index VectorIndexError::EmptyIndex (types.rs)."""

    code = -6


class DimensionMismatch(CudaError):
    """vector-index VectorIndexError::DimensionMismatch{expected, got} (types.rs)."""

    code = -5

    def __init__(self, expected: int, got: int):
        super().__init__(f"dimension mismatch: expected {expected}, got {got}")
        self.expected = expected
        self.got = got


_ERRORS = {c.code: c for c in (DeviceNotFound, DriverError, HardwareNotAvailable, InvalidConfig, EmptyIndex)}


def _check(status: int):
    if status == 0:
        return
    msg = (_lib.vhip_last_error() or b"").decode()
    if status == InsufficientDevices.code:
        r = _sz()
        a = _sz()
        _lib.vhip_last_error_devices(ctypes.byref(r), ctypes.byref(a))
        raise InsufficientDevices(r.value, a.value, msg)
    if status == DeviceNotFound.code:
        raise DeviceNotFound(int(_lib.vhip_last_error_ordinal()), msg)
    raise _ERRORS.get(status, CudaError)(msg)


VHIP_MAX_K = 2048  # largest k one search call serves (VHIP_MAX_K of vector_hip.h)
NOALLOC_SCRATCH_BYTES = 64 << 20  # per-GPU working array of the allocation-free search (VHIP_NOALLOC_SCRATCH_BYTES)


# ---- types ------------------------------------------------------------------------------------
class DistanceMetric(enum.IntEnum):
    """vector-index/src/lib.rs:50-94 with the kernel codes of knn.rs:235-246."""

    L2Squared = 0
    DotProduct = 1
    CosineSimilarity = 2
    Manhattan = 3
    Minkowski = 4
    Chebyshev = 5
    Hamming = 6
    Mahalanobis = 7
    Jaccard = 8
    Hellinger = 9

    def higher_is_better(self) -> bool:
        return self in (DistanceMetric.DotProduct, DistanceMetric.CosineSimilarity)


class GpuShardMode(enum.IntEnum):
    """ddp/distributed_knn.rs:14-19."""

    Sharded = 0
    Replicated = 1


class SearchResult(NamedTuple):
    """vector-index/src/types.rs:12-20."""

    id: int
    distance: float


def _rows(data, dimension: Optional[int], dtype=np.float32) -> np.ndarray:
    a = np.ascontiguousarray(data, dtype=dtype)
    if a.ndim == 1:
        if dimension is None or dimension <= 0:
            raise InvalidConfig("dimension must be > 0")
        if a.size % dimension != 0:
            raise InvalidConfig(f"data length {a.size} is not a multiple of dimension {dimension}")
        a = a.reshape(-1, dimension)
    elif dimension is not None and a.shape[1] != dimension:
        raise InvalidConfig(f"rows have {a.shape[1]} elements, dimension is {dimension}")
    return a


def _p(a, t):
    return a.ctypes.data_as(t)


def _to_lists(ids, dist, lens) -> List[List[SearchResult]]:
    return [[SearchResult(int(ids[q, j]), float(dist[q, j])) for j in range(int(lens[q]))]
            for q in range(ids.shape[0])]


class CudaDeviceContext:
    """device.rs:81-256.  The constructor is with_ordinal_strict (DeviceNotFound when the ordinal
    has no usable gfx950 device); with_ordinal / new return a software-emulator descriptor
    instead, as the reference does.  A descriptor runs nothing: engines on its ordinal raise
    DeviceNotFound rather than falling back to the CPU."""

    def __init__(self, ordinal: int = 0):
        name = ctypes.create_string_buffer(256)
        mem = _sz()
        _check(_lib.vhip_device_info(ordinal, name, 256, ctypes.byref(mem)))
        self._id = ordinal
        self._name = name.value.decode()
        self._mem = mem.value
        self._hw = True

    @staticmethod
    def device_count() -> int:
        return _lib.vhip_device_count()

    @classmethod
    def with_ordinal_strict(cls, ordinal: int) -> "CudaDeviceContext":
        return cls(ordinal)

    @classmethod
    def with_ordinal(cls, ordinal: int) -> "CudaDeviceContext":
        """device.rs:188-221"""
        try:
            return cls(ordinal)
        except CudaError:
            return cls.software_emulator(ordinal)

    @classmethod
    def new(cls) -> "CudaDeviceContext":
        """device.rs:120-122"""
        return cls.with_ordinal(0)

    @classmethod
    def software_emulator(cls, ordinal: int) -> "CudaDeviceContext":
        """device.rs:173-185: a descriptor with no device and total memory 0."""
        c = cls.__new__(cls)
        c._id = ordinal
        c._name = f"HIP Software Emulator (GPU {ordinal}, no device)"
        c._mem = 0
        c._hw = False
        return c

    def device_id(self) -> int:
        return self._id

    def device_name(self) -> str:
        return self._name

    def total_memory_bytes(self) -> int:
        return self._mem

    def is_hardware_available(self) -> bool:
        return self._hw


class _Profiled:
    _prof_fn = None
    _read_fn = None

    def profile(self, enable: bool = True):
        _check(type(self)._prof_fn(self._h, int(enable)))

    def profile_read(self) -> dict:
        ms = ctypes.c_double()
        n = ctypes.c_uint64()
        w = ctypes.c_double()
        b = ctypes.c_double()
        _check(type(self)._read_fn(self._h, ctypes.byref(ms), ctypes.byref(n), ctypes.byref(w), ctypes.byref(b)))
        return {"kernel_ms": ms.value, "launches": n.value, "work": w.value, "bytes": b.value}


class CudaKnnEngine(_Profiled):
    """knn.rs:45-401: the base is uploaded once and stays resident on the GPU."""

    _prof_fn = _lib.vhip_knn_profile
    _read_fn = _lib.vhip_knn_profile_read

    def __init__(self, dataset, dimension: Optional[int] = None, metric=DistanceMetric.L2Squared, ordinal: int = 0):
        base = _rows(dataset, dimension)
        self._dim = base.shape[1]
        h = _vp()
        _check(_lib.vhip_knn_create(_p(base, _f32p), base.shape[0], self._dim, int(metric), ordinal, ctypes.byref(h)))
        self._h = h

    @classmethod
    def new(cls, dataset, dimension, metric):
        return cls(dataset, dimension, metric, 0)

    @classmethod
    def from_vecrstor(cls, path, metric=DistanceMetric.L2Squared, ordinal: int = 0) -> "CudaKnnEngine":
        """CudaKnnEngine::new over MmapStorage::open(path): the base streams from the mapped file
        to the GPU with no host copy."""
        self = cls.__new__(cls)
        n, d = ctypes.c_size_t(), ctypes.c_size_t()
        _check(_lib.vhip_vecrstor_open(_path(path), ctypes.byref(n), ctypes.byref(d)))
        h = _vp()
        _check(_lib.vhip_knn_create_from_vecrstor(_path(path), int(metric), ordinal, ctypes.byref(h)))
        self._h = h
        self._dim = d.value
        return self

    @classmethod
    def with_ordinal(cls, dataset, dimension, metric, ordinal):
        return cls(dataset, dimension, metric, ordinal)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            _lib.vhip_knn_destroy(h)
            self._h = None

    def search_batch_arrays(self, queries, k: int):
        """Returns (ids[nq, k] u32, dist[nq, k] f32, lens[nq]); entries past lens are empty."""
        q = _rows(queries, self._dim) if np.asarray(queries).size else np.zeros((0, self._dim), np.float32)
        nq = q.shape[0]
        ids = np.empty((nq, max(k, 1)), np.uint32)
        dist = np.empty((nq, max(k, 1)), np.float32)
        lens = np.zeros(nq, np.uintp)
        _check(_lib.vhip_knn_search_batch(self._h, _p(q, _f32p), nq, k, _p(ids, _u32p), _p(dist, _f32p),
                                          _p(lens, _szp)))
        return ids[:, :k], dist[:, :k], lens

    def search_batch(self, queries, k: int) -> List[List[SearchResult]]:
        return _to_lists(*self.search_batch_arrays(queries, k))

    def search(self, query, k: int) -> List[SearchResult]:
        r = self.search_batch(query, k)
        return r[0] if r else []

    def search_batch_device(self, d_queries: int, nq: int, k: int, d_ids: int, d_dist: int):
        """Queries / outputs are device pointers (ints) on the engine's GPU."""
        _check(_lib.vhip_knn_search_batch_device(self._h, d_queries, nq, k, d_ids, d_dist))

    def search_batch_device_noalloc(self, d_queries: int, nq: int, k: int, d_ids: int, d_dist: int):
        """As search_batch_device, with working memory from the library's fixed per-GPU array of
        NOALLOC_SCRATCH_BYTES (no device allocation); same results."""
        _check(_lib.vhip_knn_search_batch_device_noalloc(self._h, d_queries, nq, k, d_ids, d_dist))

    def context(self) -> CudaDeviceContext:
        """knn.rs:381-383: the context of the engine's GPU."""
        return CudaDeviceContext(_lib.vhip_knn_device_id(self._h))

    def dimension(self) -> int:
        return _lib.vhip_knn_dimension(self._h)

    def num_vectors(self) -> int:
        return _lib.vhip_knn_num_vectors(self._h)

    def metric(self) -> DistanceMetric:
        return DistanceMetric(_lib.vhip_knn_metric(self._h))

    def device_id(self) -> int:
        return _lib.vhip_knn_device_id(self._h)


class DistributedKnnEngine:
    """ddp/distributed_knn.rs:24-262 (all ranks on one GPU)."""

    def __init__(self, handle):
        self._h = handle

    @classmethod
    def _make(cls, fn, dataset, dimension, num_gpus, mode, metric):
        if num_gpus < 1:
            raise InvalidConfig("num_gpus must be at least 1")
        base = _rows(dataset, dimension) if np.asarray(dataset).size else np.zeros((0, dimension), np.float32)
        h = _vp()
        _check(fn(_p(base, _f32p), base.shape[0], base.shape[1], num_gpus, int(mode), int(metric), ctypes.byref(h)))
        e = cls(h)
        e._dim = base.shape[1]
        return e

    @classmethod
    def try_new(cls, dataset, dimension, num_gpus, mode=GpuShardMode.Sharded, metric=DistanceMetric.L2Squared):
        return cls._make(_lib.vhip_dknn_try_new, dataset, dimension, num_gpus, mode, metric)

    @classmethod
    def emulator(cls, dataset, dimension, num_gpus, mode=GpuShardMode.Sharded, metric=DistanceMetric.L2Squared):
        return cls._make(_lib.vhip_dknn_emulator, dataset, dimension, num_gpus, mode, metric)

    @classmethod
    def new(cls, dataset, dimension, num_gpus, mode=GpuShardMode.Sharded, metric=DistanceMetric.L2Squared):
        return cls.try_new(dataset, dimension, num_gpus, mode, metric)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            _lib.vhip_dknn_destroy(h)
            self._h = None

    def search_batch_arrays(self, queries, k: int):
        q = _rows(queries, self._dim) if np.asarray(queries).size else np.zeros((0, self._dim), np.float32)
        nq = q.shape[0]
        ids = np.empty((nq, max(k, 1)), np.uint32)
        dist = np.empty((nq, max(k, 1)), np.float32)
        lens = np.zeros(nq, np.uintp)
        _check(_lib.vhip_dknn_search_batch(self._h, _p(q, _f32p), nq, k, _p(ids, _u32p), _p(dist, _f32p),
                                           _p(lens, _szp)))
        return ids[:, :k], dist[:, :k], lens

    def search_batch(self, queries, k: int) -> List[List[SearchResult]]:
        return _to_lists(*self.search_batch_arrays(queries, k))

    def search(self, query, k: int) -> List[SearchResult]:
        r = self.search_batch(query, k)
        return r[0] if r else []

    def num_gpus(self) -> int:
        return _lib.vhip_dknn_num_gpus(self._h)

    def mode(self) -> GpuShardMode:
        return GpuShardMode(_lib.vhip_dknn_mode(self._h))

    def dimension(self) -> int:
        return _lib.vhip_dknn_dimension(self._h)

    def num_vectors(self) -> int:
        return _lib.vhip_dknn_num_vectors(self._h)

    def metric(self) -> DistanceMetric:
        return DistanceMetric(_lib.vhip_dknn_metric(self._h))


class CollectiveOps:
    """ddp/collective.rs: only top_k_reduce is on the single-GPU path."""

    @staticmethod
    def top_k_reduce(partial_results_per_rank: Sequence[Sequence[SearchResult]], k: int,
                     metric=DistanceMetric.L2Squared) -> List[SearchResult]:
        flat = [r for rank in partial_results_per_rank for r in rank]
        if not flat or k == 0:
            return []
        ids = np.array([r[0] for r in flat], np.uint32)
        dist = np.array([r[1] for r in flat], np.float32)
        oi = np.empty(k, np.uint32)
        od = np.empty(k, np.float32)
        m = _lib.vhip_top_k_reduce(_p(ids, _u32p), _p(dist, _f32p), ids.size, k, int(metric), _p(oi, _u32p),
                                   _p(od, _f32p))
        return [SearchResult(int(oi[i]), float(od[i])) for i in range(m)]


class HammingKnnEngine(_Profiled):
    """Packed-bit Hamming kNN over uint32 code words (extension; exact integer distances)."""

    _prof_fn = _lib.vhip_hamming_profile
    _read_fn = _lib.vhip_hamming_profile_read

    def __init__(self, codes, ordinal: int = 0):
        c = np.ascontiguousarray(codes, dtype=np.uint32)
        if c.ndim != 2:
            raise InvalidConfig("codes must be [n, words]")
        self._words = c.shape[1]
        h = _vp()
        _check(_lib.vhip_hamming_create(_p(c, _u32p), c.shape[0], c.shape[1], ordinal, ctypes.byref(h)))
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            _lib.vhip_hamming_destroy(h)
            self._h = None

    def search_batch_arrays(self, queries, k: int):
        q = np.ascontiguousarray(queries, dtype=np.uint32).reshape(-1, self._words)
        nq = q.shape[0]
        ids = np.empty((nq, max(k, 1)), np.uint32)
        dist = np.empty((nq, max(k, 1)), np.uint32)
        lens = np.zeros(nq, np.uintp)
        _check(_lib.vhip_hamming_search_batch(self._h, _p(q, _u32p), nq, k, _p(ids, _u32p), _p(dist, _u32p),
                                              _p(lens, _szp)))
        return ids[:, :k], dist[:, :k], lens

    def search_batch_device(self, d_queries: int, nq: int, k: int, d_ids: int, d_dist: int):
        _check(_lib.vhip_hamming_search_batch_device(self._h, d_queries, nq, k, d_ids, d_dist))


# ---- k-means -------------------------------------------------------------------------------
class CudaKMeansResult(NamedTuple):
    """kmeans.rs:15-35."""

    centroids: np.ndarray
    dimension: int
    k: int
    iterations: int
    inertia: float

    def centroid(self, i: int) -> np.ndarray:
        return self.centroids[i]


INIT_KMEANSPP = 0
INIT_SHUFFLE = 1


def _kmeans_fit(data, dimension, k, max_iters, tolerance, metric, init, init_mode, seed, ordinal, want_assign):
    x = _rows(data, dimension) if np.asarray(data).size else np.zeros((0, dimension), np.float32)
    n, d = x.shape
    ek = min(k, n)
    cent = np.zeros((max(ek, 1), d), np.float32)
    assign = np.zeros(max(n, 1), np.int32) if want_assign else None
    init_arr = None
    if init is not None:
        init_arr = np.ascontiguousarray(init, dtype=np.float32).reshape(-1, d)
        if init_arr.shape[0] < ek:
            raise InvalidConfig("init_centroids has fewer than min(k, n) rows")
    res = _KMeansResultC()
    _check(_lib.vhip_kmeans_fit(ordinal, _p(x, _f32p), n, d, k, max_iters, float(tolerance), int(metric),
                                _p(init_arr, _f32p) if init_arr is not None else None, init_mode, seed,
                                _p(cent, _f32p), _p(assign, _i32p) if assign is not None else None,
                                ctypes.byref(res)))
    r = CudaKMeansResult(cent[:res.k].copy(), int(res.dimension), int(res.k), int(res.iterations), float(res.inertia))
    return (r, assign[:n]) if want_assign else r


class CudaKMeansEngine:
    """kmeans.rs:37-467 -- fit() runs on the GPU; init is k-means++ seeded by `seed`
    unless explicit init centroids are given.  fit_cpu (kmeans.rs:240-357) is the reference's
    host code and is not mirrored: this binding covers the GPU path only."""

    def __init__(self, ordinal: int = 0):
        self._ord = ordinal
        self._ctx = CudaDeviceContext(ordinal)

    @classmethod
    def new(cls):
        return cls(0)

    def context(self) -> CudaDeviceContext:
        return self._ctx

    def fit(self, data, dimension, k, max_iters, tolerance, metric=DistanceMetric.L2Squared, init=None,
            seed: int = 42, return_assign: bool = False):
        return _kmeans_fit(data, dimension, k, max_iters, tolerance, metric, init, INIT_KMEANSPP, seed, self._ord,
                           return_assign)


class DistributedKMeansEngine:
    """ddp/distributed_kmeans.rs:19-541 at one GPU: try_new validates the device count and
    fit() runs on GPU 0 with a seeded shuffle init (the reference's init_random)."""

    def __init__(self, num_gpus: int):
        if num_gpus < 1:
            raise InvalidConfig("num_gpus must be at least 1")
        self._g = num_gpus

    @classmethod
    def try_new(cls, num_gpus: int):
        if num_gpus < 1:
            raise InvalidConfig("num_gpus must be at least 1")
        _check(_lib.vhip_dkmeans_check(num_gpus))
        return cls(num_gpus)

    @classmethod
    def emulator(cls, num_gpus: int):
        return cls(num_gpus)

    @classmethod
    def new(cls, num_gpus: int):
        return cls.try_new(num_gpus)

    def num_gpus(self) -> int:
        return self._g

    def fit(self, data, dimension, k, max_iters, tolerance, metric=DistanceMetric.L2Squared, init=None,
            seed: int = 42, return_assign: bool = False):
        return _kmeans_fit(data, dimension, k, max_iters, tolerance, metric, init, INIT_SHUFFLE, seed, 0,
                           return_assign)


class KMeansState(_Profiled):
    """Resident k-means state: set centroids, run iterations, read back (per-iteration
    parity checks and benchmarks)."""

    def __init__(self, data, metric=DistanceMetric.L2Squared, ordinal: int = 0):
        type(self)._prof_fn = _lib.vhip_kmeans_profile
        type(self)._read_fn = _lib.vhip_kmeans_profile_read
        x = _rows(data, None)
        self._n, self._d = x.shape
        self._k = 0
        h = _vp()
        _check(_lib.vhip_kmeans_create(ordinal, _p(x, _f32p), self._n, self._d, int(metric), ctypes.byref(h)))
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            _lib.vhip_kmeans_destroy(h)
            self._h = None

    @classmethod
    def from_vecrstor(cls, paths, metric=DistanceMetric.L2Squared, ordinal: int = 0) -> "KMeansState":
        """A state over the rows of one or more VECRSTOR files, uploaded from the mapped files one
        after another (no concatenated host copy)."""
        paths = [paths] if isinstance(paths, (str, bytes, os.PathLike)) else list(paths)
        n, d = 0, 0
        for pth in paths:
            fn, fd = ctypes.c_size_t(), ctypes.c_size_t()
            _check(_lib.vhip_vecrstor_open(_path(pth), ctypes.byref(fn), ctypes.byref(fd)))
            n, d = n + fn.value, fd.value
        arr = (ctypes.c_char_p * len(paths))(*[_path(pth) for pth in paths])
        self = cls.__new__(cls)
        type(self)._prof_fn = _lib.vhip_kmeans_profile
        type(self)._read_fn = _lib.vhip_kmeans_profile_read
        h = _vp()
        _check(_lib.vhip_kmeans_create_from_vecrstor(ordinal, arr, len(paths), int(metric), ctypes.byref(h)))
        self._h, self._n, self._d, self._k = h, n, d, 0
        return self

    def fit(self, k: int, max_iters: int, tolerance: float, init=None, init_mode: int = 0, seed: int = 42):
        """CudaKMeansEngine::fit on the resident points: (centroids [k, d], assign int32[n], result)."""
        ek = min(k, self._n)
        c = np.zeros((max(ek, 1), self._d), np.float32)
        a = np.zeros(max(self._n, 1), np.int32)
        ini = None if init is None else np.ascontiguousarray(init, dtype=np.float32).reshape(-1, self._d)
        res = _KMeansResultC()
        _check(_lib.vhip_kmeans_fit_state(self._h, k, max_iters, float(tolerance),
                                          _p(ini, _f32p) if ini is not None else None, init_mode, seed,
                                          _p(c, _f32p), _p(a, _i32p), ctypes.byref(res)))
        self._k = ek
        return c[:ek], a[:self._n], (int(res.dimension), int(res.k), int(res.iterations), float(res.inertia))

    def set_centroids(self, centroids):
        c = np.ascontiguousarray(centroids, dtype=np.float32).reshape(-1, self._d)
        self._k = c.shape[0]
        _check(_lib.vhip_kmeans_set_centroids(self._h, _p(c, _f32p), self._k))

    def run(self, iters: int = 1):
        _check(_lib.vhip_kmeans_run(self._h, iters))

    def assign_only(self, residuals: bool = False):
        """Nearest centroid of every point without an update: (assign int32[n], score f32[n],
        residual f32[n, d] or None).  Scores are the metric values KMeans::find_nearest_centroid
        returns (ivf/kmeans.rs:262-309)."""
        a = np.empty(self._n, np.int32)
        sc = np.empty(self._n, np.float32)
        r = np.empty((self._n, self._d), np.float32) if residuals else None
        _check(_lib.vhip_kmeans_assign_only(self._h, _p(a, _i32p), _p(sc, _f32p),
                                            _p(r, _f32p) if r is not None else None))
        return a, sc, r

    def read(self) -> dict:
        c = np.empty((self._k, self._d), np.float32)
        a = np.empty(self._n, np.int32)
        cnt = np.empty(self._k, np.int64)
        sh = np.empty(self._k, np.float32)
        ms = np.zeros(1, np.float32)
        ine = np.zeros(1, np.float32)
        _check(_lib.vhip_kmeans_read(self._h, _p(c, _f32p), _p(a, _i32p), _p(cnt, _i64p), _p(sh, _f32p),
                                     _p(ms, _f32p), _p(ine, _f32p)))
        return {"centroids": c, "assign": a, "counts": cnt, "shifts": sh, "max_shift": float(ms[0]),
                "inertia": float(ine[0])}


# ---- IVF coarse quantizer (ivf/mod.rs:106-133, ivf/kmeans.rs:262-356) -------------------
class IvfCoarseQuantizer:
    """The coarse stage of IvfPqIndex on the GPU: find_nearest_centroid for every vector of a
    build (plus the residuals x - c of the PQ stage) and find_top_centroids for query batches."""

    def __init__(self, centroids, dimension: int, metric=DistanceMetric.L2Squared, ordinal: int = 0):
        c = _rows(centroids, dimension)
        self._nlist, self._d = c.shape
        self.metric = DistanceMetric(int(metric))
        h = _vp()
        _check(_lib.vhip_coarse_create(_p(c, _f32p), self._nlist, self._d, int(metric), ordinal, ctypes.byref(h)))
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            _lib.vhip_coarse_destroy(h)
            self._h = None

    def nlist(self) -> int:
        return int(_lib.vhip_coarse_nlist(self._h))

    def dimension(self) -> int:
        return int(_lib.vhip_coarse_dimension(self._h))

    def assign(self, points, residuals: bool = False):
        """(cluster uint32[n], score float32[n], residual float32[n, d] or None)."""
        x = _rows(points, self._d) if np.asarray(points).size else np.zeros((0, self._d), np.float32)
        n = x.shape[0]
        cl = np.empty(n, np.uint32)
        sc = np.empty(n, np.float32)
        r = np.empty((n, self._d), np.float32) if residuals else None
        _check(_lib.vhip_coarse_assign(self._h, _p(x, _f32p), n, _p(cl, _u32p), _p(sc, _f32p),
                                       _p(r, _f32p) if r is not None else None))
        return cl, sc, r

    def find_nearest_centroid(self, vector):
        """ivf/kmeans.rs:262-309 for one vector: (index, score)."""
        cl, sc, _ = self.assign(np.asarray(vector, np.float32).reshape(1, self._d))
        return int(cl[0]), float(sc[0])

    def probe_batch(self, queries, nprobe: int):
        """find_top_centroids for each query: (ids [nq, p], scores [nq, p], lens [nq])."""
        q = _rows(queries, self._d) if np.asarray(queries).size else np.zeros((0, self._d), np.float32)
        nq = q.shape[0]
        w = max(nprobe, 1)
        ids = np.empty((max(nq, 1), w), np.uint32)
        sc = np.empty((max(nq, 1), w), np.float32)
        lens = np.zeros(max(nq, 1), np.uintp)
        _check(_lib.vhip_coarse_probe(self._h, _p(q, _f32p), nq, nprobe, _p(ids, _u32p), _p(sc, _f32p),
                                      lens.ctypes.data_as(_szp)))
        return ids[:nq, :nprobe], sc[:nq, :nprobe], lens[:nq]

    def find_top_centroids(self, query, nprobe: int):
        """ivf/kmeans.rs:311-356: [(index, score)] best first, min(nprobe, nlist) entries."""
        ids, sc, lens = self.probe_batch(np.asarray(query, np.float32).reshape(1, self._d), nprobe)
        return [(int(ids[0, j]), float(sc[0, j])) for j in range(int(lens[0]))] if nprobe else []


# ---- files of the offline trainer (storage/mmap.rs, ivf/serializer.rs) -------------------
def _path(p) -> bytes:
    return os.fsencode(os.fspath(p))


class MmapStorage:
    """VECRSTOR vector files (storage/mmap.rs:9-16): create / create_from_flat write one, open
    validates the header and maps the file read-only (numpy memmap), so as_raw_slice() is a
    view of the mapping: engines built from it upload straight from the page cache."""

    def __init__(self, data: np.ndarray, dimension: int):
        self._data = data
        self._dim = dimension

    @staticmethod
    def create(path, dimension: int, vectors) -> None:
        for v in vectors:
            if len(v) != dimension:
                raise InvalidConfig(f"dimension mismatch: expected {dimension}, got {len(v)}")
        flat = np.concatenate([np.asarray(v, np.float32) for v in vectors]) if len(vectors) else np.zeros(0, np.float32)
        MmapStorage.create_from_flat(path, dimension, flat)

    @staticmethod
    def create_from_flat(path, dimension: int, flat_data) -> None:
        f = np.ascontiguousarray(flat_data, dtype=np.float32).reshape(-1)
        if dimension == 0 or f.size % dimension:
            raise InvalidConfig(f"dimension mismatch: expected {dimension}, got {f.size % max(dimension, 1)}")
        _check(_lib.vhip_vecrstor_write(_path(path), _p(f, _f32p), f.size // dimension, dimension))

    @classmethod
    def open(cls, path) -> "MmapStorage":
        n = ctypes.c_size_t()
        d = ctypes.c_size_t()
        _check(_lib.vhip_vecrstor_open(_path(path), ctypes.byref(n), ctypes.byref(d)))
        if n.value * d.value == 0:
            return cls(np.zeros((n.value, d.value), np.float32), d.value)
        data = np.memmap(os.fspath(path), dtype="<f4", mode="r", offset=24, shape=(n.value, d.value))
        return cls(data, d.value)

    def dimension(self) -> int:
        return self._dim

    def __len__(self) -> int:
        return self._data.shape[0]

    def is_empty(self) -> bool:
        return len(self) == 0

    def get(self, i: int) -> np.ndarray:
        if not 0 <= i < len(self):
            raise IndexError(f"vector id {i} out of bounds (len={len(self)})")
        return self._data[i]

    def as_raw_slice(self) -> np.ndarray:
        return self._data.reshape(-1)


class CentroidFileData(NamedTuple):
    """ivf/serializer.rs:380-393."""

    centroids: np.ndarray
    dimension: int
    k: int
    metric: DistanceMetric
    iterations: int
    inertia: float


def save_centroid_file(path, centroids, dimension: int, k: int, metric, iterations: int, inertia: float) -> None:
    """IvfPqSerializer::save_centroid_file (ivf/serializer.rs:264-306)."""
    c = np.ascontiguousarray(centroids, dtype=np.float32).reshape(-1)
    if c.size != k * dimension:
        raise InvalidConfig("centroids must hold k x dimension floats")
    _check(_lib.vhip_centroid_file_save(_path(path), _p(c, _f32p), dimension, k, int(metric), iterations,
                                        float(inertia)))


def load_centroid_file(path) -> CentroidFileData:
    """IvfPqSerializer::load_centroid_file (ivf/serializer.rs:309-360)."""
    d, k, it = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
    m = _int()
    ine = np.zeros(1, np.float32)
    _check(_lib.vhip_centroid_file_info(_path(path), ctypes.byref(d), ctypes.byref(k), ctypes.byref(m),
                                        ctypes.byref(it), _p(ine, _f32p)))
    c = np.empty(k.value * d.value, np.float32)
    _check(_lib.vhip_centroid_file_load(_path(path), _p(c, _f32p), k.value, d.value))
    return CentroidFileData(c, d.value, k.value, DistanceMetric(m.value), it.value, float(ine[0]))


def fit_cuda_aware(all_data, dimension: int, k: int, max_iters: int, tolerance: float, metric=DistanceMetric.L2Squared,
                   num_gpus: int = 1, seed: int = 42) -> CudaKMeansResult:
    """vector-mpi fit_cuda_aware (src/distributed_kmeans.rs:375-415): one GPU runs the fit for any
    num_gpus (more than present is the emulator there, the same one GPU here)."""
    if max(num_gpus, 1) > 1:
        return DistributedKMeansEngine.emulator(num_gpus).fit(all_data, dimension, k, max_iters, tolerance, metric,
                                                              seed=seed)
    return CudaKMeansEngine(0).fit(all_data, dimension, k, max_iters, tolerance, metric, seed=seed)


def train_from_shards(data_dir, k: int = 64, max_iters: int = 30, tolerance: float = 1e-4,
                      metric=DistanceMetric.L2Squared, num_gpus: int = 1, output: str = "centroids_global.bin",
                      seed: int = 42):
    """mpi_kmeans --use-cuda (src/bin/mpi_kmeans.rs:284-364): shard_*.bin in data_dir ->
    data_dir/output.  Returns (result, number of shards read)."""
    res = _KMeansResultC()
    ns = ctypes.c_size_t()
    _check(_lib.vhip_train_from_shards(_path(data_dir), k, max_iters, float(tolerance), int(metric), num_gpus,
                                       output.encode(), seed, ctypes.byref(res), ctypes.byref(ns)))
    return (int(res.dimension), int(res.k), int(res.iterations), float(res.inertia)), int(ns.value)


# ---- product quantization and the IVF-PQ index (vector-index/src/ivf) -------------------
@dataclasses.dataclass
class IvfPqConfig:
    """IvfPqConfig (ivf/config.rs:25-154): defaults of config.rs:6-21, builder methods, validate."""

    nlist: int = 64
    nprobe: int = 8
    num_subvectors: int = 8
    sub_clusters: int = 256
    max_kmeans_iters: int = 25
    kmeans_tolerance: float = 1e-4
    max_train_points: Optional[int] = None

    def __post_init__(self):
        self.kmeans_tolerance = float(np.float32(self.kmeans_tolerance))  # an f32 field in the reference

    @classmethod
    def new(cls, nlist: int, nprobe: int, num_subvectors: int) -> "IvfPqConfig":
        return cls(nlist=nlist, nprobe=nprobe, num_subvectors=num_subvectors)

    def with_sub_clusters(self, sub_clusters: int) -> "IvfPqConfig":
        return dataclasses.replace(self, sub_clusters=sub_clusters)

    def with_max_kmeans_iters(self, iters: int) -> "IvfPqConfig":
        return dataclasses.replace(self, max_kmeans_iters=iters)

    def with_kmeans_tolerance(self, tol: float) -> "IvfPqConfig":
        return dataclasses.replace(self, kmeans_tolerance=tol)

    def with_max_train_points(self, max_points: Optional[int]) -> "IvfPqConfig":
        return dataclasses.replace(self, max_train_points=max_points)

    def sub_dimension(self, dimension: int) -> int:
        return dimension // self.num_subvectors if self.num_subvectors else 0

    def _c(self) -> "_IvfPqConfigC":
        for f in ("nlist", "nprobe", "num_subvectors", "sub_clusters", "max_kmeans_iters"):
            if getattr(self, f) < 0:
                raise InvalidConfig(f"{f} must be non-negative")
        return _IvfPqConfigC(self.nlist, self.nprobe, self.num_subvectors, self.sub_clusters, self.max_kmeans_iters,
                             float(self.kmeans_tolerance), self.max_train_points or 0)

    @classmethod
    def _from_c(cls, c) -> "IvfPqConfig":
        return cls(int(c.nlist), int(c.nprobe), int(c.num_subvectors), int(c.sub_clusters), int(c.max_kmeans_iters),
                   float(c.kmeans_tolerance), int(c.max_train_points) or None)

    def validate(self, dimension: int) -> None:
        """config.rs:96-147: raises InvalidConfig with the reference's reason."""
        c = self._c()
        _check(_lib.vhip_ivfpq_config_validate(ctypes.byref(c), dimension))


class ProductQuantizer:
    """ProductQuantizer (ivf/pq.rs:12-293): M codebooks of Ks sub-centroids over D / M dimensions.
    train / encode_batch / compute_adc_lut run on the GPU; decode and compute_distance_with_lut
    are the reference's host helpers."""

    def __init__(self, dimension: int, num_subvectors: int, sub_clusters: int, codebooks, ordinal: int = 0):
        if num_subvectors == 0 or dimension % num_subvectors:
            raise InvalidConfig(f"vector dimension ({dimension}) must be divisible by num_subvectors "
                                f"({num_subvectors})")
        cb = np.ascontiguousarray(codebooks, dtype=np.float32).reshape(-1)
        ds = dimension // num_subvectors
        if cb.size != num_subvectors * sub_clusters * ds:  # pq.rs:38-41
            raise InvalidConfig("codebooks must hold num_subvectors x sub_clusters x sub_dimension floats")
        self.dimension = dimension
        self.num_subvectors = num_subvectors
        self.sub_dimension = ds
        self.sub_clusters = sub_clusters
        self.codebooks = cb
        self.ordinal = ordinal

    @classmethod
    def new(cls, dimension: int, num_subvectors: int, sub_clusters: int, codebooks) -> "ProductQuantizer":
        return cls(dimension, num_subvectors, sub_clusters, codebooks)

    @classmethod
    def train(cls, data, dimension: int, num_subvectors: int, sub_clusters: int, max_iters: int, tolerance: float,
              metric=DistanceMetric.L2Squared, seed: int = 42, init_codebooks=None,
              ordinal: int = 0) -> "ProductQuantizer":
        """pq.rs:53-107 (sub-space k-means on the GPU; seeded init, or init_codebooks)."""
        x = _rows(data, dimension) if np.asarray(data).size else np.zeros((0, dimension), np.float32)
        if num_subvectors == 0 or dimension % num_subvectors:
            raise InvalidConfig(f"vector dimension ({dimension}) must be divisible by num_subvectors "
                                f"({num_subvectors})")
        cb = np.zeros(num_subvectors * sub_clusters * (dimension // num_subvectors), np.float32)
        ini = None if init_codebooks is None else np.ascontiguousarray(init_codebooks, dtype=np.float32).reshape(-1)
        if ini is not None and ini.size != cb.size:
            raise InvalidConfig("init_codebooks must hold num_subvectors x sub_clusters x sub_dimension floats")
        _check(_lib.vhip_pq_train(ordinal, _p(x, _f32p), x.shape[0], dimension, num_subvectors, sub_clusters,
                                  max_iters, float(tolerance), int(metric), _p(ini, _f32p) if ini is not None else None,
                                  seed, _p(cb, _f32p)))
        return cls(dimension, num_subvectors, sub_clusters, cb, ordinal)

    train_sequential = train  # pq.rs:112-165: the same result, one sub-space after another

    def get_sub_centroid(self, m: int, k: int) -> np.ndarray:
        s = (m * self.sub_clusters + k) * self.sub_dimension
        return self.codebooks[s:s + self.sub_dimension]

    def encode_batch(self, data, metric=DistanceMetric.L2Squared) -> np.ndarray:
        """pq.rs:203-214: codes [n, M] uint8."""
        x = _rows(data, self.dimension) if np.asarray(data).size else np.zeros((0, self.dimension), np.float32)
        out = np.zeros((x.shape[0], self.num_subvectors), np.uint8)
        _check(_lib.vhip_pq_encode(self.ordinal, _p(self.codebooks, _f32p), self.dimension, self.num_subvectors,
                                   self.sub_clusters, int(metric), _p(x, _f32p), x.shape[0], _p(out, _u8p)))
        return out

    def encode(self, vector, metric=DistanceMetric.L2Squared) -> np.ndarray:
        """pq.rs:178-200."""
        v = np.asarray(vector, np.float32).reshape(-1)
        if v.size != self.dimension:
            raise DimensionMismatch(self.dimension, v.size)
        return self.encode_batch(v.reshape(1, -1), metric)[0]

    def decode(self, code) -> np.ndarray:
        """pq.rs:217-229."""
        c = np.asarray(code, np.uint8).reshape(-1)
        if c.size != self.num_subvectors:
            raise InvalidConfig("code length must equal num_subvectors")
        return np.concatenate([self.get_sub_centroid(m, int(c[m])) for m in range(self.num_subvectors)])

    def compute_adc_lut_batch(self, queries, metric=DistanceMetric.L2Squared) -> np.ndarray:
        """compute_adc_lut for a batch: [nq, M * Ks]."""
        q = _rows(queries, self.dimension)
        lut = np.zeros((q.shape[0], self.num_subvectors * self.sub_clusters), np.float32)
        _check(_lib.vhip_pq_adc_lut(self.ordinal, _p(self.codebooks, _f32p), self.dimension, self.num_subvectors,
                                    self.sub_clusters, int(metric), _p(q, _f32p), q.shape[0], _p(lut, _f32p)))
        return lut

    def compute_adc_lut(self, query, metric=DistanceMetric.L2Squared) -> np.ndarray:
        """pq.rs:233-266: lut[m * Ks + k]."""
        q = np.asarray(query, np.float32).reshape(-1)
        if q.size != self.dimension:
            raise DimensionMismatch(self.dimension, q.size)
        return self.compute_adc_lut_batch(q.reshape(1, -1), metric)[0]

    def compute_distance_with_lut(self, code, lut) -> float:
        """pq.rs:270-293: quads summed as (d0 + d1) + (d2 + d3), then the remainder, in f32."""
        c = np.asarray(code, np.uint8).reshape(-1)
        t = np.asarray(lut, np.float32).reshape(-1)
        ks = self.sub_clusters
        total = np.float32(0.0)
        m = 0
        while m + 4 <= c.size:
            d = [t[(m + j) * ks + int(c[m + j])] for j in range(4)]
            total = np.float32(total + np.float32(np.float32(d[0] + d[1]) + np.float32(d[2] + d[3])))
            m += 4
        while m < c.size:
            total = np.float32(total + t[m * ks + int(c[m])])
            m += 1
        return float(total)

    def __eq__(self, other):
        return (isinstance(other, ProductQuantizer) and
                (self.dimension, self.num_subvectors, self.sub_clusters) ==
                (other.dimension, other.num_subvectors, other.sub_clusters) and
                np.array_equal(self.codebooks, other.codebooks))


@dataclasses.dataclass
class InvertedList:
    """ivf/inverted_list.rs:8-56: ids and M-byte codes of one coarse cluster."""

    ids: np.ndarray
    codes: np.ndarray  # [len, M] uint8

    def __len__(self) -> int:
        return int(self.ids.size)

    def len(self) -> int:
        return len(self)

    def is_empty(self) -> bool:
        return self.ids.size == 0

    def get_code(self, index: int, num_subvectors: int) -> np.ndarray:
        return self.codes.reshape(-1)[index * num_subvectors:(index + 1) * num_subvectors]

    def __eq__(self, other):
        return (isinstance(other, InvertedList) and np.array_equal(self.ids, other.ids) and
                np.array_equal(self.codes.reshape(-1), other.codes.reshape(-1)))


class InvertedIndex:
    """ivf/inverted_list.rs:58-120 (host view of an index's lists)."""

    def __init__(self, nlist: int, num_subvectors: int):
        self.lists = [InvertedList(np.zeros(0, np.uint32), np.zeros((0, num_subvectors), np.uint8))
                      for _ in range(nlist)]
        self.num_subvectors = num_subvectors
        self._total = 0

    def add(self, cluster_id: int, id: int, code) -> None:
        c = np.asarray(code, np.uint8).reshape(1, -1)
        if c.shape[1] != self.num_subvectors:
            raise InvalidConfig("code length must equal num_subvectors")
        L = self.lists[cluster_id]
        self.lists[cluster_id] = InvertedList(np.append(L.ids, np.uint32(id)), np.vstack([L.codes, c]))
        self._total += 1

    def total_vectors(self) -> int:
        return self._total

    def nlist(self) -> int:
        return len(self.lists)

    def get_list(self, cluster_id: int) -> InvertedList:
        return self.lists[cluster_id]

    def _csr(self):
        sizes = np.array([len(L) for L in self.lists], np.uint32)
        ids = np.concatenate([L.ids for L in self.lists]).astype(np.uint32) if self.lists else np.zeros(0, np.uint32)
        codes = (np.concatenate([L.codes.reshape(-1, self.num_subvectors) for L in self.lists]).astype(np.uint8)
                 if self.lists else np.zeros((0, self.num_subvectors), np.uint8))
        return sizes, np.ascontiguousarray(ids), np.ascontiguousarray(codes)

    @classmethod
    def from_csr(cls, sizes, ids, codes, num_subvectors) -> "InvertedIndex":
        """Lists from CSR parts: list c holds sizes[c] consecutive entries of ids / codes."""
        ix = cls(0, num_subvectors)
        codes = np.asarray(codes, np.uint8).reshape(-1, num_subvectors)
        off = 0
        for n in sizes.tolist():
            ix.lists.append(InvertedList(ids[off:off + n].copy(), codes[off:off + n].reshape(n, num_subvectors).copy()))
            off += n
        ix._total = off
        return ix

    def __eq__(self, other):
        return (isinstance(other, InvertedIndex) and self.num_subvectors == other.num_subvectors and
                self._total == other._total and self.lists == other.lists)


class IvfPqSerializer:
    """ivf/serializer.rs:23-254 (IVFPQVEC files)."""

    @staticmethod
    def save_to_file(path, config: IvfPqConfig, coarse_centroids, pq: ProductQuantizer,
                     inverted_index: InvertedIndex, dimension: int, metric) -> None:
        c = config._c()
        cc = np.ascontiguousarray(coarse_centroids, dtype=np.float32).reshape(-1)
        sizes, ids, codes = inverted_index._csr()
        _check(_lib.vhip_ivfpq_file_save(_path(path), ctypes.byref(c), dimension, int(metric), _p(cc, _f32p),
                                         cc.size // max(dimension, 1), _p(pq.codebooks, _f32p), pq.codebooks.size,
                                         _p(sizes, _u32p), sizes.size, _p(ids, _u32p), _p(codes, _u8p)))

    @staticmethod
    def load_from_file(path):
        """(config, coarse_centroids, pq, inverted_index, dimension, metric)."""
        c = _IvfPqConfigC()
        d, nc, cbl, nl, tot = (ctypes.c_size_t() for _ in range(5))
        m = _int()
        _check(_lib.vhip_ivfpq_file_info(_path(path), ctypes.byref(c), ctypes.byref(d), ctypes.byref(m),
                                         ctypes.byref(nc), ctypes.byref(cbl), ctypes.byref(nl), ctypes.byref(tot)))
        cfg = IvfPqConfig._from_c(c)
        coarse = np.zeros(nc.value * d.value, np.float32)
        cb = np.zeros(cbl.value, np.float32)
        sizes = np.zeros(nl.value, np.uint32)
        ids = np.zeros(max(tot.value, 1), np.uint32)
        codes = np.zeros(max(tot.value * cfg.num_subvectors, 1), np.uint8)
        _check(_lib.vhip_ivfpq_file_load(_path(path), _p(coarse, _f32p), _p(cb, _f32p), _p(sizes, _u32p),
                                         _p(ids, _u32p), _p(codes, _u8p)))
        pq = ProductQuantizer(d.value, cfg.num_subvectors, cfg.sub_clusters, cb)
        inv = InvertedIndex.from_csr(sizes, ids[:tot.value], codes[:tot.value * cfg.num_subvectors],
                                      cfg.num_subvectors)
        return cfg, coarse, pq, inv, d.value, DistanceMetric(m.value)


def _storage_rows(storage, dimension: Optional[int] = None) -> np.ndarray:
    if isinstance(storage, MmapStorage):
        return storage.as_raw_slice().reshape(-1, storage.dimension()) if len(storage) else np.zeros(
            (0, storage.dimension()), np.float32)
    a = np.asarray(storage, dtype=np.float32)
    if a.size == 0:
        return np.zeros((0, dimension or (a.shape[1] if a.ndim == 2 else 0)), np.float32)
    return _rows(a, dimension)


class IvfPqIndex:
    """IvfPqIndex (ivf/mod.rs:63-449) on one GPU: coarse centroids, product quantizer and
    inverted lists resident in device memory.  `storage` is an MmapStorage or an [n, d] array."""

    def __init__(self, handle, storage, config: IvfPqConfig, metric):
        self._h = handle
        self._storage = storage
        self._config = config
        self._metric = DistanceMetric(int(metric))
        info = _IvfPqDescC()
        _check(_lib.vhip_ivfpq_info(handle, ctypes.byref(info)))
        self._info = info
        self._parts = None

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            _lib.vhip_ivfpq_destroy(h)
            self._h = None

    # ---- construction (ivf/mod.rs:76-165) ----
    @classmethod
    def build(cls, storage, metric=DistanceMetric.L2Squared, dimension: Optional[int] = None, seed: int = 42,
              ordinal: int = 0) -> "IvfPqIndex":
        return cls.build_with_config(storage, IvfPqConfig(), metric, dimension, seed, ordinal)

    @classmethod
    def build_with_config(cls, storage, config: IvfPqConfig, metric=DistanceMetric.L2Squared,
                          dimension: Optional[int] = None, seed: int = 42, ordinal: int = 0) -> "IvfPqIndex":
        x = _storage_rows(storage, dimension)
        c = config._c()
        h = _vp()
        _check(_lib.vhip_ivfpq_build(ordinal, _p(x, _f32p), x.shape[0], x.shape[1], ctypes.byref(c), int(metric), seed,
                                     ctypes.byref(h)))
        return cls(h, storage, config, metric)

    build_parallel_with_config = build_with_config
    build_sequential_with_config = build_with_config  # ivf/mod.rs:173-248: the same index

    @classmethod
    def build_sequential(cls, storage, metric=DistanceMetric.L2Squared, **kw) -> "IvfPqIndex":
        return cls.build(storage, metric, **kw)

    @classmethod
    def from_parts(cls, storage, config: IvfPqConfig, coarse_centroids, pq: ProductQuantizer,
                   inverted_index: InvertedIndex, dimension: int, metric, ordinal: int = 0) -> "IvfPqIndex":
        cc = np.ascontiguousarray(coarse_centroids, dtype=np.float32).reshape(-1)
        sizes, ids, codes = inverted_index._csr()
        c = config._c()
        h = _vp()
        _check(_lib.vhip_ivfpq_create(ordinal, dimension, int(metric), ctypes.byref(c), _p(cc, _f32p),
                                      cc.size // max(dimension, 1), _p(pq.codebooks, _f32p), _p(sizes, _u32p),
                                      _p(ids, _u32p), _p(codes, _u8p), ctypes.byref(h)))
        return cls(h, storage, config, metric)

    # ---- search (ivf/mod.rs:251-345) ----
    def search(self, query, k: int) -> List[SearchResult]:
        return self.search_with_nprobe(query, k, self._config.nprobe)

    def search_with_nprobe(self, query, k: int, nprobe: int) -> List[SearchResult]:
        q = np.asarray(query, np.float32).reshape(-1)
        if q.size != self.dimension():
            raise DimensionMismatch(self.dimension(), q.size)
        return self.search_batch(q.reshape(1, -1), k, nprobe)[0]

    def search_batch(self, queries, k: int, nprobe: Optional[int] = None) -> List[List[SearchResult]]:
        ids, dist, lens = self.search_batch_arrays(queries, k, nprobe)
        return _to_lists(ids, dist, lens)

    def search_batch_arrays(self, queries, k: int, nprobe: Optional[int] = None):
        """(ids [nq, k] uint32, dist [nq, k] float32, lens [nq])."""
        q = _rows(queries, self.dimension())
        nq = q.shape[0]
        w = max(k, 1)
        ids = np.empty((max(nq, 1), w), np.uint32)
        dist = np.empty((max(nq, 1), w), np.float32)
        lens = np.zeros(max(nq, 1), np.uintp)
        np_ = self._config.nprobe if nprobe is None else nprobe
        _check(_lib.vhip_ivfpq_search_batch(self._h, _p(q, _f32p), nq, k, np_, _p(ids, _u32p), _p(dist, _f32p),
                                            lens.ctypes.data_as(_szp)))
        return ids[:nq, :k], dist[:nq, :k], lens[:nq]

    def search_batch_device(self, d_queries: int, nq: int, k: int, nprobe: int, d_ids: int, d_dist: int,
                            d_len: int) -> None:
        _check(_lib.vhip_ivfpq_search_batch_device(self._h, d_queries, nq, k, nprobe, d_ids, d_dist, d_len))

    def probe(self, queries, nprobe: int) -> np.ndarray:
        """The coarse lists the search scans: [nq, min(max(nprobe, 1), nlist)], best first."""
        q = _rows(queries, self.dimension())
        w = max(1, min(nprobe, self.nlist()))
        out = np.empty((max(q.shape[0], 1), w), np.uint32)
        _check(_lib.vhip_ivfpq_probe(self._h, _p(q, _f32p), q.shape[0], nprobe, _p(out, _u32p)))
        return out[:q.shape[0]]

    def profile(self, enable: bool = True) -> None:
        _check(_lib.vhip_ivfpq_profile(self._h, 1 if enable else 0))

    def profile_read(self):
        ms = ctypes.c_double()
        n = ctypes.c_uint64()
        _check(_lib.vhip_ivfpq_profile_read(self._h, ctypes.byref(ms), ctypes.byref(n)))
        return {"kernel_ms": ms.value, "launches": n.value}

    @staticmethod
    def evaluate_recall(ground_truth, results) -> float:
        """ivf/mod.rs:358-372."""
        if not ground_truth or not results:
            return 0.0
        k = min(len(ground_truth), len(results))
        gt = {r.id for r in list(ground_truth)[:k]}
        return sum(1 for r in list(results)[:k] if r.id in gt) / k

    # ---- persistence (ivf/mod.rs:375-408) ----
    def _export(self):
        if self._parts is None:
            i = self._info
            cc = np.zeros(i.nlist * i.dimension, np.float32)
            cb = np.zeros(i.num_subvectors * i.sub_clusters * (i.dimension // i.num_subvectors), np.float32)
            sizes = np.zeros(i.nlist, np.uint32)
            ids = np.zeros(max(i.num_vectors, 1), np.uint32)
            codes = np.zeros((max(i.num_vectors, 1), i.num_subvectors), np.uint8)
            _check(_lib.vhip_ivfpq_export(self._h, _p(cc, _f32p), _p(cb, _f32p), _p(sizes, _u32p), _p(ids, _u32p),
                                          _p(codes, _u8p)))
            self._parts = (cc, cb, sizes, ids[:i.num_vectors], codes[:i.num_vectors])
        return self._parts

    def save_to_file(self, path) -> None:
        IvfPqSerializer.save_to_file(path, self._config, self.coarse_centroids(), self.pq(), self.inverted_index(),
                                     self.dimension(), self._metric)

    @classmethod
    def load_from_file(cls, storage, path, ordinal: int = 0) -> "IvfPqIndex":
        cfg, coarse, pq, inv, dim, metric = IvfPqSerializer.load_from_file(path)
        sd = storage.dimension() if isinstance(storage, MmapStorage) else _storage_rows(storage).shape[1]
        if sd != dim:
            raise DimensionMismatch(sd, dim)
        return cls.from_parts(storage, cfg, coarse, pq, inv, dim, metric, ordinal)

    # ---- getters (ivf/mod.rs:411-449) ----
    def storage(self):
        return self._storage

    def config(self) -> IvfPqConfig:
        return self._config

    def metric(self) -> DistanceMetric:
        return self._metric

    def dimension(self) -> int:
        return int(self._info.dimension)

    def nlist(self) -> int:
        return int(self._info.nlist)

    def __len__(self) -> int:
        return int(self._info.num_vectors)

    def len(self) -> int:
        return len(self)

    def is_empty(self) -> bool:
        return len(self) == 0

    def coarse_centroids(self) -> np.ndarray:
        return self._export()[0]

    def pq(self) -> ProductQuantizer:
        i = self._info
        return ProductQuantizer(i.dimension, i.num_subvectors, i.sub_clusters, self._export()[1])

    def inverted_index(self) -> InvertedIndex:
        _, _, sizes, ids, codes = self._export()
        return InvertedIndex.from_csr(sizes, ids, codes, int(self._info.num_subvectors))


# ---- device memory for callers that stage their own inputs ----------------------------
class DeviceBuffer:
    """A raw device allocation on one GPU (for the *_device search entry points)."""

    def __init__(self, nbytes: int, ordinal: int = 0):
        self.ordinal = ordinal
        self.nbytes = nbytes
        p = _vp()
        _check(_lib.vhip_malloc(ordinal, nbytes, ctypes.byref(p)))
        self.ptr = p.value

    @classmethod
    def from_host(cls, arr: np.ndarray, ordinal: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        b = cls(a.nbytes, ordinal)
        _check(_lib.vhip_memcpy_htod(ordinal, b.ptr, a.ctypes.data, a.nbytes))
        return b

    def to_host(self, out: np.ndarray) -> np.ndarray:
        assert out.flags.c_contiguous and out.nbytes <= self.nbytes
        _check(_lib.vhip_memcpy_dtoh(self.ordinal, out.ctypes.data, self.ptr, out.nbytes))
        return out

    def copy_from(self, other: "DeviceBuffer", nbytes: Optional[int] = None):
        """Device-to-device copy of nbytes (default: all of `other`)."""
        nb = other.nbytes if nbytes is None else nbytes
        assert nb <= self.nbytes and nb <= other.nbytes
        _check(_lib.vhip_memcpy_dtod(self.ordinal, self.ptr, other.ptr, nb))

    def free(self):
        if self.ptr:
            _check(_lib.vhip_free(self.ordinal, self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize(ordinal: int = 0):
    _check(_lib.vhip_synchronize(ordinal))


def library_path() -> str:
    return LIB_PATH
