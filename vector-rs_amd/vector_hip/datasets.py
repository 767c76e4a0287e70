"""Seeded synthetic workloads for the kNN / k-means hot path.

Each generator is deterministic for a given seed (numpy PCG64), so the GPU run and
the CPU oracle see bit-identical inputs on any machine with this numpy.  Shapes and
distributions follow the benchmark workloads of the path:

* ``gaussian``         rows ~ N(0, 1) (the 10k x 128 CPU fixture; generate_dataset.py shape).
* ``uniform_int``      integer-valued entries uniform in [0, 255], stored as f32
                       (1M x 128 squared-L2 search).
* ``normalized``       N(0, 1) rows L2-normalised in float64, then cast (1M x 768 cosine).
* ``gaussian_mixture`` k-means input: centres ~ N(0, 4 I) (sigma 2), labels uniform,
                       x = centre + N(0, I) (2M x 96, 4096 components).
* ``uniform``          U[-1, 1] (500k x 128 L1 / L-inf search).
* ``packed_bits``      uniform random bits packed as uint32 words (10M x 256-bit Hamming).

Seeds used by the benchmark workloads: base 42, queries 43, mixture 44.
"""
from __future__ import annotations

import numpy as np

SEED_BASE = 42
SEED_QUERIES = 43
SEED_MIXTURE = 44


def _rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def _chunked(n: int, dim: int, fill, chunk_rows: int = 1 << 16) -> np.ndarray:
    out = np.empty((n, dim), np.float32)
    for s in range(0, n, chunk_rows):
        e = min(n, s + chunk_rows)
        out[s:e] = fill(e - s)
    return out


def gaussian(n: int, dim: int, seed: int) -> np.ndarray:
    g = _rng(seed)
    return _chunked(n, dim, lambda r: g.standard_normal((r, dim), dtype=np.float32))


def uniform_int(n: int, dim: int, seed: int, hi: int = 255) -> np.ndarray:
    g = _rng(seed)
    return _chunked(n, dim, lambda r: g.integers(0, hi + 1, size=(r, dim), dtype=np.int32).astype(np.float32))


def normalized(n: int, dim: int, seed: int) -> np.ndarray:
    g = _rng(seed)

    def fill(r):
        x = g.standard_normal((r, dim))  # float64
        x /= np.linalg.norm(x, axis=1, keepdims=True)
        return x.astype(np.float32)

    return _chunked(n, dim, fill, chunk_rows=1 << 14)


def uniform(n: int, dim: int, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    g = _rng(seed)
    return _chunked(n, dim, lambda r: g.uniform(lo, hi, size=(r, dim)).astype(np.float32))


def gaussian_mixture(n: int, dim: int, components: int, seed: int, centre_sigma: float = 2.0,
                     sigma: float = 1.0):
    """Returns (points[n, dim] f32, labels[n] int32, centres[components, dim] f32)."""
    g = _rng(seed)
    centres = (g.standard_normal((components, dim)) * centre_sigma).astype(np.float32)
    labels = g.integers(0, components, size=n, dtype=np.int32)
    pts = np.empty((n, dim), np.float32)
    step = 1 << 16
    for s in range(0, n, step):
        e = min(n, s + step)
        pts[s:e] = centres[labels[s:e]] + (g.standard_normal((e - s, dim)) * sigma).astype(np.float32)
    return pts, labels, centres


def packed_bits(n: int, bits: int, seed: int) -> np.ndarray:
    """n codes of `bits` bits (multiple of 32) as uint32[n, bits // 32]."""
    assert bits % 32 == 0
    g = _rng(seed)
    words = bits // 32
    out = np.empty((n, words), np.uint32)
    step = 1 << 20
    for s in range(0, n, step):
        e = min(n, s + step)
        out[s:e] = g.integers(0, 1 << 32, size=(e - s, words), dtype=np.uint64).astype(np.uint32)
    return out
