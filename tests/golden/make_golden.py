"""Writes the golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

Every expected value here is computed in float64 with numpy from the mathematical definition
of the metric or algorithm -- independently of the C oracle and of the HIP library -- so the
fixtures pin both.  Inputs are either stored in the fixture (small cases) or regenerated from
the seeded generators of vector_hip/datasets.py and checked against a stored SHA-256.

Fixtures:
  c1_l2_gauss_10000x128_q100_k10.npz  10,000 x 128 N(0,1) base (seed 42), 100 N(0,1) queries
                                      (seed 43), exact squared-L2 top-10 (the CPU-runnable
                                      workload; shape of generate_dataset.py's defaults).
  metrics_tiny.npz                    300 x 37 base + 6 queries, exact top-7 for all 10 metrics
                                      (definitions of vector-simd/src/scalar.rs:14-263).
  reference_inline.npz                the reference tests' inline datasets (knn.rs:416-425 and
                                      flat.rs:579-588 formulas) with exact top-k.
  kmeans_mixture.npz                  3,000 x 16 mixture of 12 clusters (datasets.gaussian_mixture,
                                      seed 7, centre sigma 3), init = first 12 points, 6 Lloyd
                                      iterations (ivf/kmeans.rs:70-155 loop body, keep-old empty
                                      clusters): assignments, centroids and best-vs-second gaps.
  hamming_packed.npz                  1,000 codes of 256 bits + 5 queries: popcount top-10.
"""
import hashlib
import importlib.util
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))


def _datasets():
    path = os.path.join(ROOT, "vector-rs_amd", "vector_hip", "datasets.py")
    spec = importlib.util.spec_from_file_location("vh_datasets", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ---- metric definitions in float64 (scalar.rs:14-263) ----------------------------------
def dist64(metric, q, X):
    """Distance of float64 query q to every row of X (float64)."""
    if metric == "l2":
        return np.sum((X - q) ** 2, axis=1)
    if metric == "dot":
        return X @ q
    if metric == "cosine":
        den = np.sqrt(np.sum(X * X, axis=1)) * math.sqrt(float(q @ q))
        dot = X @ q
        return np.where(den <= 1e-9, 0.0, dot / np.where(den <= 1e-9, 1.0, den))
    if metric == "l1":
        return np.sum(np.abs(X - q), axis=1)
    if metric == "minkowski":
        return np.sum(np.abs(X - q) ** 3, axis=1) ** (1.0 / 3.0)
    if metric == "linf":
        return np.max(np.abs(X - q), axis=1)
    if metric == "hamming":
        return np.sum(np.abs(X.astype(np.float32) - q.astype(np.float32)) > np.float32(1e-6), axis=1).astype(np.float64)
    if metric == "mahalanobis":
        return np.sqrt(np.sum((X - q) ** 2, axis=1))
    if metric == "jaccard":
        mn = np.sum(np.minimum(np.abs(X), np.abs(q)), axis=1)
        mx = np.sum(np.maximum(np.abs(X), np.abs(q)), axis=1)
        return np.where(mx <= 1e-9, 0.0, 1.0 - mn / np.where(mx <= 1e-9, 1.0, mx))
    if metric == "hellinger":
        return np.sqrt(0.5 * np.sum((np.sqrt(np.abs(X)) - np.sqrt(np.abs(q))) ** 2, axis=1))
    raise KeyError(metric)


HIGHER = {"dot", "cosine"}
METRICS = ["l2", "dot", "cosine", "l1", "minkowski", "linf", "hamming", "mahalanobis", "jaccard", "hellinger"]


def topk64(metric, Q, X, k):
    """Exact top-k per query: best first, ties broken by the lower id."""
    nq = Q.shape[0]
    ids = np.zeros((nq, k), np.int64)
    ds = np.zeros((nq, k), np.float64)
    kth = np.zeros(nq, np.float64)
    for i in range(nq):
        d = dist64(metric, Q[i].astype(np.float64), X.astype(np.float64))
        key = -d if metric in HIGHER else d
        order = np.lexsort((np.arange(len(d)), key))[:k]
        ids[i] = order
        ds[i] = d[order]
        kth[i] = d[order[-1]]
    return ids, ds, kth


def c1(ds):
    base = ds.gaussian(10_000, 128, ds.SEED_BASE)
    q = ds.gaussian(100, 128, ds.SEED_QUERIES)
    ids, d, kth = topk64("l2", q, base, 10)
    np.savez_compressed(os.path.join(HERE, "c1_l2_gauss_10000x128_q100_k10.npz"), ids=ids.astype(np.uint32),
                        dist=d, kth=kth, base_sha256=np.array(sha(base)), queries_sha256=np.array(sha(q)),
                        base_seed=np.int64(ds.SEED_BASE), query_seed=np.int64(ds.SEED_QUERIES))


def metrics_tiny():
    rng = np.random.Generator(np.random.PCG64(2024))
    X = rng.standard_normal((300, 37)).astype(np.float32)
    X[5] = 0.0                                  # zero row: cosine 0, jaccard/hellinger edge
    X[17] = X[16]                               # exact duplicate rows: ties
    X[40:60] = np.round(X[40:60] * 2) / 2       # coincident values: thresholded Hamming is meaningful
    Q = rng.standard_normal((6, 37)).astype(np.float32)
    Q[2] = np.round(Q[2] * 2) / 2
    Q[3] = X[16]                                # a query equal to a base row
    out = {"base": X, "queries": Q}
    for m in METRICS:
        ids, d, kth = topk64(m, Q, X, 7)
        out[f"{m}_ids"] = ids.astype(np.uint32)
        out[f"{m}_dist"] = d
        out[f"{m}_kth"] = kth
    np.savez_compressed(os.path.join(HERE, "metrics_tiny.npz"), **out)


def reference_inline():
    # knn.rs:416-425: 50 rows of (i*i*0.1, 2i, i+5, 3i); query = row 10, k = 5
    i = np.arange(50, dtype=np.float32)
    knn_rs = np.stack([i * i * np.float32(0.1), i * 2, i + 5, i * 3], 1).astype(np.float32)
    ids_a, d_a, _ = topk64("l2", knn_rs[10:11], knn_rs, 5)
    # flat.rs:579-588: 200 rows x 64 of ((i*7 + d*13 + 3) % 97) * 0.01; queries rows 0, 77, 199
    ii, dd = np.meshgrid(np.arange(200), np.arange(64), indexing="ij")
    flat_rs = (((ii * 7 + dd * 13 + 3) % 97) * 0.01).astype(np.float32)
    qs = flat_rs[[0, 77, 199]]
    ids_b, d_b, _ = topk64("l2", qs, flat_rs, 10)
    ids_c, d_c, _ = topk64("cosine", qs, flat_rs, 10)
    np.savez_compressed(os.path.join(HERE, "reference_inline.npz"), knn_rs=knn_rs, knn_rs_ids=ids_a.astype(np.uint32),
                        knn_rs_dist=d_a, flat_rs=flat_rs, flat_rs_queries=qs, flat_l2_ids=ids_b.astype(np.uint32),
                        flat_l2_dist=d_b, flat_cos_ids=ids_c.astype(np.uint32), flat_cos_dist=d_c)


def kmeans_mixture(ds):
    X, _, _ = ds.gaussian_mixture(3000, 16, 12, 7, centre_sigma=3.0)
    k, iters = 12, 6
    C = X[:k].astype(np.float64)
    X64 = X.astype(np.float64)
    assigns, cents, gaps = [], [], []
    for _ in range(iters):
        d = ((X64[:, None, :] - C[None, :, :]) ** 2).sum(-1)
        a = np.argmin(d, axis=1)                  # lowest index on ties, like the strict '<' scan
        srt = np.sort(d, axis=1)
        gaps.append(srt[:, 1] - srt[:, 0])        # best-vs-second gap: near-ties may flip
        newC = C.copy()
        for c in range(k):
            m = a == c
            if m.any():
                newC[c] = X64[m].mean(0)
        assigns.append(a.astype(np.int32))
        cents.append(newC.copy())
        C = newC
    np.savez_compressed(os.path.join(HERE, "kmeans_mixture.npz"), data_sha256=np.array(sha(X)),
                        assign=np.stack(assigns).astype(np.int16), centroids=np.stack(cents),
                        gap=np.stack(gaps).astype(np.float32))


def hamming_packed():
    rng = np.random.Generator(np.random.PCG64(99))
    codes = rng.integers(0, 1 << 32, size=(1000, 8), dtype=np.uint64).astype(np.uint32)
    codes[7] = codes[3]                       # duplicate code: a tie at distance 0 from the same query
    qs = rng.integers(0, 1 << 32, size=(5, 8), dtype=np.uint64).astype(np.uint32)
    qs[1] = codes[3]
    pc = np.array([bin(v).count("1") for v in range(1 << 16)], np.int64)

    def popc(x):
        x = x.astype(np.uint64)
        return pc[x & 0xFFFF] + pc[(x >> 16) & 0xFFFF]

    ids = np.zeros((5, 10), np.uint32)
    dist = np.zeros((5, 10), np.uint32)
    for i in range(5):
        d = popc(codes ^ qs[i]).sum(1)
        order = np.lexsort((np.arange(len(d)), d))[:10]
        ids[i] = order
        dist[i] = d[order]
    np.savez_compressed(os.path.join(HERE, "hamming_packed.npz"), codes=codes, queries=qs, ids=ids, dist=dist)


if __name__ == "__main__":
    ds = _datasets()
    c1(ds)
    metrics_tiny()
    reference_inline()
    kmeans_mixture(ds)
    hamming_packed()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
