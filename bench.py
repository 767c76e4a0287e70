"""Benchmark of the kNN / k-means hot path on one MI355X.

Default (no flags): exact squared-L2 kNN over a 1,000,000 x 128 fp32 base of integer values in
[0, 255], 10,000 queries drawn the same way, k = 100 -- one "step" is one full batch search of
the 10,000 queries with queries and base resident in HBM (search_batch on device pointers).
The same JSON line carries the 2,000,000 x 96, 4,096-centroid k-means workload (10 Lloyd
iterations from the first 4,096 points) under "kmeans".

Printed JSON (one line): metric/value/unit, ms_per_step, "roofline" of the dominant kernel
(FP32-MFMA distance + filter kernel, its algorithmic flops per launch divided by its average
launch time, measured with HIP events on the engine's stream over the timed region),
"cpu_baseline": the oracle's restatement of the reference CPU path (CudaKnnEngine::search_batch_cpu,
knn.rs:312-377, AVX-512 dispatch as vector-simd) timed on this host, and "parity": the timed run's
results against the oracle's (tie-aware recall >= 0.999, distances within 1e-4 relative, exact on
integer data).  The oracle searches every query when that takes at most FULL_PARITY_S seconds
(the headline workload, L1, Linf), else a strided sample that always holds the last 128 queries,
i.e. the last, partial query tile of every scan kernel; each parity object names its queries.  The
default line also carries the other workloads under "kmeans" (each of the 10 iterations checked
against the oracle's iteration from the GPU's previous centroids: <= 0.01% flips, all near-ties,
centroids within 1e-4), "cos768", "hamming" (bit-exact against the oracle's popcount search over
all 10M codes), "l1", "linf" and "ivfpq" (the IVF-PQ search on clustered data, checked against
the oracle's search_with_nprobe), each with its own roofline, CPU baseline and parity.
The process exits with status 3, after printing the line, when any parity check fails.

The default line also carries "batch_sweep" (search_batch at batch sizes 1 to 128, as the
reference's cuda_bench.rs does, each batch checked against the oracle), "kmeans_fit" (fit() with
its default k-means++ init, init timed apart from the Lloyd iterations) and "reference_published"
(the shapes of the reference's only published GPU figures: search_batch and fit() on 100,000 x 768
cosine data, beside those figures).

Other workloads: --workload cos768 | kmeans | hamming | l1 | linf | gauss (see WORKLOADS), ivf_coarse
(the IVF coarse quantizer), ivfpq (IVF-PQ search), kmeans_fit, batch_sweep, published, upload (engine builds
from VECRSTOR files), copy (counter calibration).
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "vector-rs_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

METRIC = "kNN queries/sec (1M×128 fp32, k=100) + k-means iter/sec; % FP32-MFMA/HBM roofline"
PEAK_MFMA_F32 = 157.3e12   # FLOP/s, MI355X dense FP32 matrix
PEAK_HBM = 8.0e12          # B/s
# Published vector FP32 peak of MI355X, FLOP/s.  It counts packed FMAs (2 FLOPs x 2 lanes per
# instruction lane); packed FP32 instructions are not used here, so the kernels' attainable
# non-packed rate is lower (a throughput probe measured 57.5 T lane-ops/s for v_add_f32 and 37.7 T
# for v_fma_f32 on this part).
PEAK_VECTOR_F32 = 157.3e12
PEAK_MFMA_FP4 = 10.1e15    # OP/s, MI355X dense fp4 matrix
# LDS read rate of MI355X for 4-byte words, GB/s: 256 CUs x 64 banks x 4 B x 2.4 GHz
PEAK_LDS_GBS = 256 * 64 * 4 * 2.4


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_threads() -> int:
    """Threads of the CPU baseline: every core this process may run on (its affinity mask), as
    rayon's default pool in the reference uses every logical core it is given."""
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


# rocprofv3 counter summaries (FETCH_SIZE + WRITE_SIZE of the dominant kernel, scaled by a 1 GiB
# copy) per workload; each holds a "traffic_bytes_per_launch:" line.
PROFILES = {
    "l2int": "k_mfma_hs_filter__knn_l2_int_1000000x128_q10000_k100.txt",
    "kmeans": "k_mfma_hs_assign__kmeans_l2_2000000x96_k4096.txt",
    "cos768": "k_mfma_nt_filter__knn_cosine_1000000x768_q10000_k10.txt",
    "hamming": "k_mfma_ham_wide__knn_hamming_packed256_10000000_q10000_k10.txt",
    "l1": "k_valu_filter__knn_l1_uniform_500000x128_q4096_k10.txt",
    "linf": "k_valu_filter__knn_linf_uniform_500000x128_q4096_k10.txt",
    "ivf_coarse": "k_mfma_hs_assign__ivf_coarse_l2_2000000x96_nlist4096.txt",
    "ivfpq": "k_ivfpq_lists__ivfpq_l2_mixture1024_1000000x128_nlist1024_m16_ks256_nprobe32_q10000_k10.txt",
}


def profiled_traffic(key):
    """HBM bytes per launch of the workload's dominant kernel from its committed counter summary
    (None when there is no summary)."""
    name = PROFILES.get(key)
    if not name:
        return None
    try:
        with open(os.path.join(ROOT, "profiles", name)) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def roofline(prof, bound, peak, unit, key=None):
    if not prof["launches"] or prof["kernel_ms"] <= 0:
        return None
    avg_s = prof["kernel_ms"] / prof["launches"] / 1e3
    per_launch = prof["work"] / prof["launches"]
    achieved = per_launch / avg_s
    scale = 1e12 if unit == "TFLOP/s" else 1e9
    return {"bound": bound, "achieved": round(achieved / scale, 3), "peak": round(peak / scale, 3), "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": profiled_traffic(key),
            "traffic_source": f"profiles/{PROFILES[key]}" if key in PROFILES else None,
            "work_per_launch": per_launch, "avg_launch_ms": round(avg_s * 1e3, 4), "launches": prof["launches"],
            "algorithmic_bytes_per_launch": prof["bytes"] / prof["launches"]}


# ---------------------------------------------------------------------------------------------
def run_knn(vh, base, queries, k, metric, steps, warmup, hamming=False):
    """Times `steps` device-resident batch searches; returns (ms_per_step, profile, ids, dist)."""
    nq = queries.shape[0]
    eng = vh.HammingKnnEngine(base) if hamming else vh.CudaKnnEngine(base, base.shape[1], metric)
    dq = vh.DeviceBuffer.from_host(queries)
    di = vh.DeviceBuffer(nq * k * 4)
    dd = vh.DeviceBuffer(nq * k * 4)

    def step():
        eng.search_batch_device(dq.ptr, nq, k, di.ptr, dd.ptr)

    for _ in range(warmup):
        step()
    eng.profile(True)
    vh.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step()
        log(f"  step {i + 1}/{steps} done")
    vh.synchronize()
    t1 = time.perf_counter()
    prof = eng.profile_read()
    ids = di.to_host(np.empty((nq, k), np.uint32))
    dist = dd.to_host(np.empty((nq, k), np.uint32 if hamming else np.float32))
    # the same batch through the host-buffer entry point (queries in, results out over PCIe):
    # one untimed call (its first use allocates that path's device buffers), then the median of 3
    eng.search_batch_arrays(queries, k)
    hts = []
    for _ in range(3):
        t2 = time.perf_counter()
        eng.search_batch_arrays(queries, k)
        hts.append((time.perf_counter() - t2) * 1e3)
    host_ms = float(np.median(hts))
    return (t1 - t0) * 1e3 / steps, prof, ids, dist, host_ms


CPU_TARGET_S = 10.0  # wall time the CPU baseline leg aims for (bounded sample of the workload)
FULL_PARITY_S = 20.0  # the oracle searches every query when that takes at most this long
TAIL_QUERIES = 128    # the last queries: the last (partial) query tile of every scan kernel


def parity_sample(nq, size, tail=TAIL_QUERIES):
    """Query indices of the parity leg: all nq when size >= nq, else an even stride over the
    first nq - tail queries plus the last `tail` (the last, partial query tile of every scan
    kernel, which a prefix sample never reaches), about `size` in all."""
    if size >= nq:
        return np.arange(nq)
    head = nq - tail
    stride = max(1, -(-head // max(1, size - tail)))
    return np.concatenate([np.arange(0, head, stride), np.arange(head, nq)])


def describe_sample(idx, nq):
    if len(idx) == nq:
        return f"all {nq} queries"
    stride = int(idx[1] - idx[0]) if len(idx) > 1 else 1
    head = nq - TAIL_QUERIES
    return (f"{len(idx)} of the {nq} queries: every {stride}th of queries 0..{head - 1} and all of "
            f"{head}..{nq - 1} (the last query tiles)")


def cpu_knn_baseline(base, queries, k, metric, full_under_s=FULL_PARITY_S):
    """Times the oracle's restatement of search_batch_cpu on every query when a 16-query probe
    says that takes at most full_under_s seconds on this host's threads, else on a sample sized to
    take about CPU_TARGET_S seconds (parity_sample: strided, with the last queries).  Returns the
    baseline and (oracle result, query indices), the parity leg's reference."""
    import oracle

    th = cpu_threads()
    nq = queries.shape[0]
    t0 = time.perf_counter()
    oracle.knn_search_batch(base, queries[:16], k, metric, threads=th)
    per_q = max(time.perf_counter() - t0, 1e-6) / 16
    size = nq if per_q * nq <= full_under_s else int(max(TAIL_QUERIES + 16, CPU_TARGET_S / per_q))
    idx = parity_sample(nq, size)
    t0 = time.perf_counter()
    ref = oracle.knn_search_batch(base, np.ascontiguousarray(queries[idx]), k, metric, threads=th)
    dt = time.perf_counter() - t0
    be = {0: "scalar", 1: "AVX2+FMA", 2: "AVX-512F"}[oracle.detect_backend()]
    return {"value": round(len(idx) / dt, 3), "unit": "queries/s", "cores": th, "kind": "port",
            "sample": f"{describe_sample(idx, nq)} against the full base, k={k}, {be} backend, {dt:.2f} s wall "
                      f"on {th} threads (affinity mask) ({cpu_model()})"}, (ref, idx)


def knn_parity(base, queries, ids, dist, ref, k, metric, rtol, atol, min_recall=0.999):
    """Parity of the timed GPU search with the oracle on the queries the oracle searched (ref =
    (its ids, distances and lengths, the query indices)): tie-aware recall (a returned id counts
    when its oracle value is at least as good as the oracle's k-th), every reported distance
    against the oracle's value of the same (query, id) pair within rtol / atol, the k best values
    as a multiset, and unique in-range ids.  Packed Hamming compares popcount distances."""
    import oracle

    (rids, rdist, _), idx = ref
    m = rids.shape[0]
    hib = metric in ("dot", "cosine")
    ok_ids = total = 0
    max_abs = max_rel = 0.0
    dist_ok = multiset_ok = ids_ok = True
    for q0 in range(0, m, 512):
        q1 = min(m, q0 + 512)
        qi = idx[q0:q1]
        got = ids[qi, :k].astype(np.int64)
        ids_ok = ids_ok and bool(np.all(got < base.shape[0]))
        ids_ok = ids_ok and all(len(set(r.tolist())) == k for r in got)
        got = np.minimum(got, base.shape[0] - 1)
        if metric == "hamming":
            refv = np.bitwise_count(base[got] ^ queries[qi, None, :]).sum(-1).astype(np.float64)
        else:
            qq = np.repeat(queries[qi], k, 0)
            refv = oracle.distance_rows(metric, qq, base[got.reshape(-1)]).reshape(q1 - q0, k).astype(np.float64)
        kth = rdist[q0:q1, k - 1:k].astype(np.float64)
        tol = rtol * np.abs(kth) + atol
        good = refv >= kth - tol if hib else refv <= kth + tol
        ok_ids += int(good.sum())
        total += good.size
        diff = np.abs(dist[qi, :k].astype(np.float64) - refv)
        dist_ok = dist_ok and bool(np.all(diff <= rtol * np.abs(refv) + atol))
        max_abs = max(max_abs, float(diff.max()))
        nz = np.abs(refv) > 0
        if nz.any():
            max_rel = max(max_rel, float((diff[nz] / np.abs(refv[nz])).max()))
        rs = np.sort(rdist[q0:q1, :k].astype(np.float64), 1)
        multiset_ok = multiset_ok and bool(np.all(np.abs(rs - np.sort(refv, 1)) <= rtol * np.abs(rs) + atol))
    recall = ok_ids / max(total, 1)
    ok = bool(ids_ok and dist_ok and multiset_ok and recall >= min_recall)
    nq = queries.shape[0]
    return {"queries_checked": int(m), "query_sample": describe_sample(idx, nq), "first_query": int(idx[0]),
            "last_query": int(idx[-1]), "last_tile_checked": bool(np.all(np.isin(np.arange(nq - TAIL_QUERIES, nq), idx))),
            "k": k, "recall_tie_aware": round(recall, 6), "min_recall": min_recall,
            "max_abs_dist_err": max_abs, "max_rel_dist_err": max_rel,
            "distance_tolerance": {"rtol": rtol, "atol": atol}, "distances_ok": dist_ok,
            "kbest_values_match": multiset_ok, "ids_unique_in_range": ids_ok, "ok": ok}


def kmeans_parity(data, cent, got, ref):
    """One Lloyd iteration of the GPU from centroids `cent` against the oracle's iteration from
    the same centroids (ref): assignments differ on at most 0.01% of the points and only at
    near-ties (the two centroids' oracle distances within 1e-4 relative); member counts equal the
    GPU assignment's; each centroid within 1e-4 of its norm of the oracle's update where the
    membership agrees, and of the float64 mean of the GPU's members where a flip touched it;
    inertia within 1e-4 relative."""
    import oracle

    ga, ra = got["assign"].astype(np.int64), ref["assign"].astype(np.int64)
    n, kc = len(data), len(cent)
    flips = np.nonzero(ga != ra)[0]
    near = True
    if len(flips):
        dg = oracle.distance_rows("l2", data[flips], cent[ga[flips]]).astype(np.float64)
        dr = oracle.distance_rows("l2", data[flips], cent[ra[flips]]).astype(np.float64)
        near = bool(np.all(np.abs(dg - dr) <= 1e-4 * np.maximum(1.0, np.abs(dr))))
    counts_ok = bool(np.array_equal(np.bincount(ga, minlength=kc), got["counts"]))
    touched = np.zeros(kc, bool)
    touched[np.unique(np.concatenate([ga[flips], ra[flips]]))] = True
    gc_, rc_ = got["centroids"].astype(np.float64), ref["centroids"].astype(np.float64)
    err = np.linalg.norm(gc_ - rc_, axis=1) / np.maximum(np.linalg.norm(rc_, axis=1), 1e-6)
    worst = float(err[~touched].max()) if (~touched).any() else 0.0
    if touched.any():
        # float64 means of the GPU's members of every touched cluster, in one pass over the points
        sel = touched[ga]
        sums = np.zeros((kc, data.shape[1]), np.float64)
        np.add.at(sums, ga[sel], data[sel].astype(np.float64))
        cnt = np.bincount(ga[sel], minlength=kc)
        for c in np.nonzero(touched)[0]:
            want = sums[c] / cnt[c] if cnt[c] else cent[c].astype(np.float64)
            worst = max(worst, float(np.linalg.norm(gc_[c] - want) / max(np.linalg.norm(want), 1e-6)))
    inertia_rel = abs(float(got["inertia"]) - float(ref["inertia"])) / max(abs(float(ref["inertia"])), 1e-30)
    ok = bool(len(flips) <= max(1, int(1e-4 * n)) and near and counts_ok and worst <= 1e-4 and inertia_rel <= 1e-4)
    return {"assignment_flips": int(len(flips)), "flips_all_near_ties": near, "counts_match": counts_ok,
            "max_centroid_rel_err": worst, "inertia_rel_err": inertia_rel, "ok": ok}


def bench_kmeans(vh, steps_iters, with_cpu):
    """2,000,000 x 96 mixture of 4,096 components, 4,096 centroids from the first 4,096 points,
    `steps_iters` Lloyd iterations timed back to back.  Parity (untimed, before the timed run):
    the same iterations run one at a time, each checked against the oracle's Lloyd iteration
    (KMeans::fit body) from the GPU's own previous centroids; with_cpu false checks the first
    only.  Those oracle iterations are also the CPU baseline."""
    from vector_hip import datasets as ds
    import oracle

    n, d, kc = 2_000_000, 96, 4096
    log(f"kmeans: generating {n} x {d} mixture of {kc}")
    data, _, _ = ds.gaussian_mixture(n, d, kc, ds.SEED_MIXTURE)
    init = data[:kc].copy()
    st = vh.KMeansState(data)
    th = cpu_threads()
    st.set_centroids(init)
    cent = init
    checks, cpu_s = [], []
    for it in range(steps_iters if with_cpu else 1):
        st.run(1)
        got = st.read()
        t0 = time.perf_counter()
        ref = oracle.kmeans_step(data, cent, "l2", threads=th)
        cpu_s.append(time.perf_counter() - t0)
        r = kmeans_parity(data, cent, got, ref)
        log(f"  iteration {it + 1} against the oracle: flips {r['assignment_flips']}, "
            f"centroid err {r['max_centroid_rel_err']:.2e}, ok {r['ok']}")
        checks.append(r)
        cent = got["centroids"]
    st.set_centroids(init)
    st.profile(True)
    vh.synchronize()
    t0 = time.perf_counter()
    st.run(steps_iters)
    vh.synchronize()
    t1 = time.perf_counter()
    prof = st.profile_read()
    out = st.read()
    ms_iter = (t1 - t0) * 1e3 / steps_iters
    res = {"workload": f"kmeans_l2_{n}x{d}_k{kc}_{steps_iters}iters_init_first_points",
           "value": round(1e3 / ms_iter, 3), "unit": "iterations/s", "ms_per_iteration": round(ms_iter, 3),
           "inertia": out["inertia"],
           "roofline": roofline(prof, "mfma", PEAK_MFMA_F32, "TFLOP/s", "kmeans")}
    # the update's fixed-point sums are order-independent: the timed run's centroids equal those
    # of the checked one-at-a-time iterations bit for bit
    same = len(checks) == steps_iters and bool(np.array_equal(out["centroids"].view(np.uint32), cent.view(np.uint32)))
    res["parity"] = {"iterations_checked": len(checks), "points": int(n),
                     "rule": "each iteration from the GPU's previous centroids against the oracle's: <= 0.01% "
                             "assignment flips, all near-ties; counts equal; centroids within 1e-4 of their "
                             "norm; inertia within 1e-4",
                     "max_flips": max(c["assignment_flips"] for c in checks), "max_flip_frac": 1e-4,
                     "max_centroid_rel_err": max(c["max_centroid_rel_err"] for c in checks),
                     "max_inertia_rel_err": max(c["inertia_rel_err"] for c in checks),
                     "timed_run_equals_checked_iterations": same if len(checks) == steps_iters else None,
                     "per_iteration": checks,
                     "ok": all(c["ok"] for c in checks) and (same or len(checks) < steps_iters)}
    if with_cpu:
        dt = float(np.mean(cpu_s))
        res["cpu_baseline"] = {"value": round(1.0 / dt, 5), "unit": "iterations/s", "cores": th, "kind": "port",
                               "sample": f"{len(cpu_s)} full Lloyd iterations (KMeans::fit body) over all {n} points "
                                         f"and {kc} centroids (the parity leg's), {dt:.2f} s each on average on "
                                         f"{th} threads (affinity mask) ({cpu_model()})"}
        res["speedup_vs_cpu"] = round(res["value"] / res["cpu_baseline"]["value"], 1)
    return res


def bench_ivf_coarse(vh, steps, warmup, with_cpu):
    """IVF coarse quantizer (ivf/mod.rs:106-133): the build's find_nearest_centroid over all
    2,000,000 x 96 points of the k-means workload against 4,096 centroids (points resident, one
    step = one assignment of every point; assignments and scores come back to the host), and
    find_top_centroids for 10,000 queries at nprobe = 32."""
    from vector_hip import datasets as ds

    n, d, nlist, nq, nprobe = 2_000_000, 96, 4096, 10_000, 32
    log(f"ivf_coarse: generating {n} x {d} mixture of {nlist}")
    data, _, _ = ds.gaussian_mixture(n, d, nlist, ds.SEED_MIXTURE)
    cent = data[:nlist].copy()
    q = ds.gaussian_mixture(nq, d, nlist, ds.SEED_QUERIES)[0]
    st = vh.KMeansState(data)
    st.set_centroids(cent)
    for _ in range(warmup):
        st.assign_only()
    st.profile(True)
    vh.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        st.assign_only()
        log(f"  step {i + 1}/{steps} done")
    vh.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    prof = st.profile_read()
    cq = vh.IvfCoarseQuantizer(cent, d)
    cq.probe_batch(q, nprobe)
    t0 = time.perf_counter()
    cq.probe_batch(q, nprobe)
    probe_ms = (time.perf_counter() - t0) * 1e3
    t0 = time.perf_counter()
    cq.assign(data, residuals=True)
    host_ms = (time.perf_counter() - t0) * 1e3
    out = {"metric": "IVF coarse assignment points/sec (2M x 96 -> 4096 centroids)", "value": round(n * 1e3 / ms, 1),
           "unit": "points/s", "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 3),
           "higher_is_better": True, "scaling": "strong", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
           "config": {"workload": f"ivf_coarse_assign_l2_{n}x{d}_nlist{nlist}", "parallelism": "single GPU"},
           "roofline": roofline(prof, "mfma", PEAK_MFMA_F32, "TFLOP/s", "ivf_coarse"),
           "probe": {"queries": nq, "nprobe": nprobe, "ms": round(probe_ms, 3),
                     "value": round(nq * 1e3 / probe_ms, 1), "unit": "queries/s (host buffers)"},
           "host_buffers": {"value": round(n * 1e3 / host_ms, 1), "unit": "points/s", "ms": round(host_ms, 3),
                            "note": "IvfCoarseQuantizer.assign with residuals, points and results over PCIe"}}
    if with_cpu:
        import oracle

        # the reference's build loop is serial (ivf/mod.rs:119-132): one thread
        sp = 4096
        t0 = time.perf_counter()
        oracle.kmeans_step(data[:sp], cent, "l2", threads=1)
        dt = time.perf_counter() - t0
        sp = int(min(n, max(sp, sp * CPU_TARGET_S / max(dt, 1e-6))))
        t0 = time.perf_counter()
        oracle.kmeans_step(data[:sp], cent, "l2", threads=1)
        dt = time.perf_counter() - t0
        be = {0: "scalar", 1: "AVX2+FMA", 2: "AVX-512F"}[oracle.detect_backend()]
        out["cpu_baseline"] = {"value": round(sp / dt, 1), "unit": "points/s", "cores": 1, "kind": "port",
                               "sample": f"find_nearest_centroid of {sp} of the {n} points against all {nlist} "
                                         f"centroids (the serial build loop), {be} backend, {dt:.2f} s on 1 thread "
                                         f"({cpu_model()})"}
    return out


def bench_ivfpq(vh, steps, warmup, with_cpu):
    """IVF-PQ search (ivf/mod.rs:256-345): 1,000,000 x 128 base and 10,000 queries drawn from one
    Gaussian mixture of 1,024 components (centres ~ N(0, 4 I), sigma 1), so that the index's
    recall against the exact kNN means something (uniform data has no cluster structure for the
    coarse quantizer to find); squared L2, nlist 1024, 16 sub-spaces of 256 sub-centroids, nprobe
    32, k = 10.  One step = one batch search with queries resident (coarse probe + ADC scan); the
    roofline is the ADC scan kernel's.  recall@10 is reported at nprobe 8, 32 and 128."""
    from vector_hip import datasets as ds

    n, d, nlist, m_sub, ks, nprobe, nq, k = 1_000_000, 128, 1024, 16, 256, 32, 10_000, 10
    log(f"ivfpq: generating {n} + {nq} x {d} from a 1024-component mixture")
    pts, _, _ = ds.gaussian_mixture(n + nq, d, 1024, ds.SEED_MIXTURE)
    base = np.ascontiguousarray(pts[:n])
    q = np.ascontiguousarray(pts[n:])
    del pts
    cfg = vh.IvfPqConfig.new(nlist, nprobe, m_sub).with_sub_clusters(ks).with_max_kmeans_iters(10)
    t0 = time.perf_counter()
    ix = vh.IvfPqIndex.build_with_config(base, cfg, vh.DistanceMetric.L2Squared)
    build_s = time.perf_counter() - t0
    log(f"  build {build_s:.2f} s")
    dq = vh.DeviceBuffer.from_host(q)
    di = vh.DeviceBuffer(nq * k * 4)
    dd = vh.DeviceBuffer(nq * k * 4)
    dl = vh.DeviceBuffer(nq * 4)

    def step():
        ix.search_batch_device(dq.ptr, nq, k, nprobe, di.ptr, dd.ptr, dl.ptr)

    for _ in range(warmup):
        step()
    ix.profile(True)
    vh.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step()
        log(f"  step {i + 1}/{steps} done")
    vh.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    prof = ix.profile_read()
    ids = di.to_host(np.empty((nq, k), np.uint32))
    dist = dd.to_host(np.empty((nq, k), np.float32))
    # algorithmic work of one scan launch: every (query, probed list) builds an M x Ks table over
    # D dimensions (a subtract and a multiply-add per element), every scanned code does M table
    # lookups and M adds
    probes = ix.probe(q, nprobe)
    sizes = np.array([len(L) for L in ix.inverted_index().lists], np.int64)
    scanned = int(sizes[probes].sum())
    pairs = int((sizes[probes] > 0).sum())
    work = pairs * 2.0 * ks * d + scanned * 2.0 * m_sub
    prof_full = {"kernel_ms": prof["kernel_ms"], "launches": prof["launches"], "work": work * prof["launches"],
                 "bytes": scanned * (m_sub + 0.0) * prof["launches"]}
    rl = roofline(prof_full, "valu", PEAK_VECTOR_F32, "TFLOP/s", "ivfpq")
    if rl:
        rl["unit"] = "Top/s (against the vector FP32 peak)"
        rl["work_note"] = ("VALU/LDS ops per launch: 2*Ks*D per (query, probed list) table + 2*M per scanned code; "
                           f"{pairs} tables, {scanned} codes; the M lookups are random LDS reads, which bound "
                           "the scan")
        # the same launch against the LDS: M random 4-byte table reads per scanned code, at most
        # one 4-byte word per bank per clock (256 CUs x 64 banks x 2.4 GHz)
        lookups = scanned * m_sub
        lds_gbs = lookups * 4.0 / (rl["avg_launch_ms"] * 1e-3) / 1e9
        rl["lds"] = {"bound": "lds", "achieved": round(lds_gbs, 1), "peak": PEAK_LDS_GBS, "unit": "GB/s",
                     "frac": round(lds_gbs / PEAK_LDS_GBS, 4), "lookups_per_launch": lookups,
                     "note": "M 4-byte ADC table entries per scanned code (read 16 bytes at a time: the "
                             "four pairs of a work item share each read) against the CUs' LDS read rate "
                             "(256 CUs x 64 banks x 4 B x 2.4 GHz); random entries collide in banks, so a "
                             "wave's gather takes several passes and the full rate is out of reach"}
    # recall@10 against the exact kNN (the GPU engine, itself checked against the oracle), at the
    # benchmark's nprobe and two others
    eid = vh.CudaKnnEngine(base, d, vh.DistanceMetric.L2Squared).search_batch_arrays(q, k)[0]

    def recall_of(got):
        return round(float(np.mean([len(set(got[i]) & set(eid[i])) / k for i in range(nq)])), 4)

    recall = recall_of(ids)
    sweep = {}
    for npb in (8, 128):
        ix.search_batch_device(dq.ptr, nq, k, npb, di.ptr, dd.ptr, dl.ptr)
        vh.synchronize()
        t0 = time.perf_counter()
        ix.search_batch_device(dq.ptr, nq, k, npb, di.ptr, dd.ptr, dl.ptr)
        vh.synchronize()
        ms_n = (time.perf_counter() - t0) * 1e3
        sweep[str(npb)] = {"queries_per_s": round(nq * 1e3 / ms_n, 1),
                           "recall_at_10": recall_of(di.to_host(np.empty((nq, k), np.uint32)))}
    sweep[str(nprobe)] = {"queries_per_s": round(nq * 1e3 / ms, 1), "recall_at_10": recall}
    # PQ codes rank a cluster's members only approximately: the usual measure is how many of the
    # true 10 nearest are among the index's 100 best (recall 10@100)
    d100 = vh.DeviceBuffer(nq * 100 * 4)
    i100 = vh.DeviceBuffer(nq * 100 * 4)
    ix.search_batch_device(dq.ptr, nq, 100, nprobe, i100.ptr, d100.ptr, dl.ptr)
    got100 = i100.to_host(np.empty((nq, 100), np.uint32))
    recall_10_100 = round(float(np.mean([len(set(got100[i]) & set(eid[i])) / k for i in range(nq)])), 4)
    out = {"metric": "IVF-PQ queries/sec (1M x 128, nlist 1024, PQ16x256, nprobe 32, k=10)",
           "value": round(nq * 1e3 / ms, 1), "unit": "queries/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
           "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "strong", "vs_baseline": None,
           "dtype": "f32", "data": "synthetic",
           "config": {"workload": f"ivfpq_l2_mixture1024_{n}x{d}_nlist{nlist}_m{m_sub}_ks{ks}_nprobe{nprobe}_q{nq}_k{k}",
                      "parallelism": "single GPU", "build_s": round(build_s, 2), "recall_at_10": recall,
                      "recall_10_at_100": recall_10_100,
                      "codes_scanned_per_query": round(scanned / nq, 1),
                      "nprobe_sweep": dict(sorted(sweep.items(), key=lambda kv: int(kv[0])))},
           "roofline": rl}
    if with_cpu:
        import oracle

        # IvfPqIndex::search_with_nprobe is one query on one thread (ivf/mod.rs:256-345)
        inv = ix.inverted_index()
        sz, lids, lcodes = inv._csr()
        off = np.concatenate([[0], np.cumsum(sz)]).astype(np.uint64)
        cc = ix.coarse_centroids().reshape(-1, d)
        cb = ix.pq().codebooks

        ref = []

        def run(idx):
            ref.clear()
            t = time.perf_counter()
            for i in idx:
                pr, _ = oracle.find_top_centroids(q[i], cc, nprobe, "l2")
                ri, rd = oracle.ivfpq_search(q[i], cc, cb, m_sub, ks, off, lids, lcodes, pr, k, "l2")
                ref.append((int(i), pr, ri, rd))
            return time.perf_counter() - t

        dt = run(range(16))
        idx = parity_sample(nq, int(max(TAIL_QUERIES + 16, 16 * CPU_TARGET_S / max(dt, 1e-6))))
        dt = run(idx)
        out["parity"] = ivfpq_parity(ids, dist, probes, ref, k)
        out["parity"]["query_sample"] = describe_sample(idx, nq)
        be = {0: "scalar", 1: "AVX2+FMA", 2: "AVX-512F"}[oracle.detect_backend()]
        out["cpu_baseline"] = {"value": round(len(idx) / dt, 2), "unit": "queries/s", "cores": 1, "kind": "port",
                               "sample": f"{describe_sample(idx, nq)} through the oracle's find_top_centroids + "
                                         f"search_with_nprobe on the built index, {be} backend, {dt:.2f} s on "
                                         f"1 thread ({cpu_model()})"}
    return out


def ivfpq_parity(ids, dist, probes, ref, k):
    """Parity of the timed IVF-PQ search with the oracle's search_with_nprobe on the oracle's own
    probes (ref: (query index, probes, ids, distances) per sampled query).  A query whose GPU probe set differs
    from the oracle's (a near-tie at the nprobe-th centroid) is counted and skipped.  Otherwise
    the result counts must match, the distances as sorted lists within 1e-4 relative to the
    largest, and an id outside the oracle's k best may only tie with its k-th distance."""
    checked = probe_ties = 0
    dist_ok = ids_ok = True
    max_err = 0.0
    for i, pr, ri, rd in ref:
        if set(np.asarray(pr).tolist()) != set(probes[i].tolist()):
            probe_ties += 1
            continue
        checked += 1
        n = len(ri)
        gi, gd = ids[i, :n].astype(np.int64), dist[i, :n].astype(np.float64)
        if n < k and not (np.all(ids[i, n:] == 0xFFFFFFFF) and np.all(np.isnan(dist[i, n:]))):
            ids_ok = False
        if n == 0:
            continue
        rd = np.asarray(rd, np.float64)
        tol = 1e-4 * max(1.0, float(np.max(np.abs(rd))))
        err = float(np.max(np.abs(np.sort(gd) - np.sort(rd))))
        max_err = max(max_err, err)
        dist_ok = dist_ok and err <= tol and len(set(gi.tolist())) == n
        extra = set(gi.tolist()) - set(np.asarray(ri).tolist())
        if extra:
            ids_ok = ids_ok and all(abs(gd[list(gi).index(v)] - rd[n - 1]) <= tol for v in extra)
    ok = bool(dist_ok and ids_ok and checked >= 0.99 * len(ref))
    return {"queries_checked": checked, "probe_ties_skipped": probe_ties, "k": k, "max_abs_dist_err": max_err,
            "distance_tolerance": "1e-4 x max(1, |largest distance|)", "distances_ok": dist_ok,
            "ids_ok_up_to_ties": ids_ok, "ok": ok}


def bench_kmeans_fit(vh, with_cpu):
    """CudaKMeansEngine::fit end to end with its default seeded k-means++ init (kmeans.rs:58-97,
    409-460), the init timed apart from the Lloyd iterations:
    (a) the 2,000,000 x 96, 4,096-centroid mixture, 10 iterations (tol < 0), points resident
        (KMeansState.fit), plus the whole host-buffer fit; the init's HBM bound is one read of the
        points per drawn centre after the first, (K - 1) n dpad 4 B / 8 TB/s;
    (b) cuda_bench.rs:156-211's shape: 10,000 x 768 U[-1, 1], cosine, K = 16 .. 256, at most 15
        iterations, tol 1e-4, through CudaKMeansEngine.fit (host data in, centroids out), beside
        the oracle's KMeans::fit body from the same initial centroids on the host threads."""
    from vector_hip import datasets as ds
    import oracle

    def timed(fn, reps=1):
        fn()
        ts = []
        for _ in range(reps):
            vh.synchronize()
            t0 = time.perf_counter()
            r = fn()
            vh.synchronize()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts)), r

    n, d, kc = 2_000_000, 96, 4096
    log(f"kmeans_fit: {n} x {d} mixture, K = {kc}")
    data, _, _ = ds.gaussian_mixture(n, d, kc, ds.SEED_MIXTURE)
    st = vh.KMeansState(data)
    t_init, _ = timed(lambda: st.fit(kc, 0, -1.0, init_mode=vh.INIT_KMEANSPP, seed=42), reps=3)
    t_fit, (_, _, (_, _, iters, inertia)) = timed(lambda: st.fit(kc, 10, -1.0, init_mode=vh.INIT_KMEANSPP, seed=42),
                                                  reps=3)
    eng = vh.CudaKMeansEngine()
    t_host, _ = timed(lambda: eng.fit(data, d, kc, 10, -1.0))
    bound = (kc - 1) * n * d * 4 / PEAK_HBM
    big = {"workload": f"kmeans_l2_{n}x{d}_k{kc}_10iters_kmeanspp", "init_ms": round(t_init * 1e3, 2),
           "init_hbm_bound_ms": round(bound * 1e3, 2), "init_over_bound": round(t_init / bound, 3),
           "fit_ms": round(t_fit * 1e3, 2), "lloyd_ms": round((t_fit - t_init) * 1e3, 2), "iterations": iters,
           "inertia": inertia, "host_fit_ms": round(t_host * 1e3, 2),
           "note": "fit_ms: KMeansState.fit (points resident), median of 3; host_fit_ms: CudaKMeansEngine.fit with "
                   "the 768 MB of points uploaded and the centroids returned"}
    small = []
    dn, dd = 10_000, 768
    x = ds.uniform(dn, dd, ds.SEED_BASE)
    th = cpu_threads()
    for kk in (16, 32, 64, 128, 256):
        t_i, r0 = timed(lambda: eng.fit(x, dd, kk, 0, 1e-4, vh.DistanceMetric.CosineSimilarity), reps=5)
        t_f, r = timed(lambda: eng.fit(x, dd, kk, 15, 1e-4, vh.DistanceMetric.CosineSimilarity), reps=5)
        row = {"k": kk, "fit_ms": round(t_f * 1e3, 3), "init_ms": round(t_i * 1e3, 3), "iterations": r.iterations}
        if with_cpu:
            t0 = time.perf_counter()
            ref = oracle.kmeans_fit(x, r0.centroids, 15, 1e-4, "cosine", threads=th)
            row["cpu_lloyd_ms"] = round((time.perf_counter() - t0) * 1e3, 2)
            row["cpu_iterations"] = ref["iterations"]
        small.append(row)
        log(f"  k={kk}: {row}")
    out = {"metric": "CudaKMeansEngine::fit with k-means++ init (ms)", "value": big["fit_ms"], "unit": "ms",
           "n_gpus": 1, "steps": 3, "warmup": 1, "ms_per_step": big["fit_ms"], "higher_is_better": False,
           "scaling": "strong", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
           "config": {"workload": big["workload"], "parallelism": "single GPU"},
           "kmeans_2m": big, "cuda_bench_shape": {"data": f"{dn} x {dd} U[-1,1], cosine, at most 15 iterations, "
                                                          f"tol 1e-4, host buffers", "rows": small}}
    if with_cpu:
        out["cuda_bench_shape"]["cpu_note"] = (f"cpu_lloyd_ms: the oracle's KMeans::fit body from the GPU's k-means++ "
                                               f"centroids on {th} threads (affinity mask) ({cpu_model()})")
    return out


SWEEP_BATCHES = (1, 2, 4, 8, 16, 32, 64, 128)


def bench_batch_sweep(vh, reps, with_cpu):
    """cuda_bench.rs:41-55, 98-152: DistributedKnnEngine::search_batch at G = 1 over batch sizes 1 to
    128 with k = 10, on its default 10,000 x 768 U[-1, 1] base under cosine, and on the headline
    1,000,000 x 128 integer base under squared L2.  Per batch size: the host-buffer call (the
    reference's path: queries in, results out over PCIe) and the device-resident call, each the
    median of `reps` calls after two warm-up calls, against one pass over the base at 8 TB/s; every
    batch checked against the oracle (tie-aware recall, distances within 1e-4).  The host-buffer leg
    goes through DistributedKnnEngine.search_batch_arrays (the same C call as search_batch, without
    building Python result objects)."""
    from vector_hip import datasets as ds
    import oracle

    shapes = [("cos768_10k", ds.uniform(10_000, 768, ds.SEED_BASE), ds.uniform(128, 768, ds.SEED_QUERIES),
               vh.DistanceMetric.CosineSimilarity, "cosine"),
              ("l2int_1m", ds.uniform_int(1_000_000, 128, ds.SEED_BASE), ds.uniform_int(128, 128, ds.SEED_QUERIES),
               vh.DistanceMetric.L2Squared, "l2")]
    k = 10
    th = cpu_threads()
    out_shapes = {}
    all_ok = True
    for name, base, qs, metric, mname in shapes:
        n, d = base.shape
        log(f"batch_sweep: {name}")
        eng = vh.DistributedKnnEngine.try_new(base, d, 1, vh.GpuShardMode.Sharded, metric)
        dev = vh.CudaKnnEngine(base, d, metric)
        bound_us = n * d * 4 / PEAK_HBM * 1e6
        rows = []
        for b in SWEEP_BATCHES:
            q = np.ascontiguousarray(qs[:b])
            dq = vh.DeviceBuffer.from_host(q)
            di = vh.DeviceBuffer(b * k * 4)
            dd = vh.DeviceBuffer(b * k * 4)

            def med(fn):
                for _ in range(2):
                    fn()
                ts = []
                for _ in range(reps):
                    vh.synchronize()
                    t0 = time.perf_counter()
                    fn()
                    ts.append(time.perf_counter() - t0)
                return float(np.median(ts)) * 1e6

            # the host-buffer C call through the array binding (search_batch builds Python result
            # objects on top, which is the binding's cost, not the library's)
            host_us = med(lambda: eng.search_batch_arrays(q, k))
            dev_us = med(lambda: dev.search_batch_device(dq.ptr, b, k, di.ptr, dd.ptr))
            ids, dist, _ = dev.search_batch_arrays(q, k)
            ref = oracle.knn_search_batch(base, q, k, mname, threads=th)
            par = knn_parity(base, q, ids, dist, (ref, np.arange(b)), k, mname, 0.0 if mname == "l2" else 1e-4,
                             0.0 if mname == "l2" else 1e-6)
            host_res = eng.search_batch(q, k)
            # top_k_reduce may order equal distances differently: compare each query's id set
            same = all({r.id for r in host_res[i]} == set(ids[i].tolist()) for i in range(b))
            all_ok = all_ok and par["ok"] and same
            row = {"batch": b, "host_us": round(host_us, 1), "host_qps": round(b / host_us * 1e6, 1),
                   "device_us": round(dev_us, 1), "device_qps": round(b / dev_us * 1e6, 1),
                   "device_over_bound": round(dev_us / bound_us, 2), "parity_ok": par["ok"] and same}
            if with_cpu:
                t0 = time.perf_counter()
                oracle.knn_search_batch(base, q, k, mname, threads=th)
                row["cpu_us"] = round((time.perf_counter() - t0) * 1e6, 1)
            rows.append(row)
            log(f"  {name} batch {b}: {row}")
        out_shapes[name] = {"base": f"{n} x {d}", "metric": mname, "k": k, "one_pass_bound_us": round(bound_us, 2),
                            "rows": rows}
    b1 = out_shapes["cos768_10k"]["rows"][0]
    return {"metric": "kNN batch latency sweep (cuda_bench shape)", "value": b1["host_qps"], "unit": "queries/s",
            "n_gpus": 1, "steps": reps, "warmup": 2, "ms_per_step": round(b1["host_us"] / 1e3, 4),
            "higher_is_better": True, "scaling": "strong", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "batch_sweep_cos768_10k_and_l2int_1m_k10", "batches": list(SWEEP_BATCHES),
                       "parallelism": "single GPU"},
            "shapes": out_shapes,
            "cpu_note": f"cpu_us: the oracle's search_batch_cpu on {th} threads (affinity mask) ({cpu_model()})",
            "parity": {"ok": all_ok, "rule": "every batch against the oracle (tie-aware recall >= 0.999, distances "
                                             "exact for l2 integer data, 1e-4 for cosine); host-buffer ids equal "
                                             "the device call's"}}


# The reference's only published GPU figures (scripts/benchmarks/cuda_benchmark.svg:143, 262 on
# one NVIDIA T4; they equal the fallback values cuda_benchmark.py:110, 135 substitutes when criterion
# output is missing, so they are quoted for comparison, never as vs_baseline)
PUBLISHED_KNN_QPS = 45152.0      # batch kNN, cosine, N = 100,000, D = 768, k = 10, best batch (32)
PUBLISHED_KMEANS_FIT_S = 7.480   # CudaKMeansEngine::fit, cosine, N = 100,000, D = 768, K = 1024, 15 iters
PUBLISHED_BATCHES = (1, 2, 4, 8, 16, 32, 64, 128, 256, 512)


def bench_reference_published(vh, reps):
    """The reference's published GPU rows at their own shapes (cuda_benchmark.py:40-51 run
    cuda_bench.rs with N = 100,000, D = 768, cosine, U[-1, 1] data from generate_flat_vectors):
    * DistributedKnnEngine::search_batch at G = 1, k = 10, host slices in and results out, over
      batch sizes 1 to 512 (each the median of `reps` calls after two warm-ups); the batch of 32
      is checked against the oracle;
    * CudaKMeansEngine::fit with its default k-means++ init, K = 1024, 15 iterations at most,
      tolerance 1e-4, host data in and centroids out (median of 3 after one warm-up)."""
    from vector_hip import datasets as ds
    import oracle

    n, d, k = 100_000, 768, 10
    log(f"reference_published: {n} x {d} U[-1, 1], cosine")
    base = ds.uniform(n, d, ds.SEED_BASE)
    qs = ds.uniform(max(PUBLISHED_BATCHES), d, ds.SEED_QUERIES)
    cos = vh.DistanceMetric.CosineSimilarity
    eng = vh.DistributedKnnEngine.try_new(base, d, 1, vh.GpuShardMode.Sharded, cos)
    rows = []
    par = None
    for b in PUBLISHED_BATCHES:
        q = np.ascontiguousarray(qs[:b])
        for _ in range(2):
            eng.search_batch_arrays(q, k)
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            eng.search_batch_arrays(q, k)
            ts.append(time.perf_counter() - t0)
        us = float(np.median(ts)) * 1e6
        rows.append({"batch": b, "us": round(us, 1), "qps": round(b / us * 1e6, 1)})
        log(f"  knn batch {b}: {rows[-1]}")
        if b == 32:
            ids, dist, _ = eng.search_batch_arrays(q, k)
            ref = oracle.knn_search_batch(base, q, k, "cosine", threads=cpu_threads())
            par = knn_parity(base, q, ids, dist, (ref, np.arange(b)), k, "cosine", 1e-4, 1e-6)
    b32 = next(r for r in rows if r["batch"] == 32)
    best = max(rows, key=lambda r: r["qps"])
    knn = {"workload": f"search_batch_cosine_uniform_{n}x{d}_k{k}", "rows": rows,
           "batch32_qps": b32["qps"], "best": best, "published_t4_batch32_qps": PUBLISHED_KNN_QPS,
           "batch32_over_published": round(b32["qps"] / PUBLISHED_KNN_QPS, 2),
           "parity_batch32": {kk: par[kk] for kk in ("ok", "recall_tie_aware", "max_rel_dist_err")}}
    kc = 1024
    log(f"  kmeans fit K = {kc}")
    x = base
    fe = vh.CudaKMeansEngine()
    fe.fit(x, d, kc, 15, 1e-4, cos)
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        r = fe.fit(x, d, kc, 15, 1e-4, cos)
        ts.append(time.perf_counter() - t0)
    fit_s = float(np.median(ts))
    km = {"workload": f"kmeans_fit_cosine_uniform_{n}x{d}_k{kc}_15iters_tol1e-4", "fit_s": round(fit_s, 4),
          "iterations": r.iterations, "inertia": r.inertia, "published_t4_fit_s": PUBLISHED_KMEANS_FIT_S,
          "published_over_this": round(PUBLISHED_KMEANS_FIT_S / fit_s, 1)}
    log(f"  kmeans fit: {km}")
    return {"note": "the reference's only published GPU figures, one NVIDIA T4 (cuda_benchmark.svg:143, 262; "
                    "they equal cuda_benchmark.py's fallback values, so they are quoted, not a baseline)",
            "knn": knn, "kmeans_fit": km,
            "parity": {"ok": bool(par["ok"]), "rule": "batch of 32 against the oracle (tie-aware recall >= 0.999, "
                                                      "distances within 1e-4)"}}


def bench_copy(vh, nbytes=1 << 30, reps=5):
    """Plain device-to-device copy of `nbytes` (the runtime's blit kernel).  Its FETCH_SIZE and
    WRITE_SIZE counters calibrate the HBM traffic figures of the other kernels."""
    a = vh.DeviceBuffer(nbytes)
    b = vh.DeviceBuffer(nbytes)
    b.copy_from(a)
    vh.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        b.copy_from(a)
    vh.synchronize()
    dt = (time.perf_counter() - t0) / reps
    return {"metric": "device copy GB/s (read + write)", "value": round(2 * nbytes / dt / 1e9, 1), "unit": "GB/s",
            "n_gpus": 1, "steps": reps, "warmup": 1, "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True,
            "scaling": "strong", "vs_baseline": None, "dtype": "u8", "data": "synthetic",
            "config": {"workload": f"copy_{nbytes >> 20}MiB", "bytes_per_copy": nbytes}}


PEAK_PCIE5_X16 = 64.0e9   # B/s per direction, PCIe 5.0 x16 (the host link of one MI355X)


def bench_upload(vh, steps, warmup):
    """Engine builds from VECRSTOR files.  The reference reads each file into a Vec and uploads
    that (mpi_kmeans.rs:307-325, knn.rs:111-122); here the file is mapped and streamed through the
    pinned staging ring.  Legs, each the median of `steps` full engine builds (allocation, H2D,
    on-device row preparation) with the file warm in the page cache: the mapped file; the same
    rows already resident in a host array; and the reference's flow, read the file into an array
    then build.  Plus k-means over the 2M x 96 point set split into 8 shard files (segments) versus
    reading and concatenating the shards first."""
    import shutil
    import tempfile

    from vector_hip import datasets as ds

    def median_s(fn):
        for _ in range(warmup):
            fn()
        ts = []
        for _ in range(steps):
            vh.synchronize()
            t0 = time.perf_counter()
            e = fn()
            vh.synchronize()
            ts.append(time.perf_counter() - t0)
            del e
        return float(np.median(ts))

    n, d = 1_000_000, 128
    base = ds.uniform_int(n, d, ds.SEED_BASE)
    tmp = tempfile.mkdtemp(prefix="vh_upload_", dir=os.environ.get("TMPDIR", "/tmp"))
    try:
        p = os.path.join(tmp, "base.bin")
        vh.MmapStorage.create_from_flat(p, d, base)
        nbytes = n * d * 4
        log("upload: knn engine from mapped file / array / read-then-build")
        t_map = median_s(lambda: vh.CudaKnnEngine.from_vecrstor(p))
        t_arr = median_s(lambda: vh.CudaKnnEngine(base, d))
        t_read = median_s(lambda: vh.CudaKnnEngine(np.fromfile(p, dtype="<f4", offset=24).reshape(n, d), d))
        kn, kd, ns = 2_000_000, 96, 8
        log(f"upload: k-means state over {ns} shard files of a {kn} x {kd} mixture")
        pts, _, _ = ds.gaussian_mixture(kn, kd, 4096, ds.SEED_MIXTURE)
        paths = []
        for i, part in enumerate(np.array_split(pts, ns)):
            sp = os.path.join(tmp, f"shard_{i}.bin")
            vh.MmapStorage.create_from_flat(sp, kd, part)
            paths.append(sp)
        del pts

        def read_concat():
            return vh.KMeansState(np.concatenate([np.fromfile(sp, dtype="<f4", offset=24).reshape(-1, kd)
                                                  for sp in paths]))

        t_seg = median_s(lambda: vh.KMeansState.from_vecrstor(paths))
        t_cat = median_s(read_concat)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    kbytes = kn * kd * 4
    gbs = round(nbytes / t_map / 1e9, 2)
    return {"metric": "engine build GB/s from a VECRSTOR file (1M x 128 fp32 base)", "value": gbs, "unit": "GB/s",
            "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(t_map * 1e3, 2),
            "higher_is_better": True, "scaling": "strong", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "upload_vecrstor_1000000x128_knn_and_2000000x96_8shards_kmeans",
                       "page_cache": "warm", "parallelism": "single GPU"},
            "roofline": {"bound": "pcie", "achieved": gbs, "peak": PEAK_PCIE5_X16 / 1e9, "unit": "GB/s",
                         "frac": round(nbytes / t_map / PEAK_PCIE5_X16, 3), "traffic": None},
            "legs_ms": {"knn_mapped_file": round(t_map * 1e3, 2), "knn_host_array": round(t_arr * 1e3, 2),
                        "knn_read_then_build": round(t_read * 1e3, 2),
                        "kmeans_8_mapped_shards": round(t_seg * 1e3, 2),
                        "kmeans_read_concat_then_build": round(t_cat * 1e3, 2)},
            "legs_gbs": {"knn_mapped_file": gbs, "knn_host_array": round(nbytes / t_arr / 1e9, 2),
                         "knn_read_then_build": round(nbytes / t_read / 1e9, 2),
                         "kmeans_8_mapped_shards": round(kbytes / t_seg / 1e9, 2),
                         "kmeans_read_concat_then_build": round(kbytes / t_cat / 1e9, 2)}}


WORKLOADS = {
    "l2int": dict(n=1_000_000, d=128, nq=10_000, k=100, metric="l2", gen="uniform_int",
                  name="knn_l2_int0-255_1000000x128_q10000_k100"),
    "cos768": dict(n=1_000_000, d=768, nq=10_000, k=10, metric="cosine", gen="normalized",
                   name="knn_cosine_normalized_1000000x768_q10000_k10"),
    "gauss": dict(n=10_000, d=128, nq=100, k=10, metric="l2", gen="gaussian", name="knn_l2_gauss_10000x128_q100_k10"),
    "l1": dict(n=500_000, d=128, nq=4096, k=10, metric="l1", gen="uniform", name="knn_l1_uniform_500000x128_q4096_k10"),
    "linf": dict(n=500_000, d=128, nq=4096, k=10, metric="linf", gen="uniform",
                 name="knn_linf_uniform_500000x128_q4096_k10"),
    "hamming": dict(n=10_000_000, d=8, nq=10_000, k=10, metric="hamming", gen="packed_bits",
                    name="knn_hamming_packed256_10000000_q10000_k10"),
}


def bench_knn_workload(vh, key, steps, warmup, with_cpu):
    from vector_hip import datasets as ds

    w = WORKLOADS[key]
    log(f"{key}: generating base {w['n']} x {w['d']} ({w['gen']})")
    gen = getattr(ds, w["gen"])
    if w["gen"] == "packed_bits":
        base = gen(w["n"], 32 * w["d"], ds.SEED_BASE)
        q = gen(w["nq"], 32 * w["d"], ds.SEED_QUERIES)
    else:
        base = gen(w["n"], w["d"], ds.SEED_BASE)
        q = gen(w["nq"], w["d"], ds.SEED_QUERIES)
    names = {"l2": "L2Squared", "dot": "DotProduct", "cosine": "CosineSimilarity", "l1": "Manhattan",
             "linf": "Chebyshev"}
    metric = vh.DistanceMetric[names[w["metric"]]] if w["metric"] != "hamming" else None
    ham = w["metric"] == "hamming"
    ms, prof, ids, dist, host_ms = run_knn(vh, base, q, w["k"], metric, steps, warmup, hamming=ham)
    gemm = w["metric"] in ("l2", "dot", "cosine")
    if gemm:
        rl = roofline(prof, "mfma", PEAK_MFMA_F32, "TFLOP/s", key)
    elif ham and os.environ.get("VHIP_HAMMING_KERNEL") != "popcount":
        # packed codes run on the fp4 matrix cores: 2 K operations per (query, row), K = the
        # padded code bits (a power of two, at least 64)
        rl = roofline(dict(prof), "mfma", PEAK_MFMA_FP4, "TFLOP/s", key)
        if rl:
            rl["unit"] = "TOP/s (fp4 MFMA)"
    else:
        # VALU-bound: work counts element (or word) operations, each two VALU operations (a
        # subtract and an add or max with the |.| modifier; XOR and bit count for packed words),
        # against the published vector FP32 peak
        p2 = dict(prof)
        p2["work"] = prof["work"] * 2.0
        rl = roofline(p2, "valu", PEAK_VECTOR_F32, "TFLOP/s", key)
        if rl:
            rl["unit"] = "Top/s (against the vector FP32 peak)"
    out = {"metric": METRIC, "value": round(w["nq"] * 1e3 / ms, 2), "unit": "queries/s", "n_gpus": 1,
           "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 3), "higher_is_better": True,
           "scaling": "strong", "vs_baseline": None,
           "dtype": ("u32" if os.environ.get("VHIP_HAMMING_KERNEL") == "popcount" else "fp4") if ham else "f32",
           "data": "synthetic",
           "config": {"workload": w["name"], "base_rows": w["n"], "dim": w["d"] * (32 if ham else 1),
                      "queries": w["nq"], "k": w["k"], "metric": w["metric"], "parallelism": "single GPU"},
           "roofline": rl,
           "host_buffers": {"value": round(w["nq"] * 1e3 / host_ms, 2), "unit": "queries/s", "ms": round(host_ms, 3),
                            "note": "one batch through the host-buffer entry point (PCIe copies included), "
                                    "median of 3 after a warm-up call; not the headline value"}}
    import oracle

    k = w["k"]
    if ham:
        if with_cpu:
            sub = 500_000
            un_b = oracle.unpack_bits(base[:sub])
            un_q = oracle.unpack_bits(q)
            cb, _ = cpu_knn_baseline(un_b, un_q, k, "hamming", full_under_s=0.0)
            del un_b, un_q
            cb["value"] = round(cb["value"] * sub / w["n"], 4)
            cb["sample"] = (f"reference semantics (thresholded float Hamming over codes unpacked to 0/1 floats) "
                            f"against {sub} of the {w['n']} codes, rate scaled by {sub}/{w['n']}; " + cb["sample"])
            out["cpu_baseline"] = cb
        # parity over the full base: the oracle's popcount search on a strided query sample with
        # the last queries, bit-exact
        idx = parity_sample(w["nq"], 640 if with_cpu else 192)
        ref = (oracle.hamming_packed_knn(base, np.ascontiguousarray(q[idx]), k, threads=cpu_threads()), idx)
        out["parity"] = knn_parity(base, q, ids, dist, ref, k, "hamming", 0.0, 0.0, min_recall=1.0)
    else:
        if with_cpu:
            out["cpu_baseline"], ref = cpu_knn_baseline(base, q, k, w["metric"])
        else:
            idx = parity_sample(w["nq"], 192)
            ref = (oracle.knn_search_batch(base, np.ascontiguousarray(q[idx]), k, w["metric"], threads=cpu_threads()),
                   idx)
        # distances within 1e-4 relative; integer data is exact in every summation order
        exact = w["gen"] == "uniform_int"
        out["parity"] = knn_parity(base, q, ids, dist, ref, k, w["metric"], 0.0 if exact else 1e-4,
                                   0.0 if exact else 1e-6)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="default",
                    choices=["default", "kmeans", "kmeans_fit", "batch_sweep", "published", "copy", "ivf_coarse", "ivfpq",
                             "upload"] + sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the library has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)
    import vector_hip as vh

    if vh.CudaDeviceContext.device_count() < 1:
        print("no gfx950 GPU visible", file=sys.stderr)
        sys.exit(1)
    ctx = vh.CudaDeviceContext(0)
    if args.workload == "copy":
        out = bench_copy(vh)
    elif args.workload == "ivf_coarse":
        out = bench_ivf_coarse(vh, args.steps, args.warmup, not args.no_cpu)
    elif args.workload == "ivfpq":
        out = bench_ivfpq(vh, args.steps, args.warmup, not args.no_cpu)
    elif args.workload == "upload":
        out = bench_upload(vh, args.steps, args.warmup)
    elif args.workload == "kmeans_fit":
        out = bench_kmeans_fit(vh, not args.no_cpu)
    elif args.workload == "batch_sweep":
        out = bench_batch_sweep(vh, max(args.steps, 20), not args.no_cpu)
    elif args.workload == "published":
        r = bench_reference_published(vh, max(args.steps, 20))
        out = {"metric": "the reference's published GPU rows at their shapes", "value": r["knn"]["batch32_qps"],
               "unit": "queries/s", "n_gpus": 1, "steps": max(args.steps, 20), "warmup": 2,
               "ms_per_step": round(32 / r["knn"]["batch32_qps"] * 1e3, 4), "higher_is_better": True,
               "scaling": "strong", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
               "config": {"workload": r["knn"]["workload"], "parallelism": "single GPU"}, **r}
    elif args.workload == "kmeans":
        r = bench_kmeans(vh, 10, not args.no_cpu)
        out = {"metric": METRIC, "value": r["value"], "unit": r["unit"], "n_gpus": 1, "steps": 10, "warmup": 1,
               "ms_per_step": r["ms_per_iteration"], "higher_is_better": True, "scaling": "strong",
               "vs_baseline": None, "dtype": "f32", "data": "synthetic",
               "config": {"workload": r["workload"], "parallelism": "single GPU"}, "roofline": r["roofline"],
               "cpu_baseline": r.get("cpu_baseline"), "parity": r["parity"]}
    else:
        key = "l2int" if args.workload == "default" else args.workload
        out = bench_knn_workload(vh, key, args.steps, args.warmup, not args.no_cpu)
        if args.workload == "default":
            out["kmeans"] = bench_kmeans(vh, 10, not args.no_cpu)
            # the other benchmark workloads, each with its roofline, CPU baseline and parity
            for extra in ("cos768", "hamming", "l1", "linf"):
                r = bench_knn_workload(vh, extra, args.steps, args.warmup, not args.no_cpu)
                out[extra] = {kk: r[kk] for kk in ("value", "unit", "ms_per_step", "dtype", "config", "roofline",
                                                   "host_buffers", "cpu_baseline", "parity") if kk in r}
            r = bench_ivfpq(vh, args.steps, args.warmup, not args.no_cpu)
            out["ivfpq"] = {kk: r[kk] for kk in ("metric", "value", "unit", "ms_per_step", "dtype", "config",
                                                 "roofline", "cpu_baseline", "parity") if kk in r}
            # the reference benchmark's own shapes: search_batch over batch sizes 1..128, and fit()
            # with its default k-means++ init
            r = bench_batch_sweep(vh, 20, not args.no_cpu)
            out["batch_sweep"] = {kk: r[kk] for kk in ("metric", "config", "shapes", "cpu_note", "parity")}
            r = bench_kmeans_fit(vh, not args.no_cpu)
            out["kmeans_fit"] = {kk: r[kk] for kk in ("metric", "kmeans_2m", "cuda_bench_shape")}
            out["reference_published"] = bench_reference_published(vh, 20)
    out["config"]["device"] = ctx.device_name()
    print(json.dumps(out))
    bad = [name for name, part in [("top", out)] + [(kk, v) for kk, v in out.items() if isinstance(v, dict)]
           if isinstance(part.get("parity"), dict) and not part["parity"]["ok"]]
    if bad:
        log(f"parity check failed: {bad}")
        sys.exit(3)


if __name__ == "__main__":
    main()
