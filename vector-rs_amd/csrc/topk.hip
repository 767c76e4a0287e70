// topk.hip -- per-query top-k maintenance between filter rounds.
//
// A search runs the base in rounds of geometrically growing row ranges.  The filter
// kernels (knn_gemm.hip, knn_valu.hip, hamming.hip) append every (score, id) with
// score <= tau[q] to the query's candidate list; k_topk_merge then selects the best k of the
// running top-k and those candidates (64-bit keys: ordered score << 32 | id, so ties break
// towards the lower id).  The new tau is the k-th score, an
// upper bound of the final k-th score, so no true neighbour can be filtered out later.
// This replaces knn_topk_select (knn.cu:206-305) and its K <= 128 clamp.
#include <algorithm>

#include "vh_common.h"

namespace vh {

typedef unsigned long long u64;

__global__ void k_topk_init(int nq, float *tau, uint32_t *have, uint32_t *cnt, uint32_t *flags, uint32_t *mflag,
                            uint32_t *nflag, uint32_t cnt0, uint32_t *pad) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q < nq) {
        tau[q] = INFINITY;
        have[q] = 0;
        cnt[q] = cnt0;
        flags[q] = 0;
        mflag[q] = 0;
        if (pad && q < kSmallPadQueries) pad[(size_t)q * kSmallPadStride] = 0;
    }
    if (q < 2) nflag[q] = 0;
}

__global__ void k_fill_f32(float *p, size_t count, float v) {
    const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i < count) p[i] = v;
}

void launch_fill(float *p, size_t count, float v, hipStream_t s) {
    if (count == 0) return;
    hipLaunchKernelGGL(k_fill_f32, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, p, count, v);
}

__global__ void k_fill_u32(uint32_t *p, size_t count, uint32_t v) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < count; i += (size_t)gridDim.x * blockDim.x)
        p[i] = v;
}

void launch_fill_u32(uint32_t *p, size_t count, uint32_t v, hipStream_t s) {
    if (count == 0) return;
    size_t blocks = (count + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)blocks), dim3(256), 0, s, p, count, v);
}

void launch_topk_init(int nq, float *tau, uint32_t *have, uint32_t *cnt, uint32_t *flags, uint32_t *mflag,
                      uint32_t *nflag, uint32_t cnt0, uint32_t *pad, hipStream_t s) {
    if (nq <= 0) return;
    hipLaunchKernelGGL(k_topk_init, dim3(ceil_div(nq, 256)), dim3(256), 0, s, nq, tau, have, cnt, flags, mflag, nflag,
                       cnt0, pad);
}

// A 64-bit key from lane (this lane ^ mask) of the wave.
__device__ __forceinline__ u64 shfl_xor_u64(u64 v, int mask) {
    const uint32_t lo = __shfl_xor((uint32_t)v, mask, 64), hi = __shfl_xor((uint32_t)(v >> 32), mask, 64);
    return ((u64)hi << 32) | lo;
}

// Bitonic sort of P (power of two) keys in LDS, ascending.  Must be called by all threads.
__device__ __forceinline__ void bitonic_sort_lds(u64 *buf, int P) {
    const int tid = threadIdx.x, nt = blockDim.x;
    if (P <= 128) {
        // Up to 128 keys: one wave sorts them in registers, two a lane (key i in lane i % 64,
        // register i / 64), exchanging through shuffles, so the network's stages need no
        // workgroup barrier; the other waves wait at the one barrier after it.
        if (tid < 64) {
            u64 a0 = tid < P ? buf[tid] : ~0ull, a1 = tid + 64 < P ? buf[tid + 64] : ~0ull;
            for (int size = 2; size <= P; size <<= 1) {
                for (int stride = size >> 1; stride > 0; stride >>= 1) {
                    if (stride == 64) {  // size 128: keys i and i + 64 meet within the lane, ascending
                        const u64 mn = a0 < a1 ? a0 : a1, mx = a0 < a1 ? a1 : a0;
                        a0 = mn;
                        a1 = mx;
                        continue;
                    }
                    // key i keeps the smaller of it and key i ^ stride when it is the lower of the
                    // two in an ascending block, or the upper in a descending one
                    const bool low = (tid & stride) == 0;
                    const u64 b0 = shfl_xor_u64(a0, stride), b1 = shfl_xor_u64(a1, stride);
                    const bool min0 = low == ((tid & size) == 0), min1 = low == (((tid + 64) & size) == 0);
                    a0 = min0 ? (a0 < b0 ? a0 : b0) : (a0 < b0 ? b0 : a0);
                    a1 = min1 ? (a1 < b1 ? a1 : b1) : (a1 < b1 ? b1 : a1);
                }
            }
            if (tid < P) buf[tid] = a0;
            if (tid + 64 < P) buf[tid + 64] = a1;
        }
        __syncthreads();
        return;
    }
    for (int size = 2; size <= P; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < (P >> 1); i += nt) {
                const int lo = ((i & ~(stride - 1)) << 1) | (i & (stride - 1));
                const int hi = lo + stride;
                const bool asc = (lo & size) == 0;
                const u64 a = buf[lo], b = buf[hi];
                if ((a > b) == asc) {
                    buf[lo] = b;
                    buf[hi] = a;
                }
            }
            __syncthreads();
        }
    }
}

// ---- merge: running top-k + this round's candidates -> new top-k -------------------------
// Element i of query q is the running entry topk[q][i] for i < have[q], else candidate
// cand[q][i - have[q]]; its 64-bit key is (score key << 32) | vector id.  Keys are unique (every
// base row is scanned by exactly one round), so "the k smallest keys" is well defined.
//
// Small merges (T = have + c <= kMergeDirect, sorted by one wave in registers) sort everything.
// Larger ones select first: a histogram of the 32-bit score keys over kMergeBins equal-width
// buckets of [min, max] finds the bucket holding the k-th smallest; the elements below it (fewer
// than k) and those in it are gathered into LDS and only they are sorted.  When the boundary bucket is
// too large for the buffer (massive score ties) the merge falls back to sorting chunks of the
// elements against the running best k.
constexpr int kMergeBins = 1024;
// Selecting first pays from about a hundred entries on: with 400 entries (a k = 100 round), the
// select and a 128-key register sort take 58 us a merge of 10,000 queries, a 512-key LDS sort 81.
constexpr int kMergeDirect = 128;
constexpr int kMergeCached = 16;  // list entries per thread held in registers through the select

// The minimum of lo and the maximum of hi over the workgroup, in one round of LDS (red: 2 words
// per wave).
__device__ __forceinline__ void block_minmax_u32(uint32_t &lo, uint32_t &hi, uint32_t *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = (int)(blockDim.x >> 6);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        lo = min(lo, __shfl_xor(lo, o, 64));
        hi = max(hi, __shfl_xor(hi, o, 64));
    }
    __syncthreads();
    if (lane == 0) {
        red[wave] = lo;
        red[nw + wave] = hi;
    }
    __syncthreads();
    lo = red[0];
    hi = red[nw];
    for (int w = 1; w < nw; ++w) {
        lo = min(lo, red[w]);
        hi = max(hi, red[nw + w]);
    }
}

// buf holds `bufn` u64 entries (dynamic LDS, bufn >= 2 * pow2(kc), >= kMergeDirect).  NT threads
// per query: 256, or 1024 for a dense round of many rows, whose selection passes over all its
// scores are latency-bound (each thread keeps four independent loads in flight).
template <int NT>
__global__ __launch_bounds__(NT) void k_topk_merge(int k, int kc, int bufn, const uint2 *__restrict__ cand,
                                                    uint32_t *__restrict__ cnt, int cnt_stride, int cap,
                                                    const uint32_t *__restrict__ perm, u64 *__restrict__ topk,
                                                    uint32_t *__restrict__ have, float *__restrict__ tau,
                                                    uint32_t *__restrict__ flags, uint32_t *__restrict__ nflagged,
                                                    const float *__restrict__ qerr, uint32_t *__restrict__ mflag,
                                                    uint32_t *__restrict__ mcount) {
    extern __shared__ u64 buf[];
    __shared__ uint32_t hist[kMergeBins];
    __shared__ uint32_t red[2 * (NT / 64)];
    __shared__ uint32_t s_part[NT / 64];
    __shared__ uint32_t s_sel[4];  // boundary bucket, count below it, gather counters
    const int q = blockIdx.x, tid = threadIdx.x;
    uint32_t *const cq_cnt = cnt + (size_t)q * cnt_stride;  // this query's candidate count
    const uint32_t c_all = *cq_cnt;
    if (flags[q] || c_all == 0) {
        __syncthreads();
        if (tid == 0) {
            *cq_cnt = 0;
            // the last round counts the margin flags as they stand (an overflowed query is re-run
            // and counted again afterwards)
            if (mcount && !flags[q] && mflag[q]) atomicAdd(mcount, 1u);
        }
        return;
    }
    // entries to keep: k, or kc when the scores carry a selection error
    const float e2 = qerr ? 2.0f * qerr[q] : 0.0f;
    const uint32_t kk = e2 > 0.0f ? (uint32_t)kc : (uint32_t)k;
    const bool overflow = c_all > (uint32_t)cap;
    const uint32_t c = overflow ? (uint32_t)cap : c_all;
    u64 *tk = topk + (size_t)q * kc;
    const uint2 *cq = cand + (size_t)q * cap;
    const uint32_t h = have[q];
    const uint32_t T = h + c;
    auto key32 = [&](uint32_t i) -> uint32_t { return i < h ? (uint32_t)(tk[i] >> 32) : cq[i - h].x; };
    auto key64 = [&](uint32_t i) -> u64 {
        if (i < h) return tk[i];
        const uint2 e = cq[i - h];
        return ((u64)e.x << 32) | (u64)perm[e.y];  // base position -> vector id
    };

    uint32_t hn = 0;  // entries of the new kept list, sorted in buf[0 .. hn)
    bool done = false;
    if (T > (uint32_t)kMergeDirect && T > kk) {
        // ---- bucket select ----
        // Up to kMergeCached keys per thread stay in registers for the three passes (one read of
        // the list); longer lists are read in each pass, four keys in flight per thread.
        const bool cached = T <= (uint32_t)(kMergeCached * NT);
        uint32_t kv[kMergeCached];
        if (cached) {
#pragma unroll
            for (int u = 0; u < kMergeCached; ++u) {
                const uint32_t i = tid + u * NT;
                kv[u] = i < T ? key32(i) : 0u;
            }
        }
        // fn(i, score key) for every entry i of this thread
        auto visit = [&](auto fn) {
            if (cached) {
#pragma unroll
                for (int u = 0; u < kMergeCached; ++u)
                    if (tid + u * NT < T) fn(tid + u * NT, kv[u]);
            } else {
                for (uint32_t i0 = tid; i0 < T; i0 += 4 * NT) {
                    uint32_t v[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) v[u] = i0 + u * NT < T ? key32(i0 + u * NT) : 0u;
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (i0 + u * NT < T) fn(i0 + u * NT, v[u]);
                }
            }
        };
        uint32_t lo = 0xffffffffu, hi = 0u;
        visit([&](uint32_t, uint32_t v) {
            lo = min(lo, v);
            hi = max(hi, v);
        });
        block_minmax_u32(lo, hi, red);
        if (lo < hi) {
            const float scale = (float)kMergeBins / ((float)(hi - lo) + 1.0f);
            auto bucket = [&](uint32_t v) { return min(kMergeBins - 1, (int)((float)(v - lo) * scale)); };
            for (int i = tid; i < kMergeBins; i += NT) hist[i] = 0;
            __syncthreads();
            visit([&](uint32_t, uint32_t v) { atomicAdd(&hist[bucket(v)], 1u); });
            __syncthreads();
            // bucket b* holding the kk-th smallest: cum(b*) < kk <= cum(b*) + hist[b*].  Each thread
            // sums its run of bins; the runs' exclusive prefix comes from a wave scan (shuffles) and
            // the waves' totals.
            constexpr int per = kMergeBins / NT;
            uint32_t loc = 0;
#pragma unroll
            for (int j = 0; j < per; ++j) loc += hist[tid * per + j];
            const int lane = tid & 63, wave = tid >> 6;
            uint32_t incl = loc;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_up(incl, o, 64);
                if (lane >= o) incl += t;
            }
            if (lane == 63) s_part[wave] = incl;
            __syncthreads();
            for (int w = 0; w < wave; ++w) incl += s_part[w];
            uint32_t cum = incl - loc;  // elements in buckets before this thread's bins
#pragma unroll
            for (int j = 0; j < per; ++j) {
                const uint32_t hb = hist[tid * per + j];
                if (cum < kk && kk <= cum + hb) {
                    s_sel[0] = (uint32_t)(tid * per + j);
                    s_sel[1] = cum;
                }
                cum += hb;
            }
            if (tid == 0) {
                s_sel[2] = 0;
                s_sel[3] = 0;
            }
            __syncthreads();
            const int bstar = (int)s_sel[0];
            const uint32_t below = s_sel[1];
            const uint32_t inb = hist[bstar];
            if (below + inb <= (uint32_t)bufn) {
                visit([&](uint32_t i, uint32_t v) {
                    const int b = bucket(v);
                    if (b < bstar) buf[atomicAdd(&s_sel[2], 1u)] = key64(i);
                    else if (b == bstar) buf[below + atomicAdd(&s_sel[3], 1u)] = key64(i);
                });
                const uint32_t total = below + inb;
                int P = 2;
                while ((uint32_t)P < total) P <<= 1;
                for (uint32_t i = total + tid; i < (uint32_t)P; i += NT) buf[i] = ~0ull;
                __syncthreads();
                bitonic_sort_lds(buf, P);
                hn = kk;
                done = true;
            }
        }
    }
    if (!done) {
        // ---- sort everything, in chunks against the running best kk ----
        uint32_t hh = 0, next = 0;
        while (next < T || hh == 0) {
            const uint32_t take = min(T - next, (uint32_t)bufn - hh);
            for (uint32_t i = tid; i < take; i += NT) buf[hh + i] = key64(next + i);
            const uint32_t total = hh + take;
            int P = 2;
            while ((uint32_t)P < total) P <<= 1;
            for (uint32_t i = total + tid; i < (uint32_t)P; i += NT) buf[i] = ~0ull;
            __syncthreads();
            bitonic_sort_lds(buf, P);
            hh = min(total, kk);
            next += take;
            if (next >= T) break;
        }
        hn = hh;
    }
    __syncthreads();
    for (uint32_t i = tid; i < hn; i += NT) tk[i] = buf[i];
    if (tid == 0) {
        have[q] = hn;
        *cq_cnt = 0;
        if (overflow) {
            // The list is incomplete: stop filtering for this query; the host re-runs it
            // with a capacity that cannot overflow.
            flags[q] = 1;
            tau[q] = -INFINITY;
            atomicAdd(nflagged, 1u);
        } else if (hn < (uint32_t)k) {
            tau[q] = INFINITY;
            if (mflag) mflag[q] = 0;
        } else {
            // Later rows can only matter when they score within the margin of the k-th; once
            // kk entries are kept, also only when they beat the kk-th.
            const float sk = key_score((uint32_t)(buf[k - 1] >> 32));
            float t = sk + e2;
            bool cut = false;
            if (kk > (uint32_t)k && hn >= kk) {
                const float skk = key_score((uint32_t)(buf[kk - 1] >> 32));
                cut = skk <= t;
                t = fminf(t, skk);
            }
            // a NaN k-th score (fewer than k rows with a finite score so far) filters nothing yet
            tau[q] = t == t ? t : INFINITY;
            if (mflag) mflag[q] = cut ? 1u : 0u;
            if (mcount && cut) atomicAdd(mcount, 1u);
        }
    }
}

int merge_buffer_entries(int kc) {
    int p = 1;
    while (p < kc) p <<= 1;
    return std::max(2 * p, 1024);
}

template <int NT>
static void launch_merge_nt(int nq, int k, int kc, const uint2 *cand, uint32_t *cnt, int cnt_stride, int cap,
                            const uint32_t *perm,
                            unsigned long long *topk, uint32_t *have, float *tau, uint32_t *flags, uint32_t *nflagged,
                            const float *qerr, uint32_t *mflag, uint32_t *mcount, hipStream_t s) {
    const int bufn = merge_buffer_entries(kc);
    const size_t lds = (size_t)bufn * sizeof(u64);
    static bool attr_set = false;
    if (!attr_set && lds > 65536) {
        // more than 64 KB of dynamic LDS (gfx950 offers 160 KB per workgroup)
        (void)hipFuncSetAttribute((const void *)k_topk_merge<NT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)(merge_buffer_entries(kMaxKeep) * sizeof(u64)));
        (void)hipGetLastError();
        attr_set = true;
    }
    hipLaunchKernelGGL(k_topk_merge<NT>, dim3(nq), dim3(NT), lds, s, k, kc, bufn, cand, cnt, cnt_stride, cap, perm,
                       topk, have, tau, flags, nflagged, qerr, mflag, mcount);
}

void launch_topk_merge(int nq, int k, int kc, const uint2 *cand, uint32_t *cnt, int cnt_stride, int cap,
                       const uint32_t *perm, unsigned long long *topk, uint32_t *have, float *tau, uint32_t *flags,
                       uint32_t *nflagged, const float *qerr, uint32_t *mflag, uint32_t *mcount, bool wide,
                       hipStream_t s) {
    if (nq <= 0) return;
    if (wide)
        launch_merge_nt<1024>(nq, k, kc, cand, cnt, cnt_stride, cap, perm, topk, have, tau, flags, nflagged, qerr, mflag, mcount,
                              s);
    else
        launch_merge_nt<256>(nq, k, kc, cand, cnt, cnt_stride, cap, perm, topk, have, tau, flags, nflagged, qerr, mflag, mcount,
                             s);
}

__global__ void k_count_flags(const uint32_t *__restrict__ flags, int n, uint32_t *__restrict__ count) {
    __shared__ uint32_t red[4];
    uint32_t c = 0;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) c += flags[i] != 0;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = c;
    __syncthreads();
    if (threadIdx.x == 0) *count = red[0] + red[1] + red[2] + red[3];
}

void launch_count_flags(const uint32_t *flags, int n, uint32_t *count, hipStream_t s) {
    hipLaunchKernelGGL(k_count_flags, dim3(1), dim3(256), 0, s, flags, n, count);
}

// Row r of a re-run batch (kept entries at stride ks, count, margin flag) back into query idx[r]
// of the main batch (stride kd >= the entries copied).  A null src_mflag clears the flag.
__global__ __launch_bounds__(256) void k_scatter_topk(const u64 *__restrict__ src, int ks,
                                                      const uint32_t *__restrict__ src_have,
                                                      const uint32_t *__restrict__ src_mflag,
                                                      const uint32_t *__restrict__ idx, u64 *__restrict__ dst, int kd,
                                                      uint32_t *__restrict__ dst_have,
                                                      uint32_t *__restrict__ dst_mflag) {
    const int r = blockIdx.x;
    const uint32_t q = idx[r];
    const uint32_t h = min(src_have[r], (uint32_t)min(ks, kd));
    for (uint32_t j = threadIdx.x; j < h; j += blockDim.x) dst[(size_t)q * kd + j] = src[(size_t)r * ks + j];
    if (threadIdx.x == 0) {
        dst_have[q] = h;
        dst_mflag[q] = src_mflag ? src_mflag[r] : 0u;
    }
}

void launch_scatter_topk(const unsigned long long *src, int ks, const uint32_t *src_have, const uint32_t *src_mflag,
                         const uint32_t *idx, int m, unsigned long long *dst, int kd, uint32_t *dst_have,
                         uint32_t *dst_mflag, hipStream_t s) {
    if (m <= 0) return;
    hipLaunchKernelGGL(k_scatter_topk, dim3(m), dim3(256), 0, s, src, ks, src_have, src_mflag, idx, dst, kd, dst_have,
                       dst_mflag);
}

__global__ __launch_bounds__(256) void k_gather_rows(const float *__restrict__ src, const uint32_t *__restrict__ idx,
                                                     size_t rows, int width, float *__restrict__ dst) {
    const size_t total = rows * (size_t)width;
    for (size_t t = blockIdx.x * 256 + threadIdx.x; t < total; t += (size_t)gridDim.x * 256) {
        const size_t r = t / width, c = t - r * width;
        dst[t] = src[(size_t)idx[r] * width + c];
    }
}

void launch_gather_rows(const float *src, const uint32_t *idx, size_t rows, int width, float *dst, hipStream_t s) {
    if (rows == 0) return;
    const unsigned blocks = (unsigned)std::min<size_t>(4096, (rows * width + 255) / 256);
    hipLaunchKernelGGL(k_gather_rows, dim3(blocks), dim3(256), 0, s, src, idx, rows, width, dst);
}

// The search's two flag counters (device) copied to pinned host memory by one thread of the final
// kernel, with a system-scope release, so that the host reads them after the stream's sync with no
// copy of their own.
__device__ __forceinline__ void publish_flags(const FlagPublish &p) {
    if (p.host) {
        __hip_atomic_store(p.host, p.src[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(p.host + 1, p.src[1], __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

__global__ void k_topk_finalize(int nq, int kc, int kout, int metric, const u64 *__restrict__ topk,
                                const uint32_t *__restrict__ have, uint32_t *__restrict__ out_ids,
                                float *__restrict__ out_dist, uint32_t *__restrict__ out_dist_u32, int ostride,
                                FlagPublish pub) {
    const long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (i == 0) publish_flags(pub);
    if (i >= (long)nq * kout) return;
    const int q = (int)(i / kout), j = (int)(i % kout);
    const size_t o = (size_t)q * ostride + j;
    if ((uint32_t)j < have[q]) {
        const u64 e = topk[(size_t)q * kc + j];
        const float sc = key_score((uint32_t)(e >> 32));
        const float d = (metric == DOT || metric == COS) ? -sc + 0.0f : sc;
        out_ids[o] = (uint32_t)e;
        if (out_dist) out_dist[o] = d;
        if (out_dist_u32) out_dist_u32[o] = (uint32_t)d;
    } else {
        out_ids[o] = 0xffffffffu;
        if (out_dist) out_dist[o] = __builtin_nanf("");
        if (out_dist_u32) out_dist_u32[o] = 0xffffffffu;
    }
}

void launch_topk_finalize(int nq, int kc, int kout, int metric, const unsigned long long *topk,
                          const uint32_t *have, uint32_t *out_ids, float *out_dist, uint32_t *out_dist_u32,
                          int ostride, const FlagPublish &pub, hipStream_t s) {
    const long total = std::max((long)nq * kout, 1L);
    hipLaunchKernelGGL(k_topk_finalize, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, nq, kc, kout, metric,
                       topk, have, out_ids, out_dist, out_dist_u32, ostride, pub);
}

// Final pass for the GEMM-form metrics.  The selection used the GEMM-form score (the norm form
// ||q'||^2 + ||x'||^2 - 2 q'.x' of shifted operands for squared L2, the dot product of normalised
// rows for cosine), which differs from the reference CPU engine's direct form by at most the
// query's selection error bound; the kept entries hold every row within twice that bound of the
// k-th.  For each of them the distance is recomputed in the direct form (sum (q-x)^2 of the
// unshifted operands, sum q*x, or dot / (sqrt(|q|^2) sqrt(|x|^2)) with the 1e-9 guard,
// scalar.rs:14-75), the entries are re-sorted by (distance, id), and the best k written out.
// One workgroup per query: its threads first fetch every kept neighbour's id and stored row at
// once (the id -> row lookup is a dependent load), then groups of 16 lanes evaluate one neighbour
// each, 16 at a time, with float4 reads of the row and the query (lane s sums pieces s, s + 16,
// ... in order) and a fixed xor butterfly.  A query with a zero bound (squared L2 or dot product
// on integer rows within 2^24) skips the recomputation: its scores are already the exact values.
// Sort-buffer entries of the refine: a power of two holding kc keys (at least 2).
__host__ __device__ __forceinline__ int refine_sort_entries(int kc) {
    int p = 2;
    while (p < kc) p <<= 1;
    return p;
}

__global__ __launch_bounds__(256) void k_topk_refine(int k, int kc, int kout, int metric,
                                                     const float *__restrict__ qrows, const float *__restrict__ base,
                                                     const float *__restrict__ shift,
                                                     const uint32_t *__restrict__ inv_perm, int dpad,
                                                     const float *__restrict__ qnorm, const float *__restrict__ bnorm,
                                                     const u64 *__restrict__ topk, const uint32_t *__restrict__ have,
                                                     const float *__restrict__ qerr, uint32_t *__restrict__ out_ids,
                                                     float *__restrict__ out_dist, int ostride, FlagPublish pub) {
    // dynamic LDS sized by the launch for kc: the sort buffer (refine_sort_entries(kc), a power of
    // two >= kc) and the kept entries' rows (kc), so a small kc keeps many workgroups per CU
    extern __shared__ u64 buf[];
    uint32_t *s_row = (uint32_t *)(buf + refine_sort_entries(kc));
    if (blockIdx.x == 0 && threadIdx.x == 0) publish_flags(pub);
    __shared__ int s_h;
    const int q = blockIdx.x, tid = threadIdx.x;
    const u64 *tq = topk + (size_t)q * kc;
    const int h_all = (int)have[q];
    if (qerr && qerr[q] == 0.0f && metric != COS) {
        // No selection error: squared L2 or dot product on integer rows whose every intermediate
        // stays below 2^24 (the bound is 0 only then), so the scan's scores are the direct form's
        // exact values and the merge's list, sorted by (score, id), is already the result.
        const int hk = h_all < k ? h_all : k;
        for (int j = tid; j < kout; j += 256) {
            const size_t o = (size_t)q * ostride + j;
            if (j < hk) {
                const u64 e = tq[j];
                const float sc = key_score((uint32_t)(e >> 32));
                out_ids[o] = (uint32_t)e;
                out_dist[o] = metric == L2 ? sc : -sc + 0.0f;
            } else {
                out_ids[o] = 0xffffffffu;
                out_dist[o] = __builtin_nanf("");
            }
        }
        return;
    }
    if (tid == 0) s_h = h_all;
    __syncthreads();
    if (h_all > k && qerr) {
        // entries past the k-th count while their score is within the margin of the k-th (the
        // list is sorted by score)
        const float lim = key_score((uint32_t)(tq[k - 1] >> 32)) + 2.0f * qerr[q];
        for (int j = k + tid; j < h_all; j += 256)
            if (key_score((uint32_t)(tq[j] >> 32)) > lim) atomicMin(&s_h, j);
        __syncthreads();
    }
    const int h = s_h;
    for (int j = tid; j < h; j += 256) {
        const uint32_t id = (uint32_t)tq[j];
        s_row[j] = inv_perm[id];
        buf[j] = id;
    }
    __syncthreads();
    const int grp = tid >> 4, s = tid & 15, n4 = dpad >> 2;  // dpad is a multiple of 32
    const float4 *qv = (const float4 *)(qrows + (size_t)q * dpad);
    for (int j = grp; j < h; j += 16) {
        const uint32_t row = s_row[j];
        const float4 *xv = (const float4 *)(base + (size_t)row * dpad);
        float a = 0.0f, nq = 0.0f, nx = 0.0f;
        for (int d = s; d < n4; d += 16) {
            float4 x = xv[d];
            const float4 y = qv[d];
            if (shift) {  // squared L2 over shifted rows that give back the unshifted ones exactly
                const float4 m = ((const float4 *)shift)[d];
                x.x += m.x;
                x.y += m.y;
                x.z += m.z;
                x.w += m.w;
            }
            if (metric == L2) {
                const float t0 = y.x - x.x, t1 = y.y - x.y, t2 = y.z - x.z, t3 = y.w - x.w;
                a = fmaf(t0, t0, a);
                a = fmaf(t1, t1, a);
                a = fmaf(t2, t2, a);
                a = fmaf(t3, t3, a);
            } else {
                a = fmaf(y.x, x.x, fmaf(y.y, x.y, fmaf(y.z, x.z, fmaf(y.w, x.w, a))));
                nq = fmaf(y.x, y.x, fmaf(y.y, y.y, fmaf(y.z, y.z, fmaf(y.w, y.w, nq))));
                nx = fmaf(x.x, x.x, fmaf(x.y, x.y, fmaf(x.z, x.z, fmaf(x.w, x.w, nx))));
            }
        }
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) {
            a += __shfl_xor(a, o, 16);
            if (metric != L2) {
                nq += __shfl_xor(nq, o, 16);
                nx += __shfl_xor(nx, o, 16);
            }
        }
        float sc;
        if (metric == L2) {
            sc = a;
        } else if (metric == DOT) {
            sc = -a + 0.0f;
        } else {
            // rows and queries are stored L2-normalised; the zero-norm rule uses the original norms
            const float den = sqrtf(nq) * sqrtf(nx);
            sc = (den <= 1e-9f || qnorm[q] * bnorm[row] <= 1e-9f) ? 0.0f : -(a / den) + 0.0f;
        }
        if (s == 0) buf[j] = ((u64)score_key(nan_last(sc)) << 32) | (uint32_t)buf[j];
    }
    int P = 2;
    while (P < h) P <<= 1;
    for (int i = h + tid; i < P; i += 256) buf[i] = ~0ull;
    __syncthreads();
    bitonic_sort_lds(buf, P);
    const int hk = h < k ? h : k;
    for (int j = tid; j < kout; j += 256) {
        const size_t o = (size_t)q * ostride + j;
        if (j < hk) {
            const float sc = key_score((uint32_t)(buf[j] >> 32));
            out_ids[o] = (uint32_t)buf[j];
            out_dist[o] = metric == L2 ? sc : -sc + 0.0f;
        } else {
            out_ids[o] = 0xffffffffu;
            out_dist[o] = __builtin_nanf("");
        }
    }
}

void launch_topk_refine(int nq, int k, int kc, int kout, int metric, const float *qrows, const float *base,
                        const float *shift, const uint32_t *inv_perm, int dpad, const float *qnorm, const float *bnorm,
                        const unsigned long long *topk, const uint32_t *have, const float *qerr, uint32_t *out_ids,
                        float *out_dist, int ostride, const FlagPublish &pub, hipStream_t s) {
    if (nq <= 0) return;
    // at most kMaxKeep entries: 4096 x 8 + 2304 x 4 bytes, within the default 64 KB
    const size_t lds = (size_t)refine_sort_entries(kc) * sizeof(u64) + (size_t)kc * sizeof(uint32_t);
    hipLaunchKernelGGL(k_topk_refine, dim3(nq), dim3(256), lds, s, k, kc, kout, metric, qrows, base, shift, inv_perm,
                       dpad, qnorm, bnorm, topk, have, qerr, out_ids, out_dist, ostride, pub);
}

}  // namespace vh
