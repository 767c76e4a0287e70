// topk.hip -- per-query top-k maintenance between filter rounds.
//
// A search runs the base in rounds of geometrically growing row ranges.  The filter
// kernels (knn_gemm.hip, knn_valu.hip, hamming.hip) append every (score, id) with
// score <= tau[q] to the query's candidate list; k_topk_merge then sorts the running
// top-k together with those candidates (64-bit keys: ordered score << 32 | id, so ties
// break towards the lower id) and keeps the best k.  The new tau is the k-th score, an
// upper bound of the final k-th score, so no true neighbour can be filtered out later.
// This replaces knn_topk_select (knn.cu:206-305) and its K <= 128 clamp.
#include "vh_common.h"

namespace vh {

typedef unsigned long long u64;

__global__ void k_topk_init(int nq, float *tau, uint32_t *have, uint32_t *cnt, uint32_t *flags) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q < nq) {
        tau[q] = INFINITY;
        have[q] = 0;
        cnt[q] = 0;
        flags[q] = 0;
    }
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

void launch_topk_init(int nq, float *tau, uint32_t *have, uint32_t *cnt, uint32_t *flags, hipStream_t s) {
    if (nq <= 0) return;
    hipLaunchKernelGGL(k_topk_init, dim3(ceil_div(nq, 256)), dim3(256), 0, s, nq, tau, have, cnt, flags);
}

// Bitonic sort of P (power of two) keys in LDS, ascending.  Must be called by all threads.
__device__ __forceinline__ void bitonic_sort_lds(u64 *buf, int P) {
    const int tid = threadIdx.x, nt = blockDim.x;
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

__global__ __launch_bounds__(256) void k_topk_merge(int k, const uint2 *__restrict__ cand, uint32_t *__restrict__ cnt,
                                                    int cap, const uint32_t *__restrict__ perm,
                                                    u64 *__restrict__ topk, uint32_t *__restrict__ have,
                                                    float *__restrict__ tau, uint32_t *__restrict__ flags,
                                                    uint32_t *__restrict__ nflagged) {
    __shared__ u64 buf[kSortSlots];
    const int q = blockIdx.x, tid = threadIdx.x;
    const uint32_t c_all = cnt[q];
    if (flags[q] || c_all == 0) {
        __syncthreads();
        if (tid == 0) cnt[q] = 0;
        return;
    }
    const bool overflow = c_all > (uint32_t)cap;
    const uint32_t c = overflow ? (uint32_t)cap : c_all;
    u64 *tk = topk + (size_t)q * k;
    const uint2 *cq = cand + (size_t)q * cap;

    uint32_t h = have[q];
    for (uint32_t i = tid; i < h; i += 256) buf[i] = tk[i];
    uint32_t done = 0;
    while (done < c) {
        const uint32_t take = min(c - done, (uint32_t)kSortSlots - h);
        for (uint32_t i = tid; i < take; i += 256) {
            const uint2 e = cq[done + i];
            buf[h + i] = ((u64)e.x << 32) | (u64)perm[e.y];  // base position -> vector id
        }
        const uint32_t total = h + take;
        int P = 2;
        while ((uint32_t)P < total) P <<= 1;
        for (uint32_t i = total + tid; i < (uint32_t)P; i += 256) buf[i] = ~0ull;
        __syncthreads();
        bitonic_sort_lds(buf, P);
        h = min(total, (uint32_t)k);
        done += take;
    }
    for (uint32_t i = tid; i < h; i += 256) tk[i] = buf[i];
    if (tid == 0) {
        have[q] = h;
        cnt[q] = 0;
        if (overflow) {
            // The list is incomplete: stop filtering for this query; the host re-runs it
            // with a capacity that cannot overflow.
            flags[q] = 1;
            tau[q] = -INFINITY;
            atomicAdd(nflagged, 1u);
        } else {
            tau[q] = h >= (uint32_t)k ? key_score((uint32_t)(buf[k - 1] >> 32)) : INFINITY;
        }
    }
}

void launch_topk_merge(int nq, int k, const uint2 *cand, uint32_t *cnt, int cap, const uint32_t *perm,
                       unsigned long long *topk, uint32_t *have, float *tau, uint32_t *flags, uint32_t *nflagged,
                       hipStream_t s) {
    if (nq <= 0) return;
    hipLaunchKernelGGL(k_topk_merge, dim3(nq), dim3(256), 0, s, k, cand, cnt, cap, perm, topk, have, tau, flags,
                       nflagged);
}

__global__ void k_topk_finalize(int nq, int k, int kout, int metric, const u64 *__restrict__ topk,
                                const uint32_t *__restrict__ have, uint32_t *__restrict__ out_ids,
                                float *__restrict__ out_dist, uint32_t *__restrict__ out_dist_u32, int ostride) {
    const long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (i >= (long)nq * kout) return;
    const int q = (int)(i / kout), j = (int)(i % kout);
    const size_t o = (size_t)q * ostride + j;
    if ((uint32_t)j < have[q]) {
        const u64 e = topk[(size_t)q * k + j];
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

void launch_topk_finalize(int nq, int k, int kout, int metric, const unsigned long long *topk,
                          const uint32_t *have, uint32_t *out_ids, float *out_dist, uint32_t *out_dist_u32,
                          int ostride, hipStream_t s) {
    const long total = (long)nq * kout;
    if (total <= 0) return;
    hipLaunchKernelGGL(k_topk_finalize, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, nq, k, kout, metric,
                       topk, have, out_ids, out_dist, out_dist_u32, ostride);
}

// Final pass for the GEMM-form metrics: the selection used ||q||^2 + ||x||^2 - 2 q.x, whose
// cancellation error grows with the norms.  For each kept neighbour the distance is
// recomputed in the direct form of the reference CPU engine (sum (q-x)^2, sum q*x, or
// dot / (sqrt(|q|^2) sqrt(|x|^2)) with the 1e-9 guard, scalar.rs:14-75), the k entries are
// re-sorted by (distance, id), and written out.  One workgroup per query; each wave
// evaluates one neighbour at a time with a lane-strided sum and a fixed xor butterfly.
__global__ __launch_bounds__(256) void k_topk_refine(int k, int kout, int metric, const float *__restrict__ qpad,
                                                     const float *__restrict__ base,
                                                     const uint32_t *__restrict__ inv_perm, int dpad,
                                                     const float *__restrict__ qnorm, const float *__restrict__ bnorm,
                                                     const u64 *__restrict__ topk, const uint32_t *__restrict__ have,
                                                     uint32_t *__restrict__ out_ids, float *__restrict__ out_dist,
                                                     int ostride) {
    __shared__ u64 buf[kMaxK];
    const int q = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = (int)have[q];
    const float *qv = qpad + (size_t)q * dpad;
    for (int j = wave; j < h; j += 4) {
        const u64 e = topk[(size_t)q * k + j];
        const uint32_t id = (uint32_t)e;
        const uint32_t row = inv_perm[id];
        const float *xv = base + (size_t)row * dpad;
        float a = 0.0f, nq = 0.0f, nx = 0.0f;
        for (int d = lane; d < dpad; d += 64) {
            const float x = xv[d], y = qv[d];
            if (metric == L2) {
                const float t = y - x;
                a = fmaf(t, t, a);
            } else {
                a = fmaf(y, x, a);
                nq = fmaf(y, y, nq);
                nx = fmaf(x, x, nx);
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            a += __shfl_xor(a, o, 64);
            nq += __shfl_xor(nq, o, 64);
            nx += __shfl_xor(nx, o, 64);
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
        if (lane == 0) buf[j] = ((u64)score_key(sc) << 32) | id;
    }
    int P = 2;
    while (P < h) P <<= 1;
    for (int i = h + tid; i < P; i += 256) buf[i] = ~0ull;
    __syncthreads();
    bitonic_sort_lds(buf, P);
    for (int j = tid; j < kout; j += 256) {
        const size_t o = (size_t)q * ostride + j;
        if (j < h) {
            const float sc = key_score((uint32_t)(buf[j] >> 32));
            out_ids[o] = (uint32_t)buf[j];
            out_dist[o] = metric == L2 ? sc : -sc + 0.0f;
        } else {
            out_ids[o] = 0xffffffffu;
            out_dist[o] = __builtin_nanf("");
        }
    }
}

void launch_topk_refine(int nq, int k, int kout, int metric, const float *qpad, const float *base,
                        const uint32_t *inv_perm, int dpad, const float *qnorm, const float *bnorm,
                        const unsigned long long *topk, const uint32_t *have, uint32_t *out_ids, float *out_dist,
                        int ostride, hipStream_t s) {
    if (nq <= 0) return;
    hipLaunchKernelGGL(k_topk_refine, dim3(nq), dim3(256), 0, s, k, kout, metric, qpad, base, inv_perm, dpad, qnorm,
                       bnorm, topk, have, out_ids, out_dist, ostride);
}

}  // namespace vh
