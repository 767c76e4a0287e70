// knn_valu.hip -- non-contraction metrics on the vector ALUs, fused with the threshold
// filter of the round/merge top-k (topk.hip).
//
// Replaces the metric switch of knn_compute_distance_matrix (vector-cuda/src/kernels/knn.cu:84-141,
// 175-195) for squared L2 in direct form (the fallback of the GEMM-form L2 search), L1,
// Minkowski p=3, L-inf, thresholded Hamming, Mahalanobis (sqrt of direct L2), weighted Jaccard
// and Hellinger (direct L2 of sqrt|x|, then sqrt(0.5 * sum)).  Each lane owns
// one query held in registers; a workgroup of 256 lanes streams tiles of base rows through LDS and
// every wave reads each base element as a broadcast ds_read_b128 (all lanes the same address), so a
// base element costs two VALU operations per query (sub + add/max with the |x| modifier).  Values
// are computed in the direct form of the reference CPU engine (scalar.rs:81-263), so reported
// distances follow it closely.
#include <algorithm>

#include "vh_common.h"

namespace vh {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kValuRows = 16;             // base rows per LDS tile
constexpr long kValuItemRowsMax = 2048;   // base rows per work item (large rounds)

// k-means Hellinger: centroids are means of the raw data, so sqrt(|x|) of the centroid
// side is taken in the loop (the point side holds sqrt(|p|)).
constexpr int HELL_RAW = 11;

template <int M>
__device__ __forceinline__ void accum(float &a, float &b, float q, float x) {
    if constexpr (M == HELL_RAW) {
        const float d = q - sqrtf(fabsf(x));
        a = fmaf(d, d, a);
    } else if constexpr (M == L1) {
        a += fabsf(q - x);
    } else if constexpr (M == L2 || M == MAHA || M == HELL) {
        const float d = q - x;
        a = fmaf(d, d, a);
    } else if constexpr (M == LINF) {
        a = fmaxf(a, fabsf(q - x));
    } else if constexpr (M == MINK) {
        const float d = fabsf(q - x);
        a = fmaf(d * d, d, a);
    } else if constexpr (M == HAMF) {
        a += fabsf(q - x) > 1e-6f ? 1.0f : 0.0f;
    } else if constexpr (M == DOT) {
        a = fmaf(q, x, a);
    } else if constexpr (M == COS) {  // dot product and the row's squared norm
        a = fmaf(q, x, a);
        b = fmaf(x, x, b);
    } else {  // JACC: q holds |q|
        const float ax = fabsf(x);
        a += fminf(q, ax);
        b += fmaxf(q, ax);
    }
}

// Two consecutive elements; L-inf takes both in one max of three (|.| source modifiers).
template <int M>
__device__ __forceinline__ void accum2(float &a, float &b, float q0, float q1, float x0, float x1) {
    if constexpr (M == LINF) {
        a = fmaxf(a, fmaxf(fabsf(q0 - x0), fabsf(q1 - x1)));
    } else {
        accum<M>(a, b, q0, x0);
        accum<M>(a, b, q1, x1);
    }
}

template <int M>
__device__ __forceinline__ float finish(float a, float b) {
    if constexpr (M == MINK) return cbrtf(a);
    else if constexpr (M == MAHA) return sqrtf(a);
    else if constexpr (M == HELL || M == HELL_RAW) return sqrtf(0.5f * a);
    else if constexpr (M == JACC) return b <= 1e-9f ? 0.0f : 1.0f - a / b;
    else return a;
}

// DC: dimensions per chunk held in registers (64 or 128).  A wave serves 64 queries: lane (p, h)
// holds queries 2p and 2p + 1 of its wave's group over half h of each chunk (DC / 2 dimensions of
// each), so every broadcast tile read feeds two queries and a row costs DC / 8 LDS reads per lane,
// half of what one query per lane over the whole chunk needs.  After a tile the two halves meet
// with one cross-half exchange per row, and lane (p, h) finishes and filters query 2p + h.
template <int M, int DC>
__global__ __launch_bounds__(256) void k_valu_filter(const float *__restrict__ base, const float *__restrict__ shift,
                                                     const float *__restrict__ qry, const float *__restrict__ tau,
                                                     int nq, int dpad, long row_begin, long row_end, int n_qtiles,
                                                     int n_items, long item_rows, uint2 *__restrict__ cand,
                                                     uint32_t *__restrict__ cnt, int cap) {
    constexpr int V4 = DC / 4, HD = DC / 2, H4 = HD / 4;
    // rows interleaved per tile read: 4, or 2 for L-inf, whose max3 chains gain nothing from more
    // (L1 at 500k x 128, Q = 4096: 10.90 ms at 4 rows, 11.09 at 2; L-inf 10.82 at 2, 10.90 at 4)
    constexpr int RI = M == LINF ? 2 : 4;
    __shared__ floatx4 tile[kValuRows * V4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, pq = lane & 31;
    const int nchunks = (dpad + DC - 1) / DC;
    const int G = gridDim.x, g8 = G >> 3;
    const int slot = (blockIdx.x & 7) * g8 + (blockIdx.x >> 3);

    for (int item = slot; item < n_items; item += G) {
        const int qtile = item % n_qtiles;
        const long chunk = item / n_qtiles;
        const int q0 = qtile * 256 + wave * 64 + 2 * pq;  // this lane's query pair
        const int q = q0 + h;                              // the query it finishes
        const bool qv = q < nq;
        const float tq = qv ? tau[q] : -INFINITY;
        const long r_lo = row_begin + chunk * item_rows;
        const long r_hi = min(r_lo + item_rows, row_end);

        float qr[2][HD];
        auto load_q = [&](int c) {
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const bool v = q0 + e < nq;
#pragma unroll
                for (int i = 0; i < H4; ++i) {
                    const int d = c * DC + h * HD + 4 * i;
                    floatx4 x = (v && d < dpad) ? *(const floatx4 *)(qry + (long)(q0 + e) * dpad + d)
                                                : floatx4{0, 0, 0, 0};
#pragma unroll
                    for (int j = 0; j < 4; ++j) qr[e][4 * i + j] = (M == JACC) ? fabsf(x[j]) : x[j];
                }
            }
        };
        if (nchunks == 1) load_q(0);

        for (long rs = r_lo; rs < r_hi; rs += kValuRows) {
            float a[2][kValuRows], b[2][kValuRows];
#pragma unroll
            for (int r = 0; r < kValuRows; ++r) a[0][r] = a[1][r] = b[0][r] = b[1][r] = 0.0f;
            for (int c = 0; c < nchunks; ++c) {
                if (nchunks > 1) load_q(c);
                __syncthreads();
                for (int i = tid; i < kValuRows * V4; i += 256) {
                    const int row = i / V4, c4 = i % V4;
                    const long r = rs + row;
                    const int d = c * DC + 4 * c4;
                    floatx4 v = (r < r_hi && d < dpad) ? *(const floatx4 *)(base + r * (long)dpad + d)
                                                       : floatx4{0, 0, 0, 0};
                    if (shift && d < dpad) v += *(const floatx4 *)(shift + d);
                    tile[i] = v;
                }
                __syncthreads();
                // RI rows at a time: 2 RI independent accumulation chains per element
#pragma unroll
                for (int r = 0; r < kValuRows; r += RI) {
#pragma unroll
                    for (int i = 0; i < H4; ++i) {
                        floatx4 x[RI];
#pragma unroll
                        for (int u = 0; u < RI; ++u) x[u] = tile[(r + u) * V4 + h * H4 + i];
#pragma unroll
                        for (int j = 0; j < 4; j += 2)
#pragma unroll
                            for (int u = 0; u < RI; ++u)
#pragma unroll
                                for (int e = 0; e < 2; ++e)
                                    accum2<M>(a[e][r + u], b[e][r + u], qr[e][4 * i + j], qr[e][4 * i + j + 1],
                                              x[u][j], x[u][j + 1]);
                    }
                }
            }
            const int nvalid = (int)min((long)kValuRows, r_hi - rs);
#pragma unroll
            for (int r = 0; r < kValuRows; ++r) {
                // the partner half needs the other query's partial sums; this lane keeps its own
                const float sa = __shfl_xor(h ? a[0][r] : a[1][r], 32, 64);
                const float oa = h ? a[1][r] : a[0][r];
                float sb = 0.0f, ob = 0.0f;
                if constexpr (M == JACC || M == COS) {
                    sb = __shfl_xor(h ? b[0][r] : b[1][r], 32, 64);
                    ob = h ? b[1][r] : b[0][r];
                }
                const float ta = M == LINF ? fmaxf(oa, sa) : oa + sa;
                const float tb = ob + sb;
                const float v = finish<M>(ta, tb);
                if (v <= tq && r < nvalid && qv) {
                    const uint32_t at = atomicAdd(&cnt[q], 1u);
                    if (at < (uint32_t)cap) cand[(size_t)q * cap + at] = make_uint2(score_key(v), (uint32_t)(rs + r));
                }
            }
        }
    }
}

template <int M>
static void launch_m(int dpad, dim3 g, hipStream_t s, const float *base, const float *shift, const float *qry,
                     const float *tau, int nq, long rb, long re, int nqt, int items, long item_rows, uint2 *cand,
                     uint32_t *cnt, int cap) {
    if (dpad <= 128 && dpad > 64)
        scan_launch((k_valu_filter<M, 128>), g, dim3(256), 0, s, base, shift, qry, tau, nq, dpad, rb, re, nqt,
                           items, item_rows, cand, cnt, cap);
    else
        scan_launch((k_valu_filter<M, 64>), g, dim3(256), 0, s, base, shift, qry, tau, nq, dpad, rb, re, nqt,
                           items, item_rows, cand, cnt, cap);
}

void launch_valu_filter(int metric, const float *base, const float *shift, const float *qry, const float *tau,
                        int nq, int dim, int dpad, long row_begin, long row_end, uint2 *cand, uint32_t *cnt, int cap,
                        int grid_cap, hipStream_t s) {
    (void)dim;
    if (nq <= 0 || row_end <= row_begin) return;
    const int nqt = ceil_div(nq, 256);
    // rows per work item: small rounds are cut finer so that they still give every resident
    // workgroup about four items
    const long rows = row_end - row_begin;
    long item_rows = (rows * nqt + 4L * grid_cap - 1) / (4L * grid_cap);
    item_rows = std::min(kValuItemRowsMax, std::max(4L * kValuRows, (item_rows + kValuRows - 1) / kValuRows * kValuRows));
    const long n_chunks = (rows + item_rows - 1) / item_rows;
    const long items = (long)nqt * n_chunks;
    long grid = items < grid_cap ? items : grid_cap;
    grid = (grid + 7) / 8 * 8;
    const dim3 g((unsigned)grid);
    const int it = (int)items;
    switch (metric) {
        // squared L2 in direct form: the certified fallback of the GEMM-form L2 search
        case L2: launch_m<L2>(dpad, g, s, base, metric == L2 ? shift : nullptr, qry, tau, nq, row_begin, row_end, nqt, it, item_rows, cand, cnt, cap); break;
        case L1: launch_m<L1>(dpad, g, s, base, metric == L2 ? shift : nullptr, qry, tau, nq, row_begin, row_end, nqt, it, item_rows, cand, cnt, cap); break;
        case MINK: launch_m<MINK>(dpad, g, s, base, metric == L2 ? shift : nullptr, qry, tau, nq, row_begin, row_end, nqt, it, item_rows, cand,
                                          cnt, cap); break;
        case LINF: launch_m<LINF>(dpad, g, s, base, metric == L2 ? shift : nullptr, qry, tau, nq, row_begin, row_end, nqt, it, item_rows, cand,
                                          cnt, cap); break;
        case HAMF: launch_m<HAMF>(dpad, g, s, base, metric == L2 ? shift : nullptr, qry, tau, nq, row_begin, row_end, nqt, it, item_rows, cand,
                                          cnt, cap); break;
        case MAHA: launch_m<MAHA>(dpad, g, s, base, metric == L2 ? shift : nullptr, qry, tau, nq, row_begin, row_end, nqt, it, item_rows, cand,
                                          cnt, cap); break;
        case JACC: launch_m<JACC>(dpad, g, s, base, metric == L2 ? shift : nullptr, qry, tau, nq, row_begin, row_end, nqt, it, item_rows, cand,
                                          cnt, cap); break;
        case HELL: launch_m<HELL>(dpad, g, s, base, metric == L2 ? shift : nullptr, qry, tau, nq, row_begin, row_end, nqt, it, item_rows, cand,
                                          cnt, cap); break;
        default: break;
    }
}

// ---------------------------------------------------------------------------------
// k-means assignment for the non-contraction metrics (kmeans.cu:172-271): one lane per
// point (held in registers), centroid tiles broadcast from LDS, running argmin with a
// strict '<' in ascending centroid order (lowest index wins ties).  Per-point inertia is the
// metric value (kmeans.cu convention).
// ---------------------------------------------------------------------------------
template <int M, int DC>
__global__ __launch_bounds__(256) void k_kmeans_assign_valu(const float *__restrict__ cent, int k,
                                                            const float *__restrict__ pts, int n, int dpad,
                                                            int n_tiles, int32_t *__restrict__ assign,
                                                            float *__restrict__ inertia, int32_t *__restrict__ pos,
                                                            int32_t *__restrict__ counts) {
    constexpr int V4 = DC / 4;
    __shared__ floatx4 tile[kValuRows * V4];
    const int tid = threadIdx.x;
    const int nchunks = (dpad + DC - 1) / DC;
    for (int t = blockIdx.x; t < n_tiles; t += gridDim.x) {
        const int p = t * 256 + tid;
        const bool pv = p < n;
        float pr[DC];
        auto load_p = [&](int c) {
#pragma unroll
            for (int i = 0; i < V4; ++i) {
                const int d = c * DC + 4 * i;
                floatx4 v = (pv && d < dpad) ? *(const floatx4 *)(pts + (long)p * dpad + d) : floatx4{0, 0, 0, 0};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    pr[4 * i + j] = (M == JACC) ? fabsf(v[j]) : (M == HELL_RAW ? sqrtf(fabsf(v[j])) : v[j]);
            }
        };
        if (nchunks == 1) load_p(0);
        float best = INFINITY;
        int bi = 0;
        for (int cs = 0; cs < k; cs += kValuRows) {
            float a[kValuRows], b[kValuRows];
#pragma unroll
            for (int r = 0; r < kValuRows; ++r) a[r] = b[r] = 0.0f;
            for (int c = 0; c < nchunks; ++c) {
                if (nchunks > 1) load_p(c);
                __syncthreads();
                for (int i = tid; i < kValuRows * V4; i += 256) {
                    const int row = i / V4, c4 = i % V4;
                    const int r = cs + row;
                    const int d = c * DC + 4 * c4;
                    tile[i] = (r < k && d < dpad) ? *(const floatx4 *)(cent + (long)r * dpad + d)
                                                  : floatx4{0, 0, 0, 0};
                }
                __syncthreads();
#pragma unroll
                for (int r = 0; r < kValuRows; ++r) {
#pragma unroll
                    for (int i = 0; i < V4; ++i) {
                        const floatx4 x = tile[r * V4 + i];
#pragma unroll
                        for (int j = 0; j < 4; ++j) accum<M>(a[r], b[r], pr[4 * i + j], x[j]);
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < kValuRows; ++r) {
                const float v = finish<M>(a[r], b[r]);
                if (v < best && cs + r < k) {
                    best = v;
                    bi = cs + r;
                }
            }
        }
        if (pv) {
            assign[p] = bi;
            inertia[p] = best;
            pos[p] = atomicAdd(&counts[bi], 1);
        }
    }
}

// ---------------------------------------------------------------------------------
// Fix-up of the MFMA k-means assignment: the points whose GEMM-form argmin could not be
// certified get the argmin of the direct-form metric over all centroids (squared L2 sum (x-c)^2,
// dot product, cosine dot / (sqrt(|x|^2) sqrt(|c|^2)) with the 1e-9 guard: the formulas of
// scalar.rs:14-75 and kmeans.cu:87-170) on the unshifted points and centroids.  A work item is a
// tile of 256 listed points (one per lane, in registers) times a chunk of centroids (tiles
// broadcast from LDS); the chunk's best (score key, centroid) is folded into best[i] with a
// 64-bit atomic min, so the result is the lowest score and then the lowest index, whatever the
// order of the items.  The chunk is kFixChunk centroids, halved (down to one LDS tile) while the
// items number fewer than twice the workgroups: a short list still spreads over the GPU, and a
// centroid's score does not depend on the chunk it falls in.
// ---------------------------------------------------------------------------------
constexpr int kFixChunk = 256;
static_assert(kFixChunk % kValuRows == 0 && (kFixChunk & (kFixChunk - 1)) == 0, "chunks halve to whole LDS tiles");

__global__ void k_fix_init(const uint32_t *__restrict__ nfix, unsigned long long *__restrict__ best) {
    const uint32_t nf = *nfix;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < nf; i += gridDim.x * blockDim.x) best[i] = ~0ull;
}

template <int M, int DC>
__global__ __launch_bounds__(256) void k_fix_argmin(const float *__restrict__ pts, int dpad,
                                                    const int32_t *__restrict__ fix, const uint32_t *__restrict__ nfix,
                                                    const float *__restrict__ cent, int k,
                                                    unsigned long long *__restrict__ best) {
    constexpr int V4 = DC / 4;
    __shared__ floatx4 tile[kValuRows * V4];
    const int tid = threadIdx.x;
    const int nchunks = (dpad + DC - 1) / DC;
    const int nf = (int)*nfix;
    const int n_tiles = (nf + 255) / 256;
    int chunk = kFixChunk;
    while (chunk > kValuRows && n_tiles * ((k + chunk - 1) / chunk) < 2 * (int)gridDim.x) chunk >>= 1;
    const int n_cchunks = (k + chunk - 1) / chunk;
    const int items = n_tiles * n_cchunks;
    for (int item = blockIdx.x; item < items; item += gridDim.x) {
        const int t = item % n_tiles, cc = item / n_tiles;
        const int i = t * 256 + tid;
        const bool pv = i < nf;
        const float *prow = pts + (size_t)(pv ? fix[i] : 0) * dpad;
        float pr[DC];
        auto load_p = [&](int c) {
#pragma unroll
            for (int u = 0; u < V4; ++u) {
                const int d = c * DC + 4 * u;
                const floatx4 v = d < dpad ? *(const floatx4 *)(prow + d) : floatx4{0, 0, 0, 0};
#pragma unroll
                for (int j = 0; j < 4; ++j) pr[4 * u + j] = v[j];
            }
        };
        float pn = 0.0f;  // the point's squared norm (cosine)
        if constexpr (M == COS) {
            for (int c = 0; c < nchunks; ++c) {
                load_p(c);
#pragma unroll
                for (int j = 0; j < DC; ++j) pn = fmaf(pr[j], pr[j], pn);
            }
        }
        if (nchunks == 1) load_p(0);
        const int c0 = cc * chunk, c1 = min(k, c0 + chunk);
        float bv = INFINITY;
        int bc = c0;
        for (int cs = c0; cs < c1; cs += kValuRows) {
            float a[kValuRows], b[kValuRows];
#pragma unroll
            for (int r = 0; r < kValuRows; ++r) a[r] = b[r] = 0.0f;
            for (int c = 0; c < nchunks; ++c) {
                if (nchunks > 1) load_p(c);
                __syncthreads();
                for (int e = tid; e < kValuRows * V4; e += 256) {
                    const int row = e / V4, c4 = e % V4;
                    const int r = cs + row;
                    const int d = c * DC + 4 * c4;
                    tile[e] = (r < c1 && d < dpad) ? *(const floatx4 *)(cent + (long)r * dpad + d)
                                                   : floatx4{0, 0, 0, 0};
                }
                __syncthreads();
#pragma unroll
                for (int r = 0; r < kValuRows; ++r) {
#pragma unroll
                    for (int u = 0; u < V4; ++u) {
                        const floatx4 x = tile[r * V4 + u];
#pragma unroll
                        for (int j = 0; j < 4; ++j) accum<M>(a[r], b[r], pr[4 * u + j], x[j]);
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < kValuRows; ++r) {
                float v;
                if constexpr (M == L2) {
                    v = a[r];
                } else if constexpr (M == DOT) {
                    v = -a[r] + 0.0f;
                } else {
                    const float den = sqrtf(pn) * sqrtf(b[r]);
                    v = den <= 1e-9f ? 0.0f : -(a[r] / den) + 0.0f;
                }
                if (v < bv && cs + r < c1) {
                    bv = v;
                    bc = cs + r;
                }
            }
        }
        if (pv && c0 < c1) atomicMin(best + i, ((unsigned long long)score_key(bv) << 32) | (uint32_t)bc);
    }
}

// Assignment, ticket and inertia (-dot, 1 - cos; squared L2 leaves it to the update) of the fixed
// points; squared L2 also raises its cluster's deviation bound.
__global__ void k_fix_finish(int metric, const uint32_t *__restrict__ nfix, const int32_t *__restrict__ fix,
                             const unsigned long long *__restrict__ best, int32_t *__restrict__ assign,
                             float *__restrict__ inertia, int32_t *__restrict__ pos, int32_t *__restrict__ counts,
                             float *__restrict__ devmax) {
    const uint32_t nf = *nfix;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < nf; i += gridDim.x * blockDim.x) {
        const unsigned long long e = best[i];
        const int p = fix[i], c = (int)(uint32_t)e;
        const float v = key_score((uint32_t)(e >> 32));
        assign[p] = c;
        pos[p] = atomicAdd(&counts[c], 1);
        if (metric == L2) atomicMax((uint32_t *)devmax + c, __float_as_uint(sqrtf(fmaxf(v, 0.0f)) * 1.0001f));
        else inertia[p] = metric == DOT ? v : 1.0f + v;
    }
}

void launch_kmeans_fix(int metric, const float *pts, int dpad, const int32_t *fix, const uint32_t *nfix,
                       const float *cent, int k, unsigned long long *best, int32_t *assign, float *inertia,
                       int32_t *pos, int32_t *counts, float *devmax, int grid_cap, hipStream_t s) {
    if (k <= 0) return;
    hipLaunchKernelGGL(k_fix_init, dim3(64), dim3(256), 0, s, nfix, best);
    const dim3 g(grid_cap), b(256);
    const bool wide = dpad <= 128 && dpad > 64;
    switch (metric) {
        case L2:
            if (wide) hipLaunchKernelGGL((k_fix_argmin<L2, 128>), g, b, 0, s, pts, dpad, fix, nfix, cent, k, best);
            else hipLaunchKernelGGL((k_fix_argmin<L2, 64>), g, b, 0, s, pts, dpad, fix, nfix, cent, k, best);
            break;
        case DOT:
            if (wide) hipLaunchKernelGGL((k_fix_argmin<DOT, 128>), g, b, 0, s, pts, dpad, fix, nfix, cent, k, best);
            else hipLaunchKernelGGL((k_fix_argmin<DOT, 64>), g, b, 0, s, pts, dpad, fix, nfix, cent, k, best);
            break;
        default:
            if (wide) hipLaunchKernelGGL((k_fix_argmin<COS, 128>), g, b, 0, s, pts, dpad, fix, nfix, cent, k, best);
            else hipLaunchKernelGGL((k_fix_argmin<COS, 64>), g, b, 0, s, pts, dpad, fix, nfix, cent, k, best);
            break;
    }
    hipLaunchKernelGGL(k_fix_finish, dim3(64), dim3(256), 0, s, metric, nfix, fix, best, assign, inertia, pos, counts,
                       devmax);
}

// ---------------------------------------------------------------------------------
// Small point sets.  The MFMA assignment spreads 128-point column tiles over the CUs and pads the
// centroid rows to 256, so below 128 points per CU most of the GPU idles, and a small k wastes
// most of each tile.  There every point takes the fix-up's direct form instead, which needs no
// selection bound: L lanes per point, each holding a strided slice of its dimensions (NS float4
// at most) in registers, 64 / L points per wave; the centroids stream through L1 four at a
// time, each lane adding its slice's terms and the L lanes combining them with a fixed xor tree.
// ---------------------------------------------------------------------------------
constexpr int kAssignSmallMaxK = 256;           // centroids per point in the direct form, at most
constexpr long kAssignSmallMaxPairs = 1000000;  // and (point, centroid) pairs: the direct form costs
// about 1.4 us per centroid at 10,000 x 768 (its lanes' work grows with k), the MFMA scan about
// 115 us plus its fix-up whatever k up to 256 (its tiles pad k to 256), so the two meet near
// n k = 1e6

template <int M, int L, int NS>
__global__ __launch_bounds__(256) void k_kmeans_assign_small(const float *__restrict__ pts, int dpad, int n,
                                                             const float *__restrict__ cent, int k,
                                                             int32_t *__restrict__ assign, float *__restrict__ inertia,
                                                             int32_t *__restrict__ pos, int32_t *__restrict__ counts,
                                                             float *__restrict__ devmax) {
    constexpr int PPW = 64 / L;
    const int lane = threadIdx.x & 63, sub = lane & (L - 1);
    const int p = (blockIdx.x * 4 + (threadIdx.x >> 6)) * PPW + lane / L;
    const int pc = min(p, n - 1);  // lanes past the end repeat the last point, unstored
    const int nc4 = dpad >> 2;
    const floatx4 *prow = reinterpret_cast<const floatx4 *>(pts + (size_t)pc * dpad);
    floatx4 x[NS];
    float pn = 0.0f;  // the point's squared norm (cosine)
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int j = sub + s * L;
        x[s] = j < nc4 ? prow[j] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (M == COS)
#pragma unroll
            for (int e = 0; e < 4; ++e) pn = fmaf(x[s][e], x[s][e], pn);
    }
    if constexpr (M == COS)
#pragma unroll
        for (int o = L / 2; o > 0; o >>= 1) pn += __shfl_xor(pn, o, 64);
    float bv = INFINITY;
    int bc = 0;
    for (int c0 = 0; c0 < k; c0 += 4) {
        float a[4] = {0.0f, 0.0f, 0.0f, 0.0f}, b[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int j = min(sub + s * L, nc4 - 1);  // past the row's end: a zero slice of x
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const floatx4 cv = reinterpret_cast<const floatx4 *>(cent + (size_t)min(c0 + u, k - 1) * dpad)[j];
                const bool in = sub + s * L < nc4;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (in) accum<M>(a[u], b[u], x[s][e], cv[e]);
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
#pragma unroll
            for (int o = L / 2; o > 0; o >>= 1) {
                a[u] += __shfl_xor(a[u], o, 64);
                if constexpr (M == COS) b[u] += __shfl_xor(b[u], o, 64);
            }
            float v;
            if constexpr (M == L2) {
                v = a[u];
            } else if constexpr (M == DOT) {
                v = -a[u] + 0.0f;
            } else {
                const float den = sqrtf(pn) * sqrtf(b[u]);
                v = den <= 1e-9f ? 0.0f : -(a[u] / den) + 0.0f;
            }
            if (v < bv && c0 + u < k) {
                bv = v;
                bc = c0 + u;
            }
        }
    }
    if (sub == 0 && p < n) {
        assign[p] = bc;
        pos[p] = atomicAdd(&counts[bc], 1);
        if constexpr (M == L2) atomicMax((uint32_t *)devmax + bc, __float_as_uint(sqrtf(fmaxf(bv, 0.0f)) * 1.0001f));
        else inertia[p] = M == DOT ? bv : 1.0f + bv;  // -dot, 1 - cos
    }
}

// (dpad <= 1024 always holds for k-means, which rejects larger dimensions; it bounds NS at 16)
bool kmeans_assign_small_ok(int n, int k, int dpad, int cus) {
    return n > 0 && n < 128 * cus && k >= 1 && k <= kAssignSmallMaxK && (long)n * k <= kAssignSmallMaxPairs &&
           dpad <= 1024;
}

template <int M, int L>
static void launch_small_l(int dpad, const float *pts, int n, const float *cent, int k, int32_t *assign,
                           float *inertia, int32_t *pos, int32_t *counts, float *devmax, hipStream_t s) {
    const dim3 g(ceil_div(n, 4 * (64 / L)));
    const int ns = ceil_div(dpad / 4, L);
#define VH_AS(NS)                                                                                                 \
    scan_launch((k_kmeans_assign_small<M, L, NS>), g, dim3(256), 0, s, pts, dpad, n, cent, k, assign,     \
                       inertia, pos, counts, devmax)
    if (ns <= 2) VH_AS(2);
    else if (ns <= 4) VH_AS(4);
    else if (ns <= 8) VH_AS(8);
    else if (ns <= 12) VH_AS(12);
    else VH_AS(16);
#undef VH_AS
}

template <int M>
static void launch_small_m(int dpad, const float *pts, int n, const float *cent, int k, int32_t *assign,
                           float *inertia, int32_t *pos, int32_t *counts, float *devmax, hipStream_t s) {
    // 8 lanes per point up to 128 dimensions (at most 4 float4 each), 16 above (dpad <= 1024)
    if (dpad <= 128) launch_small_l<M, 8>(dpad, pts, n, cent, k, assign, inertia, pos, counts, devmax, s);
    else launch_small_l<M, 16>(dpad, pts, n, cent, k, assign, inertia, pos, counts, devmax, s);
}

void launch_kmeans_assign_small(int metric, const float *pts, int dpad, int n, const float *cent, int k,
                                int32_t *assign, float *inertia, int32_t *pos, int32_t *counts, float *devmax,
                                hipStream_t s) {
    if (n <= 0 || k <= 0) return;
    switch (metric) {
        case L2: launch_small_m<L2>(dpad, pts, n, cent, k, assign, inertia, pos, counts, devmax, s); break;
        case DOT: launch_small_m<DOT>(dpad, pts, n, cent, k, assign, inertia, pos, counts, devmax, s); break;
        default: launch_small_m<COS>(dpad, pts, n, cent, k, assign, inertia, pos, counts, devmax, s); break;
    }
}

template <int M>
static void launch_km(int dpad, dim3 g, hipStream_t s, const float *cent, int k, const float *pts, int n, int tiles,
                      int32_t *assign, float *inertia, int32_t *pos, int32_t *counts) {
    if (dpad <= 128 && dpad > 64)
        scan_launch((k_kmeans_assign_valu<M, 128>), g, dim3(256), 0, s, cent, k, pts, n, dpad, tiles, assign,
                           inertia, pos, counts);
    else
        scan_launch((k_kmeans_assign_valu<M, 64>), g, dim3(256), 0, s, cent, k, pts, n, dpad, tiles, assign,
                           inertia, pos, counts);
}

void launch_kmeans_assign_valu(int metric, const float *cent, int k, const float *pts, int n, int dpad,
                               int32_t *assign, float *inertia, int32_t *pos, int32_t *counts, int grid_cap,
                               hipStream_t s) {
    if (n <= 0 || k <= 0) return;
    const int tiles = ceil_div(n, 256);
    const dim3 g(tiles < grid_cap ? tiles : grid_cap);
    switch (metric) {
        case L1: launch_km<L1>(dpad, g, s, cent, k, pts, n, tiles, assign, inertia, pos, counts); break;
        case MINK: launch_km<MINK>(dpad, g, s, cent, k, pts, n, tiles, assign, inertia, pos, counts); break;
        case LINF: launch_km<LINF>(dpad, g, s, cent, k, pts, n, tiles, assign, inertia, pos, counts); break;
        case HAMF: launch_km<HAMF>(dpad, g, s, cent, k, pts, n, tiles, assign, inertia, pos, counts); break;
        case MAHA: launch_km<MAHA>(dpad, g, s, cent, k, pts, n, tiles, assign, inertia, pos, counts); break;
        case JACC: launch_km<JACC>(dpad, g, s, cent, k, pts, n, tiles, assign, inertia, pos, counts); break;
        case HELL: launch_km<HELL_RAW>(dpad, g, s, cent, k, pts, n, tiles, assign, inertia, pos, counts); break;
        default: break;
    }
}

}  // namespace vh
