// knn_gemm.hip -- fused FP32-MFMA distance tiles + per-query threshold filter.
//
// Replaces knn_compute_distance_matrix + knn_topk_select (vector-cuda/src/kernels/knn.cu:21-305)
// for the GEMM-form metrics (squared L2, dot product, cosine).  Instead of writing the
// Q x N distance matrix, every workgroup keeps its 128 queries' current threshold tau in
// registers and emits only the (score, id) pairs with score <= tau into a per-query
// candidate list; topk.hip merges those lists into the running top-k between rounds.
//
// Tiling (gfx950, wave64): a workgroup of 4 waves owns a 128-row x 128-query tile; each
// wave owns a 64 x 64 sub-tile made of 2 x 2 v_mfma_f32_32x32x2f32 blocks (rows = base
// vectors on the A side, columns = queries on the B side).  Base rows and queries stream
// through double-buffered LDS in K-chunks of 32 floats; one ds_read_b128 per operand feeds
// four MFMA k-steps (both operands use the same k permutation, so the contraction is
// unchanged).  The grid is persistent and XCD-aware: work items (query tile, row chunk) are
// handed out so that the workgroups resident on one XCD walk the same base rows together
// and share them through that XCD's L2.
#include "vh_common.h"

namespace vh {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kLdsStride = kKChunk + 4;  // 36 floats: 144 B rows keep b128 reads conflict-free
constexpr int kItemStages = 16;          // 128-row stages per work item (2048 base rows)

// ---------------------------------------------------------------------------------
// Row preparation: pad to dpad, optional permutation gather, per-row norm.
// norm_kind: 0 none, 1 squared L2 norm, 2 L2 norm (cosine).
// One wave per row; the norm is a lane-strided sum followed by a fixed xor butterfly,
// so it is deterministic.
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rows_prep(const float *__restrict__ in, size_t n, int dim, int dpad,
                                                   const uint32_t *__restrict__ perm, float *__restrict__ out,
                                                   float *__restrict__ norm, int norm_kind, int transform) {
    const int lane = threadIdx.x & 63;
    const size_t wave = (blockIdx.x * (size_t)blockDim.x + threadIdx.x) >> 6;
    const size_t nwaves = (gridDim.x * (size_t)blockDim.x) >> 6;
    for (size_t p = wave; p < n; p += nwaves) {
        const size_t src = perm ? perm[p] : p;
        const float *row = in + src * (size_t)dim;
        float *orow = out + p * (size_t)dpad;
        float ss = 0.0f;
        for (int d = lane; d < dpad; d += 64) {
            float v = d < dim ? row[d] : 0.0f;
            if (transform) v = sqrtf(fabsf(v));
            orow[d] = v;
            ss = fmaf(v, v, ss);
        }
        if (norm_kind) {
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
            if (lane == 0) norm[p] = norm_kind == 2 ? sqrtf(ss) : ss;
        }
    }
}

void launch_rows_prep(const float *in, size_t n, int dim, int dpad, const uint32_t *perm, float *out, float *norm,
                      int norm_kind, int transform, hipStream_t s) {
    if (n == 0) return;
    size_t blocks = (n + 3) / 4;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_rows_prep, dim3((unsigned)blocks), dim3(256), 0, s, in, n, dim, dpad, perm, out, norm,
                       norm_kind, transform);
}

// ---------------------------------------------------------------------------------
// Score of one (query, base row) pair; smaller is better.
//   L2 : ||q||^2 + ||x||^2 - 2 q.x clamped at 0        (knn.cu:158-163 form)
//   DOT: -q.x                                           (argmax similarity)
//   COS: -q.x / (||q|| ||x||), 0 when the product <= 1e-9 (knn.cu:168-173)
// ---------------------------------------------------------------------------------
template <int M>
__device__ __forceinline__ float pair_score(float dot, float qn, float xn) {
    if constexpr (M == L2) {
        return fmaxf(fmaf(-2.0f, dot, qn + xn), 0.0f);
    } else if constexpr (M == DOT) {
        return -dot;
    } else {
        float den = qn * xn;
        return den > 1e-9f ? -(dot / den) : -0.0f;
    }
}

struct Stage {
    floatx4 a[4];  // 4 x float4 of the base tile chunk per thread
    floatx4 b[4];  // 4 x float4 of the query tile chunk per thread
};

__device__ __forceinline__ void load_chunk(Stage &st, const float *__restrict__ base, const float *__restrict__ qry,
                                           long rs, long r_hi, int q0, int nq, int dpad, int k0) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int f = tid + 256 * i;
        const int row = f >> 3, c4 = f & 7;
        const long r = rs + row;
        st.a[i] = r < r_hi ? *(const floatx4 *)(base + r * (long)dpad + k0 + 4 * c4) : floatx4{0, 0, 0, 0};
        const int q = q0 + row;
        st.b[i] = q < nq ? *(const floatx4 *)(qry + (long)q * dpad + k0 + 4 * c4) : floatx4{0, 0, 0, 0};
    }
}

__device__ __forceinline__ void store_chunk(const Stage &st, float *sA, float *sB) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int f = tid + 256 * i;
        const int row = f >> 3, c4 = f & 7;
        *(floatx4 *)(sA + row * kLdsStride + 4 * c4) = st.a[i];
        *(floatx4 *)(sB + row * kLdsStride + 4 * c4) = st.b[i];
    }
}

template <int M>
__global__ __launch_bounds__(256) void k_gemm_filter(
    const float *__restrict__ base, const float *__restrict__ bnorm, const uint32_t *__restrict__ perm,
    const float *__restrict__ qry, const float *__restrict__ qnorm, const float *__restrict__ tau, int nq, int dpad,
    long row_begin, long row_end, int n_qtiles, int n_items, uint2 *__restrict__ cand, uint32_t *__restrict__ cnt,
    int cap) {
    __shared__ __attribute__((aligned(16))) float sA[2][kTileRows * kLdsStride];
    __shared__ __attribute__((aligned(16))) float sB[2][kTileCols * kLdsStride];
    __shared__ __attribute__((aligned(16))) float sN[kTileRows];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave & 1, wc = wave >> 1;
    const int l32 = lane & 31, h = lane >> 5;
    const int nk = dpad / kKChunk;
    const long item_rows = (long)kItemStages * kTileRows;

    // XCD-aware persistent schedule: gridDim.x is a multiple of 8 and workgroup b runs on
    // XCD b % 8.  At step t the XCD x takes the contiguous item block
    // [t*G + x*G/8, t*G + (x+1)*G/8), so its workgroups share row chunks.
    const int G = gridDim.x, g8 = G >> 3;
    const int slot = (blockIdx.x & 7) * g8 + (blockIdx.x >> 3);

    for (int item = slot; item < n_items; item += G) {
        const int qtile = item % n_qtiles;
        const long chunk = item / n_qtiles;
        const int q0 = qtile * kTileCols;
        const long r_lo = row_begin + chunk * item_rows;
        const long r_hi = min(r_lo + item_rows, row_end);

        float qn[2], tq[2];
        int qi[2];
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const int q = q0 + 64 * wc + 32 * cb + l32;
            qi[cb] = q;
            qn[cb] = q < nq ? qnorm[q] : 0.0f;
            tq[cb] = q < nq ? tau[q] : -INFINITY;
        }

        for (long rs = r_lo; rs < r_hi; rs += kTileRows) {
            floatx16 acc[2][2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = floatx16{0};

            Stage st;
            load_chunk(st, base, qry, rs, r_hi, q0, nq, dpad, 0);
            if (tid < kTileRows) sN[tid] = (rs + tid < r_hi) ? bnorm[rs + tid] : 0.0f;
            store_chunk(st, sA[0], sB[0]);
            __syncthreads();

            for (int kc = 0; kc < nk; ++kc) {
                const int buf = kc & 1;
                if (kc + 1 < nk) load_chunk(st, base, qry, rs, r_hi, q0, nq, dpad, (kc + 1) * kKChunk);
                const float *A = sA[buf];
                const float *B = sB[buf];
#pragma unroll
                for (int g = 0; g < kKChunk / 8; ++g) {
                    const int ko = 8 * g + 4 * h;
                    const floatx4 a0 = *(const floatx4 *)(A + (64 * wr + l32) * kLdsStride + ko);
                    const floatx4 a1 = *(const floatx4 *)(A + (64 * wr + 32 + l32) * kLdsStride + ko);
                    const floatx4 b0 = *(const floatx4 *)(B + (64 * wc + l32) * kLdsStride + ko);
                    const floatx4 b1 = *(const floatx4 *)(B + (64 * wc + 32 + l32) * kLdsStride + ko);
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[t], b0[t], acc[0][0], 0, 0, 0);
                        acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[t], b1[t], acc[0][1], 0, 0, 0);
                        acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[t], b0[t], acc[1][0], 0, 0, 0);
                        acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[t], b1[t], acc[1][1], 0, 0, 0);
                    }
                }
                if (kc + 1 < nk) store_chunk(st, sA[buf ^ 1], sB[buf ^ 1]);
                __syncthreads();
            }

            // Epilogue: accumulator register r of block (rb, cb) holds row
            // 64*wr + 32*rb + 8*(r/4) + 4*h + r%4 of the stage and query column l32.
            const int nvalid = (int)min((long)kTileRows, r_hi - rs);
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int rl0 = 64 * wr + 32 * rb + 8 * g + 4 * h;
                    const floatx4 n4 = *(const floatx4 *)(sN + rl0);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
#pragma unroll
                        for (int cb = 0; cb < 2; ++cb) {
                            const float s = pair_score<M>(acc[rb][cb][4 * g + j], qn[cb], n4[j]);
                            if (s <= tq[cb] && rl0 + j < nvalid && qi[cb] < nq) {
                                const uint32_t at = atomicAdd(&cnt[qi[cb]], 1u);
                                if (at < (uint32_t)cap)
                                    cand[(size_t)qi[cb] * cap + at] = make_uint2(score_key(s), perm[rs + rl0 + j]);
                            }
                        }
                    }
                }
            }
            __syncthreads();  // sN / LDS buffers are rewritten by the next stage
        }
    }
}

// ---------------------------------------------------------------------------------
// k-means assignment (replaces the per-thread loop of kmeans_assign_and_accumulate,
// vector-cuda/src/kernels/kmeans.cu:38-285): the same MFMA tiles with centroids as the
// A operand (streamed, L2-resident) and each workgroup's 128 points as the B operand.
// Every lane keeps a running (score, centroid) minimum over its rows, visiting rows in
// ascending order with a strict '<', so the lowest index wins ties as in kmeans.cu:110-114;
// partial minima are combined lexicographically.  Scores: L2 ||c||^2 - 2 x.c (the point's
// own norm is constant), DOT -x.c, COS -x.c/(||x|| ||c||) with the 1e-9 guard.
// Writes assign[p], the per-point inertia in the kmeans.cu convention (L2^2, -dot, 1-cos)
// and pos[p] = the point's slot inside its cluster (an atomic ticket on counts[c]).
// ---------------------------------------------------------------------------------
template <int M>
__global__ __launch_bounds__(256) void k_kmeans_assign(const float *__restrict__ cent, const float *__restrict__ cnorm,
                                                       int k, const float *__restrict__ pts,
                                                       const float *__restrict__ pnorm, int n, int dpad,
                                                       int n_tiles, int32_t *__restrict__ assign,
                                                       float *__restrict__ inertia, int32_t *__restrict__ pos,
                                                       int32_t *__restrict__ counts) {
    __shared__ __attribute__((aligned(16))) float sA[2][kTileRows * kLdsStride];
    __shared__ __attribute__((aligned(16))) float sB[2][kTileCols * kLdsStride];
    __shared__ __attribute__((aligned(16))) float sN[kTileRows];
    __shared__ float xs[2][64];
    __shared__ int xi[2][64];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave & 1, wc = wave >> 1;
    const int l32 = lane & 31, h = lane >> 5;
    const int nk = dpad / kKChunk;

    for (int tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
        const int p0 = tile * kTileCols;
        float pn[2], bs[2];
        int bi[2];
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const int p = p0 + 64 * wc + 32 * cb + l32;
            pn[cb] = p < n ? pnorm[p] : 0.0f;
            bs[cb] = INFINITY;
            bi[cb] = 0;
        }
        for (long rs = 0; rs < k; rs += kTileRows) {
            floatx16 acc[2][2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = floatx16{0};
            Stage st;
            load_chunk(st, cent, pts, rs, k, p0, n, dpad, 0);
            if (tid < kTileRows) sN[tid] = (rs + tid < k) ? cnorm[rs + tid] : 0.0f;
            store_chunk(st, sA[0], sB[0]);
            __syncthreads();
            for (int kc = 0; kc < nk; ++kc) {
                const int buf = kc & 1;
                if (kc + 1 < nk) load_chunk(st, cent, pts, rs, k, p0, n, dpad, (kc + 1) * kKChunk);
                const float *A = sA[buf];
                const float *B = sB[buf];
#pragma unroll
                for (int g = 0; g < kKChunk / 8; ++g) {
                    const int ko = 8 * g + 4 * h;
                    const floatx4 a0 = *(const floatx4 *)(A + (64 * wr + l32) * kLdsStride + ko);
                    const floatx4 a1 = *(const floatx4 *)(A + (64 * wr + 32 + l32) * kLdsStride + ko);
                    const floatx4 b0 = *(const floatx4 *)(B + (64 * wc + l32) * kLdsStride + ko);
                    const floatx4 b1 = *(const floatx4 *)(B + (64 * wc + 32 + l32) * kLdsStride + ko);
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[t], b0[t], acc[0][0], 0, 0, 0);
                        acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[t], b1[t], acc[0][1], 0, 0, 0);
                        acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[t], b0[t], acc[1][0], 0, 0, 0);
                        acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[t], b1[t], acc[1][1], 0, 0, 0);
                    }
                }
                if (kc + 1 < nk) store_chunk(st, sA[buf ^ 1], sB[buf ^ 1]);
                __syncthreads();
            }
            const int nvalid = (int)min((long)kTileRows, (long)k - rs);
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int rl0 = 64 * wr + 32 * rb + 8 * g + 4 * h;
                    const floatx4 n4 = *(const floatx4 *)(sN + rl0);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
#pragma unroll
                        for (int cb = 0; cb < 2; ++cb) {
                            const float dot = acc[rb][cb][4 * g + j];
                            float sc;
                            if constexpr (M == L2) {
                                sc = fmaf(-2.0f, dot, n4[j]);
                            } else if constexpr (M == DOT) {
                                sc = -dot;
                            } else {
                                const float den = pn[cb] * n4[j];
                                sc = den > 1e-9f ? -(dot / den) : -0.0f;
                            }
                            if (sc < bs[cb] && rl0 + j < nvalid) {
                                bs[cb] = sc;
                                bi[cb] = (int)rs + rl0 + j;
                            }
                        }
                    }
                }
            }
            __syncthreads();
        }
        // combine the two row halves held by lanes l and l^32, then the two row waves
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const float os = __shfl_xor(bs[cb], 32, 64);
            const int oi = __shfl_xor(bi[cb], 32, 64);
            if (os < bs[cb] || (os == bs[cb] && oi < bi[cb])) {
                bs[cb] = os;
                bi[cb] = oi;
            }
        }
        if (wr == 1 && h == 0) {
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                xs[wc][32 * cb + l32] = bs[cb];
                xi[wc][32 * cb + l32] = bi[cb];
            }
        }
        __syncthreads();
        if (wr == 0 && h == 0) {
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                const float os = xs[wc][32 * cb + l32];
                const int oi = xi[wc][32 * cb + l32];
                if (os < bs[cb] || (os == bs[cb] && oi < bi[cb])) {
                    bs[cb] = os;
                    bi[cb] = oi;
                }
                const int p = p0 + 64 * wc + 32 * cb + l32;
                if (p < n) {
                    const int c = bi[cb];
                    assign[p] = c;
                    float in;
                    if constexpr (M == L2) in = fmaxf(pn[cb] + bs[cb], 0.0f);
                    else if constexpr (M == DOT) in = bs[cb];
                    else in = 1.0f + bs[cb];
                    inertia[p] = in;
                    pos[p] = atomicAdd(&counts[c], 1);
                }
            }
        }
        __syncthreads();
    }
}

void launch_kmeans_assign(int metric, const float *cent, const float *cnorm, int k, const float *pts,
                          const float *pnorm, int n, int dpad, int32_t *assign, float *inertia, int32_t *pos,
                          int32_t *counts, int grid_cap, hipStream_t s) {
    if (n <= 0 || k <= 0) return;
    const int tiles = ceil_div(n, kTileCols);
    const int grid = tiles < grid_cap ? tiles : grid_cap;
    const dim3 g(grid), b(256);
    switch (metric) {
        case L2:
            hipLaunchKernelGGL(k_kmeans_assign<L2>, g, b, 0, s, cent, cnorm, k, pts, pnorm, n, dpad, tiles, assign,
                               inertia, pos, counts);
            break;
        case DOT:
            hipLaunchKernelGGL(k_kmeans_assign<DOT>, g, b, 0, s, cent, cnorm, k, pts, pnorm, n, dpad, tiles, assign,
                               inertia, pos, counts);
            break;
        default:
            hipLaunchKernelGGL(k_kmeans_assign<COS>, g, b, 0, s, cent, cnorm, k, pts, pnorm, n, dpad, tiles, assign,
                               inertia, pos, counts);
            break;
    }
}

void launch_gemm_filter(int metric, const float *base, const float *bnorm, const uint32_t *perm, const float *qry,
                        const float *qnorm, const float *tau, int nq, int dpad, long row_begin, long row_end,
                        uint2 *cand, uint32_t *cnt, int cap, int grid_cap, hipStream_t s) {
    if (nq <= 0 || row_end <= row_begin) return;
    const int n_qtiles = ceil_div(nq, kTileCols);
    const long item_rows = (long)kItemStages * kTileRows;
    const long n_chunks = (row_end - row_begin + item_rows - 1) / item_rows;
    const long n_items = (long)n_qtiles * n_chunks;
    long grid = n_items < grid_cap ? n_items : grid_cap;
    grid = (grid + 7) / 8 * 8;
    const dim3 g((unsigned)grid), b(256);
    switch (metric) {
        case L2:
            hipLaunchKernelGGL(k_gemm_filter<L2>, g, b, 0, s, base, bnorm, perm, qry, qnorm, tau, nq, dpad, row_begin,
                               row_end, n_qtiles, (int)n_items, cand, cnt, cap);
            break;
        case DOT:
            hipLaunchKernelGGL(k_gemm_filter<DOT>, g, b, 0, s, base, bnorm, perm, qry, qnorm, tau, nq, dpad,
                               row_begin, row_end, n_qtiles, (int)n_items, cand, cnt, cap);
            break;
        default:
            hipLaunchKernelGGL(k_gemm_filter<COS>, g, b, 0, s, base, bnorm, perm, qry, qnorm, tau, nq, dpad,
                               row_begin, row_end, n_qtiles, (int)n_items, cand, cnt, cap);
            break;
    }
}

}  // namespace vh
