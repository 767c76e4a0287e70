// knn_small.hip -- the FP32-MFMA kNN scan for batches of at most kSmallCols queries.
//
// The batch kernels (knn_gemm.hip) give a workgroup 128 (or 32) query columns times hundreds of
// base rows per work item, so a round of a few thousand rows runs on a handful of CUs, each at
// one CU's MFMA rate: at one query per batch a 10,000 x 768 cosine search took about 55 us per
// round whatever the round's size.  Here the unit of work is one wave's 32-row block against the
// batch's single 32-query tile (held in LDS, swizzled as in the batch kernels), and the
// workgroups stride over the row blocks, so every round spreads over all CUs: a round costs about
// one block's MFMA time plus the launch, and the largest rounds stream the base rows once at HBM
// rate.  The epilogues are those of the batch kernels' DENSE and FILTER modes (the same score
// formulas and candidate lists), with a passing pair appended straight to its query's global list.
#include <algorithm>

#include "vh_common.h"

namespace vh {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(4))) const float cfloat;  // read through the scalar cache

constexpr int kSmallWaves = 8;  // waves per workgroup
constexpr int kSmallDense = 2, kSmallFilter = 0;
// FILTER: LDS candidate slots per query and workgroup.  Passing pairs are appended with LDS
// atomics and flushed once, at the workgroup's end, with one global atomic per query (on that
// query's own counter line): a returning global atomic in the loop would wait for every A
// prefetch issued before it.  A workgroup covers
// a few hundred rows of a round whose expected passes per query are at most a quarter of the
// candidate capacity, so it rarely meets more than a couple per query; a full list spills to the
// global list directly.
constexpr int kSmallSlots = 16;
// LDS of one workgroup: the query tile (kSmallCols x dpad floats, dynamic), the K-split's partial
// sums (dynamic, when ksplit > 1) and the static arrays (at most the FILTER counts and slots) share
// the 160 KiB of a CU; a dispatch asking for more is not valid.
constexpr size_t kLdsPerWorkgroup = 160 * 1024;
constexpr size_t kSmallStaticMax = kSmallCols * sizeof(uint32_t) + kSmallCols * kSmallSlots * 8;
constexpr size_t kSmallSplitBytes = (size_t)kSmallWaves * 16 * 64 * 4;
constexpr size_t kSmallDynamicMax = kLdsPerWorkgroup - kSmallStaticMax;
static_assert((size_t)kSmallCols * kSmallMaxDpad * 4 <= kSmallDynamicMax, "the widest tile fits without a K-split");

struct SmallArgs {
    const float *A;      // base rows (dpad floats each; the row count padded to 256 with NaN rows)
    const float *anorm;  // per-row norm: squared L2 norm, or the cosine norm before normalisation
    const float *B;      // queries (dpad floats each; rows past ncols are zero, up to a multiple of 32)
    const float *bnorm;  // per-query norm of the same kind
    int dpad, ncols;
    long row_begin, row_end;
    int row_blocks;      // 32-row blocks covering [row_begin, row_end)
    int ksplit;          // waves per block (K-slices): 1, 2, 4 or 8, dividing dpad / 32
    const float *tau;    // FILTER: per-query threshold
    uint2 *cand;
    uint32_t *pad;       // FILTER: per-query reservation counters, kSmallPadStride words apart
    int cap;
};

// float4 index of (query r, K-chunk kc, 16-byte slot c4) in the swizzled tile: row parity picks
// the bank half (for an even chunk count) and (r >> 1) & 7 XORs the slot, so the 16 lanes of a
// ds_read_b128 pass (16 queries, one slot each) cover all 64 banks.
__device__ __forceinline__ int small_bidx(int r, int kc, int c4, int nk) {
    const int pch = (nk & 1) == 0 ? (kc ^ (r & 1)) : kc;
    return r * (8 * nk) + pch * 8 + (c4 ^ ((r >> 1) & 7));
}

// The waves of a workgroup split each 32-row block's K range ksplit ways (1, 2, 4 or 8, dividing the
// chunk count): a group is 8 / ksplit blocks, wave w computes block w / ksplit over K-slice
// w % ksplit, and the slices meet in LDS (summed in slice order) for the epilogue of the slice-0
// wave.  Small rounds split K so that their few blocks still occupy many waves; large rounds
// (ksplit 1) keep one block per wave.  Each wave streams its (group, chunk) sequence with the A
// operand loaded two chunks ahead, across block boundaries, so the next block's first loads run
// under the current block's last MFMAs and its epilogue.
template <int MODE, int M>
__global__ __launch_bounds__(512) void k_mfma_small(SmallArgs a) {
    extern __shared__ floatx4 sB[];  // kSmallCols x dpad floats, then (ksplit > 1) 8 x 16 x 64 partial sums
    // the wave index as a scalar, so that every block index below is one too
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int nk = a.dpad >> 5;
    const int S = a.ksplit, bpg = kSmallWaves / S;
    const int my_b = wave / S, my_s = wave % S;
    const int nc = nk / S, c_lo = my_s * nc;
    const int n_groups = (a.row_blocks + bpg - 1) / bpg;
    const int col0 = blockIdx.y * kSmallCols;
    {
        // the tile: every load issued before the first LDS store, so they overlap
        constexpr int FMAX = kSmallCols * 8 * (kSmallMaxDpad / 32) / 512;
        const int nf = kSmallCols * 8 * nk;
        floatx4 v[FMAX];
#pragma unroll
        for (int i = 0; i < FMAX; ++i) {
            const int f = tid + 512 * i, r = f / (8 * nk), rem = f % (8 * nk);
            if (f < nf) v[i] = *(const floatx4 *)(a.B + (long)(col0 + r) * a.dpad + 4 * rem);
        }
#pragma unroll
        for (int i = 0; i < FMAX; ++i) {
            const int f = tid + 512 * i, r = f / (8 * nk), rem = f % (8 * nk);
            if (f < nf) sB[small_bidx(r, rem >> 3, rem & 7, nk)] = v[i];
        }
    }
    float *red = (float *)(sB + kSmallCols * 8 * nk);
    const int q = col0 + l32;
    const bool qv = q < a.ncols;
    const float cn = qv ? a.bnorm[q] : 0.0f;
    const float tq = (MODE == kSmallFilter && qv) ? a.tau[q] : -INFINITY;
    __shared__ uint32_t s_cnt[MODE == kSmallFilter ? kSmallCols : 1];
    __shared__ uint2 s_slot[MODE == kSmallFilter ? kSmallCols * kSmallSlots : 1];
    if (MODE == kSmallFilter && tid < kSmallCols) s_cnt[tid] = 0;
    __syncthreads();

    // this wave's stream: element t is chunk c_lo + t % nc of block b(t / nc); a block past the
    // round reads the round's first block (in bounds) and is not evaluated
    const int my_groups = blockIdx.x < n_groups ? (n_groups - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
    const int T = my_groups * nc;
    auto block_of = [&](int i) {
        const int b = ((int)blockIdx.x + i * (int)gridDim.x) * bpg + my_b;
        return b < a.row_blocks ? b : -1;
    };
    auto load = [&](floatx4 (&r)[4], int t) {
        const int b = block_of(t / nc);
        const long row0 = a.row_begin + 32L * (b < 0 ? 0 : b);
        const float *p = a.A + (row0 + l32) * (long)a.dpad + 32 * (c_lo + t % nc) + 4 * h;
#pragma unroll
        for (int g = 0; g < 4; ++g) r[g] = *(const floatx4 *)(p + 8 * g);
    };
    floatx16 c0 = floatx16{0}, c1 = floatx16{0};
    // one stream element: the MFMAs of chunk t on `cur`, after issuing the load of element t + 2
    // into `fill`; at the last chunk of a block, its epilogue.  The loop below rotates three
    // register sets through the roles, so no register is copied (a copy would wait for its load).
    auto step = [&](const floatx4 (&cur)[4], floatx4 (&fill)[4], int t) {
        // branch-free: near the end it re-reads the last element (in bounds, unused), so the
        // compiler's wait counts see the same loads in flight on every path
        load(fill, min(t + 2, T - 1));
        const int kc = c_lo + t % nc;
        // the chunk's four tile operands read up front, so that one LDS wait covers them all
        floatx4 bq[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) bq[g] = sB[small_bidx(l32, kc, 2 * g + h, nk)];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x2f32(cur[g][0], bq[g][0], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x2f32(cur[g][1], bq[g][1], c1, 0, 0, 0);
            c0 = __builtin_amdgcn_mfma_f32_32x32x2f32(cur[g][2], bq[g][2], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x2f32(cur[g][3], bq[g][3], c1, 0, 0, 0);
        }
        if (t % nc != nc - 1) return;
        // ---- end of this wave's part of a block ----
        floatx16 acc = c0 + c1;
        c0 = floatx16{0};
        c1 = floatx16{0};
        if (S > 1) {
#pragma unroll
            for (int r = 0; r < 16; ++r) red[(wave * 16 + r) * 64 + lane] = acc[r];
            __syncthreads();
            if (my_s == 0) {
                for (int s2 = 1; s2 < S; ++s2) {
                    float part[16];
#pragma unroll
                    for (int r = 0; r < 16; ++r) part[r] = red[((wave + s2) * 16 + r) * 64 + lane];
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[r] += part[r];
                }
            }
            __syncthreads();
        }
        const int b = block_of(t / nc);
        if (my_s != 0 || b < 0 || !qv) return;
        const long row0 = a.row_begin + 32L * b;
        uint2 *dst = a.cand + (size_t)q * a.cap;
        // The block's 32 row norms through the scalar cache: a vector load here, issued after the
        // A prefetches, could only be waited for together with them (the vector-memory counter
        // retires in order).
        const cfloat *nb = (const cfloat *)(a.anorm + row0);
        float nv[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) nv[i] = nb[i];
        // accumulator 4 g + j of lane (l32, h): row row0 + 8 g + 4 h + j, query column l32
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const long row = row0 + 8 * g + 4 * h;
            floatx4 n4;
#pragma unroll
            for (int j = 0; j < 4; ++j) n4[j] = h ? nv[8 * g + 4 + j] : nv[8 * g + j];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float dot = acc[4 * g + j];
                float sc;
                if constexpr (M == L2) {
                    const float v = fmaf(-2.0f, dot, cn + n4[j]);
                    sc = v == v ? fmaxf(v, 0.0f) : v;
                } else if constexpr (M == DOT) {
                    sc = -dot + 0.0f;
                } else {
                    sc = cn * n4[j] > 1e-9f ? -dot + 0.0f : 0.0f * dot + 0.0f;
                }
                if (row + j >= a.row_end) continue;
                if constexpr (MODE == kSmallDense) {
                    ((gu64 *)dst)[row + j - a.row_begin] = pack_u2(score_key(nan_last(sc)), (uint32_t)(row + j));
                } else {
                    if (sc <= tq) {
                        const uint32_t r = atomicAdd(&s_cnt[l32], 1u);
                        if (r < (uint32_t)kSmallSlots) {
                            s_slot[l32 * kSmallSlots + r] = make_uint2(score_key(sc), (uint32_t)(row + j));
                        } else {
                            const uint32_t at = __hip_atomic_fetch_add(a.pad + (size_t)q * kSmallPadStride, 1u,
                                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            if (at < (uint32_t)a.cap)
                                ((gu64 *)dst)[at] = pack_u2(score_key(sc), (uint32_t)(row + j));
                        }
                    }
                }
            }
        }
    };
    if (T > 0) {
        floatx4 r0[4], r1[4], r2[4];
        load(r0, 0);
        load(r1, min(1, T - 1));
        int t = 0;
        for (; t + 3 <= T; t += 3) {
            step(r0, r2, t);
            step(r1, r0, t + 1);
            step(r2, r1, t + 2);
        }
        if (t < T) step(r0, r2, t);
        if (t + 1 < T) step(r1, r0, t + 1);
    }
    if constexpr (MODE == kSmallFilter) {
        // flush: each query's staged pairs take one reservation on its own counter.  The counters
        // of a batch's queries sit on separate 128-byte lines (the merge reads them there): on one
        // line (cnt), the reservations of the ~1,000 workgroups of a 1M-row round queued up at one
        // L2 atomic unit, and a 32-query round took 215 us against 99 with none.
        __syncthreads();
        for (int qi = wave; qi < kSmallCols; qi += kSmallWaves) {
            const int qq = col0 + qi;
            const uint32_t n = min(s_cnt[qi], (uint32_t)kSmallSlots);
            if (n == 0 || qq >= a.ncols) continue;
            uint32_t base = 0;
            if (lane == 0)
                base = __hip_atomic_fetch_add(a.pad + (size_t)qq * kSmallPadStride, n, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
            base = __shfl(base, 0, 64);
            if (lane < (int)n && base + lane < (uint32_t)a.cap) {
                const uint2 e = s_slot[qi * kSmallSlots + lane];
                ((gu64 *)(a.cand + (size_t)qq * a.cap))[base + lane] = pack_u2(e.x, e.y);
            }
        }
    }
}

template <int MODE, int M>
static void launch_small_m(const SmallArgs &a, dim3 grid, size_t lds, hipStream_t s) {
    // more than 64 KB of dynamic LDS (the tile at dpad > 512) has to be allowed per kernel
    static bool attr = false;
    if (lds > 65536 && !attr) {
        if (hipFuncSetAttribute((const void *)k_mfma_small<MODE, M>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)kSmallDynamicMax) == hipSuccess)
            attr = true;
        else
            (void)hipGetLastError();
    }
    scan_launch((k_mfma_small<MODE, M>), grid, dim3(512), lds, s, a);
}

void launch_small_scan(int metric, bool dense, const float *base, const float *bnorm, const float *qry,
                       const float *qnorm, const float *tau, int nq, int dpad, long row_begin, long row_end,
                       long plan_rows, uint2 *cand, uint32_t *pad, int cap, int grid_cap, hipStream_t s) {
    if (nq <= 0 || row_end <= row_begin) return;
    SmallArgs a{};
    a.A = base;
    a.anorm = bnorm;
    a.B = qry;
    a.bnorm = qnorm;
    a.dpad = dpad;
    a.ncols = nq;
    a.row_begin = row_begin;
    a.row_end = row_end;
    a.row_blocks = (int)((row_end - row_begin + 31) / 32);
    a.tau = tau;
    a.cand = cand;
    a.pad = pad;
    a.cap = cap;
    const int n_ctiles = ceil_div(nq, kSmallCols);
    const int per_tile = std::max(1, grid_cap / n_ctiles);
    // K-split: the largest of 8, 4, 2 dividing the chunk count while the round's blocks times the
    // split stay within about two waves per SIMD of the chip (grid_cap workgroups of 8 waves).  The
    // blocks are those of the whole round (plan_rows), not of this piece of it, so a score's partial
    // sums meet in the same order however the round was cut.
    const int nk = dpad / 32;
    const size_t tile = (size_t)kSmallCols * dpad * sizeof(float);
    const long plan_blocks = (std::max(plan_rows, row_end - row_begin) + 31) / 32;
    int ks = 1;
    // (the partial sums must fit beside the tile: not at dpad 992 and 1024)
    while (ks < kSmallWaves && nk % (2 * ks) == 0 && plan_blocks * 2 * ks <= (long)grid_cap * kSmallWaves / 2 &&
           tile + kSmallSplitBytes <= kSmallDynamicMax)
        ks *= 2;
    a.ksplit = ks;
    const int groups = ceil_div(a.row_blocks, kSmallWaves / ks);
    const size_t lds = tile + (ks > 1 ? kSmallSplitBytes : 0);
    // one workgroup of 8 waves per block group up to four per CU (twice grid_cap): at about 60
    // VGPRs a SIMD then holds 8 waves, whose loads cover each other's memory latency.  No more
    // workgroups than the CUs' LDS holds at once: past that they would run in a second wave, each
    // filling the query tile again, where the resident ones stride on over more block groups
    // with their tile in place and their loads running ahead across blocks.
    const int per_cu = std::max(1, std::min(4, (int)(kLdsPerWorkgroup / (lds + kSmallStaticMax))));
    const int resident = std::max(1, (grid_cap / 2) * per_cu / n_ctiles);
    const dim3 grid((unsigned)std::min({groups, 2 * per_tile, resident}), (unsigned)n_ctiles);
    if (dense) {
        if (metric == L2) launch_small_m<kSmallDense, L2>(a, grid, lds, s);
        else if (metric == DOT) launch_small_m<kSmallDense, DOT>(a, grid, lds, s);
        else launch_small_m<kSmallDense, COS>(a, grid, lds, s);
    } else {
        if (metric == L2) launch_small_m<kSmallFilter, L2>(a, grid, lds, s);
        else if (metric == DOT) launch_small_m<kSmallFilter, DOT>(a, grid, lds, s);
        else launch_small_m<kSmallFilter, COS>(a, grid, lds, s);
    }
}

}  // namespace vh
