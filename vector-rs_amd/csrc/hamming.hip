// hamming.hip -- packed-bit Hamming distance (popcount of XOR) fused with the threshold
// filter of the round/merge top-k.
//
// The reference only has the thresholded float Hamming (vector-simd/src/scalar.rs:143-153,
// knn.cu:107-115) over f32 vectors; on 0/1 codes it equals popcount(a ^ b), which is what
// this kernel computes on 32-bit words (v_xor_b32 + v_bcnt_u32_b32 per word, two VALU
// operations per word per query).  Each lane owns one query's W words in registers; tiles of
// base codes are staged in LDS and read as broadcasts.  Distances are exact integers.  The
// threshold test is batched over 4 rows (one wave-uniform branch per 4 rows) and the grid runs
// 8 workgroups per CU, so tile loads of one workgroup hide behind the others' popcounts.
#include <algorithm>

#include "vh_common.h"

namespace vh {

constexpr int kHamRows = 128;
constexpr long kHamItemRowsMax = 8192;

template <int W>
__global__ __launch_bounds__(256) void k_hamming_filter(const uint32_t *__restrict__ codes,
                                                        const uint32_t *__restrict__ qry,
                                                        const float *__restrict__ tau, int nq, int wpad,
                                                        long row_begin, long row_end, int n_qtiles, int n_items,
                                                        long item_rows, uint2 *__restrict__ cand,
                                                        uint32_t *__restrict__ cnt, int cap) {
    __shared__ uint32_t tile[kHamRows * W];
    const int tid = threadIdx.x;
    const int G = gridDim.x, g8 = G >> 3;
    const int slot = (blockIdx.x & 7) * g8 + (blockIdx.x >> 3);

    for (int item = slot; item < n_items; item += G) {
        const int qtile = item % n_qtiles;
        const long chunk = item / n_qtiles;
        const int q = qtile * 256 + tid;
        const bool qv = q < nq;
        // tau is a float score; distances are integers, so compare against floor(tau).
        const float tf = qv ? tau[q] : -1.0f;
        const uint32_t tq = tf < 0.0f ? 0u : (tf >= 4294967040.0f ? 0xffffffffu : (uint32_t)tf);
        const bool any = qv && tf >= 0.0f;
        const long r_lo = row_begin + chunk * item_rows;
        const long r_hi = min(r_lo + item_rows, row_end);

        uint32_t qw[W];
#pragma unroll
        for (int w = 0; w < W; ++w) qw[w] = (qv && w < wpad) ? qry[(long)q * wpad + w] : 0u;

        for (long rs = r_lo; rs < r_hi; rs += kHamRows) {
            __syncthreads();
            if constexpr (W >= 4) {
                // rows are W words (W = wpad here), so the tile is a contiguous run of uint4
                for (int i = tid; i < kHamRows * W / 4; i += 256) {
                    const long r = rs + (i * 4) / W;
                    ((uint4 *)tile)[i] = r < r_hi ? ((const uint4 *)(codes + rs * W))[i] : make_uint4(0, 0, 0, 0);
                }
            } else {
                for (int i = tid; i < kHamRows * W; i += 256) {
                    const int row = i / W, w = i % W;
                    const long r = rs + row;
                    tile[i] = (r < r_hi && w < wpad) ? codes[r * wpad + w] : 0u;
                }
            }
            __syncthreads();
            const int nvalid = (int)min((long)kHamRows, r_hi - rs);
#pragma unroll 2
            for (int r = 0; r < kHamRows; r += 4) {
                uint32_t d[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    d[i] = 0;
#pragma unroll
                    for (int w = 0; w < W; ++w) d[i] += (uint32_t)__popc(qw[w] ^ tile[(r + i) * W + w]);
                }
                const bool p = any && (d[0] <= tq || d[1] <= tq || d[2] <= tq || d[3] <= tq);
                if (__builtin_amdgcn_ballot_w64(p)) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if (any && d[i] <= tq && r + i < nvalid) {
                            const uint32_t at = atomicAdd(&cnt[q], 1u);
                            if (at < (uint32_t)cap)
                                cand[(size_t)q * cap + at] = make_uint2(score_key((float)d[i]), (uint32_t)(rs + r + i));
                        }
                    }
                }
            }
        }
    }
}

int hamming_word_pad(int words) {
    int w = 1;
    while (w < words) w <<= 1;
    return w;
}

void launch_hamming_filter(const uint32_t *codes, const uint32_t *qry, const float *tau,
                           int nq, int wpad, long row_begin, long row_end, uint2 *cand, uint32_t *cnt, int cap,
                           int grid_cap, hipStream_t s) {
    if (nq <= 0 || row_end <= row_begin) return;
    const int nqt = ceil_div(nq, 256);
    const long resident = 4L * grid_cap;  // 8 workgroups per CU
    // rows per work item: small rounds are cut finer so every resident workgroup gets work
    const long rows = row_end - row_begin;
    long item_rows = (rows * nqt + 2 * resident - 1) / (2 * resident);
    item_rows = std::min(kHamItemRowsMax, std::max((long)kHamRows, (item_rows + kHamRows - 1) / kHamRows * kHamRows));
    const long n_chunks = (rows + item_rows - 1) / item_rows;
    const long items = (long)nqt * n_chunks;
    long grid = items < resident ? items : resident;
    grid = (grid + 7) / 8 * 8;
    const dim3 g((unsigned)grid), b(256);
    const int it = (int)items;
#define VH_HAM(W)                                                                                              \
    scan_launch(k_hamming_filter<W>, g, b, 0, s, codes, qry, tau, nq, wpad, row_begin, row_end, nqt, \
                       it, item_rows, cand, cnt, cap)
    switch (wpad) {
        case 1: VH_HAM(1); break;
        case 2: VH_HAM(2); break;
        case 4: VH_HAM(4); break;
        case 8: VH_HAM(8); break;
        case 16: VH_HAM(16); break;
        default: VH_HAM(32); break;
    }
#undef VH_HAM
}

}  // namespace vh
