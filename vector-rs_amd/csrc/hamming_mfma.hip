// hamming_mfma.hip -- packed-bit Hamming kNN on the fp4 matrix cores.
//
// The popcount kernel (hamming.hip) runs at the VALU issue limit: two VALU operations (XOR,
// bit count) per 32-bit word per query.  Here each bit of a code is expanded once to one fp4
// (e2m1) value, x = 1 - 2 b (+1.0 for 0, -1.0 for 1), two to a byte.  For K-bit codes a and b
// the expanded vectors give x . y = K - 2 popcount(a ^ b), so the Hamming distance is
// (K - x . y) / 2.  Every product is +-1 and every partial sum an integer of magnitude <= K <=
// 1024, so the f32 accumulation is exact, and the scan becomes an fp4 GEMM on
// v_mfma_scale_f32_32x32x64_f8f6f4 (block scales fixed at 2^0) fused with the same threshold
// filter as the FP32 kernels.  That instruction takes 64 K per 32 x 32 tile in the issue time
// of the int8 one's 32 K, and its operands are half the bytes.  The reference's thresholded
// float Hamming (scalar.rs:143-153) equals this distance on 0/1 codes.
//
// Tiling: a workgroup of 8 waves owns a work item of 128 query columns (their expanded rows
// resident in LDS, 16-byte slots XOR-swizzled by column so a 16-lane pass of ds_read_b128 is
// conflict-free) x item_rows base rows, in stages of 512 rows; every wave streams its own 64
// rows from L2 straight into registers, three K-chunks ahead (the base is stored in the A
// operand's lane order, so each load is 1 KB contiguous), and computes a 64 x 128 block as 2 x 4
// 32 x 32 tiles, so each base code feeds 128 queries from registers.  The grid is persistent
// and XCD-aware like the FP32 kernels.  FILTER keeps (distance, row) pairs with distance <= tau
// in per-query LDS slots flushed once per item; DENSE (the first round) writes every pair.
#include <algorithm>
#include <climits>

#include "vh_common.h"

namespace vh {

typedef int intx4 __attribute__((ext_vector_type(4)));
typedef int intx8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int kHmCols = 128;             // query columns per work item
constexpr int kHmStage = 512;            // base rows per stage: 8 waves x 64
constexpr int kHmSlots = kGemmSlotsReg;  // LDS candidate slots per query per work item
constexpr int kHmFilter = 0, kHmDense = 1;

struct HamArgs {
    const int8_t *A;  // expanded base codes, 32 KC bytes per row, rows readable up to row_end + kHmStage
    const int8_t *B;  // expanded query codes, 32 KC bytes per row, rows padded to a multiple of 128
    const float *tau;
    int nq, n_ctiles, n_items;
    long row_begin, row_end, item_rows;
    uint2 *cand;
    uint32_t *cnt;
    int cap;
};

// Expands rows of `words` packed uint32 (row stride wstride) to one fp4 value per bit, two to a
// byte (bit i of word w -> nibble 32 w + i, the low nibble of a byte first): 0x2 (+1.0) for a
// clear bit, 0xA (-1.0) for a set one.  Words from `words` up to `wout` (even) and rows at or past
// `rows` read as clear bits.  A row is wout / 2 K-chunks of 32 bytes (64 bits).  One thread
// writes the 4 bytes that hold one byte of a code.
//  * tiled = false: row-major (the query tiles, staged through LDS).
//  * tiled = true: the layout of the MFMA A operand, so that one 16-byte load per lane of a wave
//    reads 1 KB contiguous (8 whole cache lines, not 32 partial ones): byte b of row r sits at
//    ((r / 32) * KC + b / 32) * 1024 + ((b / 16) & 1) * 512 + (r % 32) * 16 + b % 16.
__global__ __launch_bounds__(256) void k_ham_expand(const uint32_t *__restrict__ src, size_t rows, int words,
                                                    int wout, int wstride, size_t rows_out, bool tiled,
                                                    uint32_t *__restrict__ dst) {
    const size_t per_row = (size_t)wout * 4, total = rows_out * per_row;  // 4-byte units
    const int kc = wout >> 1;
    for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < total; t += (size_t)gridDim.x * blockDim.x) {
        const size_t r = t / per_row;
        const int rem = (int)(t - r * per_row), w = rem >> 2, sel = rem & 3;
        const uint32_t word = r < rows && w < words ? src[r * (size_t)wstride + w] : 0u;
        const uint32_t b = (word >> (8 * sel)) & 255u;
        uint32_t out = 0x22222222u;
#pragma unroll
        for (int i = 0; i < 8; ++i) out |= ((b >> i) & 1u) << (4 * i + 3);
        size_t o = t;
        if (tiled) {
            const int byte = 4 * rem;  // first of the 4 bytes within the row
            const size_t blk = (r >> 5) * (size_t)kc + (size_t)(byte >> 5);
            o = (blk * 1024 + (size_t)((byte >> 4) & 1) * 512 + (r & 31) * 16 + (byte & 15)) >> 2;
        }
        dst[o] = out;
    }
}

// the fp4 operand: 32 nibbles in the low four registers (the upper four are not read)
__device__ __forceinline__ intx8 fp4_operand(const intx4 &v) {
    return __builtin_shufflevector(v, v, 0, 1, 2, 3, -1, -1, -1, -1);
}

__device__ __forceinline__ int ham_first_item() { return (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3); }

template <int MODE, int KC>
__global__ __launch_bounds__(512, 1) void k_mfma_ham(HamArgs a) {
    constexpr int K = 64 * KC, RB = 32 * KC, NS = RB / 16;  // bits (K), bytes and 16-byte slots per row
    constexpr int SW = NS < 16 ? NS - 1 : 15;
    __shared__ intx4 sB[kHmCols * NS];
    __shared__ uint32_t s_qcnt[MODE == kHmFilter ? kHmCols : 1];
    __shared__ uint2 s_slot[MODE == kHmFilter ? kHmCols * kHmSlots : 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    int item = ham_first_item();
    if (item >= a.n_items) return;

    auto bslot = [](int c, int s) { return c * NS + (s ^ (c & SW)); };
    auto decode = [&](int it, int &c0, long &lo, long &hi) {
        const int ct = it % a.n_ctiles;
        const long chunk = it / a.n_ctiles;
        c0 = ct * kHmCols;
        lo = a.row_begin + chunk * a.item_rows;
        hi = min(lo + a.item_rows, a.row_end);
    };
    auto fill_b = [&](int c0) {
        for (int f = tid; f < kHmCols * NS; f += 512) {
            const int c = f / NS, sidx = f - c * NS;
            sB[bslot(c, sidx)] = *(const intx4 *)(a.B + (size_t)(c0 + c) * RB + 16 * sidx);
        }
    };
    // the two 16-byte operands of K-chunk kc for this wave's rows rs + 64 wave + 32 rb + l32
    // (tiled layout: 32-row blocks of KC chunks of 1 KB, lane-contiguous)
    auto load_a = [&](intx4 (&r)[2], long rs, int kc) {
        const int8_t *p = a.A + ((size_t)((rs + 64 * wave) >> 5) * KC + kc) * 1024 + 16 * lane;
        r[0] = *(const intx4 *)p;
        r[1] = *(const intx4 *)(p + (size_t)KC * 1024);
    };

    int col0;
    long r_lo, r_hi;
    decode(item, col0, r_lo, r_hi);
    fill_b(col0);
    if constexpr (MODE == kHmFilter) {
        if (tid < kHmCols) s_qcnt[tid] = 0;
    }
    // per column: distance <= tq  <=>  dot >= T = K - 2 floor(tq) (distances are integers)
    float T[4];
    auto item_begin = [&]() {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            const int q = col0 + 32 * cb + l32;
            const float t = q < a.nq ? a.tau[q] : -1.0f;
            T[cb] = (float)(t < 0.0f ? K + 1 : (t >= (float)K ? -K : K - 2 * (int)t));
        }
    };
    item_begin();
    long rs = r_lo;
    // A operands in a ring of RING K-chunks, loaded RING - 1 chunks ahead (across stages): a
    // chunk is only 8 MFMAs, too short to cover an L2 round trip on its own.  RING divides KC,
    // so every ring index is a compile-time constant.
    constexpr int RING = KC < 4 ? KC : 4, PD = RING - 1;
    intx4 ring[RING][2];
#pragma unroll
    for (int c = 0; c < PD; ++c) load_a(ring[c], rs, c);
    __syncthreads();

    for (;;) {
        long nrs = rs + kHmStage;
        int nitem = item, ncol0 = col0;
        long nlo = r_lo, nhi = r_hi;
        const bool item_end = nrs >= r_hi;
        bool more = true;
        if (item_end) {
            nitem = item + (int)gridDim.x;
            more = nitem < a.n_items;
            if (more) {
                decode(nitem, ncol0, nlo, nhi);
                nrs = nlo;
            }
        }
        floatx16 acc[2][4];
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) acc[rb][cb] = floatx16{0.0f};
        // the wave in its MFMA block issues first: the other wave of the SIMD fills the matrix
        // pipe's gaps with its epilogue (3% faster than equal priorities)
        __builtin_amdgcn_s_setprio(1);
        // B operands one K-chunk ahead (the LDS read of chunk kc + 1 overlaps the MFMAs of kc)
        intx4 bq[2][4];
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) bq[0][cb] = sB[bslot(32 * cb + l32, h)];
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
            if constexpr (PD > 0) {
                // past the last item this re-reads the current stage (in bounds, never used):
                // no branch inside the unrolled K loop
                if (kc + PD < KC) load_a(ring[(kc + PD) % RING], rs, kc + PD);
                else load_a(ring[(kc + PD) % RING], more ? nrs : rs, kc + PD - KC);
            }
            if (kc + 1 < KC) {
#pragma unroll
                for (int cb = 0; cb < 4; ++cb) bq[(kc + 1) & 1][cb] = sB[bslot(32 * cb + l32, 2 * (kc + 1) + h)];
            }
            const intx4 (&b)[4] = bq[kc & 1];
            if constexpr (PD == 0) load_a(ring[0], rs, kc);  // KC == 1
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                for (int cb = 0; cb < 4; ++cb)
                    acc[rb][cb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        fp4_operand(ring[kc % RING][rb]), fp4_operand(b[cb]), acc[rb][cb], 4, 4, 0, 127, 0, 127);
        }
        // all eight tiles complete here: without this the compiler sinks the second row block's
        // products below the first block's filter branch, keeping every K-chunk's query operands
        // live across it (spills at 512 bits and up)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) asm volatile("" : "+v"(acc[rb][cb]));
        __builtin_amdgcn_s_setprio(0);
        // ---- epilogue: register 4g+j of tile (rb, cb) holds row rs + 64 wave + 32 rb + 8 g + 4 h + j
        // and column 32 cb + l32 ----
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            if constexpr (MODE == kHmFilter) {
                // first each column's best over all 16 rows of the tile half: one compare per
                // column; only a half with some candidate lane takes the per-group tests
                uint64_t m = 0;
#pragma unroll
                for (int cb = 0; cb < 4; ++cb) {
                    const floatx16 &v = acc[rb][cb];
                    float mx = v[0];
#pragma unroll
                    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, v[i]);
                    m |= __builtin_amdgcn_ballot_w64(mx >= T[cb]);
                }
                if (m == 0) continue;
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const long row0 = rs + 64 * wave + 32 * rb + 8 * g + 4 * h;
                if constexpr (MODE == kHmDense) {
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb) {
                        const int q = col0 + 32 * cb + l32;
                        if (q >= a.nq) continue;
                        uint2 *dst = a.cand + (size_t)q * a.cap;
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const long row = row0 + j;
                            if (row < r_hi) {
                                const float dist = ((float)K - acc[rb][cb][4 * g + j]) * 0.5f;
                                dst[row - a.row_begin] = make_uint2(score_key(dist), (uint32_t)row);
                            }
                        }
                    }
                } else {
                    uint64_t m = 0;
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb) {
                        const floatx16 &v = acc[rb][cb];
                        const float mx = fmaxf(fmaxf(v[4 * g], v[4 * g + 1]), fmaxf(v[4 * g + 2], v[4 * g + 3]));
                        m |= __builtin_amdgcn_ballot_w64(mx >= T[cb]);
                    }
                    if (m == 0) continue;
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const float dot = acc[rb][cb][4 * g + j];
                            const long row = row0 + j;
                            if (dot < T[cb] || row >= r_hi) continue;
                            const int ql = 32 * cb + l32;
                            const uint32_t key = score_key(((float)K - dot) * 0.5f);
                            const uint32_t rii = (uint32_t)(row - r_lo);
                            const uint32_t r = atomicAdd(&s_qcnt[ql], 1u);
                            if (r < (uint32_t)kHmSlots) {
                                s_slot[ql * kHmSlots + r] = make_uint2(key, rii);
                            } else {
                                // rare overflow: straight to the global list, drained here so no
                                // store is pending where this path rejoins the loop
                                const int q = col0 + ql;
                                const uint32_t at = __hip_atomic_fetch_add((gu32 *)a.cnt + q, 1u, __ATOMIC_RELAXED,
                                                                           __HIP_MEMORY_SCOPE_AGENT);
                                if (at < (uint32_t)a.cap)
                                    ((gu64 *)a.cand)[(size_t)q * a.cap + at] = pack_u2(key, (uint32_t)row);
                                __builtin_amdgcn_s_waitcnt(VH_VMCNT(0));
                            }
                        }
                }
            }
        }
        if (item_end) {
            __syncthreads();  // every wave is past this item's tile and slot appends
            if constexpr (MODE == kHmFilter) {
                if (tid < kHmCols) {
                    uint32_t c = s_qcnt[tid];
                    if (c) {
                        s_qcnt[tid] = 0;
                        c = min(c, (uint32_t)kHmSlots);
                        const int q = col0 + tid;
                        const uint32_t base = atomicAdd(&a.cnt[q], c);
                        for (uint32_t j = 0; j < c; ++j)
                            if (base + j < (uint32_t)a.cap) {
                                const uint2 e = s_slot[tid * kHmSlots + j];
                                a.cand[(size_t)q * a.cap + base + j] = make_uint2(e.x, (uint32_t)(r_lo + e.y));
                            }
                    }
                }
            }
            if (!more) break;
            fill_b(ncol0);
            __syncthreads();
            item = nitem;
            col0 = ncol0;
            r_lo = nlo;
            r_hi = nhi;
            item_begin();
        }
        rs = nrs;
    }
}

// =========================================================================================
// Wide filter kernel (codes of at most 256 bits, filter rounds).  The kernel above streams each
// wave's base rows from L2 into registers and shares a 128-query tile through LDS: every base
// byte then crosses the L2 -> L1 path once per 128 queries, and that feed (not the matrix pipe)
// bounds it.  Here the roles swap.  A work item is 1024 query columns; each of the 8 waves keeps
// its 128 columns' expanded codes in registers for the whole item (4 tiles x KC chunks x 16
// bytes per lane), and the base passes through a ring of 64-row stages in LDS, copied by
// global_load_lds (one 1 KB piece per wave and stage), which all 8 waves read.  Each base byte
// then feeds 1024 queries per fetch.  Every wave scores each stage as two halves of 32 rows, and
// interleaves the MFMAs of one half with the threshold pre-test of the other (the previous
// stage's second half, or this stage's first), so the epilogue's VALU work runs in the matrix
// pipe's shadow.
// Ring protocol: one LDS barrier every kHwSync stages, in the middle of stage t (t a multiple of
// kHwSync), after the wave's reads of stage t's first half.  Before it each wave waits for its
// own DMAs (stages up to t + kHwSync, issued at the previous barrier); after it every wave's
// pieces of those stages are visible and every wave is done with the stages before t, so the
// DMAs of stages t + kHwSync + 1 .. t + 2 kHwSync go into those slots (2 kHwSync + 1 slots keep
// stages t .. t + 2 kHwSync apart).  Sparse barriers let a wave that appends candidates in one
// stage catch up in the next ones instead of holding all eight waves at every stage.
// =========================================================================================
constexpr int kHwCols = ham_wide_cols();    // query columns per work item: 8 waves x 128
constexpr int kHwStage = 64;                 // base rows per stage (all 8 waves score the same rows)
constexpr int kHwSync = 4;                   // stages per workgroup barrier
constexpr int kHwRing = 2 * kHwSync + 1;     // LDS ring stages (see k_mfma_ham_wide)
constexpr int kHwSlots = ham_wide_slots();   // LDS candidate slots per query per work item
constexpr int kHwHalf = kHwSlots / 2;        // of them, per query and accumulator row half (h)
static_assert(kHwCols == 8 * 128, "one 128-column block per wave");

template <int KC>
__global__ __launch_bounds__(512, 1) void k_mfma_ham_wide(HamArgs a) {
    constexpr int K = 64 * KC, RB = 32 * KC, SB = kHwStage * RB;  // bits, bytes per row, bytes per stage
    constexpr int NPIECE = 2 * KC;                                 // 1 KB pieces per stage
    static_assert(KC == 1 || KC == 2 || KC == 4, "codes of 64 to 256 expanded bits");
    __shared__ __attribute__((aligned(16))) int8_t s_ring[kHwRing * SB];
    // Candidate slots: a query column ql belongs to lanes l32 and l32 + 32 of one wave (rows of
    // the two accumulator halves h), so each (column, h) gets kHwHalf slots of its own, counted
    // in a register of its lane (no LDS atomics).  The counts reach LDS at the item's end.
    __shared__ uint32_t s_hcnt[kHwCols * 2];
    __shared__ uint2 s_slot[kHwCols * kHwSlots];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const int G = gridDim.x;
    int item = ham_first_item();
    if (item >= a.n_items) return;  // uniform over the workgroup

    auto decode = [&](int it, int &c0, long &lo, long &hi) {
        const int ct = it % a.n_ctiles;
        const long chunk = it / a.n_ctiles;
        c0 = ct * kHwCols;
        lo = a.row_begin + chunk * a.item_rows;
        hi = min(lo + a.item_rows, a.row_end);
    };
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)&s_ring[0];
    // The DMA cursor runs up to 2 kHwSync stages ahead of the scored stage over the same sequence
    // of (item, stage).  Past the last stage it keeps re-reading the last one (in bounds, never
    // scored), so every wave issues exactly one DMA per stage and its vmcnt waits stay constant.
    int d_item = item;
    long d_rs, d_hi;
    {
        int c0;
        long lo;
        decode(d_item, c0, lo, d_hi);
        d_rs = lo;
    }
    auto dma_stage = [&](int t) {
        if (wave_u < NPIECE)
            dma_lds16(a.A + ((size_t)(d_rs >> 5) * KC) * 1024 + 1024 * wave_u + 16 * lane,
                      ring_lds + (uint32_t)((t % kHwRing) * SB + 1024 * wave_u));
    };
    auto d_advance = [&]() {
        const long n = d_rs + kHwStage;
        if (n < d_hi) {
            d_rs = n;
        } else if (d_item + G < a.n_items) {
            d_item += G;
            int c0;
            long lo;
            decode(d_item, c0, lo, d_hi);
            d_rs = lo;
        }
    };
    // the A operand of half hf, K-chunk kc of the stage in ring slot t % kHwRing
    auto read_a = [&](int t, int hf, int kc) {
        return *(const intx4 *)(s_ring + (t % kHwRing) * SB + (hf * KC + kc) * 1024 + 16 * lane);
    };

    int col0;
    long r_lo, r_hi;
    decode(item, col0, r_lo, r_hi);
    // this wave's 128 columns: query operands in registers, thresholds per column
    // (distance <= tq  <=>  dot >= T = K - 2 floor(tq); columns past nq never pass)
    intx4 bq[4][KC];
    float T[4];
    int TI[4];  // the pre-test's integer form of T
    bool active = false;
    auto item_begin = [&]() {
        // A wave whose columns all lie past nq (the last column block) skips its MFMAs and drops
        // its masks; its operands are zeroed so that no register is read undefined.
        active = col0 + 128 * wave_u < a.nq;  // rows of B are allocated up to a multiple of 128
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
#pragma unroll
            for (int kc = 0; kc < KC; ++kc)
                bq[cb][kc] = active ? *(const intx4 *)(a.B + (size_t)(col0 + 128 * wave + 32 * cb + l32) * RB +
                                                       32 * kc + 16 * h)
                                    : intx4{0, 0, 0, 0};
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            const int q = col0 + 128 * wave + 32 * cb + l32;
            const float t = q < a.nq ? a.tau[q] : -1.0f;
            T[cb] = (float)(t < 0.0f ? K + 1 : (t >= (float)K ? -K : K - 2 * (int)t));
            TI[cb] = T[cb] > 0.0f ? __builtin_bit_cast(int, T[cb]) : INT_MIN;
        }
    };
    item_begin();
    uint32_t cnt4 = 0;  // this lane's slots used per tile cb, 8 bits each (at most kHwHalf)
    // prologue: stages 0 .. kHwSync (and the query operands) landed and visible
    int t = 0;  // stages scored so far by this workgroup (ring slot t % kHwRing)
#pragma unroll
    for (int i = 0; i <= kHwSync; ++i) {
        dma_stage(i);
        d_advance();
    }
    __builtin_amdgcn_s_waitcnt(VH_VMCNT(0));
    lds_barrier();

    floatx16 acc[2][4];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[hf][cb] = floatx16{0.0f};
    // Threshold pre-test of tile cb of a half: some value of the lane's column among the tile's
    // 16 rows may reach T.  The values are integers in [-K, K] held as floats.  For T > 0 the
    // test runs on their bit patterns as signed integers: non-negative floats order like their
    // patterns, and negative ones read as negative integers, below every positive T.  That makes
    // the maximum one tree of 8 integer max3 operations (no NaN canonicalisation, 3 deep).  For
    // T <= 0 (a threshold of at least K / 2 bits, early rounds only) TI = INT_MIN sends the half
    // to the exact per-row tests.
    auto pretest = [&](const floatx16 &v, int cb) {
        int x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            // through a scalar: this compiler's __builtin_bit_cast of a vector-element expression
            // reads element 0 whatever the index
            const float f = v[i];
            x[i] = __builtin_bit_cast(int, f);
        }
        auto m3 = [](int a, int b, int c) { return max(max(a, b), c); };
        const int a0 = m3(x[0], x[1], x[2]), a1 = m3(x[3], x[4], x[5]), a2 = m3(x[6], x[7], x[8]);
        const int a3 = m3(x[9], x[10], x[11]), a4 = m3(x[12], x[13], x[14]);
        const int mx = max(m3(a0, a1, a2), m3(a3, a4, x[15]));
        return __builtin_amdgcn_ballot_w64(mx >= TI[cb]);
    };
    // Per-row tests and LDS slot appends of a half whose pre-test passed; mk[cb] holds the lanes
    // of tile cb whose column may pass, so only those tiles are examined.  Register 4g+j of tile
    // cb holds row srs + 32 hf + 8 g + 4 h + j and column 128 wave + 32 cb + l32.
    auto append = [&](const floatx16 (&ac)[4], long srs, int hf, const uint64_t (&mk)[4]) {
        // the lane's first row as an offset within the item, and how many rows from it lie inside
        const uint32_t rel0 = (uint32_t)(srs - r_lo) + 32 * hf + 4 * h;
        const int room = (int)((uint32_t)(r_hi - r_lo) - rel0);
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            if (mk[cb] == 0) continue;
            const floatx16 &v = ac[cb];
            const int ql = 128 * wave + 32 * cb + l32;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float mx = fmaxf(fmaxf(v[4 * g], v[4 * g + 1]), fmaxf(v[4 * g + 2], v[4 * g + 3]));
                if (__builtin_amdgcn_ballot_w64(mx >= T[cb]) == 0) continue;
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const float dot = v[4 * g + jj];
                    const int off = 8 * g + jj;  // row of this register after the lane's first
                    if (dot < T[cb] || off >= room) continue;
                    const uint32_t key = score_key(((float)K - dot) * 0.5f);
                    const uint32_t r = (cnt4 >> (8 * cb)) & 255u;
                    if (r < (uint32_t)kHwHalf) {
                        s_slot[(2 * ql + h) * kHwHalf + r] = make_uint2(key, rel0 + off);
                        cnt4 += 1u << (8 * cb);
                    } else {
                        // rare overflow: straight to the global list, drained here so no store
                        // is pending where this path rejoins the loop
                        const int q = col0 + ql;
                        const uint32_t at = __hip_atomic_fetch_add((gu32 *)a.cnt + q, 1u, __ATOMIC_RELAXED,
                                                                   __HIP_MEMORY_SCOPE_AGENT);
                        if (at < (uint32_t)a.cap)
                            ((gu64 *)a.cand)[(size_t)q * a.cap + at] = pack_u2(key, (uint32_t)(r_lo + rel0 + off));
                        __builtin_amdgcn_s_waitcnt(VH_VMCNT(0));
                    }
                }
            }
        }
    };
    // one step: the 4 MFMAs of (half hf, chunk kc) on operand `cur`, interleaved with the
    // pre-test of the tiles [4 kc / KC, 4 (kc + 1) / KC) of the other half's accumulators `oth`
    // into mask[cb] (unconditional, so it stays in the MFMAs' basic block; the caller ignores the
    // masks of a half that holds no scores)
    auto step = [&](floatx16 (&ac)[4], const intx4 &cur, int kc, const floatx16 (&oth)[4], uint64_t (&mask)[4]) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
            ac[cb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fp4_operand(cur), fp4_operand(bq[cb][kc]),
                                                                     kc == 0 ? floatx16{0.0f} : ac[cb], 4, 4, 0, 127,
                                                                     0, 127);
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
            if (cb >= 4 * kc / KC && cb < 4 * (kc + 1) / KC) mask[cb] = pretest(oth[cb], cb);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        }
    };

    long rs = r_lo, prs = 0;
    bool prev = false;  // the previous stage's second half still awaits its pre-test
    intx4 cur = read_a(0, 0, 0);
    for (;;) {
        long nrs = rs + kHwStage;
        int nitem = item, ncol0 = col0;
        long nlo = r_lo, nhi = r_hi;
        const bool item_end = nrs >= r_hi;
        bool more = true;
        if (item_end) {
            nitem = item + G;
            more = nitem < a.n_items;
            if (more) {
                decode(nitem, ncol0, nlo, nhi);
                nrs = nlo;
            }
        }
        // ---- half 0: MFMAs into acc[0]; pre-test of the previous stage's half 1 ----
        uint64_t m1[4] = {0, 0, 0, 0};
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
            const intx4 nxt = kc + 1 < KC ? read_a(t, 0, kc + 1) : read_a(t, 1, 0);
            if (active) step(acc[0], cur, kc, acc[1], m1);
            cur = nxt;
        }
        // acc[1] holds scores of this item's previous stage (and real columns) only if prev && active
        const bool any1 = prev && active && (m1[0] | m1[1] | m1[2] | m1[3]) != 0;
        if (t % kHwSync == 0) {
            __builtin_amdgcn_s_waitcnt(VH_VMCNT(0));  // this wave's pieces of stages <= t + kHwSync
            lds_barrier();
#pragma unroll
            for (int i = 1; i <= kHwSync; ++i) {
                dma_stage(t + kHwSync + i);
                d_advance();
            }
        }
        if (any1) append(acc[1], prs, 1, m1);
        // ---- half 1: MFMAs into acc[1]; pre-test of this stage's half 0 ----
        uint64_t m0[4] = {0, 0, 0, 0};
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
            // stage t + 1 is visible since the last barrier; past the last stage this reads a
            // slot's stale data, never used
            const intx4 nxt = kc + 1 < KC ? read_a(t, 1, kc + 1) : read_a(t + 1, 0, 0);
            if (active) step(acc[1], cur, kc, acc[0], m0);
            cur = nxt;
        }
        const bool any0 = active && (m0[0] | m0[1] | m0[2] | m0[3]) != 0;
        if (any0) append(acc[0], rs, 0, m0);
        prev = true;
        prs = rs;
        ++t;
        if (item_end) {
            // drain: this stage's half 1, then the item's candidate flush
            if (active) {
                uint64_t m[4];
#pragma unroll
                for (int cb = 0; cb < 4; ++cb) m[cb] = pretest(acc[1][cb], cb);
                if ((m[0] | m[1] | m[2] | m[3]) != 0) append(acc[1], rs, 1, m);
            }
            prev = false;
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) s_hcnt[2 * (128 * wave + 32 * cb + l32) + h] = (cnt4 >> (8 * cb)) & 255u;
            cnt4 = 0;
            lds_barrier();  // every wave's slot appends and counts of this item are in LDS
            for (int ql = tid; ql < kHwCols; ql += 512) {
                const uint32_t c0 = s_hcnt[2 * ql], c1 = s_hcnt[2 * ql + 1];
                if (c0 + c1) {
                    const int q = col0 + ql;
                    const uint32_t base = atomicAdd(&a.cnt[q], c0 + c1);
                    for (uint32_t j = 0; j < c0 + c1; ++j)
                        if (base + j < (uint32_t)a.cap) {
                            const uint2 e = s_slot[j < c0 ? 2 * ql * kHwHalf + j : (2 * ql + 1) * kHwHalf + (j - c0)];
                            a.cand[(size_t)q * a.cap + base + j] = make_uint2(e.x, (uint32_t)(r_lo + e.y));
                        }
                }
            }
            lds_barrier();  // the slots are read before the next item's appends
            if (!more) break;
            item = nitem;
            col0 = ncol0;
            r_lo = nlo;
            r_hi = nhi;
            item_begin();
        }
        rs = nrs;
    }
    // the re-reads past the last stage still write this workgroup's LDS: let them land first
    __builtin_amdgcn_s_waitcnt(VH_VMCNT(0));
}

}  // namespace

size_t ham_mfma_rows(size_t n) { return round_up(n, kHmStage) + kHmStage; }

bool ham_mfma_supported(int wpad) { return wpad >= 1 && wpad <= 32; }

// 64-bit K-chunks per expanded row (a 32-bit code is padded with one clear word)
static int ham_chunks(int wpad) { return wpad < 2 ? 1 : wpad / 2; }

size_t ham_mfma_row_bytes(int wpad) { return 32 * (size_t)ham_chunks(wpad); }

void launch_ham_expand(const uint32_t *src, size_t rows, int wpad, int wstride, size_t rows_out, bool tiled,
                       int8_t *dst, hipStream_t s) {
    const int wout = 2 * ham_chunks(wpad);
    const size_t total = rows_out * (size_t)wout * 4;
    if (total == 0) return;
    const unsigned blocks = (unsigned)std::min<size_t>(65536, (total + 255) / 256);
    hipLaunchKernelGGL(k_ham_expand, dim3(blocks), dim3(256), 0, s, src, rows, wpad, wout, wstride, rows_out, tiled,
                       (uint32_t *)dst);
}

void launch_ham_mfma(bool dense, long item_rows, const int8_t *base8, const int8_t *qry8, int wpad,
                     const float *tau, int nq, long row_begin, long row_end, uint2 *cand, uint32_t *cnt, int cap,
                     int grid_cap, hipStream_t s) {
    if (nq <= 0 || row_end <= row_begin) return;
    HamArgs a{};
    a.A = base8;
    a.B = qry8;
    a.tau = tau;
    a.nq = nq;
    a.n_ctiles = ceil_div(nq, kHmCols);
    a.item_rows = item_rows;
    a.row_begin = row_begin;
    a.row_end = row_end;
    const long n_chunks = (row_end - row_begin + item_rows - 1) / item_rows;
    a.n_items = (int)((long)a.n_ctiles * n_chunks);
    a.cand = cand;
    a.cnt = cnt;
    a.cap = cap;
    const int cus = grid_cap / 2;
    long g = a.n_items < cus ? a.n_items : cus;
    const dim3 grid((unsigned)((g + 7) / 8 * 8)), block(512);
#define VH_HM(MODE, KC) scan_launch((k_mfma_ham<MODE, KC>), grid, block, 0, s, a)
#define VH_HM_K(MODE)                 \
    switch (ham_chunks(wpad)) {        \
        case 1: VH_HM(MODE, 1); break; \
        case 2: VH_HM(MODE, 2); break; \
        case 4: VH_HM(MODE, 4); break; \
        case 8: VH_HM(MODE, 8); break; \
        default: VH_HM(MODE, 16); break; \
    }
    if (dense) {
        VH_HM_K(kHmDense)
    } else {
        VH_HM_K(kHmFilter)
    }
#undef VH_HM_K
#undef VH_HM
}

bool ham_wide_supported(int wpad) { return ham_mfma_supported(wpad) && ham_chunks(wpad) <= 4; }

void launch_ham_mfma_wide(long item_rows, const int8_t *base8, const int8_t *qry8, int wpad, const float *tau, int nq,
                          long row_begin, long row_end, uint2 *cand, uint32_t *cnt, int cap, int grid_cap,
                          hipStream_t s) {
    if (nq <= 0 || row_end <= row_begin) return;
    HamArgs a{};
    a.A = base8;
    a.B = qry8;
    a.tau = tau;
    a.nq = nq;
    a.n_ctiles = ceil_div(nq, kHwCols);
    a.item_rows = item_rows;
    a.row_begin = row_begin;
    a.row_end = row_end;
    const long n_chunks = (row_end - row_begin + item_rows - 1) / item_rows;
    a.n_items = (int)((long)a.n_ctiles * n_chunks);
    a.cand = cand;
    a.cnt = cnt;
    a.cap = cap;
    const int cus = grid_cap / 2;
    long g = a.n_items < cus ? a.n_items : cus;
    const dim3 grid((unsigned)((g + 7) / 8 * 8)), block(512);
    switch (ham_chunks(wpad)) {
        case 1: scan_launch((k_mfma_ham_wide<1>), grid, block, 0, s, a); break;
        case 2: scan_launch((k_mfma_ham_wide<2>), grid, block, 0, s, a); break;
        default: scan_launch((k_mfma_ham_wide<4>), grid, block, 0, s, a); break;
    }
}

}  // namespace vh
