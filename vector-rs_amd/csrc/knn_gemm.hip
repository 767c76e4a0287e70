// knn_gemm.hip -- FP32-MFMA distance tiles fused with the kNN threshold filter or the
// k-means argmin.
//
// Replaces knn_compute_distance_matrix + knn_topk_select (vector-cuda/src/kernels/knn.cu:21-305)
// for the GEMM-form metrics (squared L2, dot product, cosine) and the per-thread centroid loop
// of kmeans_assign_and_accumulate (kmeans.cu:38-285).  The Q x N distance matrix is never
// written: in FILTER mode every workgroup keeps its 128 queries' current threshold tau in
// registers and stages only the (score, row) pairs with score <= tau; in ASSIGN mode every
// lane keeps a running (score, centroid) minimum; DENSE mode (the first, small round of a
// search) writes every score of its rows.
//
// Operands: A = rows (resident base vectors, or centroids), B = columns (queries, or points),
// both row-major with `dpad` floats per row (a multiple of 32, zero filled).  A's row count is
// padded to a multiple of 256 with NaN rows, so every score they produce is NaN and fails every
// comparison; B's row count is padded to a multiple of 128.  The inner loop has no bounds checks.
//
// Two kernels share the epilogues:
//  * k_mfma_hs (dpad <= 128): a workgroup of 8 waves owns a work item of 128 columns whose
//    128 x dpad tile stays resident in LDS; each wave streams its own rows of A straight from
//    L2 into registers one step ahead, so waves need no barrier inside an item, and computes its
//    64 x 64 tile in two 32-row halves so that the epilogue of one half runs under the MFMAs of
//    the other.
//  * k_mfma_pnl (dpad a multiple of 128 above 128): the same per-wave register feed of A; the
//    column tile passes through double-buffered LDS in K-panels of 128 floats, copied by
//    global_load_lds one panel ahead, with one barrier per panel.
//  * k_mfma_stream (other dpad > 128): a workgroup of 4 waves streams 128-row x 128-column
//    stages of both operands through double-buffered LDS in K-chunks (32 flop per byte), two
//    workgroups per CU.
// Each wave owns a 64 x 64 sub-tile of 2 x 2 v_mfma_f32_32x32x2f32 blocks.  LDS tiles are
// swizzled for gfx950's LDS (64 banks; a ds_read_b128 serves 16 lanes per pass): within 16
// consecutive rows, row parity selects the 128-byte half of the banks and (row >> 1) & 7 XORs
// the 16-byte slot, so the b128 operand reads and the b128 tile stores are conflict-free.
// The grid is persistent and XCD-aware: work items are handed out so that the workgroups
// resident on one XCD walk the same base rows together and share them through that XCD's L2.
//
// FILTER epilogue: scores are tested against a slightly loose threshold, per group of 8 (4 rows x
// 2 columns per lane) first on each column's best value (two compares per group); only a group
// in which some lane may pass takes the per-score and exact tests.  In k_mfma_hs the squared-L2
// accumulators start from the row norms and the column tile holds -2 q, so the accumulator is
// the test value ||x||^2 - 2 q.x itself (exact for integer data in [0, 255] at dpad <= 128: every
// partial sum stays below 2^24 in magnitude).  Passing
// (score, row) pairs are appended to per-query LDS slots (LDS atomics) and flushed to the
// global per-query candidate lists once per work item, with one global atomic per query.  The
// host sizes each round's work items so that the expected passes per query and item stay well
// below the slot count.
#include "vh_common.h"

namespace vh {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kFilter = 0, kAssign = 1, kDense = 2;
constexpr int kRegSlots = kGemmSlotsReg;     // LDS candidate slots per query per work item (register-fed kernel)
constexpr int kPnlSlots = kGemmSlotsPanel;   // same for the panel kernel
constexpr int kStrSlots = kGemmSlotsStream;  // same for the streaming kernel (two workgroups share a CU's LDS)
constexpr int kNtSlots = kGemmSlotsNarrow;   // same for the narrow resident-tile kernel

// float4 index of (row, c4) in a 32-float-wide swizzled tile
__device__ __forceinline__ int swz(int row, int c4) { return row * 8 + (c4 ^ ((row >> 1) & 7)); }

// ---------------------------------------------------------------------------------
// Row preparation (see RowPrep): one wave per row; the norm is a lane-strided sum followed by
// a fixed xor butterfly, so it is deterministic.
// ---------------------------------------------------------------------------------
constexpr int kPrepRegs = 16;  // rows of up to 64 * 16 floats are held in registers

__global__ __launch_bounds__(256) void k_rows_prep(RowPrep a) {
    const int lane = threadIdx.x & 63;
    const size_t wave = (blockIdx.x * (size_t)blockDim.x + threadIdx.x) >> 6;
    const size_t nwaves = (gridDim.x * (size_t)blockDim.x) >> 6;
    const int dim = a.dim, dpad = a.dpad;
    for (size_t p = wave; p < a.n_out; p += nwaves) {
        float *orow = a.out + p * (size_t)dpad;
        float *rrow = a.raw_out ? a.raw_out + p * (size_t)dpad : nullptr;
        if (p >= a.n) {
            for (int d = lane; d < dpad; d += 64) {
                orow[d] = a.pad_fill;
                if (rrow) rrow[d] = a.pad_fill;
            }
            if (lane == 0) {
                if (a.norm) a.norm[p] = a.pad_fill;
                if (a.err) a.err[p] = 0.0f;
            }
            continue;
        }
        if (a.init.tau && lane < 2) {
            // the run's reset (see launch_topk_init): query p, and the two flag counters at row 0
            if (lane == 0) {
                a.init.tau[p] = INFINITY;
                a.init.have[p] = 0;
                a.init.cnt[p] = a.init.cnt0;
                a.init.flags[p] = 0;
                a.init.mflag[p] = 0;
                if (a.init.pad && p < (size_t)kSmallPadQueries) a.init.pad[p * kSmallPadStride] = 0;
            }
            if (p == 0) a.init.nflag[lane] = 0;
        }
        const size_t src = a.perm ? a.perm[p] : p;
        const float *row = a.in + src * (size_t)dim;
        float ss = 0.0f;
        bool whole = true, exact = true;
        if (dpad <= 64 * kPrepRegs) {
            // the whole row in registers: every load in flight at once, one pass for the norm and the
            // (normalized) output; the sum in the order d, as below
            float xs[kPrepRegs], sh[kPrepRegs];
#pragma unroll
            for (int r = 0; r < kPrepRegs; ++r) {
                const int d = lane + 64 * r;
                xs[r] = d < dim ? row[d] : 0.0f;
                sh[r] = (a.shift && d < dpad) ? a.shift[d] : 0.0f;
            }
#pragma unroll
            for (int r = 0; r < kPrepRegs; ++r) {
                const int d = lane + 64 * r;
                if (d >= dpad) continue;
                const float x = xs[r];
                whole = whole && x == rintf(x);
                if (rrow) rrow[d] = x;
                float v = a.shift ? x - sh[r] : x;
                exact = exact && (!a.shift || v + sh[r] == x);
                if (a.transform) v = sqrtf(fabsf(v));
                if (!a.normalize) orow[d] = v;
                ss = fmaf(v, v, ss);
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
            if (a.normalize) {  // as the pass below: the raw value (transformed), times 1 / norm
                const float nr = sqrtf(ss);
                const float inv = nr > 0.0f ? 1.0f / nr : 0.0f;
#pragma unroll
                for (int r = 0; r < kPrepRegs; ++r) {
                    const int d = lane + 64 * r;
                    if (d >= dpad) continue;
                    float v = xs[r];
                    if (a.transform) v = sqrtf(fabsf(v));
                    orow[d] = v * inv;
                }
            }
        } else {
            // four elements per lane in flight at a time (the loads first), the sum in the order d
            for (int d0 = lane; d0 < dpad; d0 += 256) {
                float xs[4], sh[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int d = d0 + 64 * u;
                    xs[u] = d < dim ? row[d] : 0.0f;
                    sh[u] = (a.shift && d < dpad) ? a.shift[d] : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int d = d0 + 64 * u;
                    if (d >= dpad) break;
                    const float x = xs[u];
                    whole = whole && x == rintf(x);
                    if (rrow) rrow[d] = x;
                    float v = a.shift ? x - sh[u] : x;
                    exact = exact && (!a.shift || v + sh[u] == x);
                    if (a.transform) v = sqrtf(fabsf(v));
                    if (!a.normalize) orow[d] = v;
                    ss = fmaf(v, v, ss);
                }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
            if (a.normalize) {
                const float nr = sqrtf(ss);
                const float inv = nr > 0.0f ? 1.0f / nr : 0.0f;
                for (int d0 = lane; d0 < dpad; d0 += 256) {
                    float xs[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int d = d0 + 64 * u;
                        xs[u] = d < dim ? row[d] : 0.0f;
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int d = d0 + 64 * u;
                        if (d >= dpad) break;
                        float v = xs[u];
                        if (a.transform) v = sqrtf(fabsf(v));
                        orow[d] = v * inv;
                    }
                }
            }
        }
        const bool row_int = __builtin_amdgcn_ballot_w64(!whole) == 0;
        const bool row_exact = __builtin_amdgcn_ballot_w64(!exact) == 0;
        if (lane == 0) {
            if (a.norm_kind && a.norm) a.norm[p] = a.norm_kind == 2 ? sqrtf(ss) : ss;
            if (a.nonint && !row_int) atomicOr(a.nonint, 1u);
            if (a.inexact && !row_exact) atomicOr(a.inexact, 1u);
            if (a.err) {
                const bool ints = row_int && a.base_integral;
                float e = 0.0f;
                if (a.err_mode == 1) {
                    const float r = sqrtf(ss) + sqrtf(a.err_nmax);
                    e = (ints && r * r < 0x1.fep23f) ? 0.0f : a.err_coeff * r * r;
                } else if (a.err_mode == 2) {
                    const float r = sqrtf(ss) * sqrtf(a.err_nmax);
                    e = (ints && r < 0x1.fep23f) ? 0.0f : a.err_coeff * r;
                } else if (a.err_mode == 3) {
                    e = a.err_coeff;
                }
                a.err[p] = e;
            }
        }
    }
}

void launch_rows_prep(const RowPrep &a, hipStream_t s) {
    if (a.n_out == 0) return;
    size_t blocks = (a.n_out + 3) / 4;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_rows_prep, dim3((unsigned)blocks), dim3(256), 0, s, a);
}

void launch_rows_prep(const float *in, size_t n, size_t n_out, int dim, int dpad, const uint32_t *perm, float *out,
                      float *norm, int norm_kind, int transform, int normalize, float pad_fill, hipStream_t s) {
    RowPrep a;
    a.in = in;
    a.n = n;
    a.n_out = n_out;
    a.dim = dim;
    a.dpad = dpad;
    a.perm = perm;
    a.out = out;
    a.norm = norm;
    a.norm_kind = norm_kind;
    a.transform = transform;
    a.normalize = normalize;
    a.pad_fill = pad_fill;
    launch_rows_prep(a, s);
}

// ---------------------------------------------------------------------------------
// Per-dimension shift (the column means): block b sums rows [b*chunk, ...) of every column in
// double (thread t owns columns t, t + 256, ...) and counts them, skipping non-finite values, and
// flags non-integer finite values; one more kernel adds the nparts partials per column in a fixed
// order.  A NaN or infinity then affects only the distances of its own row, as in the reference,
// instead of turning its whole column's shift (and so every shifted row) non-finite.
// ---------------------------------------------------------------------------------
constexpr int kColParts = 512;
size_t col_shift_scratch_bytes(int dim) { return 2 * (size_t)kColParts * (size_t)dim * sizeof(double); }

__global__ __launch_bounds__(256) void k_col_partial(const float *__restrict__ x, size_t n, int dim, size_t chunk,
                                                     double *__restrict__ partial, uint32_t *__restrict__ nonint) {
    const size_t r0 = blockIdx.x * chunk, r1 = min(n, r0 + chunk);
    double *__restrict__ count = partial + (size_t)kColParts * dim;
    bool whole = true;
    for (int d = threadIdx.x; d < dim; d += 256) {
        // 8 rows in flight per step, each into its own accumulator
        double s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        uint32_t c = 0;
        size_t r = r0;
        for (; r + 8 <= r1; r += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = x[(r + j) * (size_t)dim + d];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const bool fin = __builtin_isfinite(v[j]);
                whole = whole && (!fin || v[j] == rintf(v[j]));
                s[j] += fin ? (double)v[j] : 0.0;
                c += fin ? 1u : 0u;
            }
        }
        for (; r < r1; ++r) {
            const float v = x[r * (size_t)dim + d];
            const bool fin = __builtin_isfinite(v);
            whole = whole && (!fin || v == rintf(v));
            s[0] += fin ? (double)v : 0.0;
            c += fin ? 1u : 0u;
        }
        partial[(size_t)blockIdx.x * dim + d] = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
        count[(size_t)blockIdx.x * dim + d] = (double)c;
    }
    if (!whole) atomicOr(nonint, 1u);
}

__global__ __launch_bounds__(256) void k_col_finish(const double *__restrict__ partial, int dim, int dpad,
                                                    const uint32_t *__restrict__ nonint, float *__restrict__ shift) {
    const int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= dpad) return;
    if (d >= dim) {
        shift[d] = 0.0f;
        return;
    }
    const double *count = partial + (size_t)kColParts * dim;
    double s = 0.0, c = 0.0;
    for (int b = 0; b < kColParts; ++b) {
        s += partial[(size_t)b * dim + d];
        c += count[(size_t)b * dim + d];
    }
    // a column with no finite value keeps no shift
    const double m = c > 0.0 ? s / c : 0.0;
    shift[d] = *nonint ? (float)m : (float)rint(m);
}

void launch_col_shift(const float *x, size_t n, int dim, int dpad, double *partial, uint32_t *nonint, float *shift,
                      hipStream_t s) {
    const size_t chunk = (n + kColParts - 1) / kColParts;
    hipLaunchKernelGGL(k_col_partial, dim3(kColParts), dim3(256), 0, s, x, n, dim, chunk, partial, nonint);
    hipLaunchKernelGGL(k_col_finish, dim3((unsigned)((dpad + 255) / 256)), dim3(256), 0, s, partial, dim, dpad,
                       nonint, shift);
}

// ---------------------------------------------------------------------------------
// Kernel arguments.  Work item i covers column tile (i % n_ctiles) and the row range
// [row_begin + (i / n_ctiles) * item_rows, min(.. + item_rows, row_end)); row_begin and
// item_rows are multiples of 256 and row_end is a multiple of 256 or the padded end.
// ---------------------------------------------------------------------------------
struct ScanArgs {
    const float *A;      // rows: base vectors / centroids
    const float *anorm;  // per-row epilogue value: L2 squared norm, cosine norm (NaN on padding rows)
    const float *B;      // columns: queries / points
    const float *bnorm;  // per-column norm: L2 squared norm, cosine norm
    int dpad;
    int ncols;  // real number of columns
    int n_ctiles;
    int n_items;
    long row_begin, row_end;
    long item_rows;
    // FILTER
    const float *tau;
    uint2 *cand;
    uint32_t *cnt;
    int cap;
    float anorm_max;  // largest row value of anorm (L2 slack bound)
    float anorm_min;  // smallest row norm (cosine zero-norm guard)
    // ASSIGN
    int32_t *assign;
    float *inertia;
    int32_t *pos;
    int32_t *counts;
    // ASSIGN certification: a point whose best and second-best scores lie within twice its
    // selection error bound goes to the fix-up list (fix, nfix) instead of taking its ticket
    float err_coeff;      // selection error coefficient (sel_err_coeff)
    const float *cmax;    // device scalar: largest centroid norm value (cnorm units)
    int32_t *fix;
    uint32_t *nfix;
    float *devmax;        // squared L2: per-cluster bound of |x_d - c_d| over its points
    int nrows_valid;      // rows past this (padding) never take a point
};

// -0.0 and +0.0 are the same distance; give them one key.
__device__ __forceinline__ float canon(float s) { return s + 0.0f; }

// 4 x 16 = 64 MFMAs per wave on one K-chunk.  A / B point at the chunk's float4 rows; `bidx`
// maps (column row, c4) to the B tile's float4 index.
template <class BIdx>
__device__ __forceinline__ void mfma_chunk(floatx16 (&acc)[2][2], const floatx4 *__restrict__ A,
                                           const floatx4 *__restrict__ B, BIdx bidx, int wr, int wc, int l32,
                                           int h) {
    const int ra0 = 64 * wr + l32, ra1 = ra0 + 32;
    const int rb0 = 64 * wc + l32, rb1 = rb0 + 32;
#pragma unroll
    for (int g = 0; g < kKChunk / 8; ++g) {
        const int c4 = 2 * g + h;
        const floatx4 a0 = A[swz(ra0, c4)];
        const floatx4 a1 = A[swz(ra1, c4)];
        const floatx4 b0 = B[bidx(rb0, c4)];
        const floatx4 b1 = B[bidx(rb1, c4)];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[t], b0[t], acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[t], b1[t], acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[t], b0[t], acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[t], b1[t], acc[1][1], 0, 0, 0);
        }
    }
}

// ---- per-item epilogue state -----------------------------------------------------------
struct EpiState {
    float tau_e[2], T[2], cn[2];  // FILTER: exact threshold, loose "may pass" threshold, column norm
    bool guard;                   // FILTER cosine: some column may meet a near-zero-norm row
    float bs[2], bs2[2];          // ASSIGN: running best (score, row) and second-best score
    int bi[2];
};

// CB: the wave's 32-column blocks (2, or 1 in the narrow-tile kernel).
template <int MODE, int M, int CB = 2>
__device__ __forceinline__ void item_begin(EpiState &st, const ScanArgs &a, int col0, int wc, int l32) {
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        const int q = col0 + 64 * wc + 32 * cb + l32;
        const bool v = q < a.ncols;
        st.cn[cb] = v ? a.bnorm[q] : 0.0f;
        if constexpr (MODE == kFilter) {
            const float t = v ? a.tau[q] : -INFINITY;
            st.tau_e[cb] = t;
            if constexpr (M == L2) {
                // The loose test compares u = xn - 2 q.x (as computed) with T; the exact score is
                // fl(qn + u) (register kernel) or fl(fl(qn + xn) - 2 q.x) (the others), which
                // differ from qn + u by at most 2^-21 (qn + xn + |t|); the slack doubles that.
                st.T[cb] = (t < INFINITY && t > -INFINITY)
                               ? (t - st.cn[cb]) + 0x1p-19f * (st.cn[cb] + a.anorm_max + fabsf(t))
                               : t;
            } else {
                st.T[cb] = -t;  // score = -dot <= tau  <=>  dot >= -tau (exact)
            }
        } else if constexpr (MODE == kAssign) {
            st.bs[cb] = INFINITY;
            st.bs2[cb] = INFINITY;
            st.bi[cb] = 0;
        }
    }
    st.guard = false;
    if constexpr (MODE == kFilter && M == COS) {
        const bool g0 = (col0 + 64 * wc + l32 < a.ncols) && st.cn[0] * a.anorm_min <= 1e-9f;
        const bool g1 = CB > 1 && (col0 + 64 * wc + 32 + l32 < a.ncols) && st.cn[1] * a.anorm_min <= 1e-9f;
        st.guard = __builtin_amdgcn_ballot_w64(g0 || g1) != 0;
    }
}

// Appends (key, row) to query column ql's LDS slots; a full slot list spills to the global
// candidate list with one atomic per entry.  The spill path (rare: the host sizes work items so
// that the expected passes stay well below SLOTS) waits for its own store, so no vector-memory
// store is pending where it rejoins the main loop: with loads alone in flight the compiler can
// wait for exactly the operand loads each MFMA step needs, rather than for all of them
// (including the prefetch of the next step).
template <int SLOTS>
__device__ __forceinline__ void append_candidate(const ScanArgs &a, int ql, uint32_t key, uint32_t row_in_item,
                                                 long r_lo, int col0, uint32_t *s_qcnt, uint2 *s_slot) {
    const uint32_t r = atomicAdd(&s_qcnt[ql], 1u);
    if (r < (uint32_t)SLOTS) {
        s_slot[ql * SLOTS + r] = make_uint2(key, row_in_item);
    } else {
        const int q = col0 + ql;
        const uint32_t at = __hip_atomic_fetch_add((gu32 *)a.cnt + q, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (at < (uint32_t)a.cap)
            ((gu64 *)a.cand)[(size_t)q * a.cap + at] = pack_u2(key, (uint32_t)(r_lo + row_in_item));
        __builtin_amdgcn_s_waitcnt(VH_VMCNT(0));
    }
}

// FILTER: stage every (score, row) of this stage with score <= tau.  Accumulator register
// 4g+j of block (rb, cb) holds row 64wr + 32rb + 8g + 4h + j of the stage and column
// 64wc + 32cb + l32 of the tile.  `nf(rb, g)` returns the epilogue values (row norms) of rows
// rl0 .. rl0 + 3 below.  Each score costs two VALU operations against a slightly loose
// threshold; only a group of 8 scores in which some lane of the wave may pass takes the exact
// path (one wave-uniform branch per group).
template <int M, int SLOTS, class NF>
__device__ __forceinline__ void filter_stage(const floatx16 (&acc)[2][2], NF nf, const EpiState &st,
                                             const ScanArgs &a, int wr, int wc, int l32, int h, long rs, long r_lo,
                                             int col0, uint32_t *s_qcnt, uint2 *s_slot) {
    const uint32_t row0 = (uint32_t)(rs - r_lo) + 64 * wr + 4 * h;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const floatx4 n4 = nf(rb, g);
            if (!(M == COS && st.guard)) {
                // Wave test on each column's extremum over the group's 4 rows (fminf / fmaxf skip
                // the NaN of padding rows, which fail every test): a group none of whose lanes
                // can pass skips the per-score tests.
                float e[2];
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) {
                    float v[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float dot = acc[rb][cb][4 * g + j];
                        v[j] = M == L2 ? fmaf(-2.0f, dot, n4[j]) : dot;
                    }
                    e[cb] = M == L2 ? fminf(fminf(v[0], v[1]), fminf(v[2], v[3]))
                                    : fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
                }
                const uint64_t m = M == L2 ? __builtin_amdgcn_ballot_w64(e[0] <= st.T[0]) |
                                                 __builtin_amdgcn_ballot_w64(e[1] <= st.T[1])
                                           : __builtin_amdgcn_ballot_w64(e[0] >= st.T[0]) |
                                                 __builtin_amdgcn_ballot_w64(e[1] >= st.T[1]);
                if (m == 0) continue;
            }
            bool p[4][2];
            bool any = false;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) {
                    const float dot = acc[rb][cb][4 * g + j];
                    if constexpr (M == L2) p[j][cb] = fmaf(-2.0f, dot, n4[j]) <= st.T[cb];
                    else p[j][cb] = dot >= st.T[cb];
                    any = any || p[j][cb];
                }
            if (M == COS && st.guard) {
                // a (query, row) pair with ||q|| ||x|| <= 1e-9 has similarity 0 (knn.cu:168-173)
                any = false;
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) {
                        const float dot = acc[rb][cb][4 * g + j];
                        const float sc = st.cn[cb] * n4[j] > 1e-9f ? -dot : 0.0f * dot;
                        p[j][cb] = sc <= st.tau_e[cb];
                        any = any || p[j][cb];
                    }
            }
            if (__builtin_amdgcn_ballot_w64(any)) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) {
                        if (!p[j][cb]) continue;
                        const float dot = acc[rb][cb][4 * g + j];
                        float sc;
                        if constexpr (M == L2) {
                            sc = fmaxf(fmaf(-2.0f, dot, st.cn[cb] + n4[j]), 0.0f);
                            if (!(sc <= st.tau_e[cb])) continue;
                        } else if constexpr (M == DOT) {
                            sc = canon(-dot);
                        } else {
                            sc = st.guard ? (st.cn[cb] * n4[j] > 1e-9f ? canon(-dot) : 0.0f) : canon(-dot);
                        }
                        append_candidate<SLOTS>(a, 64 * wc + 32 * cb + l32, score_key(sc),
                                                row0 + 32 * rb + 8 * g + j, r_lo, col0, s_qcnt, s_slot);
                    }
            }
        }
    }
}

// FILTER item end: one global atomic per query with staged candidates.  Must be called by
// all threads; contains a barrier.
template <int SLOTS, int TC = kTileCols>
__device__ __forceinline__ void filter_flush(const ScanArgs &a, int col0, long r_lo, uint32_t *s_qcnt,
                                             uint2 *s_slot) {
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < TC) {
        uint32_t c = s_qcnt[tid];
        if (c) {
            s_qcnt[tid] = 0;
            c = min(c, (uint32_t)SLOTS);
            const int q = col0 + tid;
            const uint32_t base = atomicAdd(&a.cnt[q], c);
            for (uint32_t j = 0; j < c; ++j) {
                if (base + j < (uint32_t)a.cap) {
                    const uint2 e = s_slot[tid * SLOTS + j];
                    a.cand[(size_t)q * a.cap + base + j] = make_uint2(e.x, (uint32_t)(r_lo + e.y));
                }
            }
        }
    }
}

// DENSE: every (score, row) of the stage with row < row_end is written to
// cand[q * cap + (row - row_begin)] (the round's rows fit the per-query capacity), four
// consecutive rows of one column per pair of 16-byte stores.  Scores are the exact-path values
// of FILTER mode.
template <int M, class NF>
__device__ __forceinline__ void dense_stage(const floatx16 (&acc)[2][2], NF nf, const EpiState &st,
                                            const ScanArgs &a, int wr, int wc, int l32, int h, long rs, int col0) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        const int q = col0 + 64 * wc + 32 * cb + l32;
        if (q >= a.ncols) continue;
        uint2 *dst = a.cand + (size_t)q * a.cap;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const floatx4 n4 = nf(rb, g);
                const long row = rs + 64 * wr + 32 * rb + 8 * g + 4 * h;
                uint32_t key[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float dot = acc[rb][cb][4 * g + j];
                    float sc;
                    if constexpr (M == L2) {
                        const float v = fmaf(-2.0f, dot, st.cn[cb] + n4[j]);
                        sc = v == v ? fmaxf(v, 0.0f) : v;
                    } else if constexpr (M == DOT) {
                        sc = canon(-dot);
                    } else {
                        sc = st.cn[cb] * n4[j] > 1e-9f ? canon(-dot) : canon(0.0f * dot);
                    }
                    key[j] = score_key(nan_last(sc));
                }
                const uint32_t p0 = (uint32_t)(row - a.row_begin);
                if (row + 3 < a.row_end) {
                    *(uint4 *)(dst + p0) = make_uint4(key[0], (uint32_t)row, key[1], (uint32_t)row + 1);
                    *(uint4 *)(dst + p0 + 2) = make_uint4(key[2], (uint32_t)row + 2, key[3], (uint32_t)row + 3);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (row + j < a.row_end) dst[p0 + j] = make_uint2(key[j], (uint32_t)(row + j));
                }
            }
    }
}

// Running best and second-best of a sequence.  Dot product and cosine: the quiet NaN of padding
// rows is ignored (a compare and select per score).  Squared L2: padding centroids score FLT_MAX
// (zero rows of norm FLT_MAX), so plain max / min keep the pair.  Non-finite input makes the
// point's error bound NaN or infinite, which leaves it uncertified for the direct-form fix-up.
template <int M>
__device__ __forceinline__ void second_min(float &m, float &m2, float u) {
    if constexpr (M == L2)
        m2 = fminf(m2, fmaxf(m, u));
    else
        m2 = fminf(m2, u < m ? m : u);
    m = fminf(m, u);
}
// Folds a block's (best m, second m2) into the column's running state; `index` gives the block row
// holding m.  Blocks come in ascending row order and the strict '<' keeps the earlier row on ties
// (the tie then shows as a zero gap).
template <class IDX>
__device__ __forceinline__ void take_min(EpiState &st, int cb, float m, float m2, IDX index) {
    if (m < st.bs[cb]) {
        int idx;
        const int row = index(idx);
        st.bs2[cb] = fminf(st.bs[cb], m2);
        st.bs[cb] = m;
        st.bi[cb] = row;
    } else {
        st.bs2[cb] = fminf(st.bs2[cb], m);
    }
}
// Combines another (best, second, row) triple into the column's state: lower score, then lower row.
__device__ __forceinline__ void combine_best(EpiState &st, int cb, float os, float os2, int oi) {
    if (os < st.bs[cb] || (os == st.bs[cb] && oi < st.bi[cb])) {
        st.bs2[cb] = fminf(os2, st.bs[cb]);
        st.bs[cb] = os;
        st.bi[cb] = oi;
    } else {
        st.bs2[cb] = fminf(st.bs2[cb], os);
    }
}

// ASSIGN: per column, the minimum score over this stage's 32 rows held by the lane, then the
// first (lowest) row reaching it.  Rows are visited in ascending order with a strict '<' across
// stages, so the lowest index wins ties (kmeans.cu:110-114).
template <int M, class NF>
__device__ __forceinline__ void assign_stage(floatx16 (&acc)[2][2], NF nf, EpiState &st, int wr, int h, long rs) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        float m = INFINITY, m2 = INFINITY;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const floatx4 n4 = nf(rb, g);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float dot = acc[rb][cb][4 * g + j];
                    float u;
                    if constexpr (M == L2) {
                        u = fmaf(-2.0f, dot, n4[j]);
                    } else if constexpr (M == DOT) {
                        u = -dot;
                    } else {
                        const float den = st.cn[cb] * n4[j];
                        u = den > 1e-9f ? -(dot / den) : canon(0.0f * dot);
                    }
                    acc[rb][cb][4 * g + j] = u;
                    second_min<M>(m, m2, u);
                }
            }
        take_min(st, cb, m, m2, [&](int &idx) {
            idx = 31;
#pragma unroll
            for (int r = 31; r >= 0; --r) idx = acc[r >> 4][cb][r & 15] == m ? r : idx;
            return (int)rs + 64 * wr + 4 * h + 32 * (idx >> 4) + 8 * ((idx >> 2) & 3) + (idx & 3);
        });
    }
}

// ASSIGN item end: combine lanes l and l^32 (row halves) and the RW row waves, write the
// outputs.  Must be called by all threads; contains a barrier.  A point is certified when its
// second-best score exceeds the best by more than twice its selection error bound: then the
// GEMM-form argmin is the argmin of the exact distances, and the point takes its ticket in its
// cluster.  Otherwise (near-ties, or scores too coarse on badly conditioned data) it goes to the
// fix-up list, whose direct-form pass assigns it.
template <int M, int RW, bool PACKED = false>
__device__ __forceinline__ void assign_finish(EpiState &st, const ScanArgs &a, int col0, int wr, int wc, int l32,
                                              int h, float *s_xs, float *s_xs2, int *s_xi) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
        combine_best(st, cb, __shfl_xor(st.bs[cb], 32, 64), __shfl_xor(st.bs2[cb], 32, 64),
                     __shfl_xor(st.bi[cb], 32, 64));
    if (wr > 0 && h == 0) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const int o = (wr - 1) * kTileCols + 64 * wc + 32 * cb + l32;
            s_xs[o] = st.bs[cb];
            s_xs2[o] = st.bs2[cb];
            s_xi[o] = st.bi[cb];
        }
    }
    __syncthreads();
    if (wr == 0 && h == 0) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
            for (int w = 0; w < RW - 1; ++w) {
                const int o = w * kTileCols + 64 * wc + 32 * cb + l32;
                combine_best(st, cb, s_xs[o], s_xs2[o], s_xi[o]);
            }
            const int p = col0 + 64 * wc + 32 * cb + l32;
            if (p < a.ncols) {
                const int c = st.bi[cb];
                a.assign[p] = c;
                // selection error bound of this point's scores
                float e;
                if constexpr (M == L2) {
                    const float r = sqrtf(st.cn[cb]) + sqrtf(*a.cmax);
                    e = a.err_coeff * r * r;
                } else if constexpr (M == DOT) {
                    e = a.err_coeff * sqrtf(st.cn[cb]) * sqrtf(*a.cmax);
                } else {
                    e = a.err_coeff;
                }
                // the register-fed kernel's squared-L2 scores are packed keys (assign_half): the
                // margin also covers their 15-ulp perturbation; a padding row never certifies
                float margin = 2.0f * e;
                if constexpr (M == L2 && PACKED)
                    margin += 0x1p-18f * (fabsf(st.bs[cb]) + fabsf(st.bs2[cb])) + 0x1p-140f;
                if (!(st.bs2[cb] - st.bs[cb] > margin) || c >= a.nrows_valid) {
                    a.fix[atomicAdd(a.nfix, 1u)] = p;
                } else {
                    if constexpr (M == L2) {
                        // |x_d - c_d| <= ||x - c|| <= sqrt(score + error)
                        const float d = fmaxf(st.cn[cb] + st.bs[cb], 0.0f) + e;
                        atomicMax((uint32_t *)a.devmax + c, __float_as_uint(sqrtf(d) * 1.0001f));
                    } else {
                        a.inertia[p] = M == DOT ? st.bs[cb] : 1.0f + st.bs[cb];  // -dot, 1 - cos
                    }
                    a.pos[p] = atomicAdd(&a.counts[c], 1);
                }
            }
        }
    }
}

template <int TC = kTileCols>
__device__ __forceinline__ void decode_item(const ScanArgs &a, int it, int &c0, long &lo, long &hi) {
    const int ct = it % a.n_ctiles;
    const long chunk = it / a.n_ctiles;
    c0 = ct * TC;
    lo = a.row_begin + chunk * a.item_rows;
    hi = min(lo + a.item_rows, a.row_end);
}

// XCD-aware order: workgroup b runs on XCD b % 8; at step t the XCD x takes the contiguous
// item block [t*G + x*G/8, t*G + (x+1)*G/8) (G, the grid size, is a multiple of 8).
__device__ __forceinline__ int first_item() {
    return (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
}


// =========================================================================================
// Streaming kernel: 4 waves, 128-row stages, both operands streamed per K-chunk (any dpad).
// =========================================================================================
template <int MODE, int M>
__global__ __launch_bounds__(256, 2) void k_mfma_stream(ScanArgs a) {
    constexpr int RW = 2, TR = 128;
    __shared__ floatx4 sA[2][TR * 8];
    __shared__ floatx4 sB[2][kTileCols * 8];
    __shared__ __attribute__((aligned(16))) float sN[2][TR];
    __shared__ uint32_t s_qcnt[MODE == kFilter ? kTileCols : 1];
    __shared__ uint2 s_slot[MODE == kFilter ? kTileCols * kStrSlots : 1];
    __shared__ float s_xs[MODE == kAssign ? (RW - 1) * kTileCols : 1];
    __shared__ float s_xs2[MODE == kAssign ? (RW - 1) * kTileCols : 1];
    __shared__ int s_xi[MODE == kAssign ? (RW - 1) * kTileCols : 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave & 1, wc = wave >> 1;
    const int l32 = lane & 31, h = lane >> 5;
    const int nk = a.dpad / kKChunk;
    const int G = gridDim.x;
    int item = first_item();
    if (item >= a.n_items) return;

    auto load = [&](floatx4 (&ra)[4], floatx4 (&rb)[4], long rs, int c0, int k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int f = tid + 256 * i;
            const int row = f >> 3, c4 = f & 7;
            ra[i] = *(const floatx4 *)(a.A + (rs + row) * (long)a.dpad + k0 + 4 * c4);
            rb[i] = *(const floatx4 *)(a.B + (long)(c0 + row) * a.dpad + k0 + 4 * c4);
        }
    };
    auto store = [&](const floatx4 (&ra)[4], const floatx4 (&rb)[4], floatx4 *dA, floatx4 *dB) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int f = tid + 256 * i;
            dA[swz(f >> 3, f & 7)] = ra[i];
            dB[swz(f >> 3, f & 7)] = rb[i];
        }
    };

    int col0;
    long r_lo, r_hi;
    decode_item(a, item, col0, r_lo, r_hi);
    long rs = r_lo;
    EpiState st;
    item_begin<MODE, M>(st, a, col0, wc, l32);

    floatx4 ra[4], rbv[4];
    float rn = 0.0f;
    load(ra, rbv, rs, col0, 0);
    if (tid < TR) rn = a.anorm[rs + tid];
    store(ra, rbv, sA[0], sB[0]);
    if (tid < TR) sN[0][tid] = rn;
    if constexpr (MODE == kFilter) {
        if (tid < kTileCols) s_qcnt[tid] = 0;
    }
    __syncthreads();
    int buf = 0, sb = 0;

    for (;;) {
        long nrs = rs + TR;
        int nitem = item, ncol0 = col0;
        long nlo = r_lo, nhi = r_hi;
        const bool item_end = nrs >= r_hi;
        bool more = true;
        if (item_end) {
            nitem = item + G;
            more = nitem < a.n_items;
            if (more) {
                decode_item(a, nitem, ncol0, nlo, nhi);
                nrs = nlo;
            }
        }

        floatx16 acc[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = floatx16{0};

        for (int kc = 0; kc < nk; ++kc) {
            const bool last = kc + 1 == nk;
            if (!last) {
                load(ra, rbv, rs, col0, (kc + 1) * kKChunk);
            } else if (more) {
                load(ra, rbv, nrs, ncol0, 0);
                if (tid < TR) rn = a.anorm[nrs + tid];
            }
            mfma_chunk(acc, sA[buf], sB[buf], [](int r, int c4) { return swz(r, c4); }, wr, wc, l32, h);
            if (!last || more) {
                store(ra, rbv, sA[buf ^ 1], sB[buf ^ 1]);
                if (last && tid < TR) sN[sb ^ 1][tid] = rn;
            }
            __syncthreads();
            buf ^= 1;
        }

        const float *nrow = sN[sb];
        auto nf = [&](int rb, int g) { return *(const floatx4 *)(nrow + 64 * wr + 32 * rb + 8 * g + 4 * h); };
        if constexpr (MODE == kFilter) {
            filter_stage<M, kStrSlots>(acc, nf, st, a, wr, wc, l32, h, rs, r_lo, col0, s_qcnt, s_slot);
            if (item_end) filter_flush<kStrSlots>(a, col0, r_lo, s_qcnt, s_slot);
        } else if constexpr (MODE == kDense) {
            dense_stage<M>(acc, nf, st, a, wr, wc, l32, h, rs, col0);
        } else {
            assign_stage<M>(acc, nf, st, wr, h, rs);
            if (item_end) assign_finish<M, RW>(st, a, col0, wr, wc, l32, h, s_xs, s_xs2, s_xi);
        }

        if (!more) break;
        rs = nrs;
        sb ^= 1;
        if (item_end) {
            item = nitem;
            col0 = ncol0;
            r_lo = nlo;
            r_hi = nhi;
            item_begin<MODE, M>(st, a, col0, wc, l32);
        }
    }
}

// =========================================================================================
// Panel kernel (dpad a multiple of 128, e.g. 768): 8 waves, 256-row stages.  As in k_mfma_hs
// every wave streams its own 64 rows of A from L2 into registers one K-chunk ahead.  The
// 128-column tile is too large to stay resident, so it passes through LDS in K-panels of 128
// floats (64 KB): while panel p is multiplied, panel p+1 -- of this stage, the next stage or
// the next work item -- is copied from global memory straight into the other LDS buffer by
// global_load_lds (no VGPRs), and one barrier per panel hands the buffers over.
// =========================================================================================
template <int MODE, int M>
__global__ __launch_bounds__(512, 1) void k_mfma_pnl(ScanArgs a) {
    constexpr int RW = 4, TR = 256;
    __shared__ floatx4 sB[2][kTileCols * 32];
    __shared__ floatx4 sN[2][TR / 4];  // row epilogue values (norms) of the current / next stage
    __shared__ uint32_t s_qcnt[MODE == kFilter ? kTileCols : 1];
    __shared__ uint2 s_slot[MODE == kFilter ? kTileCols * kPnlSlots : 1];
    __shared__ float s_xs[MODE == kAssign ? (RW - 1) * kTileCols : 1];
    __shared__ float s_xs2[MODE == kAssign ? (RW - 1) * kTileCols : 1];
    __shared__ int s_xi[MODE == kAssign ? (RW - 1) * kTileCols : 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave & 3, wc = wave >> 2;
    const int l32 = lane & 31, h = lane >> 5;
    const int D = a.dpad, NK = D / kKChunk, NP = NK / 4;
    const int G = gridDim.x;
    int item = first_item();
    if (item >= a.n_items) return;

    // swizzled panel layout (row r, chunk kc of the panel, 16-byte slot c4), as k_mfma_hs with NK = 4
    auto bidx = [](int r, int kc, int c4) { return r * 32 + (kc ^ (r & 1)) * 8 + (c4 ^ ((r >> 1) & 7)); };
    // Panel p of the column tile at c0 into buffer b.  Instruction i of wave w fills LDS slots
    // [512 i + 64 w, + 64); each lane fetches the 16 bytes the swizzle puts in its slot.
    // Slot f = 512 i + tid holds row r = 16 i + (tid >> 5); its chunk and slot depend on tid only
    // (r & 1 = (tid >> 5) & 1, (r >> 1) & 7 = (tid >> 6) & 7), so one lane address plus a stride
    // of 16 rows serves all eight instructions.
    const int dr = tid >> 5, drem = tid & 31;
    const int dkc = (drem >> 3) ^ (dr & 1), dc4 = (drem & 7) ^ ((tid >> 6) & 7);
    const long dstride = 16L * D;
    // The DMAs are asm (dma_lds16): the compiler then makes no read of the other buffer wait for
    // them (it cannot tell the two buffers apart), nor counts them in the waits for the A loads.
    // Each panel ends with a full vmcnt wait and a barrier before its buffer is read.
    const uint32_t sB_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)&sB[0][0];
    const uint32_t sN_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)&sN[0][0];
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    auto dma_panel = [&](int b, int c0, int p) {
        const float *src = a.B + (long)(c0 + dr) * D + 128 * p + 32 * dkc + 4 * dc4;
        const uint32_t dst = sB_lds + (uint32_t)(b * kTileCols * 32 + 64 * wave_u) * 16u;
#pragma unroll
        for (int i = 0; i < 8; ++i) dma_lds16(src + i * dstride, dst + 512u * 16u * i);
    };
    // row epilogue values of the stage at row rs into norm buffer b (wave 0: 64 lanes x 16 bytes)
    auto dma_norms = [&](int b, long rs) {
        if (wave_u == 0) dma_lds16(a.anorm + rs + 4 * lane, sN_lds + (uint32_t)(b * (TR / 4)) * 16u);
    };
    auto load_a = [&](floatx4 (&r)[8], long rs, int kc) {
        const float *p0 = a.A + (rs + 64 * wr + l32) * (long)D + 32 * kc + 4 * h;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            r[g] = *(const floatx4 *)(p0 + 8 * g);
            r[4 + g] = *(const floatx4 *)(p0 + 32 * (long)D + 8 * g);
        }
    };

    int col0;
    long r_lo, r_hi;
    decode_item(a, item, col0, r_lo, r_hi);
    int pb = 0, sb = 0;
    dma_panel(0, col0, 0);
    dma_norms(0, r_lo);
    if constexpr (MODE == kFilter) {
        if (tid < kTileCols) s_qcnt[tid] = 0;
    }
    long rs = r_lo;
    EpiState st;
    item_begin<MODE, M>(st, a, col0, wc, l32);
    floatx4 cur[8];
    load_a(cur, rs, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    for (;;) {
        long nrs = rs + TR;
        int nitem = item, ncol0 = col0;
        long nlo = r_lo, nhi = r_hi;
        const bool item_end = nrs >= r_hi;
        bool more = true;
        if (item_end) {
            nitem = item + G;
            more = nitem < a.n_items;
            if (more) {
                decode_item(a, nitem, ncol0, nlo, nhi);
                nrs = nlo;
            }
        }
        floatx16 acc[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = floatx16{0};

        for (int p = 0; p < NP; ++p) {
            // the panel after this one goes into the other buffer (free: every wave passed the
            // barrier that ended its last use)
            if (p + 1 < NP) {
                dma_panel(pb ^ 1, col0, p + 1);
            } else if (more) {
                dma_panel(pb ^ 1, ncol0, 0);
                dma_norms(sb ^ 1, nrs);
            }
            const bool last_p = p + 1 == NP;
            const int rb0 = 64 * wc + l32, rb1 = rb0 + 32;
            // B pieces one group ahead (across K-chunks too): the LDS reads of the next group are
            // in flight while the 16 MFMAs of this one issue
            floatx4 nb0 = sB[pb][bidx(rb0, 0, h)], nb1 = sB[pb][bidx(rb1, 0, h)];
#pragma unroll
            for (int kc = 0; kc < 4; ++kc) {
                floatx4 nxt[8];
                const bool last = last_p && kc == 3;
                if (!last) load_a(nxt, rs, 4 * p + kc + 1);
                else if (more) load_a(nxt, nrs, 0);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const floatx4 a0 = cur[g], a1 = cur[4 + g];
                    const floatx4 b0 = nb0, b1 = nb1;
                    if (g < 3) {
                        nb0 = sB[pb][bidx(rb0, kc, 2 * g + 2 + h)];
                        nb1 = sB[pb][bidx(rb1, kc, 2 * g + 2 + h)];
                    } else if (kc < 3) {
                        nb0 = sB[pb][bidx(rb0, kc + 1, h)];
                        nb1 = sB[pb][bidx(rb1, kc + 1, h)];
                    }
                    __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the MFMAs
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[t], b0[t], acc[0][0], 0, 0, 0);
                        acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[t], b1[t], acc[0][1], 0, 0, 0);
                        acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[t], b0[t], acc[1][0], 0, 0, 0);
                        acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[t], b1[t], acc[1][1], 0, 0, 0);
                    }
                }
                if (!last || more) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) cur[i] = nxt[i];
                }
            }
            // this wave's share of the next panel has landed; after the barrier every wave's has,
            // and nobody reads buffer pb any more
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            pb ^= 1;
        }

        const float *nrow = (const float *)&sN[sb][0];
        auto nf = [&](int rb, int g) { return *(const floatx4 *)(nrow + 64 * wr + 32 * rb + 8 * g + 4 * h); };
        if constexpr (MODE == kFilter) {
            filter_stage<M, kPnlSlots>(acc, nf, st, a, wr, wc, l32, h, rs, r_lo, col0, s_qcnt, s_slot);
            if (item_end) filter_flush<kPnlSlots>(a, col0, r_lo, s_qcnt, s_slot);
        } else if constexpr (MODE == kDense) {
            dense_stage<M>(acc, nf, st, a, wr, wc, l32, h, rs, col0);
        } else {
            assign_stage<M>(acc, nf, st, wr, h, rs);
            if (item_end) assign_finish<M, RW>(st, a, col0, wr, wc, l32, h, s_xs, s_xs2, s_xi);
        }

        if (!more) break;
        if (item_end) {
            item = nitem;
            col0 = ncol0;
            r_lo = nlo;
            r_hi = nhi;
            item_begin<MODE, M>(st, a, col0, wc, l32);
        }
        rs = nrs;
        sb ^= 1;
    }
}

// =========================================================================================
// Half-staged register-fed kernel (dpad <= 128).  The 128-column tile of a work item stays in
// LDS; every wave loads its own rows of A from L2 into registers one step (half x K-chunk)
// ahead, and computes its 64 x 64 tile in two halves of 32 rows: while the MFMAs of one half
// run, the wave evaluates the epilogue of the other half (the previous stage's second half, or
// this stage's first half).  Both halves live in the same accumulator registers as before, so
// the epilogue's VALU work hides in the MFMA shadow without extra registers, and the two waves
// of a SIMD never sit in their epilogues while the matrix pipe idles.  There is no barrier inside
// a work item; barriers remain at item boundaries (candidate flush / argmin combine and the
// column-tile reload).
// =========================================================================================

// Epilogue pieces of one half.  acc2[cb] register 4g+j holds row rb0 + 8g + j (rb0 = the half's
// first row in this lane's layout, i.e. rs + 64 wr + 32 hf + 4 h) and column 64wc + 32cb + l32.
// For squared L2 the register kernel's accumulators start from the row norms and its column
// tile holds the queries times -2, so a register already holds u = ||x||^2 - 2 q.x and the
// score is max(||q||^2 + u, 0); for the other metrics it holds q.x.
template <int M, int SLOTS, int CB = 2>
__device__ __forceinline__ void filter_group(const floatx16 (&acc2)[CB], floatx4 n4, const EpiState &st,
                                             const ScanArgs &a, int wc, int l32, uint32_t row_g, long r_lo,
                                             int col0, uint32_t *s_qcnt, uint2 *s_slot, int g, bool enable) {
    bool p[4][CB];
    bool any = false;
    if (!(M == COS && st.guard)) {
        // Wave test on each column's extremum over the group's 4 rows: one compare per column
        // block, whose lane masks are OR-ed in scalar registers.  Only a group with some
        // candidate lane takes the per-score tests below.
        uint64_t m = 0;
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            const float v0 = acc2[cb][4 * g], v1 = acc2[cb][4 * g + 1];
            const float v2 = acc2[cb][4 * g + 2], v3 = acc2[cb][4 * g + 3];
            // fminf / fmaxf ignore the quiet NaN of padding rows
            const float e = M == L2 ? fminf(fminf(v0, v1), fminf(v2, v3)) : fmaxf(fmaxf(v0, v1), fmaxf(v2, v3));
            m |= M == L2 ? __builtin_amdgcn_ballot_w64(e <= st.T[cb]) : __builtin_amdgcn_ballot_w64(e >= st.T[cb]);
        }
        if (!(m != 0 && enable)) return;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                const float v = acc2[cb][4 * g + j];
                p[j][cb] = M == L2 ? v <= st.T[cb] : v >= st.T[cb];
            }
        any = true;
    } else {
        // a (query, row) pair with ||q|| ||x|| <= 1e-9 has similarity 0 (knn.cu:168-173)
        any = false;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                const float dot = acc2[cb][4 * g + j];
                const float sc = st.cn[cb] * n4[j] > 1e-9f ? -dot : 0.0f * dot;
                p[j][cb] = sc <= st.tau_e[cb];
                any = any || p[j][cb];
            }
    }
    if (__builtin_amdgcn_ballot_w64(any && enable)) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                if (!p[j][cb]) continue;
                const float dot = acc2[cb][4 * g + j];
                float sc;
                if constexpr (M == L2) {
                    sc = fmaxf(st.cn[cb] + dot, 0.0f);  // dot holds u (see above)
                    if (!(sc <= st.tau_e[cb])) continue;
                } else if constexpr (M == DOT) {
                    sc = canon(-dot);
                } else {
                    sc = st.guard ? (st.cn[cb] * n4[j] > 1e-9f ? canon(-dot) : 0.0f) : canon(-dot);
                }
                append_candidate<SLOTS>(a, 64 * wc + 32 * cb + l32, score_key(sc), row_g + j, r_lo, col0, s_qcnt,
                                        s_slot);
            }
    }
}

template <int M, int CB = 2>
__device__ __forceinline__ void dense_group(const floatx16 (&acc2)[CB], floatx4 n4, const EpiState &st,
                                            const ScanArgs &a, int wc, int l32, long row, int col0, int g) {
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        const int q = col0 + 64 * wc + 32 * cb + l32;
        if (q >= a.ncols) continue;
        uint2 *dst = a.cand + (size_t)q * a.cap;
        uint32_t key[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float dot = acc2[cb][4 * g + j];
            float sc;
            if constexpr (M == L2) {
                const float v = st.cn[cb] + dot;  // dot holds u (see filter_group)
                sc = v == v ? fmaxf(v, 0.0f) : v;
            } else if constexpr (M == DOT) {
                sc = canon(-dot);
            } else {
                sc = st.cn[cb] * n4[j] > 1e-9f ? canon(-dot) : canon(0.0f * dot);
            }
            key[j] = score_key(nan_last(sc));
        }
        const uint32_t p0 = (uint32_t)(row - a.row_begin);
        if (row + 3 < a.row_end) {
            *(uint4 *)(dst + p0) = make_uint4(key[0], (uint32_t)row, key[1], (uint32_t)row + 1);
            *(uint4 *)(dst + p0 + 2) = make_uint4(key[2], (uint32_t)row + 2, key[3], (uint32_t)row + 3);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (row + j < a.row_end) dst[p0 + j] = make_uint2(key[j], (uint32_t)(row + j));
        }
    }
}

// ASSIGN for one half: per column, the minimum over the half's 16 rows held by the lane, then
// the first (lowest) row reaching it; halves and stages are visited in ascending row order with
// a strict '<', so the lowest index wins ties (kmeans.cu:110-114).
template <int M, bool FUSED = false>
__device__ __forceinline__ void assign_half(floatx16 (&acc2)[2], const floatx4 (&n)[4], EpiState &st, long rb0) {
    if constexpr (M == L2) {
        // Squared L2: each score carries its row within the half (0..15) in its 4 low mantissa
        // bits, so one min yields the best score and its row, and one med3 the second best (4
        // VALU operations per score, no search for the row).  A key differs from its score by
        // at most 15 ulp; the certification at item end widens its margin by 2^-18 of the scores
        // to cover that, so a certified argmin is the argmin of the unpacked scores.  Exact ties
        // are near-ties and go to the direct-form fix-up, which applies the lowest-index rule.
        // Padding centroids score FLT_MAX (finite keys).  Denormals are preserved (the packed
        // bits of scores near zero survive the min).  Both the min and the second come from
        // v_med3 (no canonicalisation of the keys); a non-finite score only arises from
        // non-finite or overflowing input, whose margin at item end is infinite or NaN, so such a
        // point is never certified.
        // -inf the compiler cannot see, so that med3(m, key, -inf) stays a med3 (folded to a
        // min it would canonicalise every key first)
        float neg_inf;
        asm("v_mov_b32 %0, 0xff800000" : "=v"(neg_inf));
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            float m = INFINITY, m2 = INFINITY;
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // FUSED: the accumulators already hold ||c||^2 - 2 c.x
                    const float u = FUSED ? acc2[cb][4 * g + j] : fmaf(-2.0f, acc2[cb][4 * g + j], n[g][j]);
                    const float key = __uint_as_float((__float_as_uint(u) & ~15u) | (uint32_t)(4 * g + j));
                    m2 = __builtin_amdgcn_fmed3f(m, m2, key);
                    m = __builtin_amdgcn_fmed3f(m, key, neg_inf);
                }
            const uint32_t r = __float_as_uint(m) & 15u;
            const int row = (int)rb0 + 8 * (int)(r >> 2) + (int)(r & 3u);
            st.bs2[cb] = fminf(fminf(st.bs2[cb], m2), fmaxf(st.bs[cb], m));
            const bool better = m < st.bs[cb];
            st.bi[cb] = better ? row : st.bi[cb];
            st.bs[cb] = better ? m : st.bs[cb];
        }
        return;
    }
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        float m = INFINITY, m2 = INFINITY;
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float dot = acc2[cb][4 * g + j];
                float u;
                if constexpr (M == L2) {
                    u = fmaf(-2.0f, dot, n[g][j]);
                } else if constexpr (M == DOT) {
                    u = -dot;
                } else {
                    const float den = st.cn[cb] * n[g][j];
                    u = den > 1e-9f ? -(dot / den) : canon(0.0f * dot);
                }
                acc2[cb][4 * g + j] = u;
                second_min<M>(m, m2, u);
            }
        take_min(st, cb, m, m2, [&](int &idx) {
            idx = 15;
#pragma unroll
            for (int r = 15; r >= 0; --r) idx = acc2[cb][r] == m ? r : idx;
            return (int)rb0 + 8 * (idx >> 2) + (idx & 3);
        });
    }
}

template <int MODE, int M, int NK>
__global__ __launch_bounds__(512, 1) void k_mfma_hs(ScanArgs a) {
    constexpr int RW = 4, TR = 256, D = 32 * NK;
    // squared-L2 scan: accumulators start from the row norms and the column tile holds -2 q, so
    // they end as ||x||^2 - 2 q.x (the filter's test value, and the assign score) with no
    // epilogue arithmetic
    constexpr bool FUSE = M == L2;
    __shared__ floatx4 sB[kTileCols * 8 * NK];
    __shared__ uint32_t s_qcnt[MODE == kFilter ? kTileCols : 1];
    __shared__ uint2 s_slot[MODE == kFilter ? kTileCols * kRegSlots : 1];
    __shared__ float s_xs[MODE == kAssign ? (RW - 1) * kTileCols : 1];
    __shared__ float s_xs2[MODE == kAssign ? (RW - 1) * kTileCols : 1];
    __shared__ int s_xi[MODE == kAssign ? (RW - 1) * kTileCols : 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave & 3, wc = wave >> 2;
    const int l32 = lane & 31, h = lane >> 5;
    const int G = gridDim.x;
    int item = first_item();
    if (item >= a.n_items) return;

    auto bidx_kc = [](int r, int kc, int c4) {
        const int pch = (NK % 2 == 0) ? (kc ^ (r & 1)) : kc;
        return r * (8 * NK) + pch * 8 + (c4 ^ ((r >> 1) & 7));
    };
    auto fill_b = [&](int c0) {
        floatx4 rq[2 * NK];
#pragma unroll
        for (int i = 0; i < 2 * NK; ++i) {
            const int f = tid + 512 * i;
            const int r = f / (8 * NK), rem = f % (8 * NK);
            rq[i] = *(const floatx4 *)(a.B + (long)(c0 + r) * D + 4 * rem);
        }
        if constexpr (FUSE) {
#pragma unroll
            for (int i = 0; i < 2 * NK; ++i) rq[i] = rq[i] * -2.0f;  // exact
        }
#pragma unroll
        for (int i = 0; i < 2 * NK; ++i) {
            const int f = tid + 512 * i;
            const int r = f / (8 * NK), rem = f % (8 * NK);
            sB[bidx_kc(r, rem >> 3, rem & 7)] = rq[i];
        }
    };
    // A of half hf, chunk kc of the stage at rs: row rs + 64 wr + 32 hf + l32, floats 32 kc + 8 g + 4 h.
    auto load_a = [&](floatx4 (&r)[4], long rs, int hf, int kc) {
        const float *p0 = a.A + (rs + 64 * wr + 32 * hf + l32) * (long)D + 32 * kc + 4 * h;
#pragma unroll
        for (int g = 0; g < 4; ++g) r[g] = *(const floatx4 *)(p0 + 8 * g);
    };
    auto load_n = [&](floatx4 (&n)[4], long rs, int hf) {
#pragma unroll
        for (int g = 0; g < 4; ++g) n[g] = *(const floatx4 *)(a.anorm + rs + 64 * wr + 32 * hf + 8 * g + 4 * h);
    };
    // `first`: the accumulators start from `init` instead of their contents
    auto mfma_step = [&](floatx16 (&ac)[2], const floatx4 (&ra)[4], int kc, const floatx16 &init, bool first) {
        const int rb0 = 64 * wc + l32, rb1 = rb0 + 32;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int c4 = 2 * g + h;
            const floatx4 b0 = sB[bidx_kc(rb0, kc, c4)];
            const floatx4 b1 = sB[bidx_kc(rb1, kc, c4)];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const bool i0 = first && g == 0 && t == 0;
                ac[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(ra[g][t], b0[t], i0 ? init : ac[0], 0, 0, 0);
                ac[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(ra[g][t], b1[t], i0 ? init : ac[1], 0, 0, 0);
            }
        }
    };
    // the 4 x 4 row values of a half in accumulator order (register 4g+j = row 8g+j of the lane)
    auto n16 = [](const floatx4 (&n)[4]) {
        floatx16 v;
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j) v[4 * g + j] = n[g][j];
        return v;
    };

    int col0;
    long r_lo, r_hi;
    decode_item(a, item, col0, r_lo, r_hi);
    fill_b(col0);
    if constexpr (MODE == kFilter) {
        if (tid < kTileCols) s_qcnt[tid] = 0;
    }
    long rs = r_lo;
    EpiState st;
    item_begin<MODE, M>(st, a, col0, wc, l32);
    floatx4 cur[4];
    load_a(cur, rs, 0, 0);
    __syncthreads();

    floatx16 acc[2][2];  // acc[half][cb]
    floatx4 nrm[2][4];   // epilogue values of each half's rows
    bool prev = false;   // the previous stage's second half is still to be evaluated

    // Epilogue of half hf of the stage at srs, groups [g0, g1); `enable` false makes it a no-op
    // (FILTER folds it into the wave-uniform branch, so the MFMAs and the threshold tests stay in
    // one basic block and the scheduler can interleave them).
    auto epi = [&](floatx16 (&ac)[2], const floatx4 (&n)[4], long srs, int hf, int g0, int g1, bool enable) {
        if constexpr (MODE == kAssign) {
            if (g0 == 0 && enable) assign_half<M, FUSE>(ac, n, st, srs + 64 * wr + 32 * hf + 4 * h);
        } else {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                if (g < g0 || g >= g1) continue;
                if constexpr (MODE == kFilter) {
                    filter_group<M, kRegSlots>(ac, n[g], st, a, wc, l32,
                                               (uint32_t)(srs - r_lo) + 64 * wr + 32 * hf + 8 * g + 4 * h, r_lo,
                                               col0, s_qcnt, s_slot, g, enable);
                } else if (enable) {
                    dense_group<M>(ac, n[g], st, a, wc, l32, srs + 64 * wr + 32 * hf + 8 * g + 4 * h, col0, g);
                }
            }
        }
    };
    // Interleave the step's MFMAs with the epilogue's VALU work: 1 MFMA, then up to 2 VALU.
    // ASSIGN raises the wave's priority over each step's MFMAs (1% faster k-means assign); the
    // filter measured 1% slower with it and keeps equal priorities
    auto interleave = [&]() {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        }
    };

    for (;;) {
        long nrs = rs + TR;
        int nitem = item, ncol0 = col0;
        long nlo = r_lo, nhi = r_hi;
        const bool item_end = nrs >= r_hi;
        bool more = true;
        if (item_end) {
            nitem = item + G;
            more = nitem < a.n_items;
            if (more) {
                decode_item(a, nitem, ncol0, nlo, nhi);
                nrs = nlo;
            }
        }
        // ---- half 0: MFMAs into acc[0]; epilogue of the previous stage's half 1 ----
        load_n(nrm[0], rs, 0);
        if constexpr (!FUSE) {
            acc[0][0] = floatx16{0};
            acc[0][1] = floatx16{0};
        }
        const floatx16 init0 = n16(nrm[0]);
#pragma unroll
        for (int kc = 0; kc < NK; ++kc) {
            floatx4 nxt[4];
            if (kc + 1 < NK) load_a(nxt, rs, 0, kc + 1);
            else load_a(nxt, rs, 1, 0);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (MODE == kAssign) __builtin_amdgcn_s_setprio(1);
            mfma_step(acc[0], cur, kc, init0, FUSE && kc == 0);
            if constexpr (MODE == kAssign) __builtin_amdgcn_s_setprio(0);
            epi(acc[1], nrm[1], rs - TR, 1, (4 * kc) / NK, (4 * (kc + 1)) / NK, prev);
            interleave();
#pragma unroll
            for (int i = 0; i < 4; ++i) cur[i] = nxt[i];
        }
        // ---- half 1: MFMAs into acc[1]; epilogue of this stage's half 0 ----
        load_n(nrm[1], rs, 1);
        if constexpr (!FUSE) {
            acc[1][0] = floatx16{0};
            acc[1][1] = floatx16{0};
        }
        const floatx16 init1 = n16(nrm[1]);
#pragma unroll
        for (int kc = 0; kc < NK; ++kc) {
            floatx4 nxt[4];
            const bool last = kc + 1 == NK;
            if (!last) load_a(nxt, rs, 1, kc + 1);
            else if (more) load_a(nxt, nrs, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (MODE == kAssign) __builtin_amdgcn_s_setprio(1);
            mfma_step(acc[1], cur, kc, init1, FUSE && kc == 0);
            if constexpr (MODE == kAssign) __builtin_amdgcn_s_setprio(0);
            epi(acc[0], nrm[0], rs, 0, (4 * kc) / NK, (4 * (kc + 1)) / NK, true);
            interleave();
            if (!last || more) {
#pragma unroll
                for (int i = 0; i < 4; ++i) cur[i] = nxt[i];
            }
        }
        prev = true;
        if (item_end) {
            // drain: this stage's half 1, then the item's cross-wave work
            epi(acc[1], nrm[1], rs, 1, 0, 4, true);
            if constexpr (MODE == kFilter) filter_flush<kRegSlots>(a, col0, r_lo, s_qcnt, s_slot);
            else if constexpr (MODE == kAssign)
                assign_finish<M, RW, true>(st, a, col0, wr, wc, l32, h, s_xs, s_xs2, s_xi);
            if (!more) break;
            // every wave is past this item's MFMAs (barrier in the flush / combine above; DENSE
            // has none, so take one here)
            if constexpr (MODE == kDense) __syncthreads();
            fill_b(ncol0);
            __syncthreads();
            item = nitem;
            col0 = ncol0;
            r_lo = nlo;
            r_hi = nhi;
            item_begin<MODE, M>(st, a, col0, wc, l32);
            prev = false;
        }
        rs = nrs;
    }
}

// =========================================================================================
// Narrow resident-tile kernel (kNN search at dpad a multiple of 128 from 256 to 896).  A work item is
// kNtCols = 32 query columns, whose 32 x dpad tile stays resident in LDS (96 KB at dpad 768), x
// item_rows base rows in stages of 512: each of the 8 waves streams its own 64 rows of A from L2
// into registers two K-chunks ahead and computes its 64 x 32 block in two
// halves of 32 rows, the epilogue of one half running under the MFMAs of the other, as in
// k_mfma_hs.  The tile operand of each 4-MFMA group is read from LDS one group ahead.  Each half
// accumulates in two chains (even and odd K pairs) summed at its end, so that a wave's
// consecutive MFMAs do not wait for each other.  Against the panel kernel, whose 128-column
// tiles pass through LDS in K-panels, the query tile is read once per work item instead of once
// per 256-row stage, nothing inside an item takes a barrier, and the 32 workgroups of an XCD
// (32 consecutive column tiles of one row range) share each base row through its L2.
// Items are multiples of 256 rows, so a stage can reach past the item's last row: a wave whose 64
// rows start at or past it reads the item's first 64 rows instead (always inside the padded
// base) and evaluates nothing.
// =========================================================================================
template <int MODE, int M, int NK>
__global__ __launch_bounds__(512, 1) void k_mfma_nt(ScanArgs a) {
    static_assert(MODE != kAssign, "search modes only");
    constexpr int TR = 512, D = 32 * NK, TC = kNtCols;
    constexpr bool FUSE = M == L2;  // accumulators start from the row norms; the tile holds -2 q
    // prefetch distance in K-chunks: 2 (4% faster at dpad 768 than 1; 3 gains nothing at dpad 256
    // to 512), 1 in the dense round at dpad 896, whose registers would spill
    constexpr int PD = MODE == kDense && NK >= 28 ? 1 : 2;
    __shared__ floatx4 sB[TC * 8 * NK];
    __shared__ uint32_t s_qcnt[MODE == kFilter ? TC : 1];
    __shared__ uint2 s_slot[MODE == kFilter ? TC * kNtSlots : 1];

    const int tid = threadIdx.x, lane = tid & 63, wr = tid >> 6;  // wave wr: rows 64 wr .. of a stage
    const int l32 = lane & 31, h = lane >> 5;
    const int G = gridDim.x;
    int item = first_item();
    if (item >= a.n_items) return;

    // swizzled tile layout, as in k_mfma_hs (row r = query column, chunk kc, 16-byte slot c4)
    auto bidx_kc = [](int r, int kc, int c4) {
        const int pch = (NK % 2 == 0) ? (kc ^ (r & 1)) : kc;
        return r * (8 * NK) + pch * 8 + (c4 ^ ((r >> 1) & 7));
    };
    auto fill_b = [&](int c0) {
        constexpr int PER = TC * 8 * NK / 512;
        floatx4 rq[PER];
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int f = tid + 512 * i;
            const int r = f / (8 * NK), rem = f % (8 * NK);
            rq[i] = *(const floatx4 *)(a.B + (long)(c0 + r) * D + 4 * rem);
        }
        if constexpr (FUSE) {
#pragma unroll
            for (int i = 0; i < PER; ++i) rq[i] = rq[i] * -2.0f;  // exact
        }
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int f = tid + 512 * i;
            const int r = f / (8 * NK), rem = f % (8 * NK);
            sB[bidx_kc(r, rem >> 3, rem & 7)] = rq[i];
        }
    };
    // A of half hf, chunk kc of the rows at `base`: row base + 64 wr + 32 hf + l32, floats 32 kc + 8 g + 4 h.
    auto load_a = [&](floatx4 (&r)[4], long base, int hf, int kc) {
        const float *p0 = a.A + (base + 64 * wr + 32 * hf + l32) * (long)D + 32 * kc + 4 * h;
#pragma unroll
        for (int g = 0; g < 4; ++g) r[g] = *(const floatx4 *)(p0 + 8 * g);
    };
    auto load_n = [&](floatx4 (&n)[4], long base, int hf) {
#pragma unroll
        for (int g = 0; g < 4; ++g) n[g] = *(const floatx4 *)(a.anorm + base + 64 * wr + 32 * hf + 8 * g + 4 * h);
    };
    // one K-chunk of a half into its two chains; at kc = 0 chain 0 starts from `init`, chain 1 from 0.
    // bq holds the tile operand of (kc, group 0) on entry; each group reads the next group's
    // (wrapping to chunk 0, which the next half and stage start with) before its own MFMAs, so
    // the LDS latency runs under them.
    const floatx16 zero16 = floatx16{0};
    auto mfma_step = [&](floatx16 (&ch)[2], const floatx4 (&ra)[4], floatx4 &bq, int kc, const floatx16 &init) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const floatx4 b = bq;
            const int nkc = g < 3 ? kc : (kc + 1 < NK ? kc + 1 : 0);
            bq = sB[bidx_kc(l32, nkc, 2 * ((g + 1) & 3) + h)];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const bool first = kc == 0 && g == 0 && t < 2;
                ch[t & 1] = __builtin_amdgcn_mfma_f32_32x32x2f32(ra[g][t], b[t],
                                                                 first ? (t == 0 ? init : zero16) : ch[t & 1], 0, 0, 0);
            }
        }
    };
    auto n16 = [](const floatx4 (&n)[4]) {
        floatx16 v;
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j) v[4 * g + j] = n[g][j];
        return v;
    };

    int col0;
    long r_lo, r_hi;
    decode_item<TC>(a, item, col0, r_lo, r_hi);
    fill_b(col0);
    if constexpr (MODE == kFilter) {
        if (tid < TC) s_qcnt[tid] = 0;
    }
    long rs = r_lo;
    bool act = rs + 64 * wr < r_hi;  // this wave's rows of the stage belong to the item
    EpiState st;
    item_begin<MODE, M, 1>(st, a, col0, 0, l32);
    // A chunks in flight: pf[0] is this step's, pf[j] the one j steps ahead
    floatx4 pf[PD][4];
#pragma unroll
    for (int j = 0; j < PD; ++j) load_a(pf[j], act ? rs : r_lo - 64 * wr, 0, j);
    __syncthreads();
    floatx4 bq = sB[bidx_kc(l32, 0, h)];

    floatx16 ch[2];      // the running half's two chains
    floatx16 res[2][1];  // each half's summed accumulators, for its epilogue
    floatx4 nrm[2][4];   // epilogue values (row norms) of each half's rows
    bool prev = false;   // the previous stage's second half is still to be evaluated
    bool pact = false;   // ... and belonged to the item

    auto epi = [&](const floatx16 (&ac)[1], const floatx4 (&n)[4], long srs, int hf, int g0, int g1, bool enable) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            if (g < g0 || g >= g1) continue;
            if constexpr (MODE == kFilter) {
                filter_group<M, kNtSlots, 1>(ac, n[g], st, a, 0, l32,
                                             (uint32_t)(srs - r_lo) + 64 * wr + 32 * hf + 8 * g + 4 * h, r_lo, col0,
                                             s_qcnt, s_slot, g, enable);
            } else if (enable) {
                dense_group<M, 1>(ac, n[g], st, a, 0, l32, srs + 64 * wr + 32 * hf + 8 * g + 4 * h, col0, g);
            }
        }
    };
    // per group: the next group's LDS read, then 1 MFMA and up to 2 VALU.  Placed in the MFMA block
    // (before the epilogue's branches), where the scheduler applies it
    auto interleave = [&]() {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
            }
        }
    };

    for (;;) {
        long nrs = rs + TR;
        int nitem = item, ncol0 = col0;
        long nlo = r_lo, nhi = r_hi;
        const bool item_end = nrs >= r_hi;
        bool more = true;
        if (item_end) {
            nitem = item + G;
            more = nitem < a.n_items;
            if (more) {
                decode_item<TC>(a, nitem, ncol0, nlo, nhi);
                nrs = nlo;
            }
        }
        // the rows this wave reads: its own, or (an idle wave) the item's first 64
        const long base = act ? rs : r_lo - 64 * wr;
        const bool nact = nrs + 64 * wr < nhi;
        const long nbase = nact ? nrs : nlo - 64 * wr;
        // ---- half 0: MFMAs into the chains; epilogue of the previous stage's half 1 ----
        load_n(nrm[0], base, 0);
        const floatx16 init0 = FUSE ? n16(nrm[0]) : zero16;
#pragma unroll
        for (int kc = 0; kc < NK; ++kc) {
            floatx4 nn[4];
            if (kc + PD < NK) load_a(nn, base, 0, kc + PD);
            else load_a(nn, base, 1, kc + PD - NK);
            __builtin_amdgcn_sched_barrier(0);
            mfma_step(ch, pf[0], bq, kc, init0);
            interleave();
            epi(res[1], nrm[1], rs - TR, 1, (4 * kc) / NK, (4 * (kc + 1)) / NK, prev && pact);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int j = 0; j + 1 < PD; ++j) pf[j][i] = pf[j + 1][i];
                pf[PD - 1][i] = nn[i];
            }
        }
        res[0][0] = ch[0] + ch[1];
        // ---- half 1: MFMAs into the chains; epilogue of this stage's half 0 ----
        load_n(nrm[1], base, 1);
        const floatx16 init1 = FUSE ? n16(nrm[1]) : zero16;
#pragma unroll
        for (int kc = 0; kc < NK; ++kc) {
            floatx4 nn[4];
            if (kc + PD < NK) load_a(nn, base, 1, kc + PD);
            else if (more) load_a(nn, nbase, 0, kc + PD - NK);  // the next stage's first chunks
            __builtin_amdgcn_sched_barrier(0);
            mfma_step(ch, pf[0], bq, kc, init1);
            interleave();
            epi(res[0], nrm[0], rs, 0, (4 * kc) / NK, (4 * (kc + 1)) / NK, act);
#pragma unroll
            for (int i = 0; i < 4; ++i) {  // past the last stage nn is unset, and no step uses it
#pragma unroll
                for (int j = 0; j + 1 < PD; ++j) pf[j][i] = pf[j + 1][i];
                pf[PD - 1][i] = nn[i];
            }
        }
        res[1][0] = ch[0] + ch[1];
        prev = true;
        pact = act;
        if (item_end) {
            // drain: this stage's half 1, then the item's candidates
            epi(res[1], nrm[1], rs, 1, 0, 4, act);
            if constexpr (MODE == kFilter) filter_flush<kNtSlots, TC>(a, col0, r_lo, s_qcnt, s_slot);
            if (!more) break;
            // every wave is past this item's MFMAs (the flush has a barrier; DENSE takes one here)
            if constexpr (MODE == kDense) __syncthreads();
            fill_b(ncol0);
            __syncthreads();
            bq = sB[bidx_kc(l32, 0, h)];
            item = nitem;
            col0 = ncol0;
            r_lo = nlo;
            r_hi = nhi;
            item_begin<MODE, M, 1>(st, a, col0, 0, l32);
            prev = false;
        }
        rs = nrs;
        act = nact;
    }
}

// ---- launch ----------------------------------------------------------------------------
static int grid_for(long n_items, int cap) {
    long g = n_items < cap ? n_items : cap;
    return (int)((g + 7) / 8 * 8);
}

// grid_cap: 2 workgroups per CU (the streaming kernel's residency); the resident-column
// kernel runs one 8-wave workgroup per CU.
template <int MODE, int M>
static void launch_scan(const ScanArgs &a, int grid_cap, hipStream_t s) {
    const int cus = grid_cap / 2;
    const int nk = a.dpad / kKChunk;
    if (nk <= 4) {
        const dim3 g(grid_for(a.n_items, cus)), b(512);
        switch (nk) {
            case 1: scan_launch((k_mfma_hs<MODE, M, 1>), g, b, 0, s, a); break;
            case 2: scan_launch((k_mfma_hs<MODE, M, 2>), g, b, 0, s, a); break;
            case 3: scan_launch((k_mfma_hs<MODE, M, 3>), g, b, 0, s, a); break;
            default: scan_launch((k_mfma_hs<MODE, M, 4>), g, b, 0, s, a); break;
        }
    } else if (nk % 4 == 0) {
        const dim3 g(grid_for(a.n_items, cus));
        if constexpr (MODE != kAssign) {
            switch (gemm_filter_cols(a.dpad) == kNtCols ? nk : 0) {  // the narrow-tile instantiations
                case 8: scan_launch((k_mfma_nt<MODE, M, 8>), g, dim3(512), 0, s, a); return;
                case 12: scan_launch((k_mfma_nt<MODE, M, 12>), g, dim3(512), 0, s, a); return;
                case 16: scan_launch((k_mfma_nt<MODE, M, 16>), g, dim3(512), 0, s, a); return;
                case 20: scan_launch((k_mfma_nt<MODE, M, 20>), g, dim3(512), 0, s, a); return;
                case 24: scan_launch((k_mfma_nt<MODE, M, 24>), g, dim3(512), 0, s, a); return;
                case 28: scan_launch((k_mfma_nt<MODE, M, 28>), g, dim3(512), 0, s, a); return;
                default: break;
            }
        }
        scan_launch((k_mfma_pnl<MODE, M>), g, dim3(512), 0, s, a);
    } else {
        const dim3 g(grid_for(a.n_items, 2 * cus)), b(256);
        scan_launch((k_mfma_stream<MODE, M>), g, b, 0, s, a);
    }
}

template <int MODE>
static void launch_metric(int metric, const ScanArgs &a, int grid_cap, hipStream_t s) {
    switch (metric) {
        case L2: launch_scan<MODE, L2>(a, grid_cap, s); break;
        case DOT: launch_scan<MODE, DOT>(a, grid_cap, s); break;
        default: launch_scan<MODE, COS>(a, grid_cap, s); break;
    }
}

void launch_gemm_filter(int metric, bool dense, long item_rows, const float *base, const float *bnorm,
                        const float *qry, const float *qnorm, const float *tau, int nq, int dpad, long row_begin,
                        long row_end, uint2 *cand, uint32_t *cnt, int cap, float anorm_max, float anorm_min,
                        int grid_cap, hipStream_t s) {
    if (nq <= 0 || row_end <= row_begin) return;
    ScanArgs a{};
    a.A = base;
    a.anorm = bnorm;
    a.B = qry;
    a.bnorm = qnorm;
    a.dpad = dpad;
    a.ncols = nq;
    a.n_ctiles = ceil_div(nq, gemm_filter_cols(dpad));
    a.item_rows = item_rows;
    a.row_begin = row_begin;
    a.row_end = row_end;
    const long n_chunks = (row_end - row_begin + a.item_rows - 1) / a.item_rows;
    a.n_items = (int)((long)a.n_ctiles * n_chunks);
    a.tau = tau;
    a.cand = cand;
    a.cnt = cnt;
    a.cap = cap;
    a.anorm_max = anorm_max;
    a.anorm_min = anorm_min;
    if (dense) launch_metric<kDense>(metric, a, grid_cap, s);
    else launch_metric<kFilter>(metric, a, grid_cap, s);
}

void launch_kmeans_assign(int metric, const float *cent, const float *cnorm, int kpad, const float *pts,
                          const float *pnorm, int n, int dpad, int32_t *assign, float *inertia, int32_t *pos,
                          int32_t *counts, const AssignCert &cert, int grid_cap, hipStream_t s) {
    if (n <= 0 || kpad <= 0) return;
    ScanArgs a{};
    a.A = cent;
    a.anorm = cnorm;
    a.B = pts;
    a.bnorm = pnorm;
    a.dpad = dpad;
    a.ncols = n;
    a.n_ctiles = ceil_div(n, kTileCols);
    a.n_items = a.n_ctiles;
    a.row_begin = 0;
    a.row_end = kpad;
    a.item_rows = kpad;
    a.assign = assign;
    a.inertia = inertia;
    a.pos = pos;
    a.counts = counts;
    a.err_coeff = cert.err_coeff;
    a.cmax = cert.cmax;
    a.fix = cert.fix;
    a.nfix = cert.nfix;
    a.devmax = cert.devmax;
    a.nrows_valid = cert.k > 0 ? cert.k : kpad;
    launch_metric<kAssign>(metric, a, grid_cap, s);
}

}  // namespace vh
