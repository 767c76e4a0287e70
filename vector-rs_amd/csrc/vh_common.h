// vh_common.h -- shared device helpers and internal launcher declarations.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace vh {

// ---- scan-kernel launches and their timing ------------------------------------------------
// A timed region (KernelTimer::begin .. end on one host thread) hands its event pair to the scan
// launches inside it, which attach the events to their own dispatches: the first records `start`
// as its kernel begins and each records `stop` as its kernel ends.  The pair then spans the scan
// kernels alone, as a kernel trace measures them, without the launch gaps and the fill kernels
// around them.  Outside a timed region (no pair pending) this is a plain launch.
struct TimedLaunch {
    hipEvent_t start = nullptr, stop = nullptr;
    bool used = false;  // some launch of the region took the start event
};
TimedLaunch &timed_launch_slot();  // this host thread's pending pair

template <typename F, typename... Args>
inline void scan_launch(F kernel, dim3 grid, dim3 block, uint32_t shm, hipStream_t s, Args... args) {
    TimedLaunch &t = timed_launch_slot();
    hipExtLaunchKernelGGL(kernel, grid, block, shm, s, t.used ? nullptr : t.start, t.stop, 0u, args...);
    if (t.stop) t.used = true;
}

enum Metric : int {
    L2 = 0, DOT = 1, COS = 2, L1 = 3, MINK = 4, LINF = 5, HAMF = 6, MAHA = 7, JACC = 8, HELL = 9,
    HAMMING_PACKED = 10  // internal: packed-bit codes (uint32 words), popcount distance
};

constexpr int kMaxK = 2048;          // VHIP_MAX_K
constexpr int kGemmSlotsReg = 48;    // LDS candidate slots per query and work item, register-fed MFMA kernel
constexpr int kGemmSlotsPanel = 24;  // same, panel MFMA kernel (dpad a multiple of 128 above 128)
constexpr int kGemmSlotsStream = 14; // same, streaming MFMA kernel (other dpad > 128)
constexpr int kGemmSlotsNarrow = 48; // same, narrow resident-tile MFMA kernel (see gemm_filter_cols)
constexpr int kKChunk = 32;          // K (dimension) chunk of the MFMA tiles
constexpr int kTileCols = 128;       // queries (or k-means points) per MFMA work item
constexpr int kNtCols = 32;          // queries per work item of the narrow resident-tile kernel
// Query columns per work item of the MFMA search kernel that serves rows of dpad floats: the
// narrow resident-tile kernel takes dpad a multiple of 128 from 256 to 896 (its 32 x dpad query
// tile stays in LDS), the others kTileCols.
inline bool gemm_narrow(int dpad) { return dpad % 128 == 0 && dpad >= 256 && dpad <= 896; }
inline int gemm_filter_cols(int dpad) { return gemm_narrow(dpad) ? kNtCols : kTileCols; }
// LDS candidate slots of the MFMA search kernel that serves rows of dpad floats
inline int gemm_slots(int dpad) {
    return dpad <= 128 ? kGemmSlotsReg
                       : (gemm_narrow(dpad) ? kGemmSlotsNarrow : (dpad % 128 == 0 ? kGemmSlotsPanel : kGemmSlotsStream));
}
// Batches of at most kSmallCols queries (one 32-query tile), or up to four tiles over a base of at
// most kSmallBaseRows rows (where every search is bound by launches, not by scanned pairs) or of
// rows of at most 128 floats, with rows of at most kSmallMaxDpad floats take the small-batch MFMA
// scan (knn_small.hip), which spreads every round over all CUs.  (1M x 128 integer squared L2,
// k = 10: 64 queries 245 us against 432 on the batch kernels, whose 128-query tiles run half
// empty, and 128 queries 411 against 440.)
constexpr int kSmallCols = 32;
constexpr int kSmallMaxDpad = 1024;
constexpr size_t kSmallBaseRows = 262144;
inline bool small_batch(int nq, int dpad, size_t n) {
    return dpad <= kSmallMaxDpad &&
           (nq <= kSmallCols || (nq <= 4 * kSmallCols && (n <= kSmallBaseRows || dpad <= 128)));
}
constexpr int kRowAlign = 256;       // row counts of MFMA row operands and round boundaries
                                     // are multiples of this (the largest MFMA stage)

// s_waitcnt immediate that waits until at most n (< 16) vector memory operations are
// outstanding, leaving the export and LDS counters unconstrained.
#define VH_VMCNT(n) (((n) & 15) | (7 << 4) | (15 << 8))

// Global-memory views of device pointers.  Accesses through them compile to global_* rather
// than flat_* instructions: a flat access counts against both the vector-memory and the LDS
// wait counters, so one pending flat store makes the compiler wait for every outstanding load
// before the next LDS or register use.
typedef __attribute__((address_space(1))) uint32_t gu32;
typedef __attribute__((address_space(1))) uint64_t gu64;
// the 8 bytes of a uint2 {x, y} as one little-endian 64-bit word
__device__ __forceinline__ uint64_t pack_u2(uint32_t x, uint32_t y) { return (uint64_t)y << 32 | x; }

// Workgroup barrier that publishes LDS data only: the wave's LDS operations complete, its
// global->LDS DMAs in flight do not (a wave waits for the chunks it publishes with vmcnt first).
// __syncthreads() would wait for every DMA in flight, since they write LDS.  The memory clobber
// keeps the compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Global->LDS DMA of 16 (4) bytes per lane from `src` to LDS byte address m0_base + 16 (4) x lane.
// Written as asm so that the compiler neither counts the DMA among the loads it waits for nor
// makes later LDS accesses wait for it: the caller waits with vmcnt before reading the data (M0
// is restored; the DMA takes its value when issued).
__device__ __forceinline__ void dma_lds16(const void *src, uint32_t m0_base) {
    uint32_t sv;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(sv)
                 : "v"(src), "s"(m0_base)
                 : "memory");
}
__device__ __forceinline__ void dma_lds4(const void *src, uint32_t m0_base) {
    uint32_t sv;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(sv)
                 : "v"(src), "s"(m0_base)
                 : "memory");
}

// Maps a float score (smaller is better) to an unsigned key with the same order.
__host__ __device__ inline uint32_t score_key(float s) {
    uint32_t u = __builtin_bit_cast(uint32_t, s);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// Every NaN score (a row holding a NaN or an infinity) as the positive quiet NaN, whose key
// follows that of +inf: such a row ranks after every other whatever the sign bit of the NaN that
// reached it.
__host__ __device__ inline float nan_last(float s) { return s == s ? s : __builtin_nanf(""); }
__host__ __device__ inline float key_score(uint32_t k) {
    uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __builtin_bit_cast(float, u);
}

// Rounding bound of a sum of n fp32 terms in any order: gamma_n = n u / (1 - n u), u = 2^-24.
inline double gamma_n(double n) { return n * 0x1p-24 / (1.0 - n * 0x1p-24); }
// Coefficients of the GEMM-form selection error bound (2 % slack on top):
//  * squared L2 on shifted operands q' = fl(q - mu), x' = fl(x - mu): the shifts (2u), the norms
//    and the MFMA sum (2 gamma_{D+2}) and the epilogue add (u) give
//    |s~ - ||q - x||^2| <= c (||q'|| + ||x'||)^2;
//  * dot product: |s~ - q.x| <= gamma_D sum |q_i x_i| <= c ||q|| ||x||;
//  * cosine of rows normalised in fp32: the two normalisations (gamma_D + 6u) and the sum
//    (gamma_D) give an absolute bound c.
inline float sel_err_coeff(int metric, int dpad) {
    const double u = 0x1p-24, g = gamma_n(dpad + 2.0);
    const double c = metric == 0 ? 2.0 * g + 4.0 * u : (metric == 1 ? g : 2.0 * g + 8.0 * u);
    return (float)(c * 1.02);
}
// Entries kept per query by a GEMM-metric search: the k best by the GEMM-form score plus up to
// this many within the selection error bound of the k-th, which the final direct-form pass
// re-ranks.
inline int margin_cap(int k) { return k < 16 ? 16 : (k > 256 ? 256 : k); }
constexpr int kMaxKeep = kMaxK + 256;

inline int ceil_div(long a, long b) { return (int)((a + b - 1) / b); }
inline size_t round_up(size_t a, size_t b) { return (a + b - 1) / b * b; }

// ---- launchers (defined in the .hip files) ----------------------------------
// Candidate lists: every filter kernel appends (score key, row) pairs where `row` is the
// position in the resident (permuted) base; k_topk_merge maps positions to vector ids.

// knn_gemm.hip
// Row preparation.  Rows [0, n) of `dim` floats are copied into rows of `dpad` floats (zero
// fill), in the order given by `perm` (out row p = in row perm[p]) or identity if perm is null;
// `shift` (dpad floats, may be null) is subtracted from every element first; then the row is
// optionally sqrt(|x|)-transformed (transform 1, Hellinger) and L2-normalised (normalize 1).
// Rows [n, n_out) are filled with `pad_fill`.  norm_kind 1 writes per-row squared L2 norms, 2 L2
// norms (before normalisation).  With no shift, norm_kind 0, transform 0 and normalize 0 the
// copy is bit-exact, so it also moves packed uint32 codes.
//  * raw_out (may be null): the rows before the shift, padded the same way;
//  * nonint (may be null): set to 1 when some value of a real row is not an integer;
//  * err (may be null): per-row bound of the selection error of the GEMM-form score of that row
//    (as a query) against any base row, err_mode 1 squared L2 (err_coeff (||q'|| + sqrt(err_nmax))^2),
//    2 dot product (err_coeff ||q|| sqrt(err_nmax)), 3 cosine (err_coeff); 0 when every operand
//    is an integer (the row's and, by base_integral, the base's) and every partial sum stays
//    below 2^24, where the fp32 GEMM is exact.
struct RowPrep {
    const float *in = nullptr;
    size_t n = 0, n_out = 0;
    int dim = 0, dpad = 0;
    const uint32_t *perm = nullptr;
    const float *shift = nullptr;
    float *out = nullptr;
    float *raw_out = nullptr;
    float *norm = nullptr;
    int norm_kind = 0, transform = 0, normalize = 0;
    float pad_fill = 0.0f;
    uint32_t *nonint = nullptr;
    uint32_t *inexact = nullptr;  // (may be null) set to 1 when some shifted value v = fl(x - shift)
                                  // does not give back x as v + shift
    float *err = nullptr;
    int err_mode = 0;
    float err_coeff = 0.0f, err_nmax = 0.0f;
    int base_integral = 0;
    // (tau may be null) a search run's per-query state, reset in the same launch as
    // launch_topk_init would reset it for the n rows: a query batch's preparation and the reset
    // of its run, one launch instead of two on a launch-bound small search.
    struct RunInit {
        float *tau = nullptr;
        uint32_t *have = nullptr, *cnt = nullptr, *flags = nullptr, *mflag = nullptr, *nflag = nullptr;
        uint32_t *pad = nullptr;
        uint32_t cnt0 = 0;
    } init;
};
void launch_rows_prep(const RowPrep &a, hipStream_t s);
// Short form: no shift, raw copy, integer check or error bound.
void launch_rows_prep(const float *in, size_t n, size_t n_out, int dim, int dpad, const uint32_t *perm, float *out,
                      float *norm, int norm_kind, int transform, int normalize, float pad_fill, hipStream_t s);
// Per-dimension shift of n rows of `dim` floats (row-major, contiguous): the column means over
// the finite values, rounded to integers when every finite value is an integer (so that shifted
// integer data stays integer), into shift[0, dpad) (zeros past dim); nonint (device u32) is set
// to 1 when some finite value is not an integer.  partial: col_shift_scratch_bytes(dim) bytes of
// device scratch.
size_t col_shift_scratch_bytes(int dim);
void launch_col_shift(const float *x, size_t n, int dim, int dpad, double *partial, uint32_t *nonint, float *shift,
                      hipStream_t s);
// One round of the fused MFMA distance + threshold filter over base rows [row_begin, row_end)
// (row_begin a multiple of 256; rows past the real base are NaN padding up to a multiple of 256).
// `base` has its rows padded to a multiple of 256 with NaN rows; `qry` has nq rows padded to a
// multiple of 128.  anorm_max / anorm_min: extremes of bnorm over the real rows.  item_rows (a
// multiple of 256): base rows per work item.  dense: write every score of rows < row_end to
// cand[q * cap + (row - row_begin)] instead of filtering (needs row_end - row_begin <= cap; the
// caller sets cnt).  grid_cap: number of workgroups of the persistent grid.
void launch_gemm_filter(int metric, bool dense, long item_rows, const float *base, const float *bnorm,
                        const float *qry, const float *qnorm, const float *tau, int nq, int dpad, long row_begin,
                        long row_end, uint2 *cand, uint32_t *cnt, int cap, float anorm_max, float anorm_min,
                        int grid_cap, hipStream_t s);
// The same round for a small batch (small_batch(nq, dpad)): one wave per 32-row block against the
// batch's 32-query tile, DENSE or FILTER as above, squared L2, dot product or cosine.  plan_rows:
// the length of the round this launch belongs to (a round cut into pieces passes its whole
// length), which alone sets how the K range is split over the waves, and so the order in which
// each score's partial sums meet: a score comes out the same whether its round ran whole or cut.
// FILTER launches count each query's candidates on pad[q * kSmallPadStride] (one 128-byte line
// per query; pad holds min(nq, kSmallPadQueries) counters, zero before the round) instead of the
// run's cnt[q], and the round's merge reads them there (launch_topk_merge with that stride);
// DENSE launches write row - row_begin and leave the counts to the caller.
constexpr int kSmallPadStride = 32, kSmallPadQueries = 4 * kSmallCols;
void launch_small_scan(int metric, bool dense, const float *base, const float *bnorm, const float *qry,
                       const float *qnorm, const float *tau, int nq, int dpad, long row_begin, long row_end,
                       long plan_rows, uint2 *cand, uint32_t *pad, int cap, int grid_cap, hipStream_t s);

// Certification of the MFMA k-means assignment: each point's best score must beat its second
// best by more than twice the point's selection error bound (err_coeff times the norms, with
// *cmax the largest centroid norm value), else the point goes to fix[atomicAdd(nfix)] and takes
// no ticket.  Squared L2 records in devmax[c] (u32 bits of a non-negative float, atomic max) a
// bound of |x_d - c_d| over the certified points of cluster c.
struct AssignCert {
    float err_coeff = 0.0f;
    const float *cmax = nullptr;
    int32_t *fix = nullptr;
    uint32_t *nfix = nullptr;
    float *devmax = nullptr;
    int k = 0;  // real centroid rows (the rest of kpad is padding); 0: all kpad rows
};
// MFMA k-means assignment (knn_gemm.hip); metric L2 / DOT / COS.  `cent` has kpad rows
// (a multiple of 128; padding rows are NaN, or for squared L2 zero rows of norm FLT_MAX), `pts` n
// rows padded to a multiple of 128 (zeros).
// cnorm / pnorm hold squared norms for L2 and dot product and L2 norms for COS.  Certified
// points get assign, pos (ticket in counts) and, for dot / cosine, inertia (-dot, 1 - cos).
void launch_kmeans_assign(int metric, const float *cent, const float *cnorm, int kpad, const float *pts,
                          const float *pnorm, int n, int dpad, int32_t *assign, float *inertia, int32_t *pos,
                          int32_t *counts, const AssignCert &cert, int grid_cap, hipStream_t s);

// topk.hip
// Resets a run's per-query state: tau = +inf, have = flags = mflag = 0, cnt = cnt0 (the first
// round's rows when that round is dense), and the two flag counters; with `pad` (may be null) also
// the small-batch scan's counters pad[q * kSmallPadStride] for q < min(nq, kSmallPadQueries).
void launch_topk_init(int nq, float *tau, uint32_t *have, uint32_t *cnt, uint32_t *flags, uint32_t *mflag,
                      uint32_t *nflag, uint32_t cnt0, uint32_t *pad, hipStream_t s);
// Merges each query's candidates into its running best entries (row stride kc of topk).  A query
// with qerr[q] > 0 (qerr may be null: all 0) keeps its kc best entries and filters later rounds at
// tau = min(kc-th score, k-th score + 2 qerr[q]), so the final entries hold every row whose score
// lies within 2 qerr of the k-th; mflag[q] (may be null) is set when that margin may have been cut
// by the capacity kc.  Others keep k entries and filter at the k-th score.  mcount (non-null in a
// run's last round only): incremented once per query whose margin flag stands at the end of the
// round, overflowed queries excepted.  wide: 1024 threads per query instead of 256 (a dense round
// of many rows).
// cnt: query q's candidate count is cnt[q * cnt_stride] (1, or kSmallPadStride for a small-batch
// FILTER round's spread counters), cleared by the merge.
void launch_topk_merge(int nq, int k, int kc, const uint2 *cand, uint32_t *cnt, int cnt_stride, int cap,
                       const uint32_t *perm, unsigned long long *topk, uint32_t *have, float *tau, uint32_t *flags,
                       uint32_t *nflagged, const float *qerr, uint32_t *mflag, uint32_t *mcount, bool wide,
                       hipStream_t s);
// Where the final kernel of a search (refine or finalize) copies the two flag counters src[0..1]:
// host = pinned host memory, or null for no copy.
struct FlagPublish {
    const uint32_t *src = nullptr;
    uint32_t *host = nullptr;
};
// Writes results: out_ids[q*ostride + j], out_dist[...] for j < have[q]; distance is the
// metric value recovered from the score (negated for similarities, transformed for
// Minkowski / Mahalanobis / Hellinger).  Entries past have[q] are set to UINT32_MAX / NaN.
// kc is the stride of topk (kept entries per query); kout <= ostride entries are written per
// query (kout may exceed k when k was clamped to the number of base rows).
void launch_topk_finalize(int nq, int kc, int kout, int metric, const unsigned long long *topk,
                          const uint32_t *have, uint32_t *out_ids, float *out_dist, uint32_t *out_dist_u32,
                          int ostride, const FlagPublish &pub, hipStream_t s);
// GEMM metrics: recompute the kept distances in direct form, re-sort by (distance, id) and
// write the best k (same output contract as launch_topk_finalize; out_dist required).  Entries
// past the k-th count only when their GEMM-form score is within 2 qerr[q] of the k-th.  `qrows` /
// `base` are the unshifted queries and resident rows, or (shift non-null, squared L2) base +
// shift gives back the unshifted rows exactly; qnorm / bnorm are the original L2 norms (cosine
// zero-norm guard; unused for the other metrics).
void launch_topk_refine(int nq, int k, int kc, int kout, int metric, const float *qrows, const float *base,
                        const float *shift, const uint32_t *inv_perm, int dpad, const float *qnorm, const float *bnorm,
                        const unsigned long long *topk, const uint32_t *have, const float *qerr, uint32_t *out_ids,
                        float *out_dist, int ostride, const FlagPublish &pub, hipStream_t s);
// Number of nonzero flags among flags[0, n) into *count (device).
void launch_count_flags(const uint32_t *flags, int n, uint32_t *count, hipStream_t s);
// Copies the kept entries of re-run queries (row r, stride ks) back to rows idx[r] (stride kd)
// with their counts and margin flags (src_mflag null: flags cleared).
void launch_scatter_topk(const unsigned long long *src, int ks, const uint32_t *src_have, const uint32_t *src_mflag,
                         const uint32_t *idx, int m, unsigned long long *dst, int kd, uint32_t *dst_have,
                         uint32_t *dst_mflag, hipStream_t s);
// dst row r (width floats) = src row idx[r] (row stride width), for r < rows.
void launch_gather_rows(const float *src, const uint32_t *idx, size_t rows, int width, float *dst, hipStream_t s);
// hamming.hip
int hamming_word_pad(int words);
// fp4 matrix-core path of packed Hamming (hamming_mfma.hip): codes of wpad words expanded to one
// fp4 value per bit, ham_mfma_row_bytes(wpad) bytes per row (32-bit codes padded to 64 bits)
size_t ham_mfma_rows(size_t n);
bool ham_mfma_supported(int wpad);
size_t ham_mfma_row_bytes(int wpad);
void launch_ham_expand(const uint32_t *src, size_t rows, int wpad, int wstride, size_t rows_out, bool tiled,
                       int8_t *dst, hipStream_t s);
void launch_ham_mfma(bool dense, long item_rows, const int8_t *base8, const int8_t *qry8, int wpad,
                     const float *tau, int nq, long row_begin, long row_end, uint2 *cand, uint32_t *cnt, int cap,
                     int grid_cap, hipStream_t s);
// Filter rounds of codes up to 256 bits (ham_wide_supported) with many queries: work items of
// ham_wide_cols() query columns held in registers, the base through an LDS ring, and
// ham_wide_slots() LDS candidate slots per query and item.  Rows of qry8 are allocated up to a
// multiple of 128; base row starts and item_rows are multiples of 64.
bool ham_wide_supported(int wpad);
constexpr int ham_wide_cols() { return 1024; }
constexpr int ham_wide_slots() { return 8; }
void launch_ham_mfma_wide(long item_rows, const int8_t *base8, const int8_t *qry8, int wpad, const float *tau, int nq,
                          long row_begin, long row_end, uint2 *cand, uint32_t *cnt, int cap, int grid_cap,
                          hipStream_t s);
void launch_hamming_filter(const uint32_t *codes, const uint32_t *qry, const float *tau, int nq, int wpad,
                           long row_begin, long row_end, uint2 *cand, uint32_t *cnt, int cap, int grid_cap,
                           hipStream_t s);
// knn_valu.hip
void launch_kmeans_assign_valu(int metric, const float *cent, int k, const float *pts, int n, int dpad,
                               int32_t *assign, float *inertia, int32_t *pos, int32_t *counts, int grid_cap,
                               hipStream_t s);
// Fix-up of the MFMA assignment (metric L2 / DOT / COS): the listed points (fix[0, *nfix)) get the
// direct-form argmin over the k unshifted centroids (rows of dpad floats) on the unshifted points,
// their tickets, and inertia (dot / cosine) or the deviation bound (squared L2).  best: scratch of
// one u64 per listed point.
void launch_kmeans_fix(int metric, const float *pts, int dpad, const int32_t *fix, const uint32_t *nfix,
                       const float *cent, int k, unsigned long long *best, int32_t *assign, float *inertia,
                       int32_t *pos, int32_t *counts, float *devmax, int grid_cap, hipStream_t s);
// Direct-form assignment of small point sets (metric L2 / DOT / COS): every point gets what the
// fix-up gives a listed point (argmin over the k unshifted centroids, lowest index on ties, on
// the unshifted points), its ticket, and inertia (dot / cosine) or the deviation bound (squared
// L2).  kmeans_assign_small_ok says whether a shape takes this path.
bool kmeans_assign_small_ok(int n, int k, int dpad, int cus);
void launch_kmeans_assign_small(int metric, const float *pts, int dpad, int n, const float *cent, int k,
                                int32_t *assign, float *inertia, int32_t *pos, int32_t *counts, float *devmax,
                                hipStream_t s);
// shift (may be null): added to every base value as the tiles are read (the direct-form pass of
// squared L2 over shifted rows that give back the unshifted ones exactly).
void launch_valu_filter(int metric, const float *base, const float *shift, const float *qry, const float *tau, int nq,
                        int dim, int dpad, long row_begin, long row_end, uint2 *cand, uint32_t *cnt, int cap,
                        int grid_cap, hipStream_t s);
// Fills count floats (32-bit words) with v.  Kernels rather than hipMemsetAsync, so a caller may
// capture the engines' work in a HIP graph.
void launch_fill(float *p, size_t count, float v, hipStream_t s);
void launch_fill_u32(uint32_t *p, size_t count, uint32_t v, hipStream_t s);

}  // namespace vh
