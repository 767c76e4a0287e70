// knn_engine.hip -- CudaKnnEngine / DistributedKnnEngine replacements behind the C ABI.
//
// CudaKnnEngine::with_ordinal (vector-cuda/src/knn.rs:90-140) computed norms and an SoA
// transpose on one host thread and kept a host copy.  Here the base is uploaded once
// through pinned staging and laid out on the GPU: rows in a fixed pseudo-random order
// (so every prefix of the resident base is an unbiased sample of it), padded to a
// multiple of 32 floats, the row count padded to a multiple of 256 with NaN rows, with
// per-row norms computed on the device (cosine rows are stored L2-normalised).
//
// search_batch (knn.rs:151-310) materialised the Q x N distance matrix.  Here a search
// is a sequence of rounds over geometrically growing row ranges of the permuted base:
// the first round keeps every row, later rounds keep only rows whose score is <= the
// k-th best score found so far (see topk.hip).  A query whose candidate list overflows
// is re-run with a capacity equal to the largest round, which cannot overflow.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>

#include "vh_runtime.h"

namespace vh {

constexpr uint64_t kPermSeed = 0x5EEDB45E00000001ull;
constexpr size_t kQueryBatch = 16384;

bool is_gemm_metric(int m) { return m == L2 || m == DOT || m == COS; }

// Bump allocator over one device region: every buffer of a search batch is carved from it, so
// a batch costs one growable workspace buffer (or none, in the allocation-free entry point).
// With a null base it only measures: `used` is then the bytes the same carve sequence needs.
struct Arena {
    uintptr_t base = 0;
    size_t size = SIZE_MAX, used = 0;
    Arena() = default;
    Arena(void *p, size_t bytes) : base((uintptr_t)p), size(bytes) {}
    template <class T>
    T *take(size_t count) {
        const size_t b = round_up(std::max<size_t>(count * sizeof(T), 1), 256);
        T *r = (used + b <= size) ? (T *)(base + used) : nullptr;
        used += b;
        return r;
    }
    bool fits() const { return used <= size; }
};

// Buffers of one run of the search rounds over nq prepared queries.
struct RunBufs {
    uint2 *cand = nullptr;                 // nq x cap candidates
    unsigned long long *topk = nullptr;    // nq x kc kept entries
    float *tau = nullptr;                  // nq thresholds
    uint32_t *have = nullptr, *cnt = nullptr, *flags = nullptr, *mflag = nullptr;  // nq each
    uint32_t *nflag = nullptr;             // 2 counters
    int8_t *q8 = nullptr;                  // expanded query codes (packed Hamming on fp4 MFMA)
    uint32_t *spad = nullptr;              // the small-batch scan's spread counters (launch_small_scan)
};

struct Workspace {
    DevBuf arena;
    DevBuf hq, hi, hd;  // the host-buffer path's device copies of queries and results (grow-only)
};

}  // namespace vh

struct vhip_knn {
    int dev = 0;
    size_t n = 0, n_pad = 0, dim = 0, dpad = 0;
    int metric = 0;
    float norm_max = 0.0f, norm_min = 0.0f;  // extremes of the per-row norm values
    int grid_cap = 512;
    hipStream_t stream = nullptr;
    vh::DevBuf base, norm, perm, inv_perm;
    // Squared L2: the rows are stored minus a per-dimension shift (the column means, integers for
    // integer data), which keeps the norm form well conditioned on data away from the origin.  The
    // direct-form passes need the unshifted rows: when every shifted value v gives back its x
    // exactly as v + shift (integer data with an integer shift), they add the shift as they read;
    // otherwise `raw` holds the unshifted rows (same order and padding).
    vh::DevBuf shift, raw;
    bool shifted = false;
    bool integral = false;    // every base value is an integer
    float err_coeff = 0.0f;   // selection error coefficient of the GEMM-form score
    uint32_t *flags_host = nullptr;  // pinned, coherent: the flagged-query counts of the running search
    vh::DevBuf base8;  // packed Hamming on the fp4 matrix cores: one +1/-1 nibble per code bit
    bool ham8 = false;
    bool ham_wide = false;  // filter rounds may use the 1024-column fp4 kernel (codes <= 256 bits)
    std::mutex mu;
    vh::Workspace ws;
    vh::PinnedStager stager;
    vh::KernelTimer timer;
    ~vhip_knn() {
        if (stream) {
            (void)hipSetDevice(dev);
            (void)hipStreamSynchronize(stream);
            (void)hipStreamDestroy(stream);
        }
        if (flags_host) (void)hipHostFree(flags_host);
    }
};

namespace vh {

// Search rounds.  Round 0 scores rows [0, b0) with b0 about 20 k, the first 256-row multiple
// at or above it (all rows when the base has at most max(2048, 32 k)): for the GEMM metrics
// densely (every score written, no atomics), for the others through the filter with tau = +inf.
// Every later round covers about 4 times the rows seen so far (the growth factor, see
// kRoundGrowth) and keeps only rows scoring <= tau, the k-th best so far.  Because the base rows
// are in a pseudo-random order, round i passes about k * (rows_i / seen_i) ~ 3 k candidates per
// query at a rate p_i = k / seen_i per scored pair.  item_rows of the MFMA filter is sized so that a work
// item's expected passes per query, item_rows * p_i, stay at most a third of the LDS slots.
struct Round {
    long rb, re;
    bool dense;
    long item_rows;  // the slot rule's length, capped at 8192 rows
    long slot_rows;  // the slot rule's length alone
    long plan_rows = 0;  // a piece of a cut round (split_rounds): the whole round's rows
};

// Round growth: each round covers `growth` times the rows seen so far.  A round passes about
// k (growth - 1) candidates per query, so a smaller factor passes fewer in all (the filter's
// appends and the merges' sorts) at the cost of more launches and merges.  4 measured best:
// squared L2 1M x 128, Q = 10k, k = 100: 20.0 ms against 20.3 at 8 (3 alike); L1 500k x 128,
// Q = 4096: 13.3 ms against 13.8 (3 slower); fp4 Hamming 10M x 256 bits: 9.25 against 9.56
// (2 slower).
constexpr int kRoundGrowth = 4;

// Small batches (`small`: at most kSmallCols queries on the GEMM metrics) pay mostly for launches
// and merges, not for scanned pairs: their first, dense round covers kSmallDenseRows rows (all of a
// base of up to twice that), and the rest follows in one filter round when its expected passes per
// query, k (n - seen) / seen, stay within a quarter of the candidate capacity, else in rounds growing
// 16 times.  (1M rows at k = 10: 8,192 rows, then the other 991,808 with about 1,200 passes; at
// k = 100 three rounds.)  A larger first round costs more in its merge (32,768 rows: 27 us against
// about 12) than the fewer passes save.
constexpr size_t kSmallDenseRows = 8192;

static std::vector<Round> plan_rounds(size_t n, size_t k, bool gemm, int dpad, int growth, bool small = false) {
    std::vector<Round> r;
    if (n == 0) return r;
    const size_t kk = std::max<size_t>(k, 1);
    size_t b0 = std::min(n, round_up(std::max<size_t>(256, 20 * kk), kRowAlign));
    // A base within the candidate capacity's floor (round_cap) is scored in one dense round: its
    // later rounds would cost more launches than rows (the IVF coarse probe: 1,024 centroids).
    if (n <= std::max<size_t>(2048, 32 * kk)) b0 = n;
    if (small) b0 = n <= 2 * kSmallDenseRows ? n : std::max(b0, kSmallDenseRows);
    r.push_back({0, (long)b0, gemm, (long)kRowAlign, (long)kRowAlign});
    const int slots = gemm_slots(dpad);
    const size_t cap_floor = std::max<size_t>({2048, 32 * kk, b0});
    size_t seen = b0;
    while (seen < n) {
        size_t e = std::min(n, round_up(seen * growth, kRowAlign));
        if (small) e = kk * (n - seen) / seen <= cap_floor / 4 ? n : std::min(n, round_up(seen * 16, kRowAlign));
        const size_t slot_item = std::max<size_t>(kRowAlign, (size_t)slots * seen / (3 * kk) / kRowAlign * kRowAlign);
        const size_t item = std::min<size_t>(8192, slot_item);
        r.push_back({(long)seen, (long)e, false, (long)item, (long)slot_item});
        seen = e;
    }
    return r;
}

// Work-item rows for an MFMA filter round (one workgroup per CU): among multiples of `step` up to
// the slot-derived `cap_item`, the one with the least estimated time, i.e. the fewest
// item-rounds over the resident workgroups times the item length (plus a per-item cost of
// about 64 rows for the tile load and flush).  Larger items win ties.
static long balanced_item(long cap_item, long rows, int n_ctiles, int wgs, long step = kRowAlign) {
    cap_item = std::max(step, cap_item / step * step);
    long best = cap_item;
    double best_cost = 0.0;
    for (long it = cap_item; it >= step; it -= step) {
        const long items = (rows + it - 1) / it * n_ctiles;
        const double cost = (double)((items + wgs - 1) / wgs) * (double)(it + 64);
        if (it == cap_item || cost < best_cost * 0.999) {
            best_cost = cost;
            best = it;
        }
    }
    return best;
}

// Candidate capacity per query and round: the dense round's rows, and room for several times
// the ~3 k expected passes of a filter round.  A query that still overflows is re-run with a
// capacity equal to the largest round.

static int round_cap(size_t n, size_t k, bool gemm, int dpad, bool small) {
    size_t cap = std::max<size_t>(2048, 32 * std::max<size_t>(k, 1));
    for (const Round &r : plan_rounds(n, k, gemm, dpad, kRoundGrowth, small))
        if (r.rb == 0) cap = std::max(cap, (size_t)(r.re - r.rb));
    return (int)round_up(cap, kRowAlign);
}

// The engine's pseudo-random row order (positions p -> base rows perm[p], so that every round
// scores a uniform sample of the base): a 4-round Feistel network over the 2^m >= n codes (m
// even), cycle-walked back into [0, n).  The walk from x follows x's own cycle, which returns to
// x < n, so it ends; with 2^m < 4n it takes fewer than 4 steps on average.  The round function
// is the "lowbias32" integer hash (Chris Wellons).  Built on the device, with the inverse for the
// GEMM metrics' refine, so engine creation does no host shuffle and no extra upload.
struct RowShuffle {
    uint32_t half_bits, mask;
    uint32_t key[4];
};

__device__ __forceinline__ uint32_t shuffle_code(uint32_t x, const RowShuffle &f) {
    uint32_t l = x >> f.half_bits, r = x & f.mask;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t h = r ^ f.key[i];
        h ^= h >> 16;
        h *= 0x7feb352du;
        h ^= h >> 15;
        h *= 0x846ca68bu;
        h ^= h >> 16;
        const uint32_t nr = (l ^ h) & f.mask;
        l = r;
        r = nr;
    }
    return (l << f.half_bits) | r;
}

// The position index is 64-bit: with n close to 2^32 a 32-bit index stepping by the grid size
// would wrap below n and never end.
__global__ __launch_bounds__(256) void k_row_shuffle(uint32_t n, RowShuffle f, uint32_t *__restrict__ perm,
                                                     uint32_t *__restrict__ inv) {
    for (uint64_t p = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; p < n; p += (uint64_t)gridDim.x * blockDim.x) {
        uint32_t x = (uint32_t)p;
        do {
            x = shuffle_code(x, f);
        } while (x >= n);
        perm[p] = x;
        if (inv) inv[x] = (uint32_t)p;
    }
}

// Per-block maximum and minimum of the finite values of x[0, count): the host folds the
// gridDim.x pairs.  A row holding a NaN or an infinity has a non-finite norm; its scores are NaN
// or infinite and never pass a filter, so it takes no part in the bounds the extremes feed.
__global__ __launch_bounds__(256) void k_minmax_partial(const float *__restrict__ x, size_t count,
                                                        float *__restrict__ pmax, float *__restrict__ pmin) {
    __shared__ float rmax[256], rmin[256];
    float mx = 0.0f, mn = INFINITY;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < count; i += (size_t)gridDim.x * blockDim.x) {
        const float v = x[i];
        if (__builtin_isfinite(v)) {
            mx = fmaxf(mx, v);
            mn = fminf(mn, v);
        }
    }
    rmax[threadIdx.x] = mx;
    rmin[threadIdx.x] = mn;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) {
            rmax[threadIdx.x] = fmaxf(rmax[threadIdx.x], rmax[threadIdx.x + o]);
            rmin[threadIdx.x] = fminf(rmin[threadIdx.x], rmin[threadIdx.x + o]);
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        pmax[blockIdx.x] = rmax[0];
        pmin[blockIdx.x] = rmin[0];
    }
}

constexpr int kMinMaxParts = 1024;

static int build_row_order(vhip_knn *E, size_t n, bool with_inverse) {
    int m = 2;
    while (m < 32 && (1ull << m) < n) ++m;
    m += m & 1;
    RowShuffle f;
    f.half_bits = (uint32_t)(m / 2);
    f.mask = (1u << f.half_bits) - 1u;
    uint64_t st = kPermSeed;
    for (int i = 0; i < 4; ++i) f.key[i] = (uint32_t)splitmix64(st);
    VH_CHECK(E->perm.ensure(E->dev, n * sizeof(uint32_t)));
    if (with_inverse) VH_CHECK(E->inv_perm.ensure(E->dev, n * sizeof(uint32_t)));
    const unsigned blocks = (unsigned)std::min<size_t>(4096, (n + 255) / 256);
    hipLaunchKernelGGL(k_row_shuffle, dim3(blocks), dim3(256), 0, E->stream, (uint32_t)n, f, E->perm.as<uint32_t>(),
                       with_inverse ? E->inv_perm.as<uint32_t>() : nullptr);
    VH_HIP(hipGetLastError());
    return VHIP_OK;
}

// Packed Hamming keeps a second copy of the codes expanded to one fp4 value per bit (4x the packed
// bytes) for the matrix-core kernel.  The copy is made when it takes at most half of the device
// memory free at creation (the rest stays for search workspaces); otherwise the engine scans the
// packed codes with the popcount kernel.  VHIP_HAMMING_KERNEL = "popcount" or "fp4" overrides
// the choice for engines created afterwards, and "fp4-tile" takes the fp4 copy but keeps every
// round on the 128-column tile kernel (all kernels give identical results).
static bool want_fp4_copy(size_t bytes) {
    if (const char *env = std::getenv("VHIP_HAMMING_KERNEL")) {
        if (std::strcmp(env, "popcount") == 0) return false;
        if (std::strcmp(env, "fp4") == 0 || std::strcmp(env, "fp4-tile") == 0) return true;
    }
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return bytes <= free_b / 2;
}

// One batch of prepared queries: the rows the scan kernels read (shifted for squared L2), their
// norms and selection error bounds (null for the non-GEMM metrics), and the unshifted rows of
// the direct-form passes (qpad itself when the engine keeps no shift).
struct QueryRows {
    const float *qpad, *qnorm, *qerr, *qraw;
};

// Base rows of the direct-form passes: the unshifted copy when there is one, else the scan rows,
// plus direct_shift(E) when those are shifted (then base + shift is the unshifted row, exactly).
static const float *direct_rows(const vhip_knn *E) { return E->raw.p ? E->raw.as<float>() : E->base.as<float>(); }
static const float *direct_shift(const vhip_knn *E) { return E->shifted && !E->raw.p ? E->shift.as<float>() : nullptr; }

// Carves the buffers of one run over nq queries: kc kept entries and (with_cand) cap candidates
// per query.
static RunBufs carve_run(Arena &A, const vhip_knn *E, size_t nq, int kc, int cap, bool with_cand) {
    RunBufs B;
    if (with_cand) B.cand = A.take<uint2>(nq * (size_t)cap);
    B.topk = A.take<unsigned long long>(nq * (size_t)kc);
    B.tau = A.take<float>(nq);
    B.have = A.take<uint32_t>(nq);
    B.cnt = A.take<uint32_t>(nq);
    B.flags = A.take<uint32_t>(nq);
    B.mflag = A.take<uint32_t>(nq);
    B.nflag = A.take<uint32_t>(2);
    if (E->ham8) B.q8 = A.take<int8_t>(round_up(nq, kTileCols) * ham_mfma_row_bytes((int)E->dpad));
    if (is_gemm_metric(E->metric)) {
        // any run of at most kSmallPadQueries of these queries may take the small-batch scan
        B.spad = A.take<uint32_t>(std::min<size_t>(nq, kSmallPadQueries) * kSmallPadStride);
    }
    return B;
}

// Splits every round into pieces of at most max_rows rows (a multiple of kRowAlign, at least the
// first round's rows; 0 = no split).  A query's candidates from one piece cannot outnumber the
// piece's rows, so pieces no longer than the candidate capacity cannot overflow it.
static std::vector<Round> split_rounds(const std::vector<Round> &r, long max_rows) {
    if (max_rows <= 0) return r;
    std::vector<Round> out;
    for (const Round &x : r)
        for (long b = x.rb; b < x.re; b += max_rows) {
            Round p = x;
            p.rb = b;
            p.re = std::min(x.re, b + max_rows);
            p.plan_rows = x.re - x.rb;
            out.push_back(p);
        }
    return out;
}

// The round plan of a search over nq queries: the small-batch plan for at most kSmallCols queries
// on the GEMM metrics (not the direct-form re-runs).
static bool small_plan(const vhip_knn *E, size_t nq, bool direct) {
    return is_gemm_metric(E->metric) && !direct && !E->ham8 &&
           small_batch((int)std::min<size_t>(nq, 1 << 20), (int)E->dpad, E->n);
}

// The candidate count a run starts from: the first round's rows when that round is dense (every
// score is written), else 0.
static uint32_t first_count(const std::vector<Round> &rounds, const vhip_knn *E) {
    const bool dense0 = !rounds.empty() && (rounds[0].dense || (E->ham8 && rounds[0].rb == 0));
    return dense0 ? (uint32_t)(rounds[0].re - rounds[0].rb) : 0u;
}
static std::vector<Round> run_plan(const vhip_knn *E, int k, bool gemm, bool small, long max_round_rows) {
    return split_rounds(plan_rounds(E->n, (size_t)k, gemm, (int)E->dpad, kRoundGrowth, small), max_round_rows);
}

// Runs all rounds for nq prepared queries; results stay in B.topk (row stride kc) / B.have.
// `direct`: score squared L2 in direct form on the unshifted rows (VALU kernel) instead of the
// engine's own scan; it serves the queries whose GEMM-form margin could not be certified.
// `small`: the small-batch round plan (see plan_rounds; cap must be that plan's).
// max_round_rows: see split_rounds.  `timed`: the scan launches feed the engine's kernel timer.
// reset_done: the run's per-query state was reset with its queries' preparation (RowPrep::init).
static int run_rounds(vhip_knn *E, const QueryRows &Q, int nq, int k, int kc, int cap, bool direct, bool small,
                      const RunBufs &B, long max_round_rows, bool timed, bool reset_done = false) {
    hipStream_t s = E->stream;
    const bool gemm = is_gemm_metric(E->metric) && !direct;
    const std::vector<Round> rounds = run_plan(E, k, gemm, small, max_round_rows);
    if (!reset_done)
        launch_topk_init(nq, B.tau, B.have, B.cnt, B.flags, B.mflag, B.nflag, first_count(rounds, E), B.spad, s);
    if (E->ham8) {
        // the queries' +1/-1 nibbles, rows padded to the 128-query tiles
        const size_t rows = round_up((size_t)nq, kTileCols);
        launch_ham_expand((const uint32_t *)Q.qpad, (size_t)nq, (int)E->dpad, (int)E->dpad, rows, false, B.q8, s);
    }
    for (size_t ri = 0; ri < rounds.size(); ++ri) {
        const Round &rd = rounds[ri];
        const long rb = rd.rb, re = rd.re;
        const bool dense = rd.dense || (E->ham8 && rb == 0);
        // Algorithmic work per launch: 2*Q*rows*D flops (GEMM metrics), Q*rows*D element
        // operations (VALU metrics) or Q*rows*words word operations (packed Hamming); bytes
        // are the base rows and queries each launch must read once.  The direct-form passes
        // are not timed (they are not the engine's scan).
        const double rows = (double)(re - rb);
        const double work = gemm ? 2.0 * nq * rows * (double)E->dim
                                 : (E->ham8 ? 2.0 * nq * rows * 2.0 * (double)ham_mfma_row_bytes((int)E->dpad)
                                            : (double)nq * rows * (double)E->dim);
        const double bytes = E->ham8 ? (rows + nq) * (double)ham_mfma_row_bytes((int)E->dpad)  // expanded codes
                                     : rows * E->dim * 4.0 + (double)nq * E->dim * 4.0;
        if (dense && ri > 0) launch_fill_u32(B.cnt, (size_t)nq, (uint32_t)(re - rb), s);
        // the small-batch scan's FILTER rounds count candidates on B.spad (kSmallPadStride apart)
        const bool small_scan = !E->ham8 && gemm && small_batch(nq, (int)E->dpad, E->n);
        const bool spread = small_scan && !rd.dense;
        const int t = (direct || !timed) ? -1 : E->timer.begin(s);
        // the narrow resident-tile kernel (gemm_narrow) works in 512-row stages on 32-column tiles
        const bool narrow = gemm && gemm_narrow((int)E->dpad);
        const long item = gemm && !rd.dense
                              ? balanced_item(rd.item_rows, re - rb, ceil_div(nq, gemm_filter_cols((int)E->dpad)),
                                              E->grid_cap / 2, narrow ? 512 : kRowAlign)
                              : (narrow ? std::max<long>(rd.item_rows, 512) : rd.item_rows);
        if (E->ham8) {
            // fp4 matrix-core Hamming: 2 K operations per (query, row), K = the padded code bits.
            // Items up to 32768 rows where the slot rule allows: each spreads its query-tile fill
            // and flush over more 512-row stages (5% faster at 10M x 256 bits than 8192)
            // Filter rounds with at least 2048 queries whose slot rule allows items of 2048 rows
            // take the 1024-column kernel (8 candidate slots per query and item, so its items are
            // sized by the same rule with 8 slots).
            const long wide_rows = (long)ham_wide_slots() * rb / (3 * (long)std::max(k, 1)) / 512 * 512;
            if (!dense && E->ham_wide && nq >= 2048 && wide_rows >= 2048) {
                const long witem = balanced_item(std::min<long>(65536, wide_rows), re - rb,
                                                 ceil_div(nq, ham_wide_cols()), E->grid_cap / 2, 512);
                launch_ham_mfma_wide(witem, E->base8.as<int8_t>(), B.q8, (int)E->dpad, B.tau, nq, rb, re, B.cand,
                                     B.cnt, cap, E->grid_cap, s);
            } else {
                const long hitem =
                    dense ? re - rb
                          : balanced_item(std::min<long>(32768, rd.slot_rows), re - rb, ceil_div(nq, kTileCols),
                                          E->grid_cap / 2, 512);
                launch_ham_mfma(dense, hitem, E->base8.as<int8_t>(), B.q8, (int)E->dpad, B.tau, nq, rb, re, B.cand,
                                B.cnt, cap, E->grid_cap, s);
            }
        } else if (small_scan)
            launch_small_scan(E->metric, rd.dense, E->base.as<float>(), E->norm.as<float>(), Q.qpad, Q.qnorm, B.tau,
                              nq, (int)E->dpad, rb, re, rd.plan_rows ? rd.plan_rows : re - rb, B.cand, B.spad, cap,
                              E->grid_cap, s);
        else if (gemm)
            launch_gemm_filter(E->metric, rd.dense, item, E->base.as<float>(), E->norm.as<float>(), Q.qpad, Q.qnorm,
                               B.tau, nq, (int)E->dpad, rb, re, B.cand, B.cnt, cap, E->norm_max, E->norm_min,
                               E->grid_cap, s);
        else if (E->metric == HAMMING_PACKED)
            launch_hamming_filter(E->base.as<uint32_t>(), (const uint32_t *)Q.qpad, B.tau, nq, (int)E->dpad, rb, re,
                                  B.cand, B.cnt, cap, E->grid_cap, s);
        else if (direct)
            launch_valu_filter(L2, direct_rows(E), direct_shift(E), Q.qraw, B.tau, nq, (int)E->dim, (int)E->dpad, rb,
                               re, B.cand, B.cnt, cap, E->grid_cap, s);
        else
            launch_valu_filter(E->metric, E->base.as<float>(), nullptr, Q.qpad, B.tau, nq, (int)E->dim, (int)E->dpad,
                               rb, re, B.cand, B.cnt, cap, E->grid_cap, s);
        if (t >= 0) E->timer.end(t, s, work, bytes);
        VH_HIP(hipGetLastError());
        // the last round counts the standing margin flags into nflag[1]
        const bool last = ri + 1 == rounds.size();
        launch_topk_merge(nq, k, kc, B.cand, spread ? B.spad : B.cnt, spread ? kSmallPadStride : 1, cap,
                          E->perm.as<uint32_t>(), B.topk, B.have, B.tau, B.flags,
                          B.nflag, gemm ? Q.qerr : nullptr, B.mflag, last && gemm ? B.nflag + 1 : nullptr,
                          dense && re - rb > 4096, s);
        VH_HIP(hipGetLastError());
    }
    return VHIP_OK;
}

// Capacity of a candidate list that no round can overflow: the largest round's rows, of either
// round plan.
static int full_cap(const vhip_knn *E, size_t k, bool gemm) {
    long big = k;
    for (int sm = 0; sm < 2; ++sm)
        for (const Round &rd : plan_rounds(E->n, k, gemm, (int)E->dpad, kRoundGrowth, sm == 1))
            big = std::max(big, rd.re - rd.rb);
    return (int)round_up((size_t)big, kRowAlign);
}

// Buffers of a re-run of nidx queries in sub-batches of per_batch.
struct RerunMem {
    uint32_t *didx;
    float *fr, *fq, *fn, *fe;
    RunBufs F;
};
static RerunMem carve_rerun(Arena &A, const vhip_knn *E, size_t nidx, size_t per_batch, int kc_run, int cap,
                            bool direct, bool with_cand) {
    const size_t m_pad = round_up(per_batch, kTileCols);
    RerunMem r{};
    r.didx = A.take<uint32_t>(nidx);
    r.fr = A.take<float>(m_pad * E->dpad);
    if (!direct) {
        r.fq = A.take<float>(m_pad * E->dpad);
        r.fn = A.take<float>(m_pad);
        r.fe = A.take<float>(m_pad);
    }
    r.F = carve_run(A, E, per_batch, kc_run, cap, with_cand);
    return r;
}

// Re-runs the queries idx (host list) of the batch Q: `direct` as in run_rounds, and writes their
// kept entries, counts and margin flags back into the batch's buffers M (row stride kc).
//  * fixed == null: the re-run allocates candidate lists that no round can overflow.
//  * Otherwise every buffer is carved from *fixed (sized by the caller for a re-run of up to the
//    batch's query count) and the batch's own candidate buffer (cand_slots entries, no longer
//    needed) holds the candidate lists; rounds longer than each query's share of it are split
//    into pieces of that length, which cannot overflow.
static int rerun_queries(vhip_knn *E, const QueryRows &Q, const std::vector<uint32_t> &idx, int k, int kc,
                         bool direct, const RunBufs &M, const Arena *fixed, uint2 *cand, size_t cand_slots) {
    hipStream_t s = E->stream;
    const bool gemm = is_gemm_metric(E->metric) && !direct;
    const int kc_run = direct ? k : kc;
    const int cap_big = full_cap(E, (size_t)k, gemm);
    const int dp = (int)E->dpad;
    size_t per_batch = idx.size();
    int cap = cap_big;
    long max_rows = 0;
    DevBuf own;
    Arena A;
    if (fixed) {
        A = *fixed;
        cap = (int)std::min<size_t>((size_t)cap_big, cand_slots / idx.size() / kRowAlign * kRowAlign);
        if (cap < cap_big) max_rows = cap;
    } else {
        per_batch = std::min(idx.size(), std::max<size_t>(1, ((size_t)1 << 30) / ((size_t)cap_big * sizeof(uint2))));
        Arena meas;
        carve_rerun(meas, E, idx.size(), per_batch, kc_run, cap, direct, true);
        VH_CHECK(own.ensure(E->dev, meas.used));
        A = Arena(own.p, own.bytes);
    }
    RerunMem R = carve_rerun(A, E, idx.size(), per_batch, kc_run, cap, direct, fixed == nullptr);
    if (!A.fits()) return set_error(VHIP_ERR_DRIVER, "re-run workspace larger than its reserve");
    if (fixed) R.F.cand = cand;
    VH_HIP(hipMemcpyAsync(R.didx, idx.data(), idx.size() * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    for (size_t b0 = 0; b0 < idx.size(); b0 += per_batch) {
        const int m = (int)std::min(per_batch, idx.size() - b0);
        const size_t m_pad = round_up((size_t)m, kTileCols);
        const uint32_t *di = R.didx + b0;
        QueryRows F{nullptr, nullptr, nullptr, nullptr};
        launch_fill(R.fr + (size_t)m * dp, (m_pad - m) * E->dpad, 0.0f, s);
        launch_gather_rows(Q.qraw, di, (size_t)m, dp, R.fr, s);
        F.qraw = R.fr;
        if (!direct) {
            launch_fill(R.fq + (size_t)m * dp, (m_pad - m) * E->dpad, 0.0f, s);
            launch_fill(R.fn + m, m_pad - m, 0.0f, s);
            launch_fill(R.fe + m, m_pad - m, 0.0f, s);
            launch_gather_rows(Q.qpad, di, (size_t)m, dp, R.fq, s);
            launch_gather_rows(Q.qnorm, di, (size_t)m, 1, R.fn, s);
            if (Q.qerr) launch_gather_rows(Q.qerr, di, (size_t)m, 1, R.fe, s);
            F.qpad = R.fq;
            F.qnorm = R.fn;
            F.qerr = Q.qerr ? R.fe : nullptr;
        }
        VH_CHECK(run_rounds(E, F, m, k, kc_run, cap, direct, small_plan(E, per_batch, direct), R.F, max_rows,
                            fixed == nullptr));
        launch_scatter_topk(R.F.topk, kc_run, R.F.have, direct ? nullptr : R.F.mflag, di, m, M.topk, kc, M.have,
                            M.mflag, s);
        VH_HIP(hipGetLastError());
    }
    VH_HIP(hipStreamSynchronize(s));  // idx and the re-run's own buffers are released at return
    return VHIP_OK;
}

static std::vector<uint32_t> flagged(const std::vector<uint32_t> &f) {
    std::vector<uint32_t> idx;
    for (size_t q = 0; q < f.size(); ++q)
        if (f[q]) idx.push_back((uint32_t)q);
    return idx;
}

// Searches nq prepared queries for k = effective_k neighbours; writes kout >= k entries per query
// (the rest marked empty) into device arrays d_ids and d_dist or d_dist_u32 (row stride ostride).
// B: the batch's run buffers (kc entries and cap candidates per query); fixed: the re-runs' reserve
// when the search must not allocate (see rerun_queries), else null.
//  * A query whose candidate list overflowed (massive ties) is re-run with a capacity that no
//    round can overflow.
//  * GEMM metrics keep, besides the k best by GEMM-form score, every entry within twice the
//    query's selection error bound of the k-th (up to margin_cap(k) more); the direct-form refine
//    then ranks them.  A squared-L2 query whose margin did not fit is re-run in direct form on the
//    unshifted rows, so every L2 result is the exact top-k of the direct-form distances.  (For dot
//    product and cosine a direct-form pass rounds no better than the GEMM form, so a cut margin
//    keeps the kc best by GEMM score: only near-ties within the error bound are affected.)
// The counts of both kinds of flagged query come back to pinned host memory behind the final pass
// (refine or finalize), so a batch with none, the usual case, waits once, at its end; a batch with
// some waits for them, re-runs those queries and runs the final pass again.
static int search_prepared(vhip_knn *E, const QueryRows &Q, int nq, int k, int kc, int cap, bool small,
                           const RunBufs &B, const Arena *fixed, int kout, uint32_t *d_ids, float *d_dist,
                           uint32_t *d_dist_u32, int ostride) {
    hipStream_t s = E->stream;
    const bool gemm = is_gemm_metric(E->metric);
    uint32_t *nfh = E->flags_host;
    auto final_pass = [&](bool publish) -> int {
        FlagPublish pub;
        if (publish) {
            pub.src = B.nflag;
            pub.host = nfh;
        }
        if (gemm && d_dist)
            launch_topk_refine(nq, k, kc, kout, E->metric, Q.qraw, direct_rows(E), direct_shift(E),
                               E->inv_perm.as<uint32_t>(), (int)E->dpad, Q.qnorm, E->norm.as<float>(), B.topk, B.have,
                               Q.qerr, d_ids, d_dist, ostride, pub, s);
        else
            launch_topk_finalize(nq, kc, kout, E->metric, B.topk, B.have, d_ids, d_dist, d_dist_u32, ostride, pub, s);
        VH_HIP(hipGetLastError());
        return VHIP_OK;
    };
    // the run's per-query state was reset with the queries' preparation (the caller's RowPrep::init)
    VH_CHECK(run_rounds(E, Q, nq, k, kc, cap, false, small, B, 0, fixed == nullptr, true));
    volatile uint32_t *vn = nfh;
    vn[0] = vn[1] = 0xffffffffu;  // overwritten by the final kernel
    VH_CHECK(final_pass(true));
    VH_HIP(hipStreamSynchronize(s));
    uint32_t nf[2] = {vn[0], vn[1]};
    if (nf[0] == 0xffffffffu || nf[1] == 0xffffffffu)
        return set_error(VHIP_ERR_DRIVER, "the search's flag counts did not reach the host");
    if (!gemm) nf[1] = 0;
    if (!nf[0] && !(nf[1] && E->metric == L2)) return VHIP_OK;
    const size_t slots = (size_t)nq * cap;
    if (nf[0]) {
        std::vector<uint32_t> f(nq);
        VH_HIP(hipMemcpy(f.data(), B.flags, nq * sizeof(uint32_t), hipMemcpyDeviceToHost));
        VH_CHECK(rerun_queries(E, Q, flagged(f), k, kc, false, B, fixed, B.cand, slots));
        if (gemm) {
            uint32_t c = 0;
            launch_count_flags(B.mflag, nq, B.nflag + 1, s);
            VH_HIP(hipMemcpyAsync(&c, B.nflag + 1, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
            VH_HIP(hipStreamSynchronize(s));
            nf[1] = c;
        }
    }
    if (nf[1] && E->metric == L2) {
        std::vector<uint32_t> f(nq);
        VH_HIP(hipMemcpy(f.data(), B.mflag, nq * sizeof(uint32_t), hipMemcpyDeviceToHost));
        VH_CHECK(rerun_queries(E, Q, flagged(f), k, kc, true, B, fixed, B.cand, slots));
    }
    return final_pass(false);
}

static int check_search_args(vhip_knn *E, size_t k) {
    if (!E) return set_error(VHIP_ERR_INVALID_CONFIG, "null engine");
    if (k > (size_t)kMaxK)
        return set_error(VHIP_ERR_INVALID_CONFIG, "k = " + std::to_string(k) + " exceeds VHIP_MAX_K (2048)");
    return VHIP_OK;
}

// L2 and dot keep squared norms (the L2 epilogue, and both metrics' selection error bounds),
// cosine the norms before normalisation (zero-norm guard)
static int norm_kind_of(int metric) { return metric == COS ? 2 : ((metric == L2 || metric == DOT) ? 1 : 0); }
static int err_mode_of(int metric) { return metric == L2 ? 1 : (metric == DOT ? 2 : (metric == COS ? 3 : 0)); }
static int transform_of(int metric) { return metric == HELL ? 1 : 0; }
static int normalize_of(int metric) { return metric == COS ? 1 : 0; }

// Creates an engine over n rows of `dim` 32-bit elements (floats, or packed code words
// for HAMMING_PACKED, whose rows are padded to a power-of-two word count).
static int engine_create(const void *base, size_t n, size_t dim, int metric, int ordinal, vhip_knn **out) {
    clear_error();
    if (!out) return set_error(VHIP_ERR_INVALID_CONFIG, "out is null");
    *out = nullptr;
    if (dim == 0) return set_error(VHIP_ERR_INVALID_CONFIG, "dimension must be > 0");
    if (metric < 0 || metric > HAMMING_PACKED) return set_error(VHIP_ERR_INVALID_CONFIG, "unknown metric code");
    if (n > 0xffffffffull) return set_error(VHIP_ERR_INVALID_CONFIG, "more than 2^32 vectors (VectorId is u32)");
    if (n > 0 && !base) return set_error(VHIP_ERR_INVALID_CONFIG, "base is null");
    VH_CHECK(open_device(ordinal));
    std::unique_ptr<vhip_knn> E(new vhip_knn());
    E->dev = ordinal;
    E->n = n;
    E->n_pad = round_up(n, kRowAlign);
    E->dim = dim;
    E->dpad = metric == HAMMING_PACKED ? (size_t)hamming_word_pad((int)dim) : round_up(dim, kKChunk);
    E->metric = metric;
    E->grid_cap = device_grid_cap(ordinal);
    VH_HIP(hipStreamCreateWithFlags(&E->stream, hipStreamNonBlocking));
    VH_CHECK(E->stager.init(ordinal));
    // coherent: the search's final kernel stores the flag counts here directly
    VH_HIP(hipHostMalloc((void **)&E->flags_host, 2 * sizeof(uint32_t), hipHostMallocCoherent));
    if (n > 0) {
        VH_CHECK(build_row_order(E.get(), n, is_gemm_metric(metric)));
        DevBuf raw, flag;
        // the raw rows; afterwards, scratch for the norm extremes' partials
        VH_CHECK(raw.ensure(ordinal, std::max(n * dim * sizeof(float), 2 * kMinMaxParts * sizeof(float))));
        VH_CHECK(flag.ensure(ordinal, 2 * sizeof(uint32_t)));  // non-integer values, inexact shifted values
        launch_fill_u32(flag.as<uint32_t>(), 2, 0u, E->stream);
        VH_CHECK(E->stager.h2d(raw.p, base, n * dim * sizeof(float), E->stream));
        bool try_exact = false;  // the shifted rows may give back the unshifted ones (see `raw`)
        if (metric == L2) {
            // per-dimension shift: the column means (integers for integer data)
            DevBuf part;
            VH_CHECK(part.ensure(ordinal, col_shift_scratch_bytes((int)dim)));
            VH_CHECK(E->shift.ensure(ordinal, E->dpad * sizeof(float)));
            launch_col_shift(raw.as<float>(), n, (int)dim, (int)E->dpad, part.as<double>(), flag.as<uint32_t>(),
                             E->shift.as<float>(), E->stream);
            VH_HIP(hipGetLastError());
            std::vector<float> mu(E->dpad);
            uint32_t colnonint = 1;
            VH_HIP(hipMemcpyAsync(mu.data(), E->shift.p, E->dpad * sizeof(float), hipMemcpyDeviceToHost, E->stream));
            VH_HIP(hipMemcpyAsync(&colnonint, flag.p, sizeof(uint32_t), hipMemcpyDeviceToHost, E->stream));
            VH_HIP(hipStreamSynchronize(E->stream));
            for (float v : mu) E->shifted = E->shifted || v != 0.0f;
            // integer values and an integer shift: x - shift is exact unless the values are huge,
            // which the row preparation checks
            try_exact = E->shifted && colnonint == 0;
        }
        VH_CHECK(E->base.ensure(ordinal, E->n_pad * E->dpad * sizeof(float)));
        VH_CHECK(E->norm.ensure(ordinal, E->n_pad * sizeof(float)));
        if (E->shifted && !try_exact) VH_CHECK(E->raw.ensure(ordinal, E->n_pad * E->dpad * sizeof(float)));
        RowPrep rp;
        rp.in = raw.as<float>();
        rp.n = n;
        rp.n_out = E->n_pad;
        rp.dim = (int)dim;
        rp.dpad = (int)E->dpad;
        rp.perm = E->perm.as<uint32_t>();
        rp.shift = E->shifted ? E->shift.as<float>() : nullptr;
        rp.out = E->base.as<float>();
        rp.raw_out = E->raw.p ? E->raw.as<float>() : nullptr;
        rp.norm = E->norm.as<float>();
        rp.norm_kind = norm_kind_of(metric);
        rp.transform = transform_of(metric);
        rp.normalize = normalize_of(metric);
        rp.pad_fill = __builtin_nanf("");
        rp.nonint = metric == HAMMING_PACKED ? nullptr : flag.as<uint32_t>();
        rp.inexact = try_exact ? flag.as<uint32_t>() + 1 : nullptr;
        launch_rows_prep(rp, E->stream);
        VH_HIP(hipGetLastError());
        if (try_exact) {
            uint32_t inexact = 1;
            VH_HIP(hipMemcpyAsync(&inexact, flag.as<uint32_t>() + 1, sizeof(uint32_t), hipMemcpyDeviceToHost,
                                  E->stream));
            VH_HIP(hipStreamSynchronize(E->stream));
            if (inexact) {
                // some shifted value lost bits: keep the unshifted rows after all
                VH_CHECK(E->raw.ensure(ordinal, E->n_pad * E->dpad * sizeof(float)));
                rp.raw_out = E->raw.as<float>();
                rp.inexact = nullptr;
                launch_rows_prep(rp, E->stream);
                VH_HIP(hipGetLastError());
            }
        }
        const size_t rows8 = ham_mfma_rows(n);
        if (metric == HAMMING_PACKED && ham_mfma_supported((int)E->dpad) &&
            want_fp4_copy(rows8 * ham_mfma_row_bytes((int)E->dpad))) {
            VH_CHECK(E->base8.ensure(ordinal, rows8 * ham_mfma_row_bytes((int)E->dpad)));
            launch_ham_expand(E->base.as<uint32_t>(), n, (int)E->dpad, (int)E->dpad, rows8, true,
                              E->base8.as<int8_t>(), E->stream);
            VH_HIP(hipGetLastError());
            E->ham8 = true;
            const char *env = std::getenv("VHIP_HAMMING_KERNEL");
            E->ham_wide = ham_wide_supported((int)E->dpad) && !(env && std::strcmp(env, "fp4-tile") == 0);
        }
        uint32_t nonint = 1;
        VH_HIP(hipMemcpyAsync(&nonint, flag.p, sizeof(uint32_t), hipMemcpyDeviceToHost, E->stream));
        if (norm_kind_of(metric)) {
            // extremes of the row norms (the L2 filter's rounding slack, the selection error bounds
            // and the cosine zero-norm guard), reduced on the device into the raw buffer, which row
            // preparation (earlier on this stream) no longer needs
            float *part = raw.as<float>();
            hipLaunchKernelGGL(k_minmax_partial, dim3(kMinMaxParts), dim3(256), 0, E->stream, E->norm.as<float>(), n,
                               part, part + kMinMaxParts);
            VH_HIP(hipGetLastError());
            std::vector<float> ph(2 * kMinMaxParts);
            VH_HIP(hipMemcpyAsync(ph.data(), part, ph.size() * sizeof(float), hipMemcpyDeviceToHost, E->stream));
            VH_HIP(hipStreamSynchronize(E->stream));
            float mx = 0.0f, mn = INFINITY;
            for (int b = 0; b < kMinMaxParts; ++b) {
                mx = std::max(mx, ph[b]);
                mn = std::min(mn, ph[kMinMaxParts + b]);
            }
            E->norm_max = mx;
            E->norm_min = mn;
        }
        VH_HIP(hipStreamSynchronize(E->stream));
        E->integral = nonint == 0;
        E->err_coeff = sel_err_coeff(metric, (int)E->dpad);
    }
    *out = E.release();
    return VHIP_OK;
}

// Buffers of one query batch of m queries: the prepared rows and the run buffers.
struct BatchMem {
    float *qpad, *qnorm, *qerr, *qraw;
    RunBufs B;
};
static BatchMem carve_batch(Arena &A, const vhip_knn *E, size_t m, int kc, int cap) {
    const size_t m_pad = round_up(m, kTileCols);
    BatchMem b{};
    b.qpad = A.take<float>(m_pad * E->dpad);
    b.qnorm = A.take<float>(m_pad);
    b.qerr = is_gemm_metric(E->metric) ? A.take<float>(m_pad) : nullptr;
    b.qraw = E->shifted ? A.take<float>(m_pad * E->dpad) : nullptr;
    b.B = carve_run(A, E, m, kc, cap, true);
    return b;
}

// Device memory a batch of m queries needs; with_rerun adds the reserve of an allocation-free
// re-run of up to m queries (everything but the candidate lists, which reuse the batch's).
static size_t batch_bytes(const vhip_knn *E, size_t m, int kc, int cap, bool with_rerun) {
    Arena A;
    carve_batch(A, E, m, kc, cap);
    if (with_rerun) carve_rerun(A, E, m, m, kc, cap, false, false);
    return A.used;
}

// Device-side search: d_queries (nq x dim elements), outputs nq x k with row stride k.  Working
// memory comes from the engine's workspace buffer (grown as needed) or, when `scratch` is given,
// from that fixed region only, in query batches sized to fit it (no allocation, no kernel timing).
// The search itself; the caller holds E->mu.
static int engine_search_locked(vhip_knn *E, const void *d_queries, size_t nq, size_t k, uint32_t *d_ids,
                                float *d_dist, uint32_t *d_dist_u32, void *scratch, size_t scratch_bytes) {
    VH_CHECK(open_device(E->dev));
    const size_t ek = std::min(k, E->n);
    if (nq == 0 || k == 0) return VHIP_OK;
    if (ek == 0) {
        launch_fill_u32(d_ids, nq * k, 0xffffffffu, E->stream);
        VH_HIP(hipGetLastError());
        VH_HIP(hipStreamSynchronize(E->stream));
        return VHIP_OK;
    }
    const bool gemm = is_gemm_metric(E->metric);
    const int kk = (int)ek;
    const int kc = gemm ? kk + margin_cap(kk) : kk;
    size_t batch = std::min(nq, kQueryBatch);
    // every batch of the call takes the plan its first does: the buffers are sized for that plan
    bool small = small_plan(E, batch, false);
    int cap = round_cap(E->n, ek, gemm, (int)E->dpad, small);
    if (scratch && small && batch_bytes(E, batch, kc, cap, true) > scratch_bytes) {
        small = false;
        cap = round_cap(E->n, ek, gemm, (int)E->dpad, false);
    }
    if (scratch) {
        // the largest batch whose buffers and re-run reserve fit the scratch region
        if (batch_bytes(E, 1, kc, cap, true) > scratch_bytes)
            return set_error(VHIP_ERR_INVALID_CONFIG,
                             "k = " + std::to_string(k) + " over " + std::to_string(E->n) + " rows of dimension " +
                                 std::to_string(E->dim) + " needs " + std::to_string(batch_bytes(E, 1, kc, cap, true)) +
                                 " bytes of working memory per query; the allocation-free search has " +
                                 std::to_string(scratch_bytes));
        size_t lo = 1, hi = batch;
        while (lo < hi) {
            const size_t mid = (lo + hi + 1) / 2;
            if (batch_bytes(E, mid, kc, cap, true) <= scratch_bytes)
                lo = mid;
            else
                hi = mid - 1;
        }
        batch = lo;
    }
    for (size_t q0 = 0; q0 < nq; q0 += batch) {
        const int m = (int)std::min(batch, nq - q0);
        const size_t m_pad = round_up((size_t)m, kTileCols);
        Arena A;
        if (scratch) {
            A = Arena(scratch, scratch_bytes);
        } else {
            VH_CHECK(E->ws.arena.ensure(E->dev, batch_bytes(E, (size_t)m, kc, cap, false)));
            A = Arena(E->ws.arena.p, E->ws.arena.bytes);
        }
        const BatchMem bm = carve_batch(A, E, (size_t)m, kc, cap);
        const Arena reserve = A;  // the re-runs' buffers follow the batch's (allocation-free search)
        if (scratch) carve_rerun(A, E, (size_t)m, (size_t)m, kc, cap, false, false);
        if (!A.fits()) return set_error(VHIP_ERR_DRIVER, "search workspace larger than its region");
        RowPrep rp;
        rp.in = (const float *)d_queries + q0 * E->dim;
        rp.n = (size_t)m;
        rp.n_out = m_pad;
        rp.dim = (int)E->dim;
        rp.dpad = (int)E->dpad;
        rp.shift = E->shifted ? E->shift.as<float>() : nullptr;
        rp.out = bm.qpad;
        rp.raw_out = bm.qraw;
        rp.norm = bm.qnorm;
        rp.norm_kind = norm_kind_of(E->metric);
        rp.transform = transform_of(E->metric);
        rp.normalize = normalize_of(E->metric);
        rp.pad_fill = 0.0f;
        if (gemm) {
            rp.err = bm.qerr;
            rp.err_mode = err_mode_of(E->metric);
            rp.err_coeff = E->err_coeff;
            rp.err_nmax = E->norm_max;
            rp.base_integral = E->integral ? 1 : 0;
        }
        // the batch's run starts here too (search_prepared's first run_rounds skips its reset)
        rp.init = {bm.B.tau, bm.B.have, bm.B.cnt, bm.B.flags, bm.B.mflag, bm.B.nflag, bm.B.spad,
                   first_count(run_plan(E, kk, gemm, small, 0), E)};
        launch_rows_prep(rp, E->stream);
        VH_HIP(hipGetLastError());
        const QueryRows Q{bm.qpad, bm.qnorm, bm.qerr, E->shifted ? bm.qraw : bm.qpad};
        VH_CHECK(search_prepared(E, Q, m, kk, kc, cap, small, bm.B, scratch ? &reserve : nullptr, (int)k, d_ids + q0 * k,
                                 d_dist ? d_dist + q0 * k : nullptr, d_dist_u32 ? d_dist_u32 + q0 * k : nullptr,
                                 (int)k));
    }
    VH_HIP(hipStreamSynchronize(E->stream));
    E->timer.collect();
    return VHIP_OK;
}

static int engine_search_device(vhip_knn *E, const void *d_queries, size_t nq, size_t k, uint32_t *d_ids,
                                float *d_dist, uint32_t *d_dist_u32, void *scratch = nullptr,
                                size_t scratch_bytes = 0) {
    clear_error();
    VH_CHECK(check_search_args(E, k));
    std::lock_guard<std::mutex> lock(E->mu);
    return engine_search_locked(E, d_queries, nq, k, d_ids, d_dist, d_dist_u32, scratch, scratch_bytes);
}

// Host-side search through pinned staging, into the engine's own device buffers (kept between
// calls, grown as needed); the engine's lock is held for the whole call, as those buffers are
// shared by its calls.
static int engine_search_host(vhip_knn *E, const void *queries, size_t nq, size_t k, uint32_t *out_ids,
                              void *out_dist, bool dist_u32, size_t *out_len) {
    clear_error();
    VH_CHECK(check_search_args(E, k));
    if (nq == 0) return VHIP_OK;
    if (!queries || !out_len) return set_error(VHIP_ERR_INVALID_CONFIG, "null query/output pointer");
    const size_t ek = std::min(k, E->n);
    if (k == 0 || ek == 0) {
        for (size_t q = 0; q < nq; ++q) out_len[q] = 0;
        return VHIP_OK;
    }
    if (!out_ids || !out_dist) return set_error(VHIP_ERR_INVALID_CONFIG, "null output pointer");
    std::lock_guard<std::mutex> lock(E->mu);
    VH_CHECK(open_device(E->dev));
    DevBuf &dq = E->ws.hq, &di = E->ws.hi, &dd = E->ws.hd;
    VH_CHECK(dq.ensure(E->dev, nq * E->dim * sizeof(float)));
    VH_CHECK(di.ensure(E->dev, nq * k * sizeof(uint32_t)));
    VH_CHECK(dd.ensure(E->dev, nq * k * sizeof(float)));
    VH_CHECK(E->stager.h2d(dq.p, queries, nq * E->dim * sizeof(float), E->stream));
    VH_CHECK(engine_search_locked(E, dq.p, nq, k, di.as<uint32_t>(), dist_u32 ? nullptr : dd.as<float>(),
                                  dist_u32 ? dd.as<uint32_t>() : nullptr, nullptr, 0));
    VH_CHECK(E->stager.d2h_pair(out_ids, di.p, nq * k * sizeof(uint32_t), out_dist, dd.p, nq * k * sizeof(float),
                                E->stream));
    for (size_t q = 0; q < nq; ++q) out_len[q] = ek;
    return VHIP_OK;
}

// ---- allocation-free search -----------------------------------------------------------------
// The working memory is the per-device array of noalloc_scratch.hip, whose lock is held for the
// whole call.  Every exit, error paths included, first waits for the engine's stream: kernels
// this call queued read and write the array, so they must finish before another call (another
// engine, on another stream) may reuse it.
static int search_device_noalloc(vhip_knn *E, const float *d_queries, size_t nq, size_t k, uint32_t *d_ids,
                                 float *d_dist) {
    clear_error();
    if (!E) return set_error(VHIP_ERR_INVALID_CONFIG, "null engine");
    std::unique_lock<std::mutex> lock;
    void *ptr = nullptr;
    VH_CHECK(noalloc_scratch_acquire(E->dev, lock, &ptr));
    const int rc = engine_search_device(E, d_queries, nq, k, d_ids, d_dist, nullptr, ptr, VHIP_NOALLOC_SCRATCH_BYTES);
    const hipError_t se = hipSetDevice(E->dev) == hipSuccess ? hipStreamSynchronize(E->stream) : hipErrorInvalidDevice;
    if (rc != VHIP_OK) return rc;  // the first error's message stands
    if (se != hipSuccess) {
        (void)hipGetLastError();
        return set_error(VHIP_ERR_DRIVER, std::string("hipStreamSynchronize: ") + hipGetErrorString(se));
    }
    return VHIP_OK;
}

}  // namespace vh

using namespace vh;

extern "C" {

int vhip_knn_create(const float *base, size_t n, size_t dim, int metric, int ordinal, vhip_knn **out) {
    if (metric < 0 || metric > 9) {
        if (out) *out = nullptr;
        return set_error(VHIP_ERR_INVALID_CONFIG, "unknown metric code");
    }
    return engine_create(base, n, dim, metric, ordinal, out);
}

int vhip_knn_search_batch_device(vhip_knn *E, const float *d_queries, size_t nq, size_t k, uint32_t *d_ids,
                                 float *d_dist) {
    return engine_search_device(E, d_queries, nq, k, d_ids, d_dist, nullptr);
}

int vhip_knn_search_batch_device_noalloc(vhip_knn *E, const float *d_queries, size_t nq, size_t k, uint32_t *d_ids,
                                         float *d_dist) {
    return search_device_noalloc(E, d_queries, nq, k, d_ids, d_dist);
}

int vhip_knn_search_batch(vhip_knn *E, const float *queries, size_t nq, size_t k, uint32_t *out_ids, float *out_dist,
                          size_t *out_len) {
    return engine_search_host(E, queries, nq, k, out_ids, out_dist, false, out_len);
}

size_t vhip_knn_dimension(const vhip_knn *E) { return E ? E->dim : 0; }
size_t vhip_knn_num_vectors(const vhip_knn *E) { return E ? E->n : 0; }
int vhip_knn_metric(const vhip_knn *E) { return E ? E->metric : -1; }
int vhip_knn_device_id(const vhip_knn *E) { return E ? E->dev : -1; }

void vhip_knn_destroy(vhip_knn *E) { delete E; }

int vhip_knn_profile(vhip_knn *E, int enable) {
    if (!E) return set_error(VHIP_ERR_INVALID_CONFIG, "null engine");
    std::lock_guard<std::mutex> lock(E->mu);
    E->timer.enabled = enable != 0;
    E->timer.reset();
    return VHIP_OK;
}

int vhip_knn_profile_read(vhip_knn *E, double *kernel_ms, uint64_t *launches, double *work, double *bytes) {
    if (!E) return set_error(VHIP_ERR_INVALID_CONFIG, "null engine");
    std::lock_guard<std::mutex> lock(E->mu);
    if (kernel_ms) *kernel_ms = E->timer.ms;
    if (launches) *launches = E->timer.launches;
    if (work) *work = E->timer.work;
    if (bytes) *bytes = E->timer.bytes;
    return VHIP_OK;
}

// ---- packed-bit Hamming engine: the same resident layout and round pipeline over
// uint32 code words (HAMMING_PACKED) ----------------------------------------------------
struct vhip_hamming {
    vhip_knn *e = nullptr;
    ~vhip_hamming() { vhip_knn_destroy(e); }
};

int vhip_hamming_create(const uint32_t *codes, size_t n, size_t words, int ordinal, vhip_hamming **out) {
    if (!out) return set_error(VHIP_ERR_INVALID_CONFIG, "out is null");
    *out = nullptr;
    if (words == 0 || words > 32) return set_error(VHIP_ERR_INVALID_CONFIG, "words must be in 1..32 (<= 1024 bits)");
    std::unique_ptr<vhip_hamming> H(new vhip_hamming());
    VH_CHECK(engine_create(codes, n, words, HAMMING_PACKED, ordinal, &H->e));
    *out = H.release();
    return VHIP_OK;
}

int vhip_hamming_search_batch(vhip_hamming *H, const uint32_t *queries, size_t nq, size_t k, uint32_t *out_ids,
                              uint32_t *out_dist, size_t *out_len) {
    if (!H) return set_error(VHIP_ERR_INVALID_CONFIG, "null engine");
    return engine_search_host(H->e, queries, nq, k, out_ids, out_dist, true, out_len);
}

int vhip_hamming_search_batch_device(vhip_hamming *H, const uint32_t *d_queries, size_t nq, size_t k,
                                     uint32_t *d_ids, uint32_t *d_dist) {
    if (!H) return set_error(VHIP_ERR_INVALID_CONFIG, "null engine");
    return engine_search_device(H->e, d_queries, nq, k, d_ids, nullptr, d_dist);
}

int vhip_hamming_profile(vhip_hamming *H, int enable) {
    if (!H) return set_error(VHIP_ERR_INVALID_CONFIG, "null engine");
    return vhip_knn_profile(H->e, enable);
}

int vhip_hamming_profile_read(vhip_hamming *H, double *kernel_ms, uint64_t *launches, double *work, double *bytes) {
    if (!H) return set_error(VHIP_ERR_INVALID_CONFIG, "null engine");
    return vhip_knn_profile_read(H->e, kernel_ms, launches, work, bytes);
}

void vhip_hamming_destroy(vhip_hamming *H) { delete H; }

}  // extern "C"

// ============================ DistributedKnnEngine ==========================================
struct vhip_dknn {
    size_t num_gpus = 1, dim = 0, n = 0;
    int mode = VHIP_SHARD_SHARDED, metric = 0;
    std::vector<vhip_knn *> ranks;
    std::vector<size_t> offsets;
    ~vhip_dknn() {
        for (auto *r : ranks) vhip_knn_destroy(r);
    }
};

static int dknn_init(const float *base, size_t n, size_t dim, size_t num_gpus, int mode, int metric, bool emulate,
                     vhip_dknn **out) {
    // DistributedKnnEngine::init_engine (distributed_knn.rs:91-146)
    std::unique_ptr<vhip_dknn> D(new vhip_dknn());
    const size_t g = std::min(num_gpus, std::max<size_t>(n, 1));
    D->num_gpus = g;
    D->dim = dim;
    D->n = n;
    D->mode = mode;
    D->metric = metric;
    if (mode == VHIP_SHARD_SHARDED) {
        const size_t chunk = (n + g - 1) / g;
        for (size_t r = 0; r < g; ++r) {
            const size_t s0 = r * chunk;
            const size_t e0 = std::min(s0 + chunk, n);
            const size_t cnt = s0 < n ? e0 - s0 : 0;
            vhip_knn *e = nullptr;
            VH_CHECK(vhip_knn_create(cnt ? base + s0 * dim : nullptr, cnt, dim, metric, emulate ? 0 : (int)r, &e));
            D->ranks.push_back(e);
            D->offsets.push_back(s0);
        }
    } else {
        for (size_t r = 0; r < g; ++r) {
            vhip_knn *e = nullptr;
            VH_CHECK(vhip_knn_create(base, n, dim, metric, emulate ? 0 : (int)r, &e));
            D->ranks.push_back(e);
            D->offsets.push_back(0);
        }
    }
    *out = D.release();
    return VHIP_OK;
}

extern "C" {

int vhip_dknn_try_new(const float *base, size_t n, size_t dim, size_t num_gpus, int mode, int metric,
                      vhip_dknn **out) {
    clear_error();
    if (!out) return set_error(VHIP_ERR_INVALID_CONFIG, "out is null");
    *out = nullptr;
    if (num_gpus < 1) return set_error(VHIP_ERR_INVALID_CONFIG, "num_gpus must be at least 1");
    if (dim == 0) return set_error(VHIP_ERR_INVALID_CONFIG, "dimension must be > 0");
    if (mode != VHIP_SHARD_SHARDED && mode != VHIP_SHARD_REPLICATED)
        return set_error(VHIP_ERR_INVALID_CONFIG, "unknown GpuShardMode");
    const size_t avail = (size_t)device_count();
    if (num_gpus > avail) {
        set_insufficient(num_gpus, avail);
        return VHIP_ERR_INSUFFICIENT_DEVICES;
    }
    return dknn_init(base, n, dim, num_gpus, mode, metric, false, out);
}

int vhip_dknn_emulator(const float *base, size_t n, size_t dim, size_t num_gpus, int mode, int metric,
                       vhip_dknn **out) {
    clear_error();
    if (!out) return set_error(VHIP_ERR_INVALID_CONFIG, "out is null");
    *out = nullptr;
    if (num_gpus < 1) return set_error(VHIP_ERR_INVALID_CONFIG, "num_gpus must be at least 1");
    if (dim == 0) return set_error(VHIP_ERR_INVALID_CONFIG, "dimension must be > 0");
    if (mode != VHIP_SHARD_SHARDED && mode != VHIP_SHARD_REPLICATED)
        return set_error(VHIP_ERR_INVALID_CONFIG, "unknown GpuShardMode");
    return dknn_init(base, n, dim, num_gpus, mode, metric, true, out);
}

int vhip_dknn_search_batch(vhip_dknn *D, const float *queries, size_t nq, size_t k, uint32_t *out_ids,
                           float *out_dist, size_t *out_len) {
    clear_error();
    if (!D) return set_error(VHIP_ERR_INVALID_CONFIG, "null engine");
    if (nq == 0) return VHIP_OK;
    if (k == 0 || D->n == 0) {
        for (size_t q = 0; q < nq; ++q) out_len[q] = 0;
        return VHIP_OK;
    }
    const size_t g = D->ranks.size();
    const bool hib = D->metric == DOT || D->metric == COS;
    if (D->mode == VHIP_SHARD_SHARDED) {
        // distributed_knn.rs:163-199: every rank searches all queries on its shard, ids are
        // shifted by the shard offset, then each query's lists are merged by top_k_reduce.
        std::vector<std::vector<uint32_t>> rid(g, std::vector<uint32_t>(nq * k));
        std::vector<std::vector<float>> rdist(g, std::vector<float>(nq * k));
        std::vector<std::vector<size_t>> rlen(g, std::vector<size_t>(nq));
        for (size_t r = 0; r < g; ++r) {
            VH_CHECK(vhip_knn_search_batch(D->ranks[r], queries, nq, k, rid[r].data(), rdist[r].data(),
                                           rlen[r].data()));
        }
        std::vector<uint32_t> ids;
        std::vector<float> dist;
        for (size_t q = 0; q < nq; ++q) {
            ids.clear();
            dist.clear();
            for (size_t r = 0; r < g; ++r)
                for (size_t j = 0; j < rlen[r][q]; ++j) {
                    ids.push_back((uint32_t)(rid[r][q * k + j] + D->offsets[r]));
                    dist.push_back(rdist[r][q * k + j]);
                }
            out_len[q] = top_k_reduce_host(ids.data(), dist.data(), ids.size(), k, hib, out_ids + q * k,
                                           out_dist + q * k);
        }
    } else {
        // distributed_knn.rs:201-229: split queries into ceil(Q/G) chunks, concatenate.
        const size_t qc = (nq + g - 1) / g;
        for (size_t r = 0; r < g; ++r) {
            const size_t q0 = r * qc;
            if (q0 >= nq) break;
            const size_t m = std::min(qc, nq - q0);
            VH_CHECK(vhip_knn_search_batch(D->ranks[r], queries + q0 * D->dim, m, k, out_ids + q0 * k,
                                           out_dist + q0 * k, out_len + q0));
        }
    }
    return VHIP_OK;
}

size_t vhip_dknn_num_gpus(const vhip_dknn *D) { return D ? D->num_gpus : 0; }
int vhip_dknn_mode(const vhip_dknn *D) { return D ? D->mode : -1; }
size_t vhip_dknn_dimension(const vhip_dknn *D) { return D ? D->dim : 0; }
size_t vhip_dknn_num_vectors(const vhip_dknn *D) { return D ? D->n : 0; }
int vhip_dknn_metric(const vhip_dknn *D) { return D ? D->metric : -1; }
void vhip_dknn_destroy(vhip_dknn *D) { delete D; }

}  // extern "C"
