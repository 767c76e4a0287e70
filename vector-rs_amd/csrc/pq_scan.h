// pq_scan.h -- device code of product quantization: the direct-form metric accumulators and
// the fused IVF-PQ scan kernel (k_ivfpq_scan), instantiated by pq_scan_*.hip.
//
// IvfPqIndex::search_with_nprobe (vector-index/src/ivf/mod.rs:256-345) for a batch of queries,
// one workgroup per query (grid-stride over queries).  The probes are taken PG at a time (PG = 1,
// 2 or 4, as many as the LDS budget holds): the workgroup loads their list bounds, forms their
// residuals q - c and builds their PG ADC tables (ProductQuantizer::compute_adc_lut, pq.rs:233-266)
// in LDS, then the 4 / PG waves assigned to each probe scan its list.  Each list entry is scored
// with compute_distance_with_lut's summation order (pq.rs:270-293) and offered to the scanning
// wave's own candidate buffer in LDS, filtered by that wave's threshold (the k-th best it holds)
// and sorted down to its k best whenever it fills; the four buffers are sorted together at the
// end of the query.
//
// With 256 sub-centroids, code rows of 16 or 32 bytes (NV = 1 or 2 sixteen-byte pieces) and their
// vector ids stream into a per-wave ring of NB chunks of 64 rows (NB = 6 or 4) with global->LDS DMA
// (no registers held); chunks are scored two at a time, with NB - 2 chunks issued ahead of the
// pair being read.  The first NB - 2 are issued before the tables are built and land while they
// are.  A chunk is read only
// after an explicit vmcnt wait that leaves exactly the younger DMAs in flight (vector memory
// loads complete in order), through an inline-asm LDS read: the compiler's own wait insertion
// would otherwise wait for every DMA in flight before any read of the ring.  Other row sizes are
// loaded straight into registers, kScanU rows per lane per step.
//
// Candidate keys are (order-preserving score key << 32) | vector id, so the k best are unique and
// equal scores are ordered by ascending id.  The reference keeps, among entries that tie at the
// k-th score, whichever its BinaryHeap keeps; the sets differ only inside such a tie.
#pragma once

#include <algorithm>

#include "vh_common.h"

namespace vh {

// ---- IVF-PQ scan ------------------------------------------------------------------------------
constexpr int kScanThreads = 256;
constexpr int kScanWaves = kScanThreads / 64;
constexpr int kLutRegs = 128;  // codebook floats per thread in the register layout
constexpr int kScanU = 2;      // rows per lane per step on the register-load path
// DMA ring depth in chunks of 64 code rows and ids: 6 chunks of 16-byte rows (7.5 KB per wave), 4
// of 32-byte rows, so that two workgroups fit in a CU's LDS; at least 4, as chunks are scored in
// pairs with two more in flight
constexpr int ring_chunks(int nv) { return nv == 2 ? 4 : 6; }
static_assert(ring_chunks(1) >= 4 && ring_chunks(2) >= 4, "pairs of chunks with two more in flight");

struct ScanArgs {
    const float *qry;          // nq x dim
    const float *coarse;       // nlist x dim
    const uint32_t *probes;    // nq x nprobe, best first
    const uint32_t *list_off;  // nlist + 1
    const uint32_t *ids;       // n, list order
    const uint8_t *codes;      // n x m_sub, list order
    const float *cb;           // m_sub x ks x ds
    const float *cbt;          // 256 x kLutRegs thread-major register layout (register path)
    uint32_t *out_ids;         // nq x k
    float *out_dist;           // nq x k
    uint32_t *out_len;         // nq
    int nq, dim, nprobe, nlist, m_sub, ks, ds, k, metric, groups, mg;
    int capw;                  // candidate slots per wave: a power of two >= k + 64 * kScanU
    int pg;                    // probes per group: 1, 2 or 4
};

constexpr int kMetaWin = 128;  // probes whose list bounds are staged in LDS at a time

// LDS bytes of the per-wave DMA rings for code rows of NV sixteen-byte pieces and their ids.
// A ring chunk holds 64 code rows (nv pieces of 64 x 16 bytes) and their 64 vector ids.
constexpr int ring_chunk_bytes(int nv) { return nv * 1024 + 256; }
constexpr int ring_bytes(int nv) { return kScanWaves * ring_chunks(nv) * ring_chunk_bytes(nv); }

// ---- list-major scan --------------------------------------------------------------------------
// For 16-byte code rows (16 sub-spaces of 256 sub-centroids) and k <= kListMaxK the search runs
// list-major: the (query, probe) pairs are grouped by list, and a work item is one list with up to
// kListQb of the queries probing it.  The item's kListQb ADC tables are built in LDS side by side:
// entry (m, e) of the four tables is one float4 (thread j computes sub-centroid j's entries from its
// register-held codebook), so one 16-byte LDS read per code byte serves the item's four pairs.  The
// list then streams once: wave w scores rows 64 w .. 64 w + 63 of each 256-row chunk, one row a
// lane (its 16 code bytes loaded straight into registers, one chunk ahead), against the four
// tables with the summation order of compute_distance_with_lut (pq.rs:270-293), and leaves the
// four scores in LDS; after one barrier per chunk, wave q filters and offers the chunk's 256
// scores of pair q, keeping its k best.  A list's codes are therefore read once per kListQb probing
// queries instead of once per probing query, and a table entry costs a quarter of a 16-byte read
// instead of a 4-byte read (a wave's 16-byte read passes 16 lanes at a time; random entries collide
// in banks either way).  Each pair's k best go to pair_out; k_ivfpq_merge then sorts each query's
// nprobe x k keys.  Keys are unique (score, id), so the result equals the query-major scan's.
// The query's threshold carries across its pairs through tau_q: a finished pair lowers it to its
// k-th key (atomic min), and a pair starts from it and re-reads it every chunk, so only the
// first pairs of a query offer many candidates.  tau_q is always the k-th key of some of the
// query's candidates, never below the final k-th, so no key of the final k best is filtered.

// 64 KB of tables, 4 KB of candidate buffers (128 keys a wave: k kept plus one offer of 64) and
// 8 KB of chunk scores fit two workgroups per CU.
constexpr int kListThreads = 256;    // 4 pairs per item; two workgroups per CU overlap their phases
constexpr int kListQb = kListThreads / 64;
constexpr int kListChunkRows = 256;  // rows per chunk: one per lane of each wave
constexpr int kListCapw = 128;       // candidate keys per wave: k kept + one offer of 64
// The list path takes k <= 48: at larger k a wave's buffer, holding k keys after each sort, fills
// with any later offer, so nearly every offer sorts it again (1M rows, 1024-component mixture,
// nprobe 32: 13.9 ms at k = 64 against 7.8 ms for the query-major scan, 6.1 against 7.5 ms at
// k = 48).
constexpr int kListMaxK = 48;
static_assert(kListMaxK + 64 <= kListCapw, "k kept plus one offer fit a wave's buffer");
constexpr int kListMaxMerge = 8192;  // nprobe x k keys sorted per query in the merge

struct ListArgs {
    ScanArgs s;                    // queries, lists, codebooks, outputs, k, nprobe, capw
    const uint4 *items;            // (list, first pair, list's first row, its length << 3 | pair count)
    const uint4 *item_pairs;       // each item's pair ids q * nprobe + p (unused slots repeat the first)
    const uint32_t *n_items;       // device scalar: items of this search
    uint32_t *work;                // device scalar: next item to take (zero before the launch)
    unsigned long long *pair_out;  // nq * nprobe * k keys: each pair's k best, ~0 past its count
    unsigned long long *tau_q;     // nq keys (~0 before the launch): the k-th best key found so far
};

namespace {

// ---- direct-form metric of two short vectors: the formulas of scalar.rs:14-263 -------------
template <int MT>
struct Acc {
    float a = 0.0f, b = 0.0f, e = 0.0f;
    __device__ __forceinline__ void step(float x, float c) {
        if constexpr (MT == DOT) {
            a = fmaf(x, c, a);
        } else if constexpr (MT == COS) {
            a = fmaf(x, c, a);
            b = fmaf(x, x, b);
            e = fmaf(c, c, e);
        } else if constexpr (MT == L1) {
            a += fabsf(x - c);
        } else if constexpr (MT == MINK) {
            const float t = fabsf(x - c);
            a = fmaf(t * t, t, a);
        } else if constexpr (MT == LINF) {
            a = fmaxf(a, fabsf(x - c));
        } else if constexpr (MT == HAMF) {
            a += fabsf(x - c) > 1e-6f ? 1.0f : 0.0f;
        } else if constexpr (MT == JACC) {
            const float ax = fabsf(x), ac = fabsf(c);
            a += fminf(ax, ac);
            b += fmaxf(ax, ac);
        } else if constexpr (MT == HELL) {
            const float t = sqrtf(fabsf(x)) - sqrtf(fabsf(c));
            a = fmaf(t, t, a);
        } else {  // L2, MAHA
            const float t = x - c;
            a = fmaf(t, t, a);
        }
    }
    __device__ __forceinline__ float finish() const {
        if constexpr (MT == COS) {
            const float den = sqrtf(b) * sqrtf(e);
            return den <= 1e-9f ? 0.0f : a / den;
        } else if constexpr (MT == MINK) {
            return cbrtf(a);
        } else if constexpr (MT == MAHA) {
            return sqrtf(a);
        } else if constexpr (MT == JACC) {
            return b <= 1e-9f ? 0.0f : 1.0f - a / b;
        } else if constexpr (MT == HELL) {
            return sqrtf(0.5f * a);
        } else {
            return a;
        }
    }
};

constexpr bool hib_metric(int m) { return m == DOT || m == COS; }

#define VH_METRIC_SWITCH(metric, CALL) \
    switch (metric) {                  \
        case L2: CALL(L2); break;      \
        case DOT: CALL(DOT); break;    \
        case COS: CALL(COS); break;    \
        case L1: CALL(L1); break;      \
        case MINK: CALL(MINK); break;  \
        case LINF: CALL(LINF); break;  \
        case HAMF: CALL(HAMF); break;  \
        case MAHA: CALL(MAHA); break;  \
        case JACC: CALL(JACC); break;  \
        default: CALL(HELL); break;    \
    }

// Orders LDS accesses of the lanes of one wave (no other wave touches the region).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Ascending bitonic sort of s[0, P) (P a power of two) by `nthr` threads with index `tid`;
// `sync` orders the stages.
template <class Sync>
__device__ __forceinline__ void bitonic_sort_u64(unsigned long long *s, int P, int tid, int nthr, Sync sync) {
    for (int size = 2; size <= P; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = tid; t < (P >> 1); t += nthr) {
                const int lo = 2 * t - (t & (stride - 1));
                const int hi = lo + stride;
                const bool asc = (lo & size) == 0;
                const unsigned long long a = s[lo], b = s[hi];
                if ((a > b) == asc) {
                    s[lo] = b;
                    s[hi] = a;
                }
            }
            sync();
        }
    }
}

// Sorts the wave's `cnt` candidates, keeps the k best and, once k are held, tightens the
// wave's threshold to the k-th.  cnt and tau are wave-uniform.
__device__ __forceinline__ void wave_compact(unsigned long long *s_w, uint32_t &cnt, unsigned long long &tau, int k) {
    const int lane = threadIdx.x & 63;
    int P = 2;
    while (P < (int)cnt) P <<= 1;
    for (int t = (int)cnt + lane; t < P; t += 64) s_w[t] = ~0ull;
    wave_sync();
    bitonic_sort_u64(s_w, P, lane, 64, wave_sync);
    if ((int)cnt >= k) tau = s_w[k - 1];
    cnt = min((int)cnt, k);
}

// ADC tables of a group of PG probes (residuals s_r[w * dim ...], tables s_lut[w * M * Ks ...]).
// Register path (one group of sub-spaces, ks > 128): thread j holds sub-centroid j of every
// sub-space in cbr (DS floats each), so every bound is uniform.
template <int MT, int DS>
__device__ __forceinline__ void lut_build_reg(const ScanArgs &A, int pg, const float *s_r, float *s_lut,
                                              const float *cbr) {
    if ((int)threadIdx.x >= A.ks) return;
    const int j = threadIdx.x, tstride = A.m_sub * A.ks;
#pragma unroll 1
    for (int w = 0; w < pg; ++w) {  // one table at a time keeps one residual live
        const float *r = s_r + w * A.dim;
        float *lut = s_lut + w * tstride + j;
#pragma unroll
        for (int m = 0; m < kLutRegs / DS; ++m) {
            if (m < A.m_sub) {
                Acc<MT> acc;
#pragma unroll
                for (int d4 = 0; d4 < DS; d4 += 4) {  // one broadcast LDS read per 4 residual values
                    const float4 rv = *reinterpret_cast<const float4 *>(r + m * DS + d4);
                    acc.step(rv.x, cbr[m * DS + d4]);
                    acc.step(rv.y, cbr[m * DS + d4 + 1]);
                    acc.step(rv.z, cbr[m * DS + d4 + 2]);
                    acc.step(rv.w, cbr[m * DS + d4 + 3]);
                }
                lut[m * A.ks] = acc.finish();
            }
        }
    }
}

// Cached path: thread t = (group g, sub-centroid j) of 256 / ks groups reads its sub-centroids
// of the group's sub-spaces through the caches.
template <int MT>
__device__ __forceinline__ void lut_build_mem(const ScanArgs &A, int pg, const float *s_r, float *s_lut) {
    const int g = threadIdx.x / A.ks, j = threadIdx.x - g * A.ks;
    if (g >= A.groups) return;
    const int m0 = g * A.mg, m1 = min(A.m_sub, m0 + A.mg), tstride = A.m_sub * A.ks;
    for (int m = m0; m < m1; ++m) {
        const float *c = A.cb + ((size_t)m * A.ks + j) * A.ds;
        for (int w = 0; w < pg; ++w) {
            Acc<MT> acc;
            for (int d = 0; d < A.ds; ++d) acc.step(s_r[w * A.dim + m * A.ds + d], c[d]);
            s_lut[w * tstride + m * A.ks + j] = acc.finish();
        }
    }
}

__device__ __forceinline__ float adc_quad(const float *L, int ks, uint32_t w) {
    const float d0 = L[w & 255u];
    const float d1 = L[ks + ((w >> 8) & 255u)];
    const float d2 = L[2 * ks + ((w >> 16) & 255u)];
    const float d3 = L[3 * ks + (w >> 24)];
    return (d0 + d1) + (d2 + d3);
}

// compute_distance_with_lut (pq.rs:270-293) of code row `cp`.
__device__ __forceinline__ float adc_score(const uint8_t *__restrict__ cp, const float *s_lut, int m_sub, int ks) {
    float total = 0.0f;
    if ((m_sub & 15) == 0) {
        const uint4 *c4 = reinterpret_cast<const uint4 *>(cp);
        const float *L = s_lut;
        for (int v = 0; v < (m_sub >> 4); ++v) {
            const uint4 w = c4[v];
            total += adc_quad(L, ks, w.x);
            total += adc_quad(L + 4 * ks, ks, w.y);
            total += adc_quad(L + 8 * ks, ks, w.z);
            total += adc_quad(L + 12 * ks, ks, w.w);
            L += 16 * ks;
        }
    } else if ((m_sub & 3) == 0) {
        const uint32_t *c1 = reinterpret_cast<const uint32_t *>(cp);
        for (int v = 0; v < (m_sub >> 2); ++v) total += adc_quad(s_lut + 4 * v * ks, ks, c1[v]);
    } else {
        int m = 0;
        for (; m + 4 <= m_sub; m += 4) {
            const float *L = s_lut + m * ks;
            const float d0 = L[cp[m]], d1 = L[ks + cp[m + 1]], d2 = L[2 * ks + cp[m + 2]], d3 = L[3 * ks + cp[m + 3]];
            total += (d0 + d1) + (d2 + d3);
        }
        for (; m < m_sub; ++m) total += s_lut[m * ks + cp[m]];
    }
    return total;
}

// Waits until at most `younger` (<= ring_chunks(NV) - 2) chunks of NV + 1 DMAs each are still
// in flight: s_waitcnt takes its count as an immediate, hence one case per count.
template <int NV>
__device__ __forceinline__ void ring_wait(int younger) {
    constexpr int P = NV + 1;
    static_assert((ring_chunks(NV) - 2) * P < 16, "vmcnt immediates stay below 16");
    switch (younger) {
        case 0: __builtin_amdgcn_s_waitcnt(VH_VMCNT(0)); break;
        case 1: __builtin_amdgcn_s_waitcnt(VH_VMCNT(P)); break;
        case 2: __builtin_amdgcn_s_waitcnt(VH_VMCNT(2 * P)); break;
        case 3: __builtin_amdgcn_s_waitcnt(VH_VMCNT(3 * P)); break;
        case 4: __builtin_amdgcn_s_waitcnt(VH_VMCNT(4 * P)); break;
        case 5: __builtin_amdgcn_s_waitcnt(VH_VMCNT(5 * P)); break;
        default: __builtin_amdgcn_s_waitcnt(VH_VMCNT(6 * P)); break;
    }
}

// Reads 16 bytes at LDS byte address `addr` (completed before it returns).
__device__ __forceinline__ uint4 lds_read16(uint32_t addr) {
    uint4 v;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
    return v;
}
// Reads 4 bytes at LDS byte address `addr` (completed before it returns).
__device__ __forceinline__ uint32_t lds_read4(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
    return v;
}

// Offers one scored list entry (vector id `id`) to the wave's candidate buffer.
template <bool HIB>
__device__ __forceinline__ void offer(float total, bool valid, uint32_t id, unsigned long long *s_w, uint32_t &cnt,
                                      unsigned long long tau, unsigned long long lanes_below) {
    bool pass = false;
    unsigned long long cand = 0;
    if (valid) {
        const float hs = (HIB ? -total : total) + 0.0f;  // -0 sorts with +0
        cand = ((unsigned long long)score_key(hs) << 32) | id;
        pass = cand < tau;
    }
    const unsigned long long bal = __ballot(pass);
    if (pass) s_w[cnt + __popcll(bal & lanes_below)] = cand;
    cnt = __builtin_amdgcn_readfirstlane(cnt + (uint32_t)__popcll(bal));
}

// Floats of the coarse-row buffer of the DMA path: pg rows, rounded up to whole DMA instructions
// of one wave (64 lanes x 4 floats).
__host__ __device__ constexpr int coarse_rows_floats(int pg, int dim) { return (pg * dim + 255) / 256 * 256; }

// Wave 0 copies the coarse rows of probes pc[0, pg) into s_cr (row w at s_cr + w * dim) with
// global->LDS DMA; an invalid probe copies row 0 (its residual is never used).  dim % 4 == 0.
__device__ __forceinline__ void coarse_dma(const ScanArgs &A, const uint32_t *pc, float *s_cr, int pg, int lane) {
    const int pieces = pg * A.dim / 4;
    for (int i0 = 0; i0 < pieces; i0 += 64) {
        const int f = min(i0 + lane, pieces - 1);
        const int w = 4 * f / A.dim, d = 4 * f - w * A.dim;
        const uint32_t c = pc[w] != 0xffffffffu ? pc[w] : 0u;
        const uint32_t dst = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)(s_cr + 4 * i0);
        dma_lds16(A.coarse + (size_t)c * A.dim + d, __builtin_amdgcn_readfirstlane(dst));
    }
}

// Scan of one list through the DMA ring (code rows of 16 * NV bytes, 256 sub-centroids): the
// wave's chunks t < mine are chunks part + t * wpl of the list.  The table of probe slot SLOT
// sits at a compile-time LDS address (the start of dynamic LDS), so each lookup is one shift of
// a code byte plus an LDS read with the sub-space offset as its immediate.
struct RingScan {
    const uint8_t *codes;
    const uint32_t *ids;
    unsigned char *ring;   // this wave's ring (generic pointer into LDS)
    uint32_t ring_lds;     // its LDS byte address
    uint32_t beg, len;
    int part, wpl, mine, lane;
};

template <int NV>
__device__ __forceinline__ void ring_dma(const RingScan &R, int t) {
    const uint32_t i = min((uint32_t)((R.part + t * R.wpl) * 64 + R.lane), R.len - 1);
    const unsigned char *src = R.codes + (size_t)(R.beg + i) * (16 * NV);
    const uint32_t dst = __builtin_amdgcn_readfirstlane(R.ring_lds + (t % ring_chunks(NV)) * ring_chunk_bytes(NV));
#pragma unroll
    for (int v = 0; v < NV; ++v) dma_lds16(src + 16 * v, dst + v * 1024);
    dma_lds4(R.ids + R.beg + i, dst + NV * 1024);
}

// Reads the code pieces and ids of two ring chunks at LDS byte addresses a0 and a1 (lane
// offsets included) with one wait for all of them.  The outputs are early-clobber: a later read
// of the block still needs its address after an earlier one has written its result.
template <int NV>
__device__ __forceinline__ void lds_read_pair(uint32_t a0, uint32_t a1, uint32_t i0, uint32_t i1, uint4 (&w0)[NV],
                                              uint4 (&w1)[NV], uint32_t &id0, uint32_t &id1) {
    if constexpr (NV == 1) {
        asm volatile(
            "ds_read_b128 %0, %4\n\t"
            "ds_read_b128 %1, %5\n\t"
            "ds_read_b32 %2, %6\n\t"
            "ds_read_b32 %3, %7\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(w0[0]), "=&v"(w1[0]), "=&v"(id0), "=&v"(id1)
            : "v"(a0), "v"(a1), "v"(i0), "v"(i1)
            : "memory");
    } else {
        asm volatile(
            "ds_read_b128 %0, %6\n\t"
            "ds_read_b128 %1, %6 offset:1024\n\t"
            "ds_read_b128 %2, %7\n\t"
            "ds_read_b128 %3, %7 offset:1024\n\t"
            "ds_read_b32 %4, %8\n\t"
            "ds_read_b32 %5, %9\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(w0[0]), "=&v"(w0[1]), "=&v"(w1[0]), "=&v"(w1[1]), "=&v"(id0), "=&v"(id1)
            : "v"(a0), "v"(a1), "v"(i0), "v"(i1)
            : "memory");
    }
}

template <int NV>
__device__ __forceinline__ float ring_score(const float *lut, const uint4 (&w)[NV]) {
    constexpr int KS = 256;
    float total = 0.0f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        const uint32_t ww[4] = {w[v].x, w[v].y, w[v].z, w[v].w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const float *L = lut + (16 * v + 4 * h) * KS;
            const float d0 = L[ww[h] & 255u], d1 = L[KS + ((ww[h] >> 8) & 255u)];
            const float d2 = L[2 * KS + ((ww[h] >> 16) & 255u)], d3 = L[3 * KS + (ww[h] >> 24)];
            total += (d0 + d1) + (d2 + d3);
        }
    }
    return total;
}

// Chunks are taken two at a time.  Invariant: before the pair (t, t + 1) is read, the chunks
// below issued = min(t + NB - 2, mine) have been issued; after the read, the next two are.
template <int NV, int SLOT, bool HIB>
__device__ __forceinline__ void ring_scan(const ScanArgs &A, const RingScan &R, const float *s_lut0,
                                          unsigned long long *s_w, uint32_t &cnt, unsigned long long &tau, int capw,
                                          unsigned long long lanes_below) {
    constexpr int M = 16 * NV, KS = 256, NB = ring_chunks(NV), CB = ring_chunk_bytes(NV);
    const float *lut = s_lut0 + SLOT * M * KS;
    // wave-uniform loop state in scalar registers: the waits and DMA issues branch uniformly
    const int mine = __builtin_amdgcn_readfirstlane(R.mine);
    for (int t = 0; t < mine; t += 2) {
        if (cnt > (uint32_t)(capw - 128)) wave_compact(s_w, cnt, tau, A.k);
        const int issued = __builtin_amdgcn_readfirstlane(min(t + NB - 2, mine));
        const int last = __builtin_amdgcn_readfirstlane(min(t + 1, mine - 1));  // second chunk of the pair
        ring_wait<NV>(issued - 1 - last);
        const uint32_t s0 = R.ring_lds + (t % NB) * CB, s1 = R.ring_lds + (last % NB) * CB;
        uint4 w0[NV], w1[NV];
        uint32_t id0, id1;
        lds_read_pair<NV>(s0 + R.lane * 16, s1 + R.lane * 16, s0 + NV * 1024 + R.lane * 4,
                          s1 + NV * 1024 + R.lane * 4, w0, w1, id0, id1);
        if (issued < mine) ring_dma<NV>(R, issued);
        if (issued + 1 < mine) ring_dma<NV>(R, issued + 1);
        const float tot0 = ring_score<NV>(lut, w0);
        const float tot1 = ring_score<NV>(lut, w1);
        const uint32_t i0 = (uint32_t)((R.part + t * R.wpl) * 64 + R.lane);
        const uint32_t i1 = (uint32_t)((R.part + (t + 1) * R.wpl) * 64 + R.lane);
        const bool v0 = i0 < R.len, v1 = t + 1 < mine && i1 < R.len;
        // pre-filter (exact): a key below tau scores at most key_score(tau's score word)
        const float thr = key_score((uint32_t)(tau >> 32));
        const float h0 = (HIB ? -tot0 : tot0) + 0.0f, h1 = (HIB ? -tot1 : tot1) + 0.0f;
        if (__ballot((v0 && !(h0 > thr)) || (v1 && !(h1 > thr))) != 0ull) {
            offer<HIB>(tot0, v0, id0, s_w, cnt, tau, lanes_below);
            offer<HIB>(tot1, v1, id1, s_w, cnt, tau, lanes_below);
        }
    }
}

// Dynamic LDS: PG ADC tables, 4 x capw u64 candidates, the query, PG residuals and (NV > 0) the
// group's coarse rows; static LDS: the DMA rings (NV > 0) and the probe metadata of kMetaWin probes.
template <int MT, int DS, int NV>
__global__ __launch_bounds__(kScanThreads) void k_ivfpq_scan(ScanArgs A) {
    extern __shared__ unsigned long long s_dyn[];
    // the rings are their own LDS object: reads of the other LDS data then need no wait for
    // the DMAs in flight
    __shared__ __attribute__((aligned(16))) unsigned char s_ring[NV > 0 ? ring_bytes(NV) : 16];
    __shared__ uint32_t s_pc[kMetaWin], s_pb[kMetaWin], s_pl[kMetaWin];  // probe list, begin, length
    const int capw = A.capw, pg = A.pg, tstride = A.m_sub * A.ks;
    float *s_lut = reinterpret_cast<float *>(s_dyn);
    unsigned long long *s_all = reinterpret_cast<unsigned long long *>(s_lut + pg * tstride);
    float *s_q = reinterpret_cast<float *>(s_all + kScanWaves * capw);
    float *s_r = s_q + A.dim;
    float *s_cr = s_r + pg * A.dim;  // DMA path: the group's coarse rows (coarse_rows_floats)
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int slot = wave % pg, part = wave / pg, wpl = kScanWaves / pg;
    unsigned long long *s_w = s_all + wave * capw;
    unsigned char *ring = s_ring + wave * (ring_chunks(NV) * ring_chunk_bytes(NV));
    const unsigned long long lanes_below = (1ull << lane) - 1ull;

    float cbr[DS > 0 ? kLutRegs : 1];
    if constexpr (DS > 0) {
        const float4 *src = reinterpret_cast<const float4 *>(A.cbt + (size_t)threadIdx.x * kLutRegs);
#pragma unroll
        for (int v = 0; v < kLutRegs / 4; ++v) {
            const float4 f = src[v];
            cbr[4 * v] = f.x;
            cbr[4 * v + 1] = f.y;
            cbr[4 * v + 2] = f.z;
            cbr[4 * v + 3] = f.w;
        }
        // landed before any DMA is issued: the compiler would otherwise wait for them at their
        // first use with counts that also cover the DMAs, which it does not see
        __builtin_amdgcn_s_waitcnt(VH_VMCNT(0));
    }
    constexpr bool hib = hib_metric(MT);

    for (int q = blockIdx.x; q < A.nq; q += gridDim.x) {
        for (int d = threadIdx.x; d < A.dim; d += kScanThreads) s_q[d] = A.qry[(size_t)q * A.dim + d];
        uint32_t cnt = 0;
        unsigned long long tau = ~0ull;
        for (int g0 = 0; g0 < A.nprobe; g0 += pg) {
            const int wbase = g0 - g0 % kMetaWin;  // pg divides kMetaWin
            const int w0 = g0 - wbase;               // this group's first probe in the window
            lds_barrier();  // the previous group's tables, residuals and metadata are no longer read
            if (w0 == 0) {
                // probe lists and their bounds for the next kMetaWin probes (ivf/mod.rs:286-298:
                // empty lists, and slots past the last probe, get length 0)
                for (int t = threadIdx.x; t < kMetaWin; t += kScanThreads) {
                    const int p = wbase + t;
                    const uint32_t c = p < A.nprobe ? A.probes[(size_t)q * A.nprobe + p] : 0xffffffffu;
                    const bool ok = c < (uint32_t)A.nlist;  // an unfilled probe slot is skipped too
                    const uint32_t beg = ok ? A.list_off[c] : 0u;
                    s_pc[t] = ok ? c : 0xffffffffu;
                    s_pb[t] = beg;
                    s_pl[t] = ok ? A.list_off[c + 1] - beg : 0u;
                }
                if constexpr (NV > 0) {
                    lds_barrier();
                    if (wave == 0) {
                        coarse_dma(A, s_pc, s_cr, pg, lane);
                        __builtin_amdgcn_s_waitcnt(VH_VMCNT(0));
                    }
                }
                lds_barrier();
            }
            for (int t = threadIdx.x; t < pg * A.dim; t += kScanThreads) {
                const int w = t / A.dim, d = t - w * A.dim;
                const uint32_t c = s_pc[w0 + w];
                float r = 0.0f;
                if (c != 0xffffffffu) {
                    if constexpr (NV > 0)
                        r = s_q[d] - s_cr[t];
                    else
                        r = s_q[d] - A.coarse[(size_t)c * A.dim + d];
                }
                s_r[t] = r;
            }
            lds_barrier();
            // this wave's list; the DMA path scans chunks part + t * wpl (64 rows each), t < mine
            const uint32_t beg = s_pb[w0 + slot], len = s_pl[w0 + slot];
            const float *lut = s_lut + slot * tstride;
            const int nch = (int)((len + 63) / 64);
            RingScan R{A.codes, A.ids, ring, (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)ring,
                       beg, len, part, wpl, nch > part ? (nch - part + wpl - 1) / wpl : 0, lane};
            if constexpr (NV > 0) {
                // the next group's coarse rows (older than this group's ring DMAs, so landed once
                // any chunk has), then the first chunks of this wave's list: both land while the
                // tables are built
                if (wave == 0 && w0 + pg < kMetaWin && g0 + pg < A.nprobe) coarse_dma(A, s_pc + w0 + pg, s_cr, pg, lane);
                for (int t = 0; t < ring_chunks(NV) - 2 && t < R.mine; ++t) ring_dma<NV>(R, t);
            }
            if constexpr (DS > 0)
                lut_build_reg<MT, DS>(A, pg, s_r, s_lut, cbr);
            else
                lut_build_mem<MT>(A, pg, s_r, s_lut);
            lds_barrier();
            if constexpr (NV > 0) {
                const float *lut0 = reinterpret_cast<const float *>(s_dyn);
                switch (slot) {
                    case 0: ring_scan<NV, 0, hib>(A, R, lut0, s_w, cnt, tau, capw, lanes_below); break;
                    case 1: ring_scan<NV, 1, hib>(A, R, lut0, s_w, cnt, tau, capw, lanes_below); break;
                    case 2: ring_scan<NV, 2, hib>(A, R, lut0, s_w, cnt, tau, capw, lanes_below); break;
                    default: ring_scan<NV, 3, hib>(A, R, lut0, s_w, cnt, tau, capw, lanes_below); break;
                }
                __builtin_amdgcn_s_waitcnt(VH_VMCNT(0));  // every DMA of this wave has landed
            } else {
                for (uint32_t base = (uint32_t)part * 64 * kScanU; base < len;
                     base += (uint32_t)wpl * 64 * kScanU) {
                    if (cnt > (uint32_t)(capw - 64 * kScanU)) wave_compact(s_w, cnt, tau, A.k);
                    float total[kScanU];
                    uint32_t id[kScanU];
#pragma unroll
                    for (int u = 0; u < kScanU; ++u) {  // ids load with the codes
                        const uint32_t i = min(base + u * 64 + lane, len - 1);
                        id[u] = A.ids[beg + i];
                        total[u] = adc_score(A.codes + (size_t)(beg + i) * A.m_sub, lut, A.m_sub, A.ks);
                    }
#pragma unroll
                    for (int u = 0; u < kScanU; ++u) {
                        const uint32_t i = base + u * 64 + lane;
                        offer<hib>(total[u], i < len, id[u], s_w, cnt, tau, lanes_below);
                    }
                }
            }
        }
        for (int t = (int)cnt + lane; t < capw; t += 64) s_w[t] = ~0ull;
        __syncthreads();
        bitonic_sort_u64(s_all, kScanWaves * capw, threadIdx.x, kScanThreads, [] { __syncthreads(); });
        for (int j = threadIdx.x; j < A.k; j += kScanThreads) {
            const size_t o = (size_t)q * A.k + j;
            const unsigned long long cnd = s_all[j];
            if (cnd != ~0ull) {
                const float hs = key_score((uint32_t)(cnd >> 32));
                A.out_ids[o] = (uint32_t)cnd;
                A.out_dist[o] = hib ? -hs : hs;
            } else {
                A.out_ids[o] = 0xffffffffu;
                A.out_dist[o] = __builtin_nanf("");
            }
        }
        if (threadIdx.x == 0) {  // kept entries: the finite prefix of the first k
            int lo = 0, hi = A.k;
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (s_all[mid] != ~0ull) lo = mid + 1; else hi = mid;
            }
            A.out_len[q] = (uint32_t)lo;
        }
        __syncthreads();  // the candidate regions and s_q are reused by the next query
    }
}

// LDS of k_ivfpq_lists, the tables first: they lie at LDS offset 0, so a lookup takes its
// sub-space's table address as the instruction's offset.
struct ListLds {
    float4 lut[16 * 256];                                  // entry (m, e): the four pairs' values
    unsigned long long cand[kListQb * kListCapw];          // candidates (residuals before the scan)
    float score[2][kListQb][kListChunkRows];               // per chunk parity: each pair's row scores
    uint32_t item;
};

// Byte B of w times 16 (an offset into the float4 tables) in one SDWA shift.
template <int B>
__device__ __forceinline__ uint32_t byte_x16(uint32_t w) {
    uint32_t a;
    if constexpr (B == 0)
        asm("v_lshlrev_b32_sdwa %0, 4, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0" : "=v"(a) : "v"(w));
    else if constexpr (B == 1)
        asm("v_lshlrev_b32_sdwa %0, 4, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1" : "=v"(a) : "v"(w));
    else if constexpr (B == 2)
        asm("v_lshlrev_b32_sdwa %0, 4, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2" : "=v"(a) : "v"(w));
    else
        asm("v_lshlrev_b32_sdwa %0, 4, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3" : "=v"(a) : "v"(w));
    return a;
}

// The four pairs' scores of one code row (16 bytes) against the float4 tables at LDS offset 0:
// per pair, sum over words h of ((d0 + d1) + (d2 + d3)).
__device__ __forceinline__ float4 row_score4(const float4 *lut, uint4 w) {
    const char *base = reinterpret_cast<const char *>(lut);
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
    float4 total = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const char *L = base + 4 * h * 4096;
        const float4 d0 = *reinterpret_cast<const float4 *>(L + byte_x16<0>(ww[h]));
        const float4 d1 = *reinterpret_cast<const float4 *>(L + 4096 + byte_x16<1>(ww[h]));
        const float4 d2 = *reinterpret_cast<const float4 *>(L + 8192 + byte_x16<2>(ww[h]));
        const float4 d3 = *reinterpret_cast<const float4 *>(L + 12288 + byte_x16<3>(ww[h]));
        total.x += (d0.x + d1.x) + (d2.x + d3.x);
        total.y += (d0.y + d1.y) + (d2.y + d3.y);
        total.z += (d0.z + d1.z) + (d2.z + d3.z);
        total.w += (d0.w + d1.w) + (d2.w + d3.w);
    }
    return total;
}

template <int MT, int DS>
__global__ __launch_bounds__(kListThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_ivfpq_lists(ListArgs L) {
    constexpr int M = 16, KS = 256, QB = kListQb, CH = kListChunkRows;
    static_assert(kListThreads == KS && CH == 4 * 64 && QB == 4, "a thread per table entry; a row per lane");
    const ScanArgs &A = L.s;
    __shared__ __attribute__((aligned(16))) ListLds S;
    static_assert(QB * 128 * sizeof(float) <= sizeof(S.cand), "residuals of dim <= 128 fit");
    float *s_r = reinterpret_cast<float *>(S.cand);  // residuals, before the scan
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    constexpr int capw = kListCapw;
    unsigned long long *s_w = S.cand + wave * capw;
    const unsigned long long lanes_below = (1ull << lane) - 1ull;
    constexpr bool hib = hib_metric(MT);

    // sub-centroid tid of every sub-space, DS floats each (thread-major layout)
    float cbr[kLutRegs];
    {
        const float4 *src = reinterpret_cast<const float4 *>(A.cbt + (size_t)tid * kLutRegs);
#pragma unroll
        for (int v = 0; v < kLutRegs / 4; ++v) {
            const float4 f = src[v];
            cbr[4 * v] = f.x;
            cbr[4 * v + 1] = f.y;
            cbr[4 * v + 2] = f.z;
            cbr[4 * v + 3] = f.w;
        }
    }

    uint32_t next = 0;
    if (tid == 0) next = atomicAdd(L.work, 1u);
    const uint32_t n_items = *L.n_items;
    for (;;) {
        if (tid == 0) S.item = next;
        lds_barrier();  // also: every wave is past the previous item (its tables, scores and candidates)
        const uint32_t it = S.item;
        if (it >= n_items) break;
        const uint4 item = L.items[it], ip = L.item_pairs[it];
        const uint32_t list = item.x, beg = item.z, len = item.w >> 3, npairs = item.w & 7u;
        auto pair_of = [&](int sl) { return sl == 0 ? ip.x : sl == 1 ? ip.y : sl == 2 ? ip.z : ip.w; };
        const int nch = (int)((len + CH - 1) / CH);
        // residuals q - c of the item's pairs (zero rows for unused slots)
        for (int t = tid; t < QB * A.dim; t += kListThreads) {
            const int sl = t / A.dim, d = t - sl * A.dim;
            float r = 0.0f;
            if (sl < (int)npairs) {
                const uint32_t q = pair_of(sl) / (uint32_t)A.nprobe;
                r = A.qry[(size_t)q * A.dim + d] - A.coarse[(size_t)list * A.dim + d];
            }
            s_r[t] = r;
        }
        // the wave's pair (wave q offers pair q's candidates) and its query's k-th best key so far
        const bool active = wave < (int)npairs;
        const uint32_t pid = pair_of(wave);  // an unused slot repeats the first pair
        const uint32_t qid = pid / (uint32_t)A.nprobe;
        unsigned long long tau = __hip_atomic_load(L.tau_q + qid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (!active) tau = ~0ull;
        const uint32_t *tau_hi = reinterpret_cast<const uint32_t *>(L.tau_q + qid) + 1;
        // chunk c's loads: this lane's code row (row 64 wave + lane), the ids of the rows the wave
        // offers (rows lane + 64 st; rows past the list's end repeat its last row, never used) and
        // the score word of the query's k-th best key as other pairs have left it so far
        auto load_chunk = [&](int c, uint4 &w, uint32_t (&id)[4], uint32_t &th) {
            const uint32_t r = min((uint32_t)(c * CH + 64 * wave + lane), len - 1);
            w = *reinterpret_cast<const uint4 *>(A.codes + (size_t)(beg + r) * 16);
#pragma unroll
            for (int st = 0; st < 4; ++st) id[st] = A.ids[beg + min((uint32_t)(c * CH + 64 * st + lane), len - 1)];
            th = __hip_atomic_load(tau_hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        };
        uint4 wa, wb;
        uint32_t ida[4], idb[4], tha, thb;
        // the first chunk's loads are in flight during the table build, except for cosine, whose
        // build needs their registers (three sums a step) to stay at two waves per SIMD
        if constexpr (MT != COS) load_chunk(0, wa, ida, tha);
        if (tid == 0) next = atomicAdd(L.work, 1u);  // the next item's claim, in flight during the build
        lds_barrier();  // residuals visible
        // ADC tables (ProductQuantizer::compute_adc_lut, pq.rs:233-266): thread j computes entry j
        // of every sub-space for one slot at a time and stores it in component `slot` of the
        // entry's float4 (one slot at a time keeps the registers beside the codebook's few)
#pragma unroll
        for (int sl = 0; sl < QB; ++sl) {
            float e[M];
            {
                const float *r = s_r + sl * A.dim;
                constexpr int MB = 4, NR = MB * DS / 4;
#pragma unroll
                for (int m0 = 0; m0 < M; m0 += MB) {
                    float4 rv[NR];
#pragma unroll
                    for (int i = 0; i < NR; ++i) rv[i] = *reinterpret_cast<const float4 *>(r + m0 * DS + 4 * i);
#pragma unroll
                    for (int mm = 0; mm < MB; ++mm) {
                        const int m = m0 + mm;
                        Acc<MT> acc;
#pragma unroll
                        for (int d4 = 0; d4 < DS; d4 += 4) {
                            const float4 v = rv[(mm * DS + d4) / 4];
                            acc.step(v.x, cbr[m * DS + d4]);
                            acc.step(v.y, cbr[m * DS + d4 + 1]);
                            acc.step(v.z, cbr[m * DS + d4 + 2]);
                            acc.step(v.w, cbr[m * DS + d4 + 3]);
                        }
                        e[m] = acc.finish();
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < M; ++m) reinterpret_cast<float *>(&S.lut[m * KS + tid])[sl] = e[m];
        }
        if constexpr (MT == COS) load_chunk(0, wa, ida, tha);
        uint32_t cnt = 0;
        // tables visible; every residual read (the candidate buffers' LDS) done
        lds_barrier();
        // chunk c: score this wave's rows for the four pairs, then (after the barrier) offer pair
        // `wave`'s 256 scores
        auto do_chunk = [&](int c, const uint4 &w, const uint32_t (&id)[4], uint32_t ext_hi) {
            const float4 t4 = row_score4(S.lut, w);
            float *sc = &S.score[c & 1][0][64 * wave + lane];
            sc[0 * CH] = t4.x;
            sc[1 * CH] = t4.y;
            sc[2 * CH] = t4.z;
            sc[3 * CH] = t4.w;
            lds_barrier();  // the chunk's scores visible; every wave past chunk c - 2's reads
            if (active) {
                // the query's k-th best score as other pairs have left it; keys of that score pass
                // (a tie's id is not read), so the filter stays conservative
                const unsigned long long ext = ((unsigned long long)ext_hi << 32) | 0xffffffffull;
                tau = ext < tau ? ext : tau;
                float tot[4];
#pragma unroll
                for (int st = 0; st < 4; ++st) tot[st] = S.score[c & 1][wave][64 * st + lane];
                // Pre-filter: a key below tau has a score at most key_score(tau's score word) (NaN
                // scores, and tau = ~0, pass), so a chunk none of whose rows passes offers nothing.
                const float thr = key_score((uint32_t)(tau >> 32));
                bool maybe = false;
#pragma unroll
                for (int st = 0; st < 4; ++st) {
                    const float hs = (hib ? -tot[st] : tot[st]) + 0.0f;
                    maybe |= !(hs > thr) && (uint32_t)(c * CH + st * 64 + lane) < len;
                }
                if (__ballot(maybe) != 0ull) {
#pragma unroll
                    for (int st = 0; st < 4; ++st) {
                        if (cnt > (uint32_t)(capw - 64)) wave_compact(s_w, cnt, tau, A.k);
                        const uint32_t row = (uint32_t)(st * 64 + lane);
                        offer<hib>(tot[st], (uint32_t)(c * CH) + row < len, id[st], s_w, cnt, tau, lanes_below);
                    }
                }
            }
        };
        // two register sets, so that no loaded value is copied (a copy would wait for its load)
        for (int c = 0; c < nch; c += 2) {
            load_chunk(c + 1, wb, idb, thb);
            do_chunk(c, wa, ida, tha);
            load_chunk(c + 2, wa, ida, tha);
            if (c + 1 < nch) do_chunk(c + 1, wb, idb, thb);
        }
        if (active) {
            wave_compact(s_w, cnt, tau, A.k);  // sorted, at most k kept
            for (int j = lane; j < A.k; j += 64)
                L.pair_out[(size_t)pid * A.k + j] = j < (int)cnt ? s_w[j] : ~0ull;
            if (lane == 0 && cnt >= (uint32_t)A.k) atomicMin(L.tau_q + qid, s_w[A.k - 1]);
        }
    }
}

// Per query: the k best of its nprobe pairs' k best (pairs of unused probe slots count as empty);
// writes ids, distances and the count as k_ivfpq_scan does.  The query's final k best are all at
// or below tau_q (the smallest k-th key of its pairs, or ~0 while no pair held k), so only those
// keys are kept, in arbitrary order through an LDS counter, and sorted.  Dynamic LDS: P keys, P
// the power of two >= nprobe * k.
template <bool HIB>
__global__ __launch_bounds__(256) void k_ivfpq_merge(ListArgs L, int P) {
    const ScanArgs &A = L.s;
    extern __shared__ unsigned long long s_keys[];
    __shared__ uint32_t s_n;
    const int n = A.nprobe * A.k;
    for (int q = blockIdx.x; q < A.nq; q += gridDim.x) {
        const unsigned long long tq = L.tau_q[q];
        if (threadIdx.x == 0) s_n = 0;
        __syncthreads();
        for (int t = threadIdx.x; t < n; t += 256) {
            const int p = t / A.k;
            if (A.probes[(size_t)q * A.nprobe + p] < (uint32_t)A.nlist) {
                const unsigned long long key = L.pair_out[(size_t)q * n + t];
                if (key != ~0ull && key <= tq) s_keys[atomicAdd(&s_n, 1u)] = key;
            }
        }
        __syncthreads();
        const int m = (int)s_n;
        int P2 = 1;
        while (P2 < m) P2 <<= 1;
        for (int t = m + (int)threadIdx.x; t < max(P2, A.k); t += 256) s_keys[t] = ~0ull;
        __syncthreads();
        bitonic_sort_u64(s_keys, P2, threadIdx.x, 256, [] { __syncthreads(); });
        for (int j = threadIdx.x; j < A.k; j += 256) {
            const size_t o = (size_t)q * A.k + j;
            const unsigned long long cnd = s_keys[j];
            if (cnd != ~0ull) {
                const float hs = key_score((uint32_t)(cnd >> 32));
                A.out_ids[o] = (uint32_t)cnd;
                A.out_dist[o] = HIB ? -hs : hs;
            } else {
                A.out_ids[o] = 0xffffffffu;
                A.out_dist[o] = __builtin_nanf("");
            }
        }
        if (threadIdx.x == 0) A.out_len[q] = (uint32_t)min(m, A.k);
        __syncthreads();
    }
}

template <int MT>
void launch_lists_mt(const ListArgs &L, int ds, int cus, hipStream_t s) {
    // persistent: as many workgroups as fit (each CU holds 163840 bytes of LDS)
    const size_t per_cu = std::max<size_t>(1, 163840 / (sizeof(ListLds) + 256));
    const unsigned grid = (unsigned)((size_t)cus * per_cu);
    if (ds == 4)
        scan_launch((k_ivfpq_lists<MT, 4>), dim3(grid), dim3(kListThreads), 0, s, L);
    else
        scan_launch((k_ivfpq_lists<MT, 8>), dim3(grid), dim3(kListThreads), 0, s, L);
}

template <bool HIB>
void launch_lists_merge(const ListArgs &L, int cus, hipStream_t s) {
    int P = 2;
    while (P < L.s.nprobe * L.s.k) P <<= 1;
    const unsigned mg = (unsigned)std::min<long>((long)L.s.nq, 4L * cus);
    hipLaunchKernelGGL((k_ivfpq_merge<HIB>), dim3(mg), dim3(256), (size_t)P * 8, s, L, P);
}

// Launches one persistent workgroup per resident slot (the occupancy of this instantiation at
// `lds` bytes of dynamic LDS on `cus` compute units), at most one per query.
template <class K>
void launch_resident(K kernel, const ScanArgs &A, int cus, size_t lds, hipStream_t s) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kScanThreads, lds) != hipSuccess ||
        per_cu < 1) {
        (void)hipGetLastError();
        per_cu = 1;
    }
    const unsigned grid = (unsigned)std::min<long>((long)A.nq, (long)per_cu * cus);
    scan_launch(kernel, dim3(grid), dim3(kScanThreads), lds, s, A);
}

template <int MT, int DS>
void launch_scan_nv(const ScanArgs &A, int nv, int cus, size_t lds, hipStream_t s) {
    if (nv == 1)
        launch_resident(k_ivfpq_scan<MT, DS, 1>, A, cus, lds, s);
    else if (nv == 2)
        launch_resident(k_ivfpq_scan<MT, DS, 2>, A, cus, lds, s);
    else
        launch_resident(k_ivfpq_scan<MT, DS, 0>, A, cus, lds, s);
}

template <int MT>
void launch_scan_reg(const ScanArgs &A, int ds, int nv, int cus, size_t lds, hipStream_t s) {
    switch (ds) {
        case 4: launch_scan_nv<MT, 4>(A, nv, cus, lds, s); break;
        case 8: launch_scan_nv<MT, 8>(A, nv, cus, lds, s); break;
        case 16: launch_scan_nv<MT, 16>(A, nv, cus, lds, s); break;
        default: launch_scan_nv<MT, 32>(A, nv, cus, lds, s); break;
    }
}

}  // namespace

// Dynamic LDS bytes of k_ivfpq_scan (pg tables, candidates for capw slots per wave, query, pg
// residuals, coarse rows for NV > 0); the rings of NV pieces add ring_bytes(nv) of static LDS and
// the probe metadata 3 x kMetaWin words.
inline size_t scan_lds_bytes(size_t dim, size_t m_sub, size_t ks, int capw, int pg, int nv) {
    return (size_t)kScanWaves * capw * sizeof(unsigned long long) +
           ((1 + pg) * dim + pg * m_sub * ks + (nv > 0 ? coarse_rows_floats(pg, (int)dim) : 0)) * sizeof(float);
}

// Launchers (pq_scan_l2.hip, pq_scan_ip.hip, pq_scan_mem.hip).  `ds` selects the register-path
// instantiation (4, 8, 16 or 32), `nv` the DMA ring (0, 1 or 2); `cus` is the device's CU count.
void launch_ivfpq_scan_l2(const ScanArgs &A, int ds, int nv, int cus, size_t lds, hipStream_t s);
void launch_ivfpq_scan_ip(const ScanArgs &A, int ds, int nv, int cus, size_t lds, hipStream_t s);
void launch_ivfpq_scan_mem(const ScanArgs &A, int nv, int cus, size_t lds, hipStream_t s);
// List-major scan and merge (16-byte code rows, 256 sub-centroids, ds 4 or 8, k <= kListMaxK,
// nprobe * k <= kListMaxMerge); the plan (pairs, items, counters) is built by ivfpq_list_plan.
void launch_ivfpq_lists_l2(const ListArgs &L, int ds, int cus, hipStream_t s);
void launch_ivfpq_lists_ip(const ListArgs &L, int ds, int cus, hipStream_t s);
// The merge of the pairs' k best into each query's (after either list launch).
void launch_ivfpq_list_merge(const ListArgs &L, int cus, hipStream_t s);
// Groups the nq x nprobe probes by list: cnt / cursor (nlist each) must be zero; order lists the
// lists by decreasing size; writes pairs, items, *n_items (and pair_off, item_off: nlist each).
void ivfpq_list_plan(const uint32_t *probes, int nq, int nprobe, int nlist, const uint32_t *order,
                     const uint32_t *list_off, uint32_t *cnt, uint32_t *cursor, uint32_t *pair_off,
                     uint32_t *item_off, uint32_t *pairs, uint4 *items, uint4 *item_pairs, uint32_t *n_items,
                     hipStream_t s);

}  // namespace vh
