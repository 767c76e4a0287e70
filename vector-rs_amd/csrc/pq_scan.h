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
// With 256 sub-centroids, code rows of 16 or 32 bytes (NV = 1 or 2 sixteen-byte pieces) stream
// into a per-wave ring of NB chunks of 64 rows (NB = 8 or 4) with global->LDS DMA (no registers
// held), NB - 1 chunks ahead of the row being scored; the first NB - 1, which cover a wave's share
// of a typical list, are issued before the tables are built and land while they are.  A chunk is read only
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
// DMA ring depth in chunks of 64 code rows: 8 chunks of 16-byte rows (8 KB per wave), 4 of 32-byte
constexpr int ring_chunks(int nv) { return nv == 2 ? 4 : 8; }

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

// LDS bytes of the per-wave DMA rings for code rows of NV sixteen-byte pieces.
constexpr int ring_bytes(int nv) { return kScanWaves * ring_chunks(nv) * nv * 64 * 16; }

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

// s_waitcnt immediate that waits until at most n (< 16) vector memory operations are
// outstanding, leaving the export and LDS counters unconstrained.
#define VH_VMCNT(n) (((n) & 15) | (7 << 4) | (15 << 8))

// Waits until at most `younger` (<= ring_chunks(NV) - 2) chunks of NV DMAs each are still in
// flight: s_waitcnt takes its count as an immediate, hence one case per count.
template <int NV>
__device__ __forceinline__ void ring_wait(int younger) {
    static_assert((ring_chunks(NV) - 2) * NV < 16, "vmcnt immediates stay below 16");
    switch (younger) {
        case 0: __builtin_amdgcn_s_waitcnt(VH_VMCNT(0)); break;
        case 1: __builtin_amdgcn_s_waitcnt(VH_VMCNT(NV)); break;
        case 2: __builtin_amdgcn_s_waitcnt(VH_VMCNT(2 * NV)); break;
        case 3: __builtin_amdgcn_s_waitcnt(VH_VMCNT(3 * NV)); break;
        case 4: __builtin_amdgcn_s_waitcnt(VH_VMCNT(4 * NV)); break;
        case 5: __builtin_amdgcn_s_waitcnt(VH_VMCNT(5 * NV)); break;
        default: __builtin_amdgcn_s_waitcnt(VH_VMCNT(6 * NV)); break;
    }
}

// Reads 16 bytes at LDS byte address `addr` (completed before it returns).
__device__ __forceinline__ uint4 lds_read16(uint32_t addr) {
    uint4 v;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
    return v;
}

// Offers one scored row to the wave's candidate buffer.
template <bool HIB>
__device__ __forceinline__ void offer(const ScanArgs &A, float total, bool valid, uint32_t row,
                                      unsigned long long *s_w, uint32_t &cnt, unsigned long long tau,
                                      unsigned long long lanes_below) {
    bool pass = false;
    unsigned long long cand = 0;
    if (valid) {
        const float hs = (HIB ? -total : total) + 0.0f;  // -0 sorts with +0
        const uint32_t key = score_key(hs);
        if (key <= (uint32_t)(tau >> 32)) {
            cand = ((unsigned long long)key << 32) | A.ids[row];
            pass = cand < tau;
        }
    }
    const unsigned long long bal = __ballot(pass);
    if (pass) s_w[cnt + __popcll(bal & lanes_below)] = cand;
    cnt += (uint32_t)__popcll(bal);
}

// Scan of one list through the DMA ring (code rows of 16 * NV bytes, 256 sub-centroids): the
// wave's chunks t < mine are chunks part + t * wpl of the list.  The table of probe slot SLOT
// sits at a compile-time LDS address (the start of dynamic LDS), so each lookup is one shift of
// a code byte plus an LDS read with the sub-space offset as its immediate.
struct RingScan {
    const uint8_t *codes;
    unsigned char *ring;   // this wave's ring (generic pointer into LDS)
    uint32_t ring_lds;     // its LDS byte address
    uint32_t beg, len;
    int part, wpl, mine, lane;
};

template <int NV>
__device__ __forceinline__ void ring_dma(const RingScan &R, int t) {
    const uint32_t i = min((uint32_t)((R.part + t * R.wpl) * 64 + R.lane), R.len - 1);
    const unsigned char *src = R.codes + (size_t)(R.beg + i) * (16 * NV);
    unsigned char *dst = R.ring + (t % ring_chunks(NV)) * (NV * 1024);
#pragma unroll
    for (int v = 0; v < NV; ++v)
        __builtin_amdgcn_global_load_lds((const void *)(src + 16 * v),
                                         (__attribute__((address_space(3))) void *)(dst + v * 1024), 16, 0, 0);
}

template <int NV, int SLOT, bool HIB>
__device__ __forceinline__ void ring_scan(const ScanArgs &A, const RingScan &R, const float *s_lut0,
                                          unsigned long long *s_w, uint32_t &cnt, unsigned long long &tau, int capw,
                                          unsigned long long lanes_below) {
    constexpr int M = 16 * NV, KS = 256, NB = ring_chunks(NV);
    const float *lut = s_lut0 + SLOT * M * KS;
    for (int t = 0; t < R.mine; ++t) {
        if (cnt > (uint32_t)(capw - 64)) wave_compact(s_w, cnt, tau, A.k);
        ring_wait<NV>(min(NB - 2, R.mine - 1 - t));
        const uint32_t at = R.ring_lds + (t % NB) * (NV * 1024) + R.lane * 16;
        uint4 w[NV];
#pragma unroll
        for (int v = 0; v < NV; ++v) w[v] = lds_read16(at + v * 1024);
        if (t + NB - 1 < R.mine) ring_dma<NV>(R, t + NB - 1);
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
        const uint32_t i = (uint32_t)((R.part + t * R.wpl) * 64 + R.lane);
        offer<HIB>(A, total, i < R.len, R.beg + i, s_w, cnt, tau, lanes_below);
    }
}

// Dynamic LDS: PG ADC tables, 4 x capw u64 candidates, the query and PG residuals; static LDS:
// the DMA rings (NV > 0).
template <int MT, int DS, int NV>
__global__ __launch_bounds__(kScanThreads) void k_ivfpq_scan(ScanArgs A) {
    extern __shared__ unsigned long long s_dyn[];
    // the rings are their own LDS object: reads of the other LDS data then need no wait for
    // the DMAs in flight
    __shared__ __attribute__((aligned(16))) unsigned char s_ring[NV > 0 ? ring_bytes(NV) : 16];
    __shared__ uint32_t s_mc[kScanWaves], s_mb[kScanWaves], s_ml[kScanWaves];
    const int capw = A.capw, pg = A.pg, tstride = A.m_sub * A.ks;
    float *s_lut = reinterpret_cast<float *>(s_dyn);
    unsigned long long *s_all = reinterpret_cast<unsigned long long *>(s_lut + pg * tstride);
    float *s_q = reinterpret_cast<float *>(s_all + kScanWaves * capw);
    float *s_r = s_q + A.dim;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int slot = wave % pg, part = wave / pg, wpl = kScanWaves / pg;
    unsigned long long *s_w = s_all + wave * capw;
    unsigned char *ring = s_ring + wave * (ring_chunks(NV) * NV * 1024);
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
    }
    constexpr bool hib = hib_metric(MT);

    for (int q = blockIdx.x; q < A.nq; q += gridDim.x) {
        for (int d = threadIdx.x; d < A.dim; d += kScanThreads) s_q[d] = A.qry[(size_t)q * A.dim + d];
        uint32_t cnt = 0;
        unsigned long long tau = ~0ull;
        for (int g0 = 0; g0 < A.nprobe; g0 += pg) {
            __syncthreads();  // the previous group's tables are no longer read; s_q is written
            if (threadIdx.x < pg) {
                const int p = g0 + threadIdx.x;
                const uint32_t c = p < A.nprobe ? A.probes[(size_t)q * A.nprobe + p] : 0xffffffffu;
                const bool ok = c < (uint32_t)A.nlist;  // past the last probe, or an unfilled slot
                const uint32_t beg = ok ? A.list_off[c] : 0u;
                s_mc[threadIdx.x] = ok ? c : 0xffffffffu;
                s_mb[threadIdx.x] = beg;
                s_ml[threadIdx.x] = ok ? A.list_off[c + 1] - beg : 0u;
            }
            __syncthreads();
            for (int t = threadIdx.x; t < pg * A.dim; t += kScanThreads) {
                const int w = t / A.dim, d = t - w * A.dim;
                const uint32_t c = s_mc[w];
                s_r[t] = c != 0xffffffffu ? s_q[d] - A.coarse[(size_t)c * A.dim + d] : 0.0f;
            }
            // this wave's list (empty lists, ivf/mod.rs:296-298, have length 0)
            const uint32_t beg = s_mb[slot], len = s_ml[slot];
            const float *lut = s_lut + slot * tstride;
            // DMA path: the wave's chunks are part + t * wpl (64 rows each), t < mine
            const int nch = (int)((len + 63) / 64);
            RingScan R{A.codes, ring, (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)ring, beg, len,
                       part, wpl, nch > part ? (nch - part + wpl - 1) / wpl : 0, lane};
            if constexpr (NV > 0) {
                for (int t = 0; t < ring_chunks(NV) - 1 && t < R.mine; ++t) ring_dma<NV>(R, t);  // lands during the tables
            }
            __syncthreads();
            if constexpr (DS > 0)
                lut_build_reg<MT, DS>(A, pg, s_r, s_lut, cbr);
            else
                lut_build_mem<MT>(A, pg, s_r, s_lut);
            __syncthreads();
            if constexpr (NV > 0) {
                const float *lut0 = reinterpret_cast<const float *>(s_dyn);
                switch (slot) {
                    case 0: ring_scan<NV, 0, hib>(A, R, lut0, s_w, cnt, tau, capw, lanes_below); break;
                    case 1: ring_scan<NV, 1, hib>(A, R, lut0, s_w, cnt, tau, capw, lanes_below); break;
                    case 2: ring_scan<NV, 2, hib>(A, R, lut0, s_w, cnt, tau, capw, lanes_below); break;
                    default: ring_scan<NV, 3, hib>(A, R, lut0, s_w, cnt, tau, capw, lanes_below); break;
                }
            } else {
                for (uint32_t base = (uint32_t)part * 64 * kScanU; base < len;
                     base += (uint32_t)wpl * 64 * kScanU) {
                    if (cnt > (uint32_t)(capw - 64 * kScanU)) wave_compact(s_w, cnt, tau, A.k);
                    float total[kScanU];
#pragma unroll
                    for (int u = 0; u < kScanU; ++u) {
                        const uint32_t i = min(base + u * 64 + lane, len - 1);
                        total[u] = adc_score(A.codes + (size_t)(beg + i) * A.m_sub, lut, A.m_sub, A.ks);
                    }
#pragma unroll
                    for (int u = 0; u < kScanU; ++u) {
                        const uint32_t i = base + u * 64 + lane;
                        offer<hib>(A, total[u], i < len, beg + i, s_w, cnt, tau, lanes_below);
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
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kScanThreads), lds, s, A);
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

// Dynamic LDS bytes of k_ivfpq_scan (candidates for capw slots per wave, query, pg residuals and
// pg tables); the rings of NV pieces add ring_bytes(nv) of static LDS.
inline size_t scan_lds_bytes(size_t dim, size_t m_sub, size_t ks, int capw, int pg) {
    return (size_t)kScanWaves * capw * sizeof(unsigned long long) + ((1 + pg) * dim + pg * m_sub * ks) * sizeof(float);
}

// Launchers (pq_scan_l2.hip, pq_scan_ip.hip, pq_scan_mem.hip).  `ds` selects the register-path
// instantiation (4, 8, 16 or 32), `nv` the DMA ring (0, 1 or 2); `cus` is the device's CU count.
void launch_ivfpq_scan_l2(const ScanArgs &A, int ds, int nv, int cus, size_t lds, hipStream_t s);
void launch_ivfpq_scan_ip(const ScanArgs &A, int ds, int nv, int cus, size_t lds, hipStream_t s);
void launch_ivfpq_scan_mem(const ScanArgs &A, int nv, int cus, size_t lds, hipStream_t s);

}  // namespace vh
