// pq.hip -- product quantization and the IVF-PQ index on one GPU behind the C ABI.
//
// ProductQuantizer (vector-index/src/ivf/pq.rs) and IvfPqIndex (ivf/mod.rs):
//  * train: one k-means per sub-space (pq.rs:53-107) on the GPU k-means engine;
//  * encode (pq.rs:178-214): k_pq_encode, one thread per (vector, sub-space), the strict-compare
//    argmin of find_nearest_centroid (ivf/kmeans.rs:262-309) over the sub-space's codebook in LDS;
//  * compute_adc_lut (pq.rs:233-266): k_pq_lut, one thread per table entry;
//  * search (ivf/mod.rs:256-345): coarse probe through a kNN engine over the coarse centroids
//    (k = nprobe, best first), then k_ivfpq_scan: one workgroup per query walks its probed lists
//    in probe order, builds each list's ADC table in LDS from the query residual (codebooks held
//    in registers, one sub-centroid column per thread), scores every code with the reference's
//    summation order (pq.rs:270-293); each wave keeps its own threshold-filtered candidate buffer
//    in LDS, sorted down to its k best whenever it fills, and the four buffers are sorted together
//    at the end of the query.
//
// Candidate keys are (order-preserving score key << 32) | vector id, so the k best are unique
// and equal scores are ordered by ascending id.  The reference keeps, among entries that tie at
// the k-th score, whichever its BinaryHeap keeps; the sets differ only inside such a tie.
#include <algorithm>
#include <cmath>
#include <memory>
#include <vector>

#include "vh_runtime.h"

namespace vh {
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

// ---- encode -------------------------------------------------------------------------------
constexpr int kEncRegDims = 32;          // sub-vector floats held in registers
constexpr int kEncLdsFloats = 16384;     // codebooks up to 64 KB are staged in LDS

// Block (x, m): 256 vectors, sub-space m.  Codebook m in LDS when it fits (cb_lds), else read
// through the caches.
template <int MT>
__global__ __launch_bounds__(256) void k_pq_encode(const float *__restrict__ x, long n, int dim, int m_sub, int ks,
                                                   int ds, const float *__restrict__ cb, int cb_lds,
                                                   uint8_t *__restrict__ codes) {
    extern __shared__ float s_cb[];
    const int m = blockIdx.y;
    const float *cbm = cb + (size_t)m * ks * ds;
    if (cb_lds) {
        for (int t = threadIdx.x; t < ks * ds; t += 256) s_cb[t] = cbm[t];
        __syncthreads();
    }
    const float *cw = cb_lds ? s_cb : cbm;
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float *xs = x + i * dim + (long)m * ds;
    constexpr bool hib = hib_metric(MT);
    float best = hib ? -INFINITY : INFINITY;
    int bi = 0;
    if (ds <= kEncRegDims) {
        float xr[kEncRegDims];
#pragma unroll
        for (int d = 0; d < kEncRegDims; ++d) xr[d] = d < ds ? xs[d] : 0.0f;
        for (int j = 0; j < ks; ++j) {
            Acc<MT> acc;
            const float *c = cw + j * ds;
#pragma unroll
            for (int d = 0; d < kEncRegDims; ++d)
                if (d < ds) acc.step(xr[d], c[d]);
            const float v = acc.finish();
            if (hib ? v > best : v < best) {
                best = v;
                bi = j;
            }
        }
    } else {
        for (int j = 0; j < ks; ++j) {
            Acc<MT> acc;
            const float *c = cw + j * ds;
            for (int d = 0; d < ds; ++d) acc.step(xs[d], c[d]);
            const float v = acc.finish();
            if (hib ? v > best : v < best) {
                best = v;
                bi = j;
            }
        }
    }
    codes[i * m_sub + m] = (uint8_t)bi;
}

// ---- ADC table for a batch of queries: lut[q][m][j] --------------------------------------
template <int MT>
__global__ __launch_bounds__(256) void k_pq_lut(const float *__restrict__ qry, long total, int dim, int m_sub, int ks,
                                                int ds, const float *__restrict__ cb, float *__restrict__ lut) {
    const long t = (long)blockIdx.x * 256 + threadIdx.x;
    if (t >= total) return;
    const int j = (int)(t % ks);
    const long r = t / ks;
    const int m = (int)(r % m_sub);
    const long q = r / m_sub;
    const float *xs = qry + q * dim + (long)m * ds;
    const float *c = cb + ((size_t)m * ks + j) * ds;
    Acc<MT> acc;
    for (int d = 0; d < ds; ++d) acc.step(xs[d], c[d]);
    lut[t] = acc.finish();
}

// ---- IVF-PQ scan ------------------------------------------------------------------------------
constexpr int kScanThreads = 256;
constexpr int kScanWaves = kScanThreads / 64;
constexpr int kLutRegs = 128;       // codebook floats per thread in the register layout

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
    int capw;                  // candidate slots per wave, a power of two >= k + 64
};

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
__device__ void wave_compact(unsigned long long *s_w, uint32_t &cnt, unsigned long long &tau, int k) {
    const int lane = threadIdx.x & 63;
    int P = 2;
    while (P < (int)cnt) P <<= 1;
    for (int t = (int)cnt + lane; t < P; t += 64) s_w[t] = ~0ull;
    wave_sync();
    bitonic_sort_u64(s_w, P, lane, 64, wave_sync);
    if ((int)cnt >= k) tau = s_w[k - 1];
    cnt = min((int)cnt, k);
}

// ADC table of one probe: thread t = (group g, sub-centroid j) writes lut[m][j] for the group's
// sub-spaces.  Register path: DS = sub-dimension, codebook column in cbr.
template <int MT, int DS>
__device__ __forceinline__ void lut_build_reg(const ScanArgs &A, const float *s_r, float *s_lut, const float *cbr) {
    const int g = threadIdx.x / A.ks, j = threadIdx.x - g * A.ks;
    if (g >= A.groups) return;
    const int m0 = g * A.mg;
#pragma unroll
    for (int ml = 0; ml < kLutRegs / DS; ++ml) {
        if (ml < A.mg && m0 + ml < A.m_sub) {
            Acc<MT> acc;
#pragma unroll
            for (int d = 0; d < DS; ++d) acc.step(s_r[(m0 + ml) * DS + d], cbr[ml * DS + d]);
            s_lut[(m0 + ml) * A.ks + j] = acc.finish();
        }
    }
}

template <int MT>
__device__ __forceinline__ void lut_build_mem(const ScanArgs &A, const float *s_r, float *s_lut) {
    const int g = threadIdx.x / A.ks, j = threadIdx.x - g * A.ks;
    if (g >= A.groups) return;
    const int m0 = g * A.mg, m1 = min(A.m_sub, m0 + A.mg);
    for (int m = m0; m < m1; ++m) {
        const float *c = A.cb + ((size_t)m * A.ks + j) * A.ds;
        Acc<MT> acc;
        for (int d = 0; d < A.ds; ++d) acc.step(s_r[m * A.ds + d], c[d]);
        s_lut[m * A.ks + j] = acc.finish();
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

// One workgroup per query (grid-stride over queries).  Each wave scans every fourth run of 64
// list entries into its own candidate region with its own threshold, so the scan needs no
// workgroup barrier; the four regions are sorted together at the end of the query.
// Dynamic LDS: 4 x capw u64 candidates, then the query, the residual and the ADC table.
template <int MT, int DS>
__global__ __launch_bounds__(kScanThreads) void k_ivfpq_scan(ScanArgs A) {
    extern __shared__ unsigned long long s_dyn[];
    const int capw = A.capw;
    unsigned long long *s_all = s_dyn;
    float *s_q = reinterpret_cast<float *>(s_dyn + kScanWaves * capw);
    float *s_r = s_q + A.dim;
    float *s_lut = s_r + A.dim;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    unsigned long long *s_w = s_all + wave * capw;
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
        for (int p = 0; p < A.nprobe; ++p) {
            const uint32_t c = A.probes[(size_t)q * A.nprobe + p];
            if (c >= (uint32_t)A.nlist) continue;  // an unfilled probe slot
            const uint32_t beg = A.list_off[c], len = A.list_off[c + 1] - beg;
            if (len == 0) continue;  // ivf/mod.rs:296-298
            __syncthreads();         // the previous table is no longer read; s_q is written
            for (int d = threadIdx.x; d < A.dim; d += kScanThreads) s_r[d] = s_q[d] - A.coarse[(size_t)c * A.dim + d];
            __syncthreads();
            if constexpr (DS > 0)
                lut_build_reg<MT, DS>(A, s_r, s_lut, cbr);
            else
                lut_build_mem<MT>(A, s_r, s_lut);
            __syncthreads();
            for (uint32_t base = (uint32_t)wave * 64; base < len; base += kScanThreads) {
                if (cnt > (uint32_t)(capw - 64)) wave_compact(s_w, cnt, tau, A.k);
                const uint32_t i = base + lane;
                bool pass = false;
                unsigned long long cand = 0;
                if (i < len) {
                    const float total = adc_score(A.codes + (size_t)(beg + i) * A.m_sub, s_lut, A.m_sub, A.ks);
                    const float hs = (hib ? -total : total) + 0.0f;  // -0 sorts with +0
                    const uint32_t key = score_key(hs);
                    if (key <= (uint32_t)(tau >> 32)) {
                        cand = ((unsigned long long)key << 32) | A.ids[beg + i];
                        pass = cand < tau;
                    }
                }
                const unsigned long long bal = __ballot(pass);
                if (pass) s_w[cnt + __popcll(bal & lanes_below)] = cand;
                cnt += (uint32_t)__popcll(bal);
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

}  // namespace

// Register-layout eligibility: squared L2, dot or cosine, sub-dimension 4, 8, 16 or 32, and
// the group's sub-spaces fit kLutRegs floats.  Other shapes build the table from codebooks read
// through the caches.
static bool lut_reg_layout(int metric, size_t m_sub, size_t ks, size_t ds, int *groups, int *mg) {
    const int G = (int)(kScanThreads / ks);
    const int Mg = (int)((m_sub + G - 1) / G);
    *groups = G;
    *mg = Mg;
    const bool fast_metric = metric == L2 || metric == DOT || metric == COS;
    const bool pow2 = ds == 4 || ds == 8 || ds == 16 || ds == 32;
    return fast_metric && pow2 && (size_t)Mg * ds <= (size_t)kLutRegs;
}

// Candidate slots per wave for k results: room for k kept plus one 64-entry step.
static int scan_capw(size_t k) {
    int c = 256;
    while ((size_t)c < k + 64) c <<= 1;
    return c;
}

static size_t scan_lds_bytes(size_t dim, size_t m_sub, size_t ks, size_t k) {
    return (size_t)kScanWaves * scan_capw(k) * sizeof(unsigned long long) + (2 * dim + m_sub * ks) * sizeof(float);
}

}  // namespace vh

using namespace vh;

// ================================================================================================
struct vhip_ivfpq {
    int dev = 0;
    size_t dim = 0, nlist = 0, m_sub = 0, ks = 0, ds = 0, n = 0;
    int metric = 0;
    vhip_ivfpq_config cfg{};
    bool reg = false;
    int groups = 1, mg = 1;
    size_t lds_limit = 65536;  // dynamic LDS bytes per workgroup the device accepts
    std::vector<float> coarse, codebooks;  // host copies (export / save)
    std::vector<uint32_t> list_off;        // nlist + 1
    std::vector<uint32_t> ids;             // list order
    std::vector<uint8_t> codes;            // list order
    vhip_knn *probe = nullptr;
    hipStream_t stream = nullptr;
    DevBuf d_coarse, d_cb, d_cbt, d_off, d_ids, d_codes;
    DevBuf d_q, d_pid, d_pdist, d_oid, d_odist, d_olen;
    PinnedStager stager;
    KernelTimer timer;
    std::mutex mu;
    ~vhip_ivfpq() {
        if (probe) vhip_knn_destroy(probe);
        if (stream) {
            (void)hipSetDevice(dev);
            (void)hipStreamSynchronize(stream);
            (void)hipStreamDestroy(stream);
        }
    }
};

namespace vh {

static int pq_check_shape(size_t dim, size_t m_sub, size_t ks, int metric) {
    if (metric < 0 || metric > 9) return set_error(VHIP_ERR_INVALID_CONFIG, "unknown metric code");
    if (dim == 0) return set_error(VHIP_ERR_INVALID_CONFIG, "dimension must be > 0");
    if (m_sub == 0 || dim % m_sub != 0)
        return set_error(VHIP_ERR_INVALID_CONFIG, "vector dimension (" + std::to_string(dim) +
                                                      ") must be divisible by num_subvectors (" +
                                                      std::to_string(m_sub) + ")");
    if (ks == 0 || ks > 256)
        return set_error(VHIP_ERR_INVALID_CONFIG,
                         "sub_clusters must be between 1 and 256, got " + std::to_string(ks));
    return VHIP_OK;
}

// Uploads `bytes` from host to a fresh device buffer through a one-off synchronous copy.
static int upload(DevBuf &b, int dev, const void *src, size_t bytes, hipStream_t s) {
    VH_CHECK(b.ensure(dev, bytes));
    if (bytes) VH_HIP(hipMemcpyAsync(b.p, src, bytes, hipMemcpyHostToDevice, s));
    return VHIP_OK;
}

static int pq_encode_dev(int dev, const float *d_x, size_t n, size_t dim, size_t m_sub, size_t ks, int metric,
                         const float *d_cb, uint8_t *d_codes, hipStream_t s) {
    if (n == 0) return VHIP_OK;
    const size_t ds = dim / m_sub;
    const int cb_lds = ks * ds <= (size_t)kEncLdsFloats ? 1 : 0;
    const dim3 grid((unsigned)((n + 255) / 256), (unsigned)m_sub);
    const size_t lds = cb_lds ? ks * ds * sizeof(float) : 0;
#define VH_ENC(MT)                                                                                             \
    hipLaunchKernelGGL(k_pq_encode<MT>, grid, dim3(256), lds, s, d_x, (long)n, (int)dim, (int)m_sub, (int)ks, \
                       (int)ds, d_cb, cb_lds, d_codes)
    VH_METRIC_SWITCH(metric, VH_ENC)
#undef VH_ENC
    VH_HIP(hipGetLastError());
    (void)dev;
    return VHIP_OK;
}

// Thread-major register layout of the codebooks for k_ivfpq_scan: thread t = g * ks + j holds
// sub-centroid j of the sub-spaces [g * mg, (g + 1) * mg), ds floats each.
static std::vector<float> cb_thread_layout(const float *cb, size_t m_sub, size_t ks, size_t ds, int groups, int mg) {
    std::vector<float> t((size_t)kScanThreads * kLutRegs, 0.0f);
    for (int th = 0; th < kScanThreads; ++th) {
        const int g = th / (int)ks, j = th - g * (int)ks;
        if (g >= groups) continue;
        for (int ml = 0; ml < mg; ++ml) {
            const size_t m = (size_t)g * mg + ml;
            if (m >= m_sub) break;
            for (size_t d = 0; d < ds; ++d)
                t[(size_t)th * kLutRegs + ml * ds + d] = cb[(m * ks + j) * ds + d];
        }
    }
    return t;
}

// Fills an index from host parts (lists in CSR order).
static int ivfpq_init(vhip_ivfpq *X, int ordinal, size_t dim, int metric, const vhip_ivfpq_config *cfg,
                      const float *coarse, size_t nlist, const float *codebooks, const uint32_t *list_sizes,
                      const uint32_t *ids, const uint8_t *codes) {
    VH_CHECK(pq_check_shape(dim, cfg->num_subvectors, cfg->sub_clusters, metric));
    if (nlist == 0 || !coarse) return set_error(VHIP_ERR_INVALID_CONFIG, "the index needs at least one list");
    const size_t m_sub = cfg->num_subvectors, ks = cfg->sub_clusters, ds = dim / m_sub;
    if (!codebooks) return set_error(VHIP_ERR_INVALID_CONFIG, "codebooks is null");
    VH_CHECK(open_device(ordinal));
    int lim = 0;
    VH_HIP(hipDeviceGetAttribute(&lim, hipDeviceAttributeMaxSharedMemoryPerBlock, ordinal));
    X->lds_limit = (size_t)lim;
    if (scan_lds_bytes(dim, m_sub, ks, 1) > X->lds_limit)
        return set_error(VHIP_ERR_INVALID_CONFIG, "ADC table and query exceed the " + std::to_string(lim) +
                                                      " bytes of LDS of a workgroup (" + std::to_string(m_sub) +
                                                      " x " + std::to_string(ks) + " table entries, dimension " +
                                                      std::to_string(dim) + ")");
    X->dev = ordinal;
    X->dim = dim;
    X->nlist = nlist;
    X->m_sub = m_sub;
    X->ks = ks;
    X->ds = ds;
    X->metric = metric;
    X->cfg = *cfg;
    X->coarse.assign(coarse, coarse + nlist * dim);
    X->codebooks.assign(codebooks, codebooks + m_sub * ks * ds);
    X->list_off.assign(nlist + 1, 0);
    uint64_t total = 0;
    for (size_t c = 0; c < nlist; ++c) {
        total += list_sizes ? list_sizes[c] : 0;
        if (total > 0xffffffffull) return set_error(VHIP_ERR_INVALID_CONFIG, "ids are u32: at most 2^32-1 vectors");
        X->list_off[c + 1] = (uint32_t)total;
    }
    X->n = total;
    if (total && (!ids || !codes)) return set_error(VHIP_ERR_INVALID_CONFIG, "ids or codes is null");
    X->ids.assign(ids, ids + total);
    X->codes.assign(codes, codes + total * m_sub);
    for (size_t i = 0; i < total * m_sub; ++i)
        if (X->codes[i] >= ks) return set_error(VHIP_ERR_INVALID_CONFIG, "a code is not below sub_clusters");
    X->reg = lut_reg_layout(metric, m_sub, ks, ds, &X->groups, &X->mg);
    hipStream_t s;
    VH_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    X->stream = s;
    VH_CHECK(X->stager.init(ordinal));
    VH_CHECK(upload(X->d_coarse, ordinal, X->coarse.data(), X->coarse.size() * 4, s));
    VH_CHECK(upload(X->d_cb, ordinal, X->codebooks.data(), X->codebooks.size() * 4, s));
    VH_CHECK(upload(X->d_off, ordinal, X->list_off.data(), X->list_off.size() * 4, s));
    VH_CHECK(X->d_ids.ensure(ordinal, std::max<size_t>(4, total * 4)));
    VH_CHECK(X->d_codes.ensure(ordinal, std::max<size_t>(16, round_up(total * m_sub, 16))));
    if (total) {
        VH_CHECK(X->stager.h2d(X->d_ids.p, X->ids.data(), total * 4, s));
        VH_CHECK(X->stager.h2d(X->d_codes.p, X->codes.data(), total * m_sub, s));
    }
    if (X->reg) {
        std::vector<float> t = cb_thread_layout(X->codebooks.data(), m_sub, ks, ds, X->groups, X->mg);
        VH_CHECK(upload(X->d_cbt, ordinal, t.data(), t.size() * 4, s));
        VH_HIP(hipStreamSynchronize(s));
    }
    VH_HIP(hipStreamSynchronize(s));
    VH_CHECK(vhip_knn_create(X->coarse.data(), nlist, dim, metric, ordinal, &X->probe));
    return VHIP_OK;
}

// Coarse probe + scan for device-resident queries; results stay on the device.
static int ivfpq_search_dev(vhip_ivfpq *X, const float *d_q, size_t nq, size_t k, size_t nprobe, uint32_t *d_ids,
                            float *d_dist, uint32_t *d_len) {
    const size_t np = std::max<size_t>(1, std::min(nprobe, X->nlist));  // ivf/mod.rs:276
    hipStream_t s = X->stream;
    VH_CHECK(X->d_pid.ensure(X->dev, nq * np * 4));
    VH_CHECK(X->d_pdist.ensure(X->dev, nq * np * 4));
    VH_CHECK(vhip_knn_search_batch_device(X->probe, d_q, nq, np, X->d_pid.as<uint32_t>(), X->d_pdist.as<float>()));
    VH_CHECK(open_device(X->dev));
    ScanArgs A;
    A.qry = d_q;
    A.coarse = X->d_coarse.as<float>();
    A.probes = X->d_pid.as<uint32_t>();
    A.list_off = X->d_off.as<uint32_t>();
    A.ids = X->d_ids.as<uint32_t>();
    A.codes = X->d_codes.as<uint8_t>();
    A.cb = X->d_cb.as<float>();
    A.cbt = X->reg ? X->d_cbt.as<float>() : nullptr;
    A.out_ids = d_ids;
    A.out_dist = d_dist;
    A.out_len = d_len;
    A.nq = (int)nq;
    A.dim = (int)X->dim;
    A.nprobe = (int)np;
    A.nlist = (int)X->nlist;
    A.m_sub = (int)X->m_sub;
    A.ks = (int)X->ks;
    A.ds = (int)X->ds;
    A.k = (int)k;
    A.metric = X->metric;
    A.groups = X->groups;
    A.mg = X->mg;
    A.capw = scan_capw(k);
    const size_t lds = scan_lds_bytes(X->dim, X->m_sub, X->ks, k);
    if (lds > X->lds_limit)
        return set_error(VHIP_ERR_INVALID_CONFIG, "k = " + std::to_string(k) + " needs " + std::to_string(lds) +
                                                      " bytes of LDS with this index, the device allows " +
                                                      std::to_string(X->lds_limit));
    const unsigned grid = (unsigned)std::min<size_t>(nq, 3u * 256u);
    const int t = X->timer.begin(s);
    const dim3 g(grid), b(kScanThreads);
#define VH_SCAN(MT, DS) hipLaunchKernelGGL((k_ivfpq_scan<MT, DS>), g, b, lds, s, A)
#define VH_SCAN_MEM(MT) VH_SCAN(MT, 0)
#define VH_SCAN_REG(MT)                          \
    switch (X->ds) {                             \
        case 4: VH_SCAN(MT, 4); break;           \
        case 8: VH_SCAN(MT, 8); break;           \
        case 16: VH_SCAN(MT, 16); break;         \
        default: VH_SCAN(MT, 32); break;         \
    }
    if (!X->reg) {
        VH_METRIC_SWITCH(X->metric, VH_SCAN_MEM)
    } else if (X->metric == L2) {
        VH_SCAN_REG(L2)
    } else if (X->metric == DOT) {
        VH_SCAN_REG(DOT)
    } else {
        VH_SCAN_REG(COS)
    }
#undef VH_SCAN_REG
#undef VH_SCAN_MEM
#undef VH_SCAN
    VH_HIP(hipGetLastError());
    // work and bytes are filled in by the caller's accounting (scanned entries are data dependent)
    X->timer.end(t, s, 0.0, 0.0);
    return VHIP_OK;
}

static int ivfpq_validate_search(vhip_ivfpq *X, size_t nq, size_t k) {
    if (!X) return set_error(VHIP_ERR_INVALID_CONFIG, "null index");
    if (k > VHIP_IVFPQ_MAX_K)
        return set_error(VHIP_ERR_INVALID_CONFIG, "IVF-PQ search supports k <= " + std::to_string(VHIP_IVFPQ_MAX_K));
    if (nq > 0x7fffffffull) return set_error(VHIP_ERR_INVALID_CONFIG, "too many queries in one batch");
    return VHIP_OK;
}

}  // namespace vh

extern "C" {

void vhip_ivfpq_config_default(vhip_ivfpq_config *c) {
    if (!c) return;
    c->nlist = 64;  // config.rs:6-21
    c->nprobe = 8;
    c->num_subvectors = 8;
    c->sub_clusters = 256;
    c->max_kmeans_iters = 25;
    c->kmeans_tolerance = 1e-4f;
    c->max_train_points = 0;
}

int vhip_ivfpq_config_validate(const vhip_ivfpq_config *c, size_t dim) {
    clear_error();
    if (!c) return set_error(VHIP_ERR_INVALID_CONFIG, "config is null");
    if (c->nlist == 0) return set_error(VHIP_ERR_INVALID_CONFIG, "nlist must be greater than 0");
    if (c->nprobe == 0) return set_error(VHIP_ERR_INVALID_CONFIG, "nprobe must be greater than 0");
    if (c->nprobe > c->nlist)
        return set_error(VHIP_ERR_INVALID_CONFIG, "nprobe (" + std::to_string(c->nprobe) +
                                                      ") cannot be greater than nlist (" + std::to_string(c->nlist) +
                                                      ")");
    if (c->num_subvectors == 0) return set_error(VHIP_ERR_INVALID_CONFIG, "num_subvectors must be greater than 0");
    if (dim % c->num_subvectors != 0)
        return set_error(VHIP_ERR_INVALID_CONFIG, "vector dimension (" + std::to_string(dim) +
                                                      ") must be divisible by num_subvectors (" +
                                                      std::to_string(c->num_subvectors) + ")");
    if (c->sub_clusters == 0 || c->sub_clusters > 256)
        return set_error(VHIP_ERR_INVALID_CONFIG,
                         "sub_clusters must be between 1 and 256, got " + std::to_string(c->sub_clusters));
    if (c->max_kmeans_iters == 0) return set_error(VHIP_ERR_INVALID_CONFIG, "max_kmeans_iters must be greater than 0");
    if (!(c->kmeans_tolerance >= 0.0f))
        return set_error(VHIP_ERR_INVALID_CONFIG, "kmeans_tolerance must be non-negative");
    return VHIP_OK;
}

int vhip_pq_train(int ordinal, const float *data, size_t n, size_t dim, size_t m_sub, size_t ks, size_t max_iters,
                  float tol, int metric, const float *init_codebooks, uint64_t seed, float *out_codebooks) {
    clear_error();
    VH_CHECK(pq_check_shape(dim, m_sub, ks, metric));
    if (!out_codebooks) return set_error(VHIP_ERR_INVALID_CONFIG, "out_codebooks is null");
    const size_t ds = dim / m_sub;
    std::fill(out_codebooks, out_codebooks + m_sub * ks * ds, 0.0f);  // pq.rs:84-88 zero padding
    if (n == 0) return VHIP_OK;
    if (!data) return set_error(VHIP_ERR_INVALID_CONFIG, "data is null");
    std::vector<float> sub(n * ds);
    for (size_t m = 0; m < m_sub; ++m) {
        for (size_t i = 0; i < n; ++i)  // pq.rs:69-74: sub-vector m of every sample
            std::memcpy(&sub[i * ds], data + i * dim + m * ds, ds * sizeof(float));
        vhip_kmeans_result r{};
        const float *init = init_codebooks ? init_codebooks + m * ks * ds : nullptr;
        VH_CHECK(vhip_kmeans_fit(ordinal, sub.data(), n, ds, ks, max_iters, tol, metric, init, VHIP_INIT_SHUFFLE,
                                 seed + 1 + m, out_codebooks + m * ks * ds, nullptr, &r));
    }
    return VHIP_OK;
}

int vhip_pq_encode(int ordinal, const float *codebooks, size_t dim, size_t m_sub, size_t ks, int metric,
                   const float *data, size_t n, uint8_t *out_codes) {
    clear_error();
    VH_CHECK(pq_check_shape(dim, m_sub, ks, metric));
    if (n == 0) return VHIP_OK;
    if (!codebooks || !data || !out_codes) return set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    VH_CHECK(open_device(ordinal));
    hipStream_t s;
    VH_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    std::unique_ptr<ihipStream_t, hipError_t (*)(hipStream_t)> hold(s, hipStreamDestroy);
    PinnedStager st;
    VH_CHECK(st.init(ordinal));
    DevBuf x, cb, codes;
    VH_CHECK(x.ensure(ordinal, n * dim * 4));
    VH_CHECK(st.h2d(x.p, data, n * dim * 4, s));
    VH_CHECK(upload(cb, ordinal, codebooks, m_sub * ks * (dim / m_sub) * 4, s));
    VH_CHECK(codes.ensure(ordinal, n * m_sub));
    VH_CHECK(pq_encode_dev(ordinal, x.as<float>(), n, dim, m_sub, ks, metric, cb.as<float>(), codes.as<uint8_t>(), s));
    VH_CHECK(st.d2h(out_codes, codes.p, n * m_sub, s));
    VH_HIP(hipStreamSynchronize(s));
    return VHIP_OK;
}

int vhip_pq_adc_lut(int ordinal, const float *codebooks, size_t dim, size_t m_sub, size_t ks, int metric,
                    const float *queries, size_t nq, float *out_lut) {
    clear_error();
    VH_CHECK(pq_check_shape(dim, m_sub, ks, metric));
    if (nq == 0) return VHIP_OK;
    if (!codebooks || !queries || !out_lut) return set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    VH_CHECK(open_device(ordinal));
    hipStream_t s;
    VH_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    std::unique_ptr<ihipStream_t, hipError_t (*)(hipStream_t)> hold(s, hipStreamDestroy);
    DevBuf q, cb, lut;
    const size_t ds = dim / m_sub, total = nq * m_sub * ks;
    VH_CHECK(upload(q, ordinal, queries, nq * dim * 4, s));
    VH_CHECK(upload(cb, ordinal, codebooks, m_sub * ks * ds * 4, s));
    VH_CHECK(lut.ensure(ordinal, total * 4));
    const unsigned blocks = (unsigned)((total + 255) / 256);
#define VH_LUT(MT)                                                                                              \
    hipLaunchKernelGGL(k_pq_lut<MT>, dim3(blocks), dim3(256), 0, s, q.as<float>(), (long)total, (int)dim,      \
                       (int)m_sub, (int)ks, (int)ds, cb.as<float>(), lut.as<float>())
    VH_METRIC_SWITCH(metric, VH_LUT)
#undef VH_LUT
    VH_HIP(hipGetLastError());
    VH_HIP(hipMemcpyAsync(out_lut, lut.p, total * 4, hipMemcpyDeviceToHost, s));
    VH_HIP(hipStreamSynchronize(s));
    return VHIP_OK;
}

int vhip_ivfpq_create(int ordinal, size_t dim, int metric, const vhip_ivfpq_config *cfg, const float *coarse,
                      size_t nlist, const float *codebooks, const uint32_t *list_sizes, const uint32_t *ids,
                      const uint8_t *codes, vhip_ivfpq **out) {
    clear_error();
    if (!out || !cfg) return set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    *out = nullptr;
    std::unique_ptr<vhip_ivfpq> X(new vhip_ivfpq());
    VH_CHECK(ivfpq_init(X.get(), ordinal, dim, metric, cfg, coarse, nlist, codebooks, list_sizes, ids, codes));
    *out = X.release();
    return VHIP_OK;
}

int vhip_ivfpq_build(int ordinal, const float *data, size_t n, size_t dim, const vhip_ivfpq_config *cfg, int metric,
                     uint64_t seed, vhip_ivfpq **out) {
    clear_error();
    if (!out || !cfg) return set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    *out = nullptr;
    VH_CHECK(vhip_ivfpq_config_validate(cfg, dim));  // ivf/mod.rs:96
    if (metric < 0 || metric > 9) return set_error(VHIP_ERR_INVALID_CONFIG, "unknown metric code");
    if (n == 0) return set_error(VHIP_ERR_EMPTY_INDEX, "EmptyIndex: the storage holds no vectors");
    if (!data) return set_error(VHIP_ERR_INVALID_CONFIG, "data is null");
    if (n > 0xffffffffull) return set_error(VHIP_ERR_INVALID_CONFIG, "ids are u32: at most 2^32-1 vectors");
    const size_t m_sub = cfg->num_subvectors, ks = cfg->sub_clusters;
    // 1. coarse centroids (ivf/mod.rs:106-116): Lloyd from a seeded sample without replacement
    const size_t nl = std::min(cfg->nlist, n);
    std::vector<float> coarse(nl * dim);
    vhip_kmeans_result kr{};
    VH_CHECK(vhip_kmeans_fit(ordinal, data, n, dim, cfg->nlist, cfg->max_kmeans_iters, cfg->kmeans_tolerance, metric,
                             nullptr, VHIP_INIT_SHUFFLE, seed, coarse.data(), nullptr, &kr));
    // 2. assignment and residuals (:118-133)
    std::vector<int32_t> assign(n);
    std::vector<float> resid(n * dim);
    {
        vhip_kmeans *K = nullptr;
        VH_CHECK(vhip_kmeans_create(ordinal, data, n, dim, metric, &K));
        std::unique_ptr<vhip_kmeans, void (*)(vhip_kmeans *)> hold(K, vhip_kmeans_destroy);
        VH_CHECK(vhip_kmeans_set_centroids(K, coarse.data(), nl));
        VH_CHECK(vhip_kmeans_assign_only(K, assign.data(), nullptr, resid.data()));
    }
    // 3. product quantizer on the residuals (:135-144)
    std::vector<float> cb(m_sub * ks * (dim / m_sub));
    VH_CHECK(vhip_pq_train(ordinal, resid.data(), n, dim, m_sub, ks, cfg->max_kmeans_iters, cfg->kmeans_tolerance,
                           metric, nullptr, seed, cb.data()));
    // 4. codes of the residuals and inverted lists in insertion (ascending id) order (:146-153)
    std::vector<uint8_t> codes(n * m_sub);
    VH_CHECK(vhip_pq_encode(ordinal, cb.data(), dim, m_sub, ks, metric, resid.data(), n, codes.data()));
    std::vector<uint32_t> sizes(nl, 0), pos(nl + 1, 0);
    for (size_t i = 0; i < n; ++i) sizes[assign[i]] += 1;
    for (size_t c = 0; c < nl; ++c) pos[c + 1] = pos[c] + sizes[c];
    std::vector<uint32_t> ids(n);
    std::vector<uint8_t> lcodes(n * m_sub);
    for (size_t i = 0; i < n; ++i) {
        const uint32_t p = pos[assign[i]]++;
        ids[p] = (uint32_t)i;
        std::memcpy(&lcodes[(size_t)p * m_sub], &codes[i * m_sub], m_sub);
    }
    std::unique_ptr<vhip_ivfpq> X(new vhip_ivfpq());
    VH_CHECK(ivfpq_init(X.get(), ordinal, dim, metric, cfg, coarse.data(), nl, cb.data(), sizes.data(), ids.data(),
                        lcodes.data()));
    *out = X.release();
    return VHIP_OK;
}

int vhip_ivfpq_search_batch_device(vhip_ivfpq *X, const float *d_queries, size_t nq, size_t k, size_t nprobe,
                                   uint32_t *d_ids, float *d_dist, uint32_t *d_len) {
    clear_error();
    VH_CHECK(ivfpq_validate_search(X, nq, k));
    if (nq == 0 || k == 0) return VHIP_OK;
    if (X->n == 0) {
        std::lock_guard<std::mutex> lock(X->mu);
        VH_CHECK(open_device(X->dev));
        launch_fill_u32(d_len, nq, 0u, X->stream);
        launch_fill_u32(d_ids, nq * k, 0xffffffffu, X->stream);
        launch_fill(d_dist, nq * k, __builtin_nanf(""), X->stream);
        VH_HIP(hipStreamSynchronize(X->stream));
        return VHIP_OK;
    }
    std::lock_guard<std::mutex> lock(X->mu);
    VH_CHECK(ivfpq_search_dev(X, d_queries, nq, k, nprobe, d_ids, d_dist, d_len));
    VH_HIP(hipStreamSynchronize(X->stream));
    X->timer.collect();
    return VHIP_OK;
}

int vhip_ivfpq_search_batch(vhip_ivfpq *X, const float *queries, size_t nq, size_t k, size_t nprobe,
                            uint32_t *out_ids, float *out_dist, size_t *out_len) {
    clear_error();
    VH_CHECK(ivfpq_validate_search(X, nq, k));
    if (nq == 0) return VHIP_OK;
    if (!out_len) return set_error(VHIP_ERR_INVALID_CONFIG, "out_len is null");
    if (k == 0 || X->n == 0) {  // ivf/mod.rs:272-274
        for (size_t q = 0; q < nq; ++q) out_len[q] = 0;
        return VHIP_OK;
    }
    if (!queries || !out_ids || !out_dist) return set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    std::lock_guard<std::mutex> lock(X->mu);
    VH_CHECK(open_device(X->dev));
    hipStream_t s = X->stream;
    VH_CHECK(X->d_q.ensure(X->dev, nq * X->dim * 4));
    VH_CHECK(X->d_oid.ensure(X->dev, nq * k * 4));
    VH_CHECK(X->d_odist.ensure(X->dev, nq * k * 4));
    VH_CHECK(X->d_olen.ensure(X->dev, nq * 4));
    VH_CHECK(X->stager.h2d(X->d_q.p, queries, nq * X->dim * 4, s));
    VH_HIP(hipStreamSynchronize(s));
    VH_CHECK(ivfpq_search_dev(X, X->d_q.as<float>(), nq, k, nprobe, X->d_oid.as<uint32_t>(), X->d_odist.as<float>(),
                              X->d_olen.as<uint32_t>()));
    std::vector<uint32_t> len(nq);
    VH_CHECK(X->stager.d2h(out_ids, X->d_oid.p, nq * k * 4, s));
    VH_CHECK(X->stager.d2h(out_dist, X->d_odist.p, nq * k * 4, s));
    VH_HIP(hipMemcpyAsync(len.data(), X->d_olen.p, nq * 4, hipMemcpyDeviceToHost, s));
    VH_HIP(hipStreamSynchronize(s));
    X->timer.collect();
    for (size_t q = 0; q < nq; ++q) out_len[q] = len[q];
    return VHIP_OK;
}

int vhip_ivfpq_probe(vhip_ivfpq *X, const float *queries, size_t nq, size_t nprobe, uint32_t *out_lists) {
    clear_error();
    if (!X) return set_error(VHIP_ERR_INVALID_CONFIG, "null index");
    if (nq == 0) return VHIP_OK;
    const size_t np = std::max<size_t>(1, std::min(nprobe, X->nlist));
    std::vector<float> dist(nq * np);
    std::vector<size_t> lens(nq);
    std::lock_guard<std::mutex> lock(X->mu);
    return vhip_knn_search_batch(X->probe, queries, nq, np, out_lists, dist.data(), lens.data());
}

int vhip_ivfpq_info(const vhip_ivfpq *X, vhip_ivfpq_desc *info) {
    clear_error();
    if (!X || !info) return set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    info->dimension = X->dim;
    info->metric = X->metric;
    info->nlist = X->nlist;
    info->num_subvectors = X->m_sub;
    info->sub_clusters = X->ks;
    info->num_vectors = X->n;
    info->config = X->cfg;
    return VHIP_OK;
}

int vhip_ivfpq_export(const vhip_ivfpq *X, float *coarse, float *codebooks, uint32_t *list_sizes, uint32_t *ids,
                      uint8_t *codes) {
    clear_error();
    if (!X) return set_error(VHIP_ERR_INVALID_CONFIG, "null index");
    if (coarse) std::copy(X->coarse.begin(), X->coarse.end(), coarse);
    if (codebooks) std::copy(X->codebooks.begin(), X->codebooks.end(), codebooks);
    if (list_sizes)
        for (size_t c = 0; c < X->nlist; ++c) list_sizes[c] = X->list_off[c + 1] - X->list_off[c];
    if (ids) std::copy(X->ids.begin(), X->ids.end(), ids);
    if (codes) std::copy(X->codes.begin(), X->codes.end(), codes);
    return VHIP_OK;
}

int vhip_ivfpq_profile(vhip_ivfpq *X, int enable) {
    if (!X) return set_error(VHIP_ERR_INVALID_CONFIG, "null index");
    std::lock_guard<std::mutex> lock(X->mu);
    X->timer.enabled = enable != 0;
    X->timer.reset();
    return VHIP_OK;
}

int vhip_ivfpq_profile_read(vhip_ivfpq *X, double *kernel_ms, uint64_t *launches) {
    if (!X) return set_error(VHIP_ERR_INVALID_CONFIG, "null index");
    std::lock_guard<std::mutex> lock(X->mu);
    if (kernel_ms) *kernel_ms = X->timer.ms;
    if (launches) *launches = X->timer.launches;
    return VHIP_OK;
}

void vhip_ivfpq_destroy(vhip_ivfpq *X) { delete X; }

}  // extern "C"
