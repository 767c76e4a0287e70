// pq.hip -- product quantization and the IVF-PQ index on one GPU behind the C ABI.
//
// ProductQuantizer (vector-index/src/ivf/pq.rs) and IvfPqIndex (ivf/mod.rs):
//  * train: one k-means per sub-space (pq.rs:53-107) on the GPU k-means engine;
//  * encode (pq.rs:178-214): k_pq_encode, one thread per (vector, sub-space), the strict-compare
//    argmin of find_nearest_centroid (ivf/kmeans.rs:262-309) over the sub-space's codebook in LDS;
//  * compute_adc_lut (pq.rs:233-266): k_pq_lut, one thread per table entry;
//  * search (ivf/mod.rs:256-345): coarse probe through a kNN engine over the coarse centroids
//    (k = nprobe, best first), then the fused ADC scan k_ivfpq_scan (pq_scan.h).
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <vector>

#include "pq_scan.h"
#include "vh_runtime.h"

namespace vh {
namespace {

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

}  // namespace

// Register-layout eligibility: squared L2, dot or cosine, sub-dimension 4, 8, 16 or 32, more
// than 128 sub-centroids (one thread per sub-centroid) and every sub-space's column within
// kLutRegs floats (dimension <= 128).  Other shapes build the tables from codebooks read through
// the caches, the threads split into 256 / ks groups of sub-spaces.
static bool lut_reg_layout(int metric, size_t m_sub, size_t ks, size_t ds, int *groups, int *mg) {
    const int G = (int)(kScanThreads / ks);
    const int Mg = (int)((m_sub + G - 1) / G);
    *groups = G;
    *mg = Mg;
    const bool fast_metric = metric == L2 || metric == DOT || metric == COS;
    const bool pow2 = ds == 4 || ds == 8 || ds == 16 || ds == 32;
    return fast_metric && pow2 && G == 1 && m_sub * ds <= (size_t)kLutRegs;
}

// Candidate slots per wave for k results: room for k kept plus one step of 64 x kScanU entries.
static int scan_capw(size_t k) {
    int c = 256;
    while ((size_t)c < k + 64 * kScanU) c <<= 1;
    return c;
}

// Sixteen-byte pieces of a code row streamed through the DMA rings (rows of 16 or 32 bytes with
// 256 sub-centroids), 0 for the register-load path.
static int scan_nv(size_t m_sub, size_t ks) {
    return ks != 256 ? 0 : (m_sub == 16 ? 1 : (m_sub == 32 ? 2 : 0));
}

// LDS of one scan workgroup, dynamic part plus the static rings.
static size_t scan_lds_total(size_t dim, size_t m_sub, size_t ks, size_t k, int pg) {
    const int nv = scan_nv(m_sub, ks);
    return scan_lds_bytes(dim, m_sub, ks, scan_capw(k), pg, nv) + (size_t)ring_bytes(nv) + 3 * kMetaWin * 4;
}

// Probes per group: the most (4, 2, 1) whose tables leave room for two workgroups per CU
// (160 KB of LDS), else 1.
constexpr size_t kScanLdsPair = 80u * 1024u;
static int scan_pg(size_t dim, size_t m_sub, size_t ks, size_t k) {
    for (int pg = kScanWaves; pg > 1; pg >>= 1)
        if (scan_lds_total(dim, m_sub, ks, k, pg) <= kScanLdsPair) return pg;
    return 1;
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
    size_t lds_limit = 65536;  // LDS bytes per workgroup the device accepts
    int cus = 256;             // compute units of the device
    std::vector<float> coarse, codebooks;  // host copies (export / save)
    std::vector<uint32_t> list_off;        // nlist + 1
    std::vector<uint32_t> ids;             // list order
    std::vector<uint8_t> codes;            // list order
    vhip_knn *probe = nullptr;
    hipStream_t stream = nullptr;
    DevBuf d_coarse, d_cb, d_cbt, d_off, d_ids, d_codes;
    DevBuf d_q, d_pid, d_pdist, d_oid, d_odist, d_olen;
    // list-major search: lists by decreasing size, and the per-search plan and pair results
    DevBuf d_order, d_lcnt, d_loff, d_pairs, d_items, d_lctr, d_pout, d_tau;
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
    VH_HIP(hipDeviceGetAttribute(&X->cus, hipDeviceAttributeMultiprocessorCount, ordinal));
    if (scan_lds_total(dim, m_sub, ks, 1, 1) > X->lds_limit)
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
    {
        // lists by decreasing size (ties by id): the list-major search takes their work first
        std::vector<uint32_t> order(nlist);
        for (size_t c = 0; c < nlist; ++c) order[c] = (uint32_t)c;
        std::stable_sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) {
            return X->list_off[a + 1] - X->list_off[a] > X->list_off[b + 1] - X->list_off[b];
        });
        VH_CHECK(upload(X->d_order, ordinal, order.data(), nlist * 4, s));
        VH_HIP(hipStreamSynchronize(s));  // `order` is released at the end of this block
    }
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

// ---- plan of the list-major search -----------------------------------------------------------
// Pair counting and scattering per workgroup over runs of kPlanPairs pairs, aggregated in an LDS
// histogram when the lists fit it: a popular list then takes one global atomic per workgroup and
// run instead of one per pair (the per-pair atomics serialised on its counter).
constexpr int kPlanBins = 8192, kPlanPer = 16, kPlanPairs = 256 * kPlanPer;

// The list-major search's starting state in one launch: the queries' thresholds (2 nq words of
// ones: no threshold yet), the per-list pair counters and cursors (2 nlist zeros) and the item
// counters (2 zeros).
__global__ void k_list_reset(uint32_t *__restrict__ tau, size_t n_tau, uint32_t *__restrict__ cnt, size_t n_cnt,
                             uint32_t *__restrict__ ctr) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n_tau + n_cnt + 2; i += stride) {
        if (i < n_tau) tau[i] = 0xffffffffu;
        else if (i < n_tau + n_cnt) cnt[i - n_tau] = 0u;
        else ctr[i - n_tau - n_cnt] = 0u;
    }
}

__global__ __launch_bounds__(256) void k_pair_count(const uint32_t *__restrict__ probes, int total, int nlist,
                                                    uint32_t *__restrict__ cnt) {
    __shared__ uint32_t h[kPlanBins];
    const bool lds = nlist <= kPlanBins;
    const int tid = threadIdx.x;
    for (long b0 = (long)blockIdx.x * kPlanPairs; b0 < total; b0 += (long)gridDim.x * kPlanPairs) {
        if (lds) {
            for (int i = tid; i < nlist; i += 256) h[i] = 0;
            __syncthreads();
        }
        for (int j = 0; j < kPlanPer; ++j) {
            const long t = b0 + j * 256 + tid;
            if (t >= total) break;
            const uint32_t c = probes[t];
            if (c < (uint32_t)nlist) atomicAdd(lds ? &h[c] : &cnt[c], 1u);
        }
        if (lds) {
            __syncthreads();
            for (int i = tid; i < nlist; i += 256)
                if (h[i]) atomicAdd(&cnt[i], h[i]);
            __syncthreads();
        }
    }
}

// One workgroup of 1024 threads: in the order `order`, exclusive prefix sums of the lists' pair
// counts (pair_off, indexed by list) and item counts (item_off, indexed by position), and the
// number of items.
__global__ __launch_bounds__(1024) void k_list_plan(const uint32_t *__restrict__ cnt, const uint32_t *__restrict__ order,
                                                    int nlist, int qb, uint32_t *__restrict__ pair_off,
                                                    uint32_t *__restrict__ item_off, uint32_t *__restrict__ n_items) {
    __shared__ uint32_t sp[1024], si[1024];
    __shared__ uint32_t carry_p, carry_i;
    const int t = threadIdx.x;
    if (t == 0) {
        carry_p = 0;
        carry_i = 0;
    }
    __syncthreads();
    for (int base = 0; base < nlist; base += 1024) {
        const int i = base + t;
        uint32_t c = 0, l = 0;
        if (i < nlist) {
            l = order[i];
            c = cnt[l];
        }
        const uint32_t items = (c + (uint32_t)qb - 1) / (uint32_t)qb;
        sp[t] = c;
        si[t] = items;
        __syncthreads();
        for (int o = 1; o < 1024; o <<= 1) {  // inclusive scans
            const uint32_t vp = t >= o ? sp[t - o] : 0u, vi = t >= o ? si[t - o] : 0u;
            __syncthreads();
            sp[t] += vp;
            si[t] += vi;
            __syncthreads();
        }
        if (i < nlist) {
            pair_off[l] = carry_p + sp[t] - c;
            item_off[i] = carry_i + si[t] - items;
        }
        __syncthreads();
        if (t == 1023) {
            carry_p += sp[1023];
            carry_i += si[1023];
        }
        __syncthreads();
    }
    if (t == 0) *n_items = carry_i;
}

// Pair ids q * nprobe + p into their list's range (the order within a list is arbitrary: every
// pair's result is the same whichever item scans it).
__global__ __launch_bounds__(256) void k_pair_scatter(const uint32_t *__restrict__ probes, int total, int nlist,
                                                      const uint32_t *__restrict__ pair_off,
                                                      uint32_t *__restrict__ cursor, uint32_t *__restrict__ pairs) {
    __shared__ uint32_t h[kPlanBins];
    const bool lds = nlist <= kPlanBins;
    const int tid = threadIdx.x;
    for (long b0 = (long)blockIdx.x * kPlanPairs; b0 < total; b0 += (long)gridDim.x * kPlanPairs) {
        if (lds) {
            for (int i = tid; i < nlist; i += 256) h[i] = 0;
            __syncthreads();
        }
        uint32_t cc[kPlanPer], loc[kPlanPer];
        for (int j = 0; j < kPlanPer; ++j) {
            const long t = b0 + j * 256 + tid;
            cc[j] = t < total ? probes[t] : 0xffffffffu;
            loc[j] = 0;
            if (cc[j] < (uint32_t)nlist)
                loc[j] = lds ? atomicAdd(&h[cc[j]], 1u) : pair_off[cc[j]] + atomicAdd(&cursor[cc[j]], 1u);
        }
        if (lds) {
            __syncthreads();
            // each list's slots for this run: one global reservation, kept in place of its count
            for (int i = tid; i < nlist; i += 256)
                if (h[i]) h[i] = pair_off[i] + atomicAdd(&cursor[i], h[i]);
            __syncthreads();
        }
        for (int j = 0; j < kPlanPer; ++j)
            if (cc[j] < (uint32_t)nlist) pairs[(lds ? h[cc[j]] : 0u) + loc[j]] = (uint32_t)(b0 + j * 256 + tid);
        if (lds) __syncthreads();  // the next run clears h
    }
}

// Work items of each list, in the order `order`, in runs of qb pairs: (list, first pair, the
// list's first row, its length << 3 | pair count), and the item's pair ids (unused slots repeat
// the first), so that a scan reads everything an item needs in one round trip.  One thread per
// item: its list is the last position i of `order` with item_off[i] <= item (lists without items
// share their successor's offset, so the last such position is the one holding the item).
__global__ void k_item_fill(const uint32_t *__restrict__ cnt, const uint32_t *__restrict__ order,
                            const uint32_t *__restrict__ item_off, const uint32_t *__restrict__ pair_off,
                            const uint32_t *__restrict__ list_off, const uint32_t *__restrict__ pairs, int nlist,
                            int qb, const uint32_t *__restrict__ n_items, uint4 *__restrict__ items,
                            uint4 *__restrict__ item_pairs) {
    const uint32_t ni = *n_items;
    for (uint32_t it = blockIdx.x * blockDim.x + threadIdx.x; it < ni; it += gridDim.x * blockDim.x) {
        int lo = 0, hi = nlist - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (item_off[mid] <= it) lo = mid; else hi = mid - 1;
        }
        const uint32_t l = order[lo], c = cnt[l], t = it - item_off[lo];
        const uint32_t first = pair_off[l] + t * (uint32_t)qb, np = min((uint32_t)qb, c - t * (uint32_t)qb);
        const uint32_t beg = list_off[l], len = list_off[l + 1] - beg;
        items[it] = make_uint4(l, first, beg, len << 3 | np);
        uint32_t p[4];
        for (uint32_t sl = 0; sl < 4; ++sl) p[sl] = pairs[first + (sl < np ? sl : 0u)];
        item_pairs[it] = make_uint4(p[0], p[1], p[2], p[3]);
    }
}

void ivfpq_list_plan(const uint32_t *probes, int nq, int nprobe, int nlist, const uint32_t *order,
                     const uint32_t *list_off, uint32_t *cnt, uint32_t *cursor, uint32_t *pair_off,
                     uint32_t *item_off, uint32_t *pairs, uint4 *items, uint4 *item_pairs, uint32_t *n_items,
                     hipStream_t s) {
    const int total = nq * nprobe;  // at most kIvfpqChunkPairs (the caller's chunks)
    const unsigned gp = (unsigned)std::min(4096, (total + 255) / 256);
    const unsigned gr = (unsigned)std::min(1024, (total + kPlanPairs - 1) / kPlanPairs);  // runs of kPlanPairs
    hipLaunchKernelGGL(k_pair_count, dim3(gr), dim3(256), 0, s, probes, total, nlist, cnt);
    hipLaunchKernelGGL(k_list_plan, dim3(1), dim3(1024), 0, s, cnt, order, nlist, kListQb, pair_off, item_off, n_items);
    hipLaunchKernelGGL(k_pair_scatter, dim3(gr), dim3(256), 0, s, probes, total, nlist, pair_off, cursor, pairs);
    // items <= pairs: one thread per item, grid-stride over the device-side count
    hipLaunchKernelGGL(k_item_fill, dim3(gp), dim3(256), 0, s, cnt, order, item_off, pair_off, list_off, pairs, nlist,
                       kListQb, n_items, items, item_pairs);
}

// The list-major search applies to 16-byte code rows of 256 sub-centroids with the register-held
// codebook (ds 4 or 8) and k <= kListMaxK; VHIP_IVFPQ_SCAN=query forces the query-major kernel.
static bool list_path(const vhip_ivfpq *X, size_t k, size_t np) {
    if (const char *e = std::getenv("VHIP_IVFPQ_SCAN"))
        if (std::strcmp(e, "query") == 0) return false;
    return X->reg && X->ks == 256 && X->m_sub == 16 && (X->ds == 4 || X->ds == 8) && k >= 1 &&
           k <= (size_t)kListMaxK && np * k <= (size_t)kListMaxMerge &&
           sizeof(ListLds) <= X->lds_limit;
}

// (query, probe) pairs of one search chunk: pair ids are 32-bit (q * nprobe + p) and the plan's
// grids and buffers scale with them, so larger batches run as several chunks.
constexpr size_t kIvfpqChunkPairs = (size_t)1 << 22;

// Coarse probe + scan for device-resident queries of one chunk; results stay on the device.
static int ivfpq_search_chunk(vhip_ivfpq *X, const float *d_q, size_t nq, size_t k, size_t np, uint32_t *d_ids,
                              float *d_dist, uint32_t *d_len) {
    hipStream_t s = X->stream;
    VH_CHECK(X->d_pid.ensure(X->dev, nq * np * 4));
    VH_CHECK(X->d_pdist.ensure(X->dev, nq * np * 4));
    const bool lists = list_path(X, k, np);
    if (lists) {
        // the plan's buffers, cleared on this stream while the probe runs on the probe engine's
        const size_t total = nq * np;
        VH_CHECK(X->d_lcnt.ensure(X->dev, 2 * X->nlist * 4));
        VH_CHECK(X->d_loff.ensure(X->dev, 2 * X->nlist * 4));
        VH_CHECK(X->d_pairs.ensure(X->dev, total * 4));
        VH_CHECK(X->d_items.ensure(X->dev, 2 * total * sizeof(uint4)));  // records, then pair ids
        VH_CHECK(X->d_lctr.ensure(X->dev, 2 * 4));
        VH_CHECK(X->d_pout.ensure(X->dev, total * k * 8));
        VH_CHECK(X->d_tau.ensure(X->dev, nq * 8));
        VH_CHECK(open_device(X->dev));
        const size_t words = 2 * nq + 2 * X->nlist + 2;
        hipLaunchKernelGGL(k_list_reset, dim3((unsigned)std::min<size_t>(1024, (words + 255) / 256)), dim3(256), 0, s,
                           X->d_tau.as<uint32_t>(), 2 * nq, X->d_lcnt.as<uint32_t>(), 2 * X->nlist,
                           X->d_lctr.as<uint32_t>());
        VH_HIP(hipGetLastError());
    }
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
    A.pg = scan_pg(X->dim, X->m_sub, X->ks, k);
    const int nv = scan_nv(X->m_sub, X->ks);
    const size_t lds = scan_lds_bytes(X->dim, X->m_sub, X->ks, A.capw, A.pg, nv);
    if (scan_lds_total(X->dim, X->m_sub, X->ks, k, A.pg) > X->lds_limit)
        return set_error(VHIP_ERR_INVALID_CONFIG, "k = " + std::to_string(k) + " needs " + std::to_string(lds) +
                                                      " bytes of LDS with this index, the device allows " +
                                                      std::to_string(X->lds_limit));
    if (lists) {
        const size_t total = nq * np;
        uint32_t *cnt = X->d_lcnt.as<uint32_t>(), *ctr = X->d_lctr.as<uint32_t>();
        uint4 *items = X->d_items.as<uint4>(), *item_pairs = items + total;
        ivfpq_list_plan(A.probes, (int)nq, (int)np, (int)X->nlist, X->d_order.as<uint32_t>(), A.list_off, cnt,
                        cnt + X->nlist, X->d_loff.as<uint32_t>(), X->d_loff.as<uint32_t>() + X->nlist,
                        X->d_pairs.as<uint32_t>(), items, item_pairs, ctr, s);
        VH_HIP(hipGetLastError());
        ListArgs L{A, items, item_pairs, ctr, ctr + 1, X->d_pout.as<unsigned long long>(),
                   X->d_tau.as<unsigned long long>()};
        const int t = X->timer.begin(s);
        if (X->metric == L2)
            launch_ivfpq_lists_l2(L, (int)X->ds, X->cus, s);
        else
            launch_ivfpq_lists_ip(L, (int)X->ds, X->cus, s);
        VH_HIP(hipGetLastError());
        X->timer.end(t, s, 0.0, 0.0);  // the scan kernel alone
        launch_ivfpq_list_merge(L, X->cus, s);
        VH_HIP(hipGetLastError());
        return VHIP_OK;
    }
    const int t = X->timer.begin(s);
    if (!X->reg)
        launch_ivfpq_scan_mem(A, nv, X->cus, lds, s);
    else if (X->metric == L2)
        launch_ivfpq_scan_l2(A, (int)X->ds, nv, X->cus, lds, s);
    else
        launch_ivfpq_scan_ip(A, (int)X->ds, nv, X->cus, lds, s);
    VH_HIP(hipGetLastError());
    // work and bytes are filled in by the caller's accounting (scanned entries are data dependent)
    X->timer.end(t, s, 0.0, 0.0);
    return VHIP_OK;
}

// Coarse probe + scan for device-resident queries, in chunks of at most kIvfpqChunkPairs pairs.
static int ivfpq_search_dev(vhip_ivfpq *X, const float *d_q, size_t nq, size_t k, size_t nprobe, uint32_t *d_ids,
                            float *d_dist, uint32_t *d_len) {
    const size_t np = std::max<size_t>(1, std::min(nprobe, X->nlist));  // ivf/mod.rs:276
    const size_t qb = std::max<size_t>(1, kIvfpqChunkPairs / np);
    for (size_t q0 = 0; q0 < nq; q0 += qb) {
        const size_t m = std::min(qb, nq - q0);
        // the next chunk's probe (on the probe engine's own stream) rewrites the probe lists and
        // plan buffers that this stream's scan of the previous chunk reads
        if (q0 > 0) VH_HIP(hipStreamSynchronize(X->stream));
        VH_CHECK(ivfpq_search_chunk(X, d_q + q0 * X->dim, m, k, np, d_ids + q0 * k, d_dist + q0 * k, d_len + q0));
    }
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
