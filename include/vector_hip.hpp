/*
 * vector_hip.hpp -- C++ host API over the C ABI of vector_hip.h, mirroring the Rust API of the
 * reference's GPU hot path (crate vector-cuda) so that code written against it reads the same:
 *
 *   CudaDeviceContext     vector-cuda/src/device.rs:81-256      (an emulator context is a descriptor only)
 *   CudaKnnEngine         vector-cuda/src/knn.rs:45-401
 *   DistributedKnnEngine  vector-cuda/src/ddp/distributed_knn.rs:24-262, GpuShardMode :14-19
 *   CollectiveOps         vector-cuda/src/ddp/collective.rs:115-159 (top_k_reduce only)
 *   CudaKMeansEngine      vector-cuda/src/kmeans.rs:37-467, CudaKMeansResult :15-35
 *   DistributedKMeansEngine vector-cuda/src/ddp/distributed_kmeans.rs:19-541
 *   CudaError             vector-cuda/src/error.rs:7-29 (thrown; Result<T, CudaError> -> T or throw)
 *   DistanceMetric, SearchResult, VectorId   vector-index/src/lib.rs:50-94, types.rs:5-20
 *
 * Rust slices (&[f32]) become (pointer, length) pairs or std::vector; Vec<Vec<SearchResult>>
 * becomes std::vector<std::vector<SearchResult>>.  Where the Rust API panics on a violated
 * precondition (assert!), this API throws CudaError(InvalidConfig).  Where the reference
 * silently fell back to the CPU, this API throws: every call runs on the GPU or fails.
 * Extensions (no reference counterpart): explicit initial centroids and seeds for k-means,
 * and HammingKnnEngine for packed-bit codes.
 *
 * The IVF stack of vector-index (src/ivf) sits on the same library:
 *   IvfCoarseQuantizer    ivf/mod.rs:106-133, ivf/kmeans.rs:262-356
 *   IvfPqConfig           ivf/config.rs:25-154
 *   ProductQuantizer      ivf/pq.rs:12-293
 *   InvertedList/Index    ivf/inverted_list.rs
 *   IvfPqIndex            ivf/mod.rs:63-449 (storage: a flat row-major float array)
 *   IvfPqSerializer       ivf/serializer.rs:16-377 (IVFPQVEC and VRSKMEAN files)
 * VectorIndexError::EmptyIndex is CudaError(EmptyIndex); DimensionMismatch and the config's
 * reasons are CudaError(InvalidConfig).
 */
#ifndef VECTOR_HIP_HPP
#define VECTOR_HIP_HPP

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "vector_hip.h"

namespace vector_hip {

using VectorId = uint32_t;

enum class DistanceMetric : int {
    L2Squared = VHIP_METRIC_L2SQUARED,
    DotProduct = VHIP_METRIC_DOTPRODUCT,
    CosineSimilarity = VHIP_METRIC_COSINE,
    Manhattan = VHIP_METRIC_MANHATTAN,
    Minkowski = VHIP_METRIC_MINKOWSKI,
    Chebyshev = VHIP_METRIC_CHEBYSHEV,
    Hamming = VHIP_METRIC_HAMMING,
    Mahalanobis = VHIP_METRIC_MAHALANOBIS,
    Jaccard = VHIP_METRIC_JACCARD,
    Hellinger = VHIP_METRIC_HELLINGER,
};

/* DistanceMetric::higher_is_better (lib.rs:89-94) */
inline bool higher_is_better(DistanceMetric m) {
    return m == DistanceMetric::DotProduct || m == DistanceMetric::CosineSimilarity;
}

enum class GpuShardMode : int { Sharded = VHIP_SHARD_SHARDED, Replicated = VHIP_SHARD_REPLICATED };

struct SearchResult {
    VectorId id;
    float distance;
};

class CudaError : public std::runtime_error {
public:
    enum class Kind { InsufficientDevices, DeviceNotFound, DriverError, HardwareNotAvailable, InvalidConfig, EmptyIndex };
    CudaError(Kind kind, const std::string &msg, size_t requested = 0, size_t available = 0, size_t ordinal = 0)
        : std::runtime_error(msg), kind_(kind), requested_(requested), available_(available), ordinal_(ordinal) {}
    Kind kind() const { return kind_; }
    size_t requested() const { return requested_; } /* InsufficientDevices */
    size_t available() const { return available_; } /* InsufficientDevices */
    size_t ordinal() const { return ordinal_; }     /* DeviceNotFound */

private:
    Kind kind_;
    size_t requested_, available_, ordinal_;
};

namespace detail {
inline void check(int status) {
    if (status == VHIP_OK) return;
    const std::string msg = vhip_last_error();
    switch (status) {
        case VHIP_ERR_INSUFFICIENT_DEVICES: {
            size_t r = 0, a = 0;
            vhip_last_error_devices(&r, &a);
            throw CudaError(CudaError::Kind::InsufficientDevices, msg, r, a);
        }
        case VHIP_ERR_DEVICE_NOT_FOUND: {
            const int o = vhip_last_error_ordinal();
            throw CudaError(CudaError::Kind::DeviceNotFound, msg, 0, 0, o < 0 ? 0 : (size_t)o);
        }
        case VHIP_ERR_HARDWARE_NOT_AVAILABLE: throw CudaError(CudaError::Kind::HardwareNotAvailable, msg);
        case VHIP_ERR_INVALID_CONFIG: throw CudaError(CudaError::Kind::InvalidConfig, msg);
        case VHIP_ERR_EMPTY_INDEX: throw CudaError(CudaError::Kind::EmptyIndex, msg);
        default: throw CudaError(CudaError::Kind::DriverError, msg);
    }
}
inline void require(bool ok, const char *what) {
    if (!ok) throw CudaError(CudaError::Kind::InvalidConfig, what);
}
inline std::vector<std::vector<SearchResult>> to_lists(size_t nq, size_t k, const std::vector<uint32_t> &ids,
                                                       const std::vector<float> &dist,
                                                       const std::vector<size_t> &len) {
    std::vector<std::vector<SearchResult>> out(nq);
    for (size_t q = 0; q < nq; ++q) {
        out[q].reserve(len[q]);
        for (size_t j = 0; j < len[q]; ++j) out[q].push_back(SearchResult{ids[q * k + j], dist[q * k + j]});
    }
    return out;
}
}  // namespace detail

/* ---- CudaDeviceContext (device.rs:81-256) -------------------------------------------------- */
class CudaDeviceContext {
public:
    static size_t device_count() { return (size_t)vhip_device_count(); }
    /* CudaDeviceContext::new() (device.rs:120-122): with_ordinal(0) */
    CudaDeviceContext() : CudaDeviceContext(with_ordinal(0)) {}
    /* device.rs:127-170: the GPU's context, or DeviceNotFound / DriverError */
    static CudaDeviceContext with_ordinal_strict(size_t ordinal) { return CudaDeviceContext(ordinal); }
    /* device.rs:188-221: the GPU's context, or a software-emulator descriptor
     * (is_hardware_available() false) when that ordinal has no usable gfx950 device.  Engines
     * built on such an ordinal throw DeviceNotFound; nothing runs on the CPU in its place. */
    static CudaDeviceContext with_ordinal(size_t ordinal) {
        char buf[256];
        size_t mem = 0;
        if (vhip_device_info((int)ordinal, buf, sizeof buf, &mem) != VHIP_OK) return software_emulator(ordinal);
        return CudaDeviceContext(ordinal, buf, mem, true);
    }
    /* device.rs:173-185: a descriptor only (no device, total memory 0) */
    static CudaDeviceContext software_emulator(size_t ordinal) {
        return CudaDeviceContext(ordinal, "HIP Software Emulator (GPU " + std::to_string(ordinal) + ", no device)", 0,
                                 false);
    }
    size_t device_id() const { return id_; }
    const std::string &device_name() const { return name_; }
    size_t total_memory_bytes() const { return mem_; }
    bool is_hardware_available() const { return hw_; }

private:
    explicit CudaDeviceContext(size_t ordinal) : id_(ordinal) {
        char buf[256];
        detail::check(vhip_device_info((int)ordinal, buf, sizeof buf, &mem_));
        name_ = buf;
    }
    CudaDeviceContext(size_t ordinal, std::string name, size_t mem, bool hw)
        : id_(ordinal), mem_(mem), name_(std::move(name)), hw_(hw) {}
    size_t id_ = 0, mem_ = 0;
    std::string name_;
    bool hw_ = true;
};

/* ---- CudaKnnEngine (knn.rs:45-401) ------------------------------------------------------- */
class CudaKnnEngine {
public:
    /* CudaKnnEngine::new (knn.rs:85-88) */
    CudaKnnEngine(const float *dataset, size_t len, size_t dimension, DistanceMetric metric)
        : CudaKnnEngine(dataset, len, dimension, metric, 0) {}
    CudaKnnEngine(const std::vector<float> &dataset, size_t dimension, DistanceMetric metric)
        : CudaKnnEngine(dataset.data(), dataset.size(), dimension, metric, 0) {}
    /* CudaKnnEngine::new over MmapStorage::open(path).as_raw_slice(): the base streams from the
     * mapped file to the GPU with no host copy (vhip_knn_create_from_vecrstor) */
    static CudaKnnEngine from_vecrstor(const std::string &path, DistanceMetric metric, size_t ordinal = 0) {
        size_t n = 0, d = 0;
        detail::check(vhip_vecrstor_open(path.c_str(), &n, &d));
        vhip_knn *h = nullptr;
        detail::check(vhip_knn_create_from_vecrstor(path.c_str(), (int)metric, (int)ordinal, &h));
        return CudaKnnEngine(h, d);
    }
    /* CudaKnnEngine::with_ordinal (knn.rs:90-140) */
    static CudaKnnEngine with_ordinal(const std::vector<float> &dataset, size_t dimension, DistanceMetric metric,
                                      size_t ordinal) {
        return CudaKnnEngine(dataset.data(), dataset.size(), dimension, metric, ordinal);
    }

    /* knn.rs:143-149: the first query's results (empty for an empty query) */
    std::vector<SearchResult> search(const float *query, size_t len, size_t k) const {
        auto r = search_batch(query, len, k);
        return r.empty() ? std::vector<SearchResult>{} : std::move(r[0]);
    }
    std::vector<SearchResult> search(const std::vector<float> &query, size_t k) const {
        return search(query.data(), query.size(), k);
    }
    /* knn.rs:151-169: len / dimension queries, min(k, N) results each, best first */
    std::vector<std::vector<SearchResult>> search_batch(const float *queries, size_t len, size_t k) const {
        detail::require(len % dim_ == 0, "query length is not a multiple of the dimension");
        const size_t nq = len / dim_;
        if (nq == 0) return {};
        std::vector<uint32_t> ids(nq * (k ? k : 1));
        std::vector<float> dist(nq * (k ? k : 1));
        std::vector<size_t> lens(nq);
        detail::check(vhip_knn_search_batch(h_.get(), queries, nq, k, ids.data(), dist.data(), lens.data()));
        return detail::to_lists(nq, k ? k : 1, ids, dist, lens);
    }
    std::vector<std::vector<SearchResult>> search_batch(const std::vector<float> &queries, size_t k) const {
        return search_batch(queries.data(), queries.size(), k);
    }

    CudaDeviceContext context() const { return CudaDeviceContext::with_ordinal_strict(device_id()); }
    size_t device_id() const { return (size_t)vhip_knn_device_id(h_.get()); }
    size_t dimension() const { return vhip_knn_dimension(h_.get()); }
    size_t num_vectors() const { return vhip_knn_num_vectors(h_.get()); }
    DistanceMetric metric() const { return (DistanceMetric)vhip_knn_metric(h_.get()); }
    vhip_knn *raw() const { return h_.get(); }

private:
    CudaKnnEngine(const float *dataset, size_t len, size_t dimension, DistanceMetric metric, size_t ordinal)
        : dim_(dimension) {
        detail::require(dimension > 0, "dimension must be > 0");
        detail::require(len % dimension == 0, "dataset length is not a multiple of the dimension");
        vhip_knn *h = nullptr;
        detail::check(vhip_knn_create(dataset, len / dimension, dimension, (int)metric, (int)ordinal, &h));
        h_.reset(h);
    }
    CudaKnnEngine(vhip_knn *h, size_t dimension) : dim_(dimension), h_(h) {}
    struct Del {
        void operator()(vhip_knn *p) const { vhip_knn_destroy(p); }
    };
    size_t dim_;
    std::unique_ptr<vhip_knn, Del> h_;
};

/* ---- DistributedKnnEngine (ddp/distributed_knn.rs:24-262) ------------------------------- */
class DistributedKnnEngine {
public:
    /* :40-61 -- InsufficientDevices when num_gpus exceeds the device count */
    static DistributedKnnEngine try_new(const std::vector<float> &dataset, size_t dimension, size_t num_gpus,
                                        GpuShardMode mode, DistanceMetric metric) {
        return DistributedKnnEngine(dataset, dimension, num_gpus, mode, metric, false);
    }
    /* :64-74 -- no device-count check; every rank runs on GPU 0 */
    static DistributedKnnEngine emulator(const std::vector<float> &dataset, size_t dimension, size_t num_gpus,
                                         GpuShardMode mode, DistanceMetric metric) {
        return DistributedKnnEngine(dataset, dimension, num_gpus, mode, metric, true);
    }
    /* :77-89 (the Rust new() panics where try_new errs; this one throws) */
    static DistributedKnnEngine new_(const std::vector<float> &dataset, size_t dimension, size_t num_gpus,
                                     GpuShardMode mode, DistanceMetric metric) {
        return try_new(dataset, dimension, num_gpus, mode, metric);
    }

    std::vector<SearchResult> search(const std::vector<float> &query, size_t k) const {
        auto r = search_batch(query, k);
        return r.empty() ? std::vector<SearchResult>{} : std::move(r[0]);
    }
    std::vector<std::vector<SearchResult>> search_batch(const std::vector<float> &queries, size_t k) const {
        detail::require(queries.size() % dim_ == 0, "query length is not a multiple of the dimension");
        const size_t nq = queries.size() / dim_;
        if (nq == 0) return {};
        std::vector<uint32_t> ids(nq * (k ? k : 1));
        std::vector<float> dist(nq * (k ? k : 1));
        std::vector<size_t> lens(nq);
        detail::check(vhip_dknn_search_batch(h_.get(), queries.data(), nq, k, ids.data(), dist.data(), lens.data()));
        return detail::to_lists(nq, k ? k : 1, ids, dist, lens);
    }
    size_t num_gpus() const { return vhip_dknn_num_gpus(h_.get()); }
    GpuShardMode mode() const { return (GpuShardMode)vhip_dknn_mode(h_.get()); }
    size_t dimension() const { return vhip_dknn_dimension(h_.get()); }
    size_t num_vectors() const { return vhip_dknn_num_vectors(h_.get()); }
    DistanceMetric metric() const { return (DistanceMetric)vhip_dknn_metric(h_.get()); }

private:
    DistributedKnnEngine(const std::vector<float> &dataset, size_t dimension, size_t num_gpus, GpuShardMode mode,
                         DistanceMetric metric, bool emulate)
        : dim_(dimension) {
        detail::require(num_gpus >= 1, "num_gpus must be at least 1");
        detail::require(dimension > 0 && dataset.size() % dimension == 0,
                        "dataset length is not a multiple of the dimension");
        vhip_dknn *h = nullptr;
        auto fn = emulate ? vhip_dknn_emulator : vhip_dknn_try_new;
        detail::check(fn(dataset.data(), dataset.size() / dimension, dimension, num_gpus, (int)mode, (int)metric, &h));
        h_.reset(h);
    }
    struct Del {
        void operator()(vhip_dknn *p) const { vhip_dknn_destroy(p); }
    };
    size_t dim_;
    std::unique_ptr<vhip_dknn, Del> h_;
};

/* ---- CollectiveOps::top_k_reduce (ddp/collective.rs:115-159) ------------------------------ */
struct CollectiveOps {
    static std::vector<SearchResult> top_k_reduce(const std::vector<std::vector<SearchResult>> &per_rank, size_t k,
                                                  DistanceMetric metric) {
        std::vector<uint32_t> ids;
        std::vector<float> dist;
        for (const auto &r : per_rank)
            for (const auto &e : r) {
                ids.push_back(e.id);
                dist.push_back(e.distance);
            }
        if (ids.empty() || k == 0) return {};
        std::vector<uint32_t> oi(k);
        std::vector<float> od(k);
        const size_t m = vhip_top_k_reduce(ids.data(), dist.data(), ids.size(), k, (int)metric, oi.data(), od.data());
        std::vector<SearchResult> out(m);
        for (size_t i = 0; i < m; ++i) out[i] = SearchResult{oi[i], od[i]};
        return out;
    }
};

/* ---- k-means (kmeans.rs:15-467, ddp/distributed_kmeans.rs) -------------------------------- */
struct CudaKMeansResult {
    std::vector<float> centroids; /* k x dimension */
    size_t dimension = 0;
    size_t k = 0;
    size_t iterations = 0;
    float inertia = 0.0f;
    const float *centroid(size_t i) const { return centroids.data() + i * dimension; }
};

/* Extension: where the initial centroids come from (the reference drew them from an unseeded
 * thread_rng). */
struct KMeansInit {
    const float *centroids = nullptr; /* effective_k x dimension, or null for a seeded init */
    uint64_t seed = 42;
};

namespace detail {
inline CudaKMeansResult kmeans_fit(size_t ordinal, const float *data, size_t len, size_t dimension, size_t k,
                                   size_t max_iters, float tolerance, DistanceMetric metric, int init_mode,
                                   const KMeansInit &init, std::vector<int32_t> *assign) {
    require(dimension > 0, "dimension must be > 0");
    const size_t n = len / dimension;
    CudaKMeansResult r;
    r.dimension = dimension;
    if (n == 0 || k == 0) return r; /* kmeans.rs:67-76 */
    const size_t ek = k < n ? k : n;
    r.centroids.resize(ek * dimension);
    if (assign) assign->resize(n);
    vhip_kmeans_result c{};
    check(vhip_kmeans_fit((int)ordinal, data, n, dimension, k, max_iters, tolerance, (int)metric, init.centroids,
                          init_mode, init.seed, r.centroids.data(), assign ? assign->data() : nullptr, &c));
    r.k = c.k;
    r.iterations = c.iterations;
    r.inertia = c.inertia;
    return r;
}
}  // namespace detail

/* CudaKMeansEngine (kmeans.rs:36-466).  fit() runs on the GPU.  fit_cpu() (kmeans.rs:240-357)
 * is the reference's host Rust code and stays there: this header mirrors the GPU path only. */
class CudaKMeansEngine {
public:
    CudaKMeansEngine() : ctx_(CudaDeviceContext()) {}
    const CudaDeviceContext &context() const { return ctx_; }
    /* kmeans.rs:58-97 -- seeded k-means++ init (kmeans.rs:409-460) unless init.centroids is set */
    CudaKMeansResult fit(const std::vector<float> &data, size_t dimension, size_t k, size_t max_iters,
                         float tolerance, DistanceMetric metric, const KMeansInit &init = {},
                         std::vector<int32_t> *assign = nullptr) const {
        return detail::kmeans_fit(ctx_.device_id(), data.data(), data.size(), dimension, k, max_iters, tolerance,
                                  metric, VHIP_INIT_KMEANSPP, init, assign);
    }

private:
    CudaDeviceContext ctx_;
};

class DistributedKMeansEngine {
public:
    /* distributed_kmeans.rs:28-38 */
    static DistributedKMeansEngine try_new(size_t num_gpus) {
        detail::require(num_gpus >= 1, "num_gpus must be at least 1");
        detail::check(vhip_dkmeans_check(num_gpus));
        return DistributedKMeansEngine(num_gpus);
    }
    /* :41-44 */
    static DistributedKMeansEngine emulator(size_t num_gpus) {
        detail::require(num_gpus >= 1, "num_gpus must be at least 1");
        return DistributedKMeansEngine(num_gpus);
    }
    static DistributedKMeansEngine new_(size_t num_gpus) { return try_new(num_gpus); }
    size_t num_gpus() const { return g_; }
    /* :55-106 at one GPU: runs on GPU 0 (the reference ran fit_cpu), seeded shuffle init
     * (distributed_kmeans.rs:524-535) unless init.centroids is set */
    CudaKMeansResult fit(const std::vector<float> &data, size_t dimension, size_t k, size_t max_iters,
                         float tolerance, DistanceMetric metric, const KMeansInit &init = {},
                         std::vector<int32_t> *assign = nullptr) const {
        return detail::kmeans_fit(0, data.data(), data.size(), dimension, k, max_iters, tolerance, metric,
                                  VHIP_INIT_SHUFFLE, init, assign);
    }

private:
    explicit DistributedKMeansEngine(size_t g) : g_(g) {}
    size_t g_;
};

/* ---- packed-bit Hamming kNN (extension) -------------------------------------------------- */
class HammingKnnEngine {
public:
    HammingKnnEngine(const uint32_t *codes, size_t n, size_t words, size_t ordinal = 0) : words_(words) {
        vhip_hamming *h = nullptr;
        detail::check(vhip_hamming_create(codes, n, words, (int)ordinal, &h));
        h_.reset(h);
    }
    /* nq x k ids and exact integer distances, best first; lens[q] = min(k, n) */
    void search_batch(const uint32_t *queries, size_t nq, size_t k, uint32_t *ids, uint32_t *dist,
                      size_t *lens) const {
        detail::check(vhip_hamming_search_batch(h_.get(), queries, nq, k, ids, dist, lens));
    }

private:
    struct Del {
        void operator()(vhip_hamming *p) const { vhip_hamming_destroy(p); }
    };
    size_t words_;
    std::unique_ptr<vhip_hamming, Del> h_;
};

/* ---- IVF coarse quantizer (ivf/mod.rs:106-133, ivf/kmeans.rs:262-356) --------------------- */
class IvfCoarseQuantizer {
public:
    IvfCoarseQuantizer(const std::vector<float> &centroids, size_t dimension,
                       DistanceMetric metric = DistanceMetric::L2Squared, size_t ordinal = 0)
        : dim_(dimension) {
        detail::require(dimension > 0 && centroids.size() % dimension == 0, "centroids must be k x dimension");
        vhip_coarse *h = nullptr;
        detail::check(vhip_coarse_create(centroids.data(), centroids.size() / dimension, dimension, (int)metric,
                                         (int)ordinal, &h));
        h_.reset(h);
    }
    size_t nlist() const { return vhip_coarse_nlist(h_.get()); }
    size_t dimension() const { return dim_; }
    /* KMeans::find_nearest_centroid (ivf/kmeans.rs:262-309): (index, metric value) */
    std::pair<size_t, float> find_nearest_centroid(const std::vector<float> &vector) const {
        detail::require(vector.size() == dim_, "dimension mismatch");
        uint32_t c = 0;
        float sc = 0.0f;
        detail::check(vhip_coarse_assign(h_.get(), vector.data(), 1, &c, &sc, nullptr));
        return {c, sc};
    }
    /* the IVF-PQ build loop (ivf/mod.rs:119-132): cluster per point and, if asked, residuals */
    void assign(const std::vector<float> &points, std::vector<uint32_t> &cluster, std::vector<float> &score,
                std::vector<float> *residuals = nullptr) const {
        const size_t n = points.size() / dim_;
        cluster.resize(n);
        score.resize(n);
        if (residuals) residuals->resize(n * dim_);
        detail::check(vhip_coarse_assign(h_.get(), points.data(), n, cluster.data(), score.data(),
                                         residuals ? residuals->data() : nullptr));
    }
    /* KMeans::find_top_centroids (ivf/kmeans.rs:311-356): best first, min(nprobe, nlist) entries */
    std::vector<std::pair<size_t, float>> find_top_centroids(const std::vector<float> &query, size_t nprobe) const {
        detail::require(query.size() == dim_, "dimension mismatch");
        std::vector<std::pair<size_t, float>> out;
        if (nprobe == 0) return out;
        std::vector<uint32_t> ids(nprobe);
        std::vector<float> sc(nprobe);
        size_t len = 0;
        detail::check(vhip_coarse_probe(h_.get(), query.data(), 1, nprobe, ids.data(), sc.data(), &len));
        for (size_t j = 0; j < len; ++j) out.emplace_back(ids[j], sc[j]);
        return out;
    }

private:
    struct Del {
        void operator()(vhip_coarse *p) const { vhip_coarse_destroy(p); }
    };
    size_t dim_;
    std::unique_ptr<vhip_coarse, Del> h_;
};

/* ---- files of the offline trainer (storage/mmap.rs, ivf/serializer.rs) ------------------- */
/* A read-only view of n floats (the &[f32] that MmapStorage::as_raw_slice returns). */
struct FloatSlice {
    const float *ptr = nullptr;
    size_t n = 0;
    const float *data() const { return ptr; }
    size_t size() const { return n; }
    bool empty() const { return n == 0; }
    const float *begin() const { return ptr; }
    const float *end() const { return ptr + n; }
    float operator[](size_t i) const { return ptr[i]; }
};

/* MmapStorage (storage/mmap.rs:56-260): open() maps the file read-only (vhip_vecrstor_map);
 * get() and as_raw_slice() read the mapping in place, and engines built from the slice upload
 * straight from the page cache.  Copies share the mapping, which is unmapped with the last. */
class MmapStorage {
public:
    static void create(const std::string &path, size_t dimension, const std::vector<std::vector<float>> &vectors) {
        std::vector<float> flat;
        for (const auto &v : vectors) {
            detail::require(v.size() == dimension, "dimension mismatch");
            flat.insert(flat.end(), v.begin(), v.end());
        }
        create_from_flat(path, dimension, flat);
    }
    static void create_from_flat(const std::string &path, size_t dimension, const std::vector<float> &flat) {
        detail::require(dimension > 0 && flat.size() % dimension == 0, "dimension mismatch");
        detail::check(vhip_vecrstor_write(path.c_str(), flat.data(), flat.size() / dimension, dimension));
    }
    static MmapStorage open(const std::string &path) {
        MmapStorage s;
        vhip_vecrstor_view *v = nullptr;
        detail::check(vhip_vecrstor_map(path.c_str(), &s.data_, &s.n_, &s.dim_, &v));
        s.view_.reset(v, vhip_vecrstor_unmap);
        return s;
    }
    size_t dimension() const { return dim_; }
    size_t len() const { return n_; }
    bool is_empty() const { return n_ == 0; }
    const float *get(size_t id) const {
        detail::require(id < n_, "vector id out of bounds");
        return data_ + id * dim_;
    }
    FloatSlice as_raw_slice() const { return FloatSlice{data_, n_ * dim_}; }

private:
    std::shared_ptr<vhip_vecrstor_view> view_;
    const float *data_ = nullptr;
    size_t n_ = 0, dim_ = 0;
};

/* CentroidFileData (ivf/serializer.rs:380-393) */
struct CentroidFileData {
    std::vector<float> centroids;
    size_t dimension = 0;
    size_t k = 0;
    DistanceMetric metric = DistanceMetric::L2Squared;
    size_t iterations = 0;
    float inertia = 0.0f;
};

struct IvfPqSerializer {
    /* ivf/serializer.rs:264-306 */
    static void save_centroid_file(const std::string &path, const std::vector<float> &centroids, size_t dimension,
                                   size_t k, DistanceMetric metric, size_t iterations, float inertia) {
        detail::require(centroids.size() == k * dimension, "centroids must be k x dimension");
        detail::check(vhip_centroid_file_save(path.c_str(), centroids.data(), dimension, k, (int)metric, iterations,
                                              inertia));
    }
    /* ivf/serializer.rs:309-360 */
    static CentroidFileData load_centroid_file(const std::string &path) {
        CentroidFileData f;
        int m = 0;
        detail::check(vhip_centroid_file_info(path.c_str(), &f.dimension, &f.k, &m, &f.iterations, &f.inertia));
        f.metric = (DistanceMetric)m;
        f.centroids.resize(f.k * f.dimension);
        detail::check(vhip_centroid_file_load(path.c_str(), f.centroids.data(), f.k, f.dimension));
        return f;
    }
};

/* vector-mpi fit_cuda_aware (src/distributed_kmeans.rs:375-415) */
inline CudaKMeansResult fit_cuda_aware(const std::vector<float> &all_data, size_t dimension, size_t k,
                                       size_t max_iters, float tolerance, DistanceMetric metric, size_t num_gpus,
                                       uint64_t seed = 42) {
    KMeansInit ini;
    ini.seed = seed;
    if ((num_gpus ? num_gpus : 1) > 1)
        return DistributedKMeansEngine::emulator(num_gpus).fit(all_data, dimension, k, max_iters, tolerance, metric,
                                                              ini);
    return CudaKMeansEngine().fit(all_data, dimension, k, max_iters, tolerance, metric, ini);
}

/* ---- product quantization and the IVF-PQ index (vector-index/src/ivf) ------------------ */
/* IvfPqConfig (ivf/config.rs:25-154); max_train_points 0 stands for None */
struct IvfPqConfig {
    size_t nlist = 64, nprobe = 8, num_subvectors = 8, sub_clusters = 256, max_kmeans_iters = 25;
    float kmeans_tolerance = 1e-4f;
    size_t max_train_points = 0;

    static IvfPqConfig make(size_t nlist, size_t nprobe, size_t num_subvectors) {
        IvfPqConfig c;
        c.nlist = nlist;
        c.nprobe = nprobe;
        c.num_subvectors = num_subvectors;
        return c;
    }
    IvfPqConfig with_sub_clusters(size_t v) const { IvfPqConfig c = *this; c.sub_clusters = v; return c; }
    IvfPqConfig with_max_kmeans_iters(size_t v) const { IvfPqConfig c = *this; c.max_kmeans_iters = v; return c; }
    IvfPqConfig with_kmeans_tolerance(float v) const { IvfPqConfig c = *this; c.kmeans_tolerance = v; return c; }
    IvfPqConfig with_max_train_points(size_t v) const { IvfPqConfig c = *this; c.max_train_points = v; return c; }
    size_t sub_dimension(size_t dimension) const { return num_subvectors ? dimension / num_subvectors : 0; }
    vhip_ivfpq_config c() const {
        return vhip_ivfpq_config{nlist, nprobe, num_subvectors, sub_clusters, max_kmeans_iters, kmeans_tolerance,
                                 max_train_points};
    }
    static IvfPqConfig from_c(const vhip_ivfpq_config &v) {
        IvfPqConfig c;
        c.nlist = v.nlist;
        c.nprobe = v.nprobe;
        c.num_subvectors = v.num_subvectors;
        c.sub_clusters = v.sub_clusters;
        c.max_kmeans_iters = v.max_kmeans_iters;
        c.kmeans_tolerance = v.kmeans_tolerance;
        c.max_train_points = v.max_train_points;
        return c;
    }
    void validate(size_t dimension) const {
        const vhip_ivfpq_config v = c();
        detail::check(vhip_ivfpq_config_validate(&v, dimension));
    }
    bool operator==(const IvfPqConfig &o) const {
        return nlist == o.nlist && nprobe == o.nprobe && num_subvectors == o.num_subvectors &&
               sub_clusters == o.sub_clusters && max_kmeans_iters == o.max_kmeans_iters &&
               kmeans_tolerance == o.kmeans_tolerance && max_train_points == o.max_train_points;
    }
};

/* ProductQuantizer (ivf/pq.rs:12-293): training, encoding and ADC tables run on the GPU */
class ProductQuantizer {
public:
    size_t dimension = 0, num_subvectors = 0, sub_dimension = 0, sub_clusters = 0;
    std::vector<float> codebooks;  // num_subvectors x sub_clusters x sub_dimension

    ProductQuantizer() = default;
    ProductQuantizer(size_t dim, size_t m, size_t ks, std::vector<float> cb)
        : dimension(dim), num_subvectors(m), sub_dimension(m ? dim / m : 0), sub_clusters(ks), codebooks(std::move(cb)) {
        detail::require(m > 0 && dim % m == 0, "dimension must be divisible by num_subvectors");
        detail::require(codebooks.size() == m * ks * sub_dimension, "codebooks must hold M x Ks x sub_dimension floats");
    }
    /* pq.rs:53-107 */
    static ProductQuantizer train(const std::vector<float> &data, size_t dim, size_t m, size_t ks, size_t max_iters,
                                  float tolerance, DistanceMetric metric, uint64_t seed = 42, size_t ordinal = 0) {
        detail::require(m > 0 && dim % m == 0, "dimension must be divisible by num_subvectors");
        std::vector<float> cb(m * ks * (dim / m));
        detail::check(vhip_pq_train((int)ordinal, data.data(), data.size() / dim, dim, m, ks, max_iters, tolerance,
                                    (int)metric, nullptr, seed, cb.data()));
        return ProductQuantizer(dim, m, ks, std::move(cb));
    }
    const float *get_sub_centroid(size_t m, size_t k) const {
        return codebooks.data() + (m * sub_clusters + k) * sub_dimension;
    }
    /* pq.rs:203-214 */
    std::vector<uint8_t> encode_batch(const std::vector<float> &data, DistanceMetric metric, size_t ordinal = 0) const {
        const size_t n = data.size() / dimension;
        std::vector<uint8_t> codes(n * num_subvectors);
        detail::check(vhip_pq_encode((int)ordinal, codebooks.data(), dimension, num_subvectors, sub_clusters,
                                     (int)metric, data.data(), n, codes.data()));
        return codes;
    }
    /* pq.rs:178-200 */
    std::vector<uint8_t> encode(const std::vector<float> &vector, DistanceMetric metric) const {
        detail::require(vector.size() == dimension, "dimension mismatch");
        return encode_batch(vector, metric);
    }
    /* pq.rs:217-229 */
    std::vector<float> decode(const std::vector<uint8_t> &code) const {
        detail::require(code.size() == num_subvectors, "code length must equal num_subvectors");
        std::vector<float> v(dimension);
        for (size_t m = 0; m < num_subvectors; ++m)
            std::memcpy(&v[m * sub_dimension], get_sub_centroid(m, code[m]), sub_dimension * sizeof(float));
        return v;
    }
    /* pq.rs:233-266 */
    std::vector<float> compute_adc_lut(const std::vector<float> &query, DistanceMetric metric, size_t ordinal = 0) const {
        detail::require(query.size() == dimension, "dimension mismatch");
        std::vector<float> lut(num_subvectors * sub_clusters);
        detail::check(vhip_pq_adc_lut((int)ordinal, codebooks.data(), dimension, num_subvectors, sub_clusters,
                                      (int)metric, query.data(), 1, lut.data()));
        return lut;
    }
    /* pq.rs:270-293: quads as (d0 + d1) + (d2 + d3), then the remainder */
    float compute_distance_with_lut(const uint8_t *code, const std::vector<float> &lut) const {
        float total = 0.0f;
        size_t m = 0;
        for (; m + 4 <= num_subvectors; m += 4) {
            const float d0 = lut[m * sub_clusters + code[m]], d1 = lut[(m + 1) * sub_clusters + code[m + 1]];
            const float d2 = lut[(m + 2) * sub_clusters + code[m + 2]], d3 = lut[(m + 3) * sub_clusters + code[m + 3]];
            total += (d0 + d1) + (d2 + d3);
        }
        for (; m < num_subvectors; ++m) total += lut[m * sub_clusters + code[m]];
        return total;
    }
    bool operator==(const ProductQuantizer &o) const {
        return dimension == o.dimension && num_subvectors == o.num_subvectors && sub_clusters == o.sub_clusters &&
               codebooks == o.codebooks;
    }
};

/* InvertedList / InvertedIndex (ivf/inverted_list.rs:8-120) */
struct InvertedList {
    std::vector<VectorId> ids;
    std::vector<uint8_t> codes;
    size_t len() const { return ids.size(); }
    bool is_empty() const { return ids.empty(); }
    const uint8_t *get_code(size_t index, size_t num_subvectors) const { return codes.data() + index * num_subvectors; }
    bool operator==(const InvertedList &o) const { return ids == o.ids && codes == o.codes; }
};
struct InvertedIndex {
    std::vector<InvertedList> lists;
    size_t num_subvectors = 0, total_vectors = 0;
    InvertedIndex(size_t nlist = 0, size_t m = 0) : lists(nlist), num_subvectors(m) {}
    void add(size_t cluster, VectorId id, const std::vector<uint8_t> &code) {
        detail::require(code.size() == num_subvectors, "code length must equal num_subvectors");
        lists.at(cluster).ids.push_back(id);
        lists[cluster].codes.insert(lists[cluster].codes.end(), code.begin(), code.end());
        ++total_vectors;
    }
    size_t nlist() const { return lists.size(); }
    const InvertedList &get_list(size_t c) const { return lists.at(c); }
    bool operator==(const InvertedIndex &o) const {
        return num_subvectors == o.num_subvectors && total_vectors == o.total_vectors && lists == o.lists;
    }
    // CSR parts: sizes, ids, codes
    void csr(std::vector<uint32_t> &sizes, std::vector<uint32_t> &ids, std::vector<uint8_t> &codes) const {
        sizes.clear(); ids.clear(); codes.clear();
        for (const auto &l : lists) {
            sizes.push_back((uint32_t)l.ids.size());
            ids.insert(ids.end(), l.ids.begin(), l.ids.end());
            codes.insert(codes.end(), l.codes.begin(), l.codes.end());
        }
    }
    static InvertedIndex from_csr(const std::vector<uint32_t> &sizes, const uint32_t *ids, const uint8_t *codes,
                                  size_t m) {
        InvertedIndex ix(sizes.size(), m);
        size_t off = 0;
        for (size_t c = 0; c < sizes.size(); ++c) {
            ix.lists[c].ids.assign(ids + off, ids + off + sizes[c]);
            ix.lists[c].codes.assign(codes + off * m, codes + (off + sizes[c]) * m);
            off += sizes[c];
        }
        ix.total_vectors = off;
        return ix;
    }
};

/* IvfPqSerializer::save_to_file / load_from_file (ivf/serializer.rs:26-254) */
struct IvfPqFile {
    IvfPqConfig config;
    std::vector<float> coarse_centroids;
    ProductQuantizer pq;
    InvertedIndex inverted_index;
    size_t dimension = 0;
    DistanceMetric metric = DistanceMetric::L2Squared;
};
struct IvfPqFiles {
    static void save_to_file(const std::string &path, const IvfPqConfig &config, const std::vector<float> &coarse,
                             const ProductQuantizer &pq, const InvertedIndex &inv, size_t dimension,
                             DistanceMetric metric) {
        std::vector<uint32_t> sizes, ids;
        std::vector<uint8_t> codes;
        inv.csr(sizes, ids, codes);
        const vhip_ivfpq_config c = config.c();
        detail::check(vhip_ivfpq_file_save(path.c_str(), &c, dimension, (int)metric, coarse.data(),
                                           dimension ? coarse.size() / dimension : 0, pq.codebooks.data(),
                                           pq.codebooks.size(), sizes.data(), sizes.size(), ids.data(), codes.data()));
    }
    static IvfPqFile load_from_file(const std::string &path) {
        vhip_ivfpq_config c{};
        size_t dim = 0, nc = 0, cbl = 0, nl = 0, tot = 0;
        int m = 0;
        detail::check(vhip_ivfpq_file_info(path.c_str(), &c, &dim, &m, &nc, &cbl, &nl, &tot));
        IvfPqFile f;
        f.config = IvfPqConfig::from_c(c);
        f.dimension = dim;
        f.metric = (DistanceMetric)m;
        f.coarse_centroids.resize(nc * dim);
        std::vector<float> cb(cbl);
        std::vector<uint32_t> sizes(nl), ids(tot + 1);
        std::vector<uint8_t> codes(tot * c.num_subvectors + 1);
        detail::check(vhip_ivfpq_file_load(path.c_str(), f.coarse_centroids.data(), cb.data(), sizes.data(), ids.data(),
                                           codes.data()));
        f.pq = ProductQuantizer(dim, c.num_subvectors, c.sub_clusters, std::move(cb));
        f.inverted_index = InvertedIndex::from_csr(sizes, ids.data(), codes.data(), c.num_subvectors);
        return f;
    }
};

/* IvfPqIndex (ivf/mod.rs:63-449) over a flat row-major storage of `dimension` floats per vector */
class IvfPqIndex {
public:
    /* ivf/mod.rs:81-165 (parallel and sequential builds give the same index) */
    static IvfPqIndex build_with_config(const std::vector<float> &storage, size_t dimension, const IvfPqConfig &config,
                                        DistanceMetric metric, uint64_t seed = 42, size_t ordinal = 0) {
        detail::require(dimension > 0 && storage.size() % dimension == 0, "storage is not a multiple of dimension");
        const vhip_ivfpq_config c = config.c();
        vhip_ivfpq *h = nullptr;
        detail::check(vhip_ivfpq_build((int)ordinal, storage.data(), storage.size() / dimension, dimension, &c,
                                       (int)metric, seed, &h));
        return IvfPqIndex(h, config, metric);
    }
    static IvfPqIndex build(const std::vector<float> &storage, size_t dimension, DistanceMetric metric) {
        return build_with_config(storage, dimension, IvfPqConfig(), metric);
    }
    static IvfPqIndex from_parts(const IvfPqConfig &config, const std::vector<float> &coarse, const ProductQuantizer &pq,
                                 const InvertedIndex &inv, size_t dimension, DistanceMetric metric, size_t ordinal = 0) {
        std::vector<uint32_t> sizes, ids;
        std::vector<uint8_t> codes;
        inv.csr(sizes, ids, codes);
        const vhip_ivfpq_config c = config.c();
        vhip_ivfpq *h = nullptr;
        detail::check(vhip_ivfpq_create((int)ordinal, dimension, (int)metric, &c, coarse.data(), coarse.size() / dimension,
                                        pq.codebooks.data(), sizes.data(), ids.data(), codes.data(), &h));
        return IvfPqIndex(h, config, metric);
    }
    /* ivf/mod.rs:251-345 */
    std::vector<SearchResult> search(const std::vector<float> &query, size_t k) const {
        return search_with_nprobe(query, k, config_.nprobe);
    }
    std::vector<SearchResult> search_with_nprobe(const std::vector<float> &query, size_t k, size_t nprobe) const {
        detail::require(query.size() == info_.dimension, "dimension mismatch");
        return search_batch(query, k, nprobe)[0];
    }
    std::vector<std::vector<SearchResult>> search_batch(const std::vector<float> &queries, size_t k,
                                                        size_t nprobe) const {
        const size_t nq = queries.size() / info_.dimension, kk = std::max<size_t>(k, 1);
        std::vector<uint32_t> ids(nq * kk);
        std::vector<float> dist(nq * kk);
        std::vector<size_t> len(nq);
        detail::check(vhip_ivfpq_search_batch(h_.get(), queries.data(), nq, k, nprobe, ids.data(), dist.data(),
                                              len.data()));
        return detail::to_lists(nq, kk, ids, dist, len);
    }
    /* ivf/mod.rs:358-372 */
    static float evaluate_recall(const std::vector<SearchResult> &gt, const std::vector<SearchResult> &res) {
        if (gt.empty() || res.empty()) return 0.0f;
        const size_t k = std::min(gt.size(), res.size());
        size_t hit = 0;
        for (size_t i = 0; i < k; ++i)
            for (size_t j = 0; j < k; ++j)
                if (res[i].id == gt[j].id) { ++hit; break; }
        return (float)hit / (float)k;
    }
    /* ivf/mod.rs:375-408 */
    void save_to_file(const std::string &path) const {
        IvfPqFiles::save_to_file(path, config_, coarse_centroids(), pq(), inverted_index(), info_.dimension, metric_);
    }
    static IvfPqIndex load_from_file(size_t storage_dimension, const std::string &path) {
        IvfPqFile f = IvfPqFiles::load_from_file(path);
        detail::require(f.dimension == storage_dimension, "dimension mismatch");
        return from_parts(f.config, f.coarse_centroids, f.pq, f.inverted_index, f.dimension, f.metric);
    }
    /* getters (ivf/mod.rs:411-449) */
    const IvfPqConfig &config() const { return config_; }
    DistanceMetric metric() const { return metric_; }
    size_t dimension() const { return info_.dimension; }
    size_t len() const { return info_.num_vectors; }
    bool is_empty() const { return len() == 0; }
    std::vector<float> coarse_centroids() const {
        std::vector<float> c(info_.nlist * info_.dimension);
        detail::check(vhip_ivfpq_export(h_.get(), c.data(), nullptr, nullptr, nullptr, nullptr));
        return c;
    }
    ProductQuantizer pq() const {
        std::vector<float> cb(info_.num_subvectors * info_.sub_clusters * (info_.dimension / info_.num_subvectors));
        detail::check(vhip_ivfpq_export(h_.get(), nullptr, cb.data(), nullptr, nullptr, nullptr));
        return ProductQuantizer(info_.dimension, info_.num_subvectors, info_.sub_clusters, std::move(cb));
    }
    InvertedIndex inverted_index() const {
        std::vector<uint32_t> sizes(info_.nlist), ids(info_.num_vectors + 1);
        std::vector<uint8_t> codes(info_.num_vectors * info_.num_subvectors + 1);
        detail::check(vhip_ivfpq_export(h_.get(), nullptr, nullptr, sizes.data(), ids.data(), codes.data()));
        return InvertedIndex::from_csr(sizes, ids.data(), codes.data(), info_.num_subvectors);
    }

private:
    struct Del {
        void operator()(vhip_ivfpq *p) const { vhip_ivfpq_destroy(p); }
    };
    IvfPqIndex(vhip_ivfpq *h, const IvfPqConfig &c, DistanceMetric m) : h_(h), config_(c), metric_(m) {
        detail::check(vhip_ivfpq_info(h, &info_));
    }
    std::unique_ptr<vhip_ivfpq, Del> h_;
    IvfPqConfig config_;
    DistanceMetric metric_;
    vhip_ivfpq_desc info_{};
};

}  // namespace vector_hip

#endif /* VECTOR_HIP_HPP */
