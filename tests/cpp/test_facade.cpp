// C++ restatement of the reference's own tests of the GPU hot path, run against the C++ host
// API (include/vector_hip.hpp) over the C ABI.  Each test names the Rust test it restates.
//
//   test_facade --host   tests that need no GPU (error semantics, collective merge)
//   test_facade          all tests (a gfx950 GPU must be visible)
//
// Exit status 0 when every test passed; one line per test on stdout.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "vector_hip.hpp"

using namespace vector_hip;

static int g_failed = 0;
#define CHECK(cond)                                                                        \
    do {                                                                                   \
        if (!(cond)) throw std::runtime_error(std::string("check failed: ") + #cond);     \
    } while (0)

static void run(const char *name, const std::function<void()> &f) {
    try {
        f();
        std::printf("PASS %s\n", name);
    } catch (const std::exception &e) {
        ++g_failed;
        std::printf("FAIL %s: %s\n", name, e.what());
    }
    std::fflush(stdout);
}

// exact squared-L2 top-k in double with lowest-id ties (the FlatIndex answer for these data)
static std::vector<std::pair<uint32_t, double>> brute_l2(const std::vector<float> &data, size_t dim,
                                                         const float *q, size_t k) {
    const size_t n = data.size() / dim;
    std::vector<std::pair<uint32_t, double>> all;
    for (size_t i = 0; i < n; ++i) {
        double s = 0;
        for (size_t d = 0; d < dim; ++d) {
            const double t = (double)data[i * dim + d] - q[d];
            s += t * t;
        }
        all.push_back({(uint32_t)i, s});
    }
    std::stable_sort(all.begin(), all.end(), [](auto &a, auto &b) { return a.second < b.second; });
    all.resize(std::min(k, n));
    return all;
}

static std::vector<float> knn_rs_data(int n) {  // knn.rs:416-425
    std::vector<float> v;
    for (int i = 0; i < n; ++i) {
        v.push_back((float)(i * i) * 0.1f);
        v.push_back((float)i * 2.0f);
        v.push_back((float)(i + 5));
        v.push_back((float)(i * 3));
    }
    return v;
}

template <class F>
static CudaError expect_error(F f) {
    try {
        f();
    } catch (const CudaError &e) {
        return e;
    }
    throw std::runtime_error("expected a CudaError");
}

static void host_tests() {
    run("ivf_pq_config default / builders / validation (ivf/config.rs:156-240)", [] {
        IvfPqConfig d;
        CHECK(d.nlist == 64 && d.nprobe == 8 && d.num_subvectors == 8 && d.sub_clusters == 256 && d.max_kmeans_iters == 25);
        d.validate(128);
        auto c = IvfPqConfig::make(32, 4, 4).with_sub_clusters(64).with_max_kmeans_iters(15).with_kmeans_tolerance(1e-5f);
        CHECK(c.sub_dimension(128) == 32);
        c.validate(128);
        const IvfPqConfig bad[] = {IvfPqConfig::make(0, 1, 4), IvfPqConfig::make(10, 0, 4), IvfPqConfig::make(10, 11, 4),
                                   IvfPqConfig::make(10, 5, 0), IvfPqConfig::make(10, 5, 5),
                                   IvfPqConfig::make(10, 5, 4).with_sub_clusters(0),
                                   IvfPqConfig::make(10, 5, 4).with_sub_clusters(300),
                                   IvfPqConfig::make(10, 5, 4).with_max_kmeans_iters(0),
                                   IvfPqConfig::make(10, 5, 4).with_kmeans_tolerance(-1.0f)};
        for (const auto &b : bad) {
            bool threw = false;
            try { b.validate(128); } catch (const CudaError &e) { threw = e.kind() == CudaError::Kind::InvalidConfig; }
            CHECK(threw);
        }
    });
    run("pq distance_with_lut and sub-centroid accessor (ivf/pq.rs:349-426)", [] {
        ProductQuantizer pq(4, 2, 2, {0, 0, 1, 1, 0, 0, 2, 2});
        const std::vector<float> lut{2, 0, 8, 0};
        const uint8_t c11[2] = {1, 1}, c00[2] = {0, 0};
        CHECK(pq.compute_distance_with_lut(c11, lut) == 0.0f && pq.compute_distance_with_lut(c00, lut) == 10.0f);
        ProductQuantizer acc(4, 2, 2, {1, 2, 3, 4, 5, 6, 7, 8});
        CHECK(acc.get_sub_centroid(1, 0)[0] == 5.0f && acc.get_sub_centroid(0, 1)[1] == 4.0f);
        CHECK((acc.decode({1, 0}) == std::vector<float>{3, 4, 5, 6}));
    });
    run("ivf_pq serializer roundtrip (ivf/serializer.rs:438-480)", [] {
        const std::string p = "/tmp/vhip_facade_ivfpq.bin";
        auto cfg = IvfPqConfig::make(2, 1, 2).with_sub_clusters(2).with_max_kmeans_iters(10);
        std::vector<float> coarse{0, 0, 0, 0, 1, 1, 1, 1};
        ProductQuantizer pq(4, 2, 2, {0, 0, 0.5f, 0.5f, 0, 0, 0.5f, 0.5f});
        InvertedIndex inv(2, 2);
        inv.add(0, 10, {0, 1});
        inv.add(1, 20, {1, 0});
        IvfPqFiles::save_to_file(p, cfg, coarse, pq, inv, 4, DistanceMetric::L2Squared);
        auto f = IvfPqFiles::load_from_file(p);
        CHECK(f.config == cfg && f.coarse_centroids == coarse && f.pq == pq && f.inverted_index == inv);
        CHECK(f.dimension == 4 && f.metric == DistanceMetric::L2Squared);
        std::remove(p.c_str());
    });
    run("centroid_file_roundtrip (ivf/serializer.rs:552-575)", [] {
        const std::string p = "/tmp/vhip_facade_centroids.bin";
        IvfPqSerializer::save_centroid_file(p, {1, 2, 3, 4, 5, 6, 7, 8}, 4, 2, DistanceMetric::L2Squared, 15, 42.5f);
        auto f = IvfPqSerializer::load_centroid_file(p);
        CHECK((f.centroids == std::vector<float>{1, 2, 3, 4, 5, 6, 7, 8}) && f.dimension == 4 && f.k == 2);
        CHECK(f.metric == DistanceMetric::L2Squared && f.iterations == 15 && std::fabs(f.inertia - 42.5f) < 1e-6f);
        std::remove(p.c_str());
    });
    run("mmap storage round trip (storage/mmap.rs:297-310)", [] {
        const std::string p = "/tmp/vhip_facade_vectors.bin";
        MmapStorage::create_from_flat(p, 3, {1, 2, 3, 4, 5, 6});
        auto st = MmapStorage::open(p);
        CHECK(st.len() == 2 && st.dimension() == 3 && st.get(1)[0] == 4.0f && st.get(1)[2] == 6.0f);
        // as_raw_slice is the mapping itself, 24 bytes past a page boundary
        auto sl = st.as_raw_slice();
        CHECK(sl.size() == 6 && sl[5] == 6.0f && (reinterpret_cast<uintptr_t>(sl.data()) & 4095u) == 24u);
        auto copy = st;  // copies share the mapping
        CHECK(copy.as_raw_slice().data() == sl.data());
        MmapStorage::create(p, 2, {{1, 2}, {3, 4}, {5, 6}});
        auto st2 = MmapStorage::open(p);
        CHECK(st2.len() == 3 && st2.get(2)[1] == 6.0f);
        CHECK(expect_error([&] { MmapStorage::create(p, 3, {{1, 2}}); }).kind() == CudaError::Kind::InvalidConfig);
        CHECK(expect_error([&] { MmapStorage::open("/tmp/vhip_facade_missing.bin"); }).kind() == CudaError::Kind::InvalidConfig);
        std::remove(p.c_str());
    });
    run("ddp_knn_insufficient_hardware_error (distributed_knn.rs:470)", [] {
        const size_t avail = CudaDeviceContext::device_count(), req = avail + 100;
        auto e = expect_error([&] {
            DistributedKnnEngine::try_new({1, 2, 3, 4}, 2, req, GpuShardMode::Sharded, DistanceMetric::L2Squared);
        });
        CHECK(e.kind() == CudaError::Kind::InsufficientDevices);
        CHECK(e.requested() == req && e.available() == avail);
    });
    run("ddp_kmeans_insufficient_hardware_error (distributed_kmeans.rs:625)", [] {
        const size_t avail = CudaDeviceContext::device_count(), req = avail + 100;
        auto e = expect_error([&] { DistributedKMeansEngine::try_new(req); });
        CHECK(e.kind() == CudaError::Kind::InsufficientDevices && e.requested() == req && e.available() == avail);
    });
    run("strict_hardware_validation_error (integration_tests.rs:164)", [] {
        const size_t avail = CudaDeviceContext::device_count(), req = avail + 10;
        auto e = expect_error([&] { DistributedKMeansEngine::try_new(req); });
        CHECK(e.kind() == CudaError::Kind::InsufficientDevices && e.requested() == req && e.available() == avail);
    });
    run("device context with_ordinal / software_emulator (device.rs:173-221)", [] {
        const size_t missing = CudaDeviceContext::device_count() + 100;
        auto emu = CudaDeviceContext::with_ordinal(missing);
        CHECK(!emu.is_hardware_available() && emu.device_id() == missing && emu.total_memory_bytes() == 0);
        CHECK(!emu.device_name().empty());
        auto sw = CudaDeviceContext::software_emulator(3);
        CHECK(!sw.is_hardware_available() && sw.device_id() == 3 && sw.total_memory_bytes() == 0);
        auto e = expect_error([&] { CudaDeviceContext::with_ordinal_strict(missing); });
        CHECK(e.kind() == CudaError::Kind::DeviceNotFound || e.kind() == CudaError::Kind::HardwareNotAvailable);
        if (e.kind() == CudaError::Kind::DeviceNotFound) CHECK(e.ordinal() == missing);
    });
    run("ddp_kmeans_getters (distributed_kmeans.rs:619)", [] {
        CHECK(DistributedKMeansEngine::emulator(6).num_gpus() == 6);
    });
    run("num_gpus >= 1 and dimension divisibility are enforced", [] {
        CHECK(expect_error([] { DistributedKMeansEngine::emulator(0); }).kind() == CudaError::Kind::InvalidConfig);
        CHECK(expect_error([] {
                  DistributedKnnEngine::emulator({1, 2, 3}, 2, 1, GpuShardMode::Sharded, DistanceMetric::L2Squared);
              }).kind() == CudaError::Kind::InvalidConfig);
    });
    run("top_k_reduce (collective.rs:239)", [] {
        auto m = CollectiveOps::top_k_reduce({{{0, 1.0f}, {1, 5.0f}}, {{10, 0.5f}, {11, 4.0f}}}, 2,
                                             DistanceMetric::L2Squared);
        CHECK(m.size() == 2 && m[0].id == 10 && m[1].id == 0);
    });
    run("top_k_reduce_empty_and_zero_k (collective.rs:250)", [] {
        CHECK(CollectiveOps::top_k_reduce({}, 5, DistanceMetric::L2Squared).empty());
        CHECK(CollectiveOps::top_k_reduce({{{0, 1.0f}}}, 0, DistanceMetric::L2Squared).empty());
    });
    run("top_k_reduce_cosine_metric (collective.rs:260)", [] {
        auto m = CollectiveOps::top_k_reduce({{{0, 0.85f}, {1, 0.40f}}, {{2, 0.95f}, {3, 0.70f}}}, 3,
                                             DistanceMetric::CosineSimilarity);
        CHECK(m.size() == 3 && m[0].id == 2 && m[1].id == 0 && m[2].id == 3);
    });
    run("top_k_reduce_k_greater_than_total_candidates (collective.rs:274)", [] {
        auto m = CollectiveOps::top_k_reduce({{{0, 2.0f}}, {{1, 1.0f}}}, 10, DistanceMetric::L2Squared);
        CHECK(m.size() == 2 && m[0].id == 1 && m[1].id == 0);
    });
}

static void gpu_tests() {
    // ---- knn.rs:410-542 ----
    run("cuda_knn_exact_match_vs_cpu_flat (knn.rs:411)", [] {
        auto data = knn_rs_data(50);
        CudaKnnEngine e(data, 4, DistanceMetric::L2Squared);
        auto gpu = e.search(std::vector<float>(data.begin() + 40, data.begin() + 44), 5);
        auto cpu = brute_l2(data, 4, data.data() + 40, 5);
        CHECK(gpu.size() == 5);
        for (int i = 0; i < 5; ++i) CHECK(gpu[i].id == cpu[i].first && std::fabs(gpu[i].distance - cpu[i].second) < 1e-4);
    });
    run("cuda_knn_batch_queries (knn.rs:444)", [] {
        CudaKnnEngine e({0, 0, 1, 1, 2, 2}, 2, DistanceMetric::L2Squared);
        auto r = e.search_batch({0.1f, 0.1f, 1.9f, 1.9f}, 1);
        CHECK(r.size() == 2 && r[0][0].id == 0 && r[1][0].id == 2);
    });
    run("cuda_knn_empty_and_zero_k (knn.rs:458)", [] {
        CudaKnnEngine e({1, 2, 3, 4}, 2, DistanceMetric::L2Squared);
        CHECK(e.search(std::vector<float>{}, 5).empty() && e.search_batch(std::vector<float>{}, 5).empty());
        CHECK(e.search({1, 2}, 0).empty());
        auto b = e.search_batch({1, 2}, 0);
        CHECK(b.size() == 1 && b[0].empty());
    });
    run("cuda_knn_k_greater_than_num_vectors (knn.rs:475)", [] {
        CudaKnnEngine e({0, 0, 1, 1, 2, 2}, 2, DistanceMetric::L2Squared);
        CHECK(e.search({0.5f, 0.5f}, 100).size() == 3);
    });
    run("cuda_knn_cosine_similarity (knn.rs:485)", [] {
        CudaKnnEngine e({1, 0, 0, 1, -1, 0}, 2, DistanceMetric::CosineSimilarity);
        auto r = e.search({0.95f, 0.05f}, 3);
        CHECK(r.size() == 3 && r[0].id == 0 && r[2].id == 2);
    });
    run("cuda_knn_dot_product (knn.rs:502)", [] {
        CudaKnnEngine e({1, 1, 2, 2, 3, 3}, 2, DistanceMetric::DotProduct);
        auto r = e.search({2, 3}, 2);
        CHECK(r.size() == 2 && r[0].id == 2 && r[1].id == 1 && std::fabs(r[0].distance - 15.0f) < 1e-5);
    });
    run("cuda_knn_engine_getters (knn.rs:519)", [] {
        CudaKnnEngine e({1, 2, 3, 4, 5, 6}, 3, DistanceMetric::L2Squared);
        CHECK(e.dimension() == 3 && e.num_vectors() == 2 && e.metric() == DistanceMetric::L2Squared);
        CHECK(e.context().device_id() == 0);
    });
    run("cuda_knn_exact_self_query (knn.rs:531)", [] {
        std::vector<float> data{10, 20, 30, 40, 50, 60};
        CudaKnnEngine e(data, 2, DistanceMetric::L2Squared);
        for (uint32_t i = 0; i < 3; ++i) {
            auto r = e.search(std::vector<float>(data.begin() + 2 * i, data.begin() + 2 * i + 2), 1);
            CHECK(r.size() == 1 && r[0].id == i && std::fabs(r[0].distance) < 1e-4);
        }
    });
    run("engine built from a mapped VECRSTOR file (storage/mmap.rs + knn.rs:85)", [] {
        const std::string p = "/tmp/vhip_facade_base.bin";
        auto data = knn_rs_data(300);
        MmapStorage::create_from_flat(p, 4, data);
        auto st = MmapStorage::open(p);
        CudaKnnEngine a(data, 4, DistanceMetric::L2Squared);
        CudaKnnEngine b(st.as_raw_slice().data(), st.as_raw_slice().size(), 4, DistanceMetric::L2Squared);
        auto c = CudaKnnEngine::from_vecrstor(p, DistanceMetric::L2Squared);
        CHECK(c.num_vectors() == 300 && c.dimension() == 4);
        std::vector<float> q(data.begin() + 40, data.begin() + 56);
        auto ra = a.search_batch(q, 7), rb = b.search_batch(q, 7), rc = c.search_batch(q, 7);
        CHECK(ra.size() == 4 && rb.size() == 4 && rc.size() == 4);
        for (size_t i = 0; i < ra.size(); ++i)
            for (size_t j = 0; j < ra[i].size(); ++j) {
                CHECK(ra[i][j].id == rb[i][j].id && ra[i][j].distance == rb[i][j].distance);
                CHECK(ra[i][j].id == rc[i][j].id && ra[i][j].distance == rc[i][j].distance);
            }
        std::remove(p.c_str());
    });
    // ---- ddp/distributed_knn.rs:270-467 ----
    run("ddp_knn_sharded_mode_exact_match (distributed_knn.rs:271)", [] {
        auto data = knn_rs_data(60);
        auto e = DistributedKnnEngine::emulator(data, 4, 3, GpuShardMode::Sharded, DistanceMetric::L2Squared);
        CHECK(e.num_gpus() == 3 && e.num_vectors() == 60);
        auto r = e.search(std::vector<float>(data.begin() + 100, data.begin() + 104), 5);
        auto cpu = brute_l2(data, 4, data.data() + 100, 5);
        CHECK(r.size() == 5);
        for (int i = 0; i < 5; ++i) CHECK(r[i].id == cpu[i].first && std::fabs(r[i].distance - cpu[i].second) < 1e-4);
    });
    run("ddp_knn_replicated_mode (distributed_knn.rs:313)", [] {
        auto e = DistributedKnnEngine::emulator({0, 0, 1, 1, 2, 2, 3, 3}, 2, 2, GpuShardMode::Replicated,
                                                DistanceMetric::L2Squared);
        auto r = e.search_batch({0.1f, 0.1f, 2.9f, 2.9f}, 1);
        CHECK(r.size() == 2 && r[0][0].id == 0 && r[1][0].id == 3);
    });
    run("ddp_knn_empty_and_zero_k (distributed_knn.rs:334)", [] {
        for (auto mode : {GpuShardMode::Sharded, GpuShardMode::Replicated}) {
            auto e = DistributedKnnEngine::emulator({1, 2, 3, 4}, 2, 2, mode, DistanceMetric::L2Squared);
            CHECK(e.search(std::vector<float>{}, 5).empty() && e.search_batch(std::vector<float>{}, 5).empty());
            CHECK(e.search({1, 2}, 0).empty());
        }
    });
    run("ddp_knn_sharded_global_id_mapping (distributed_knn.rs:364)", [] {
        auto e = DistributedKnnEngine::emulator({10, 10, 20, 20, 30, 30, 40, 40}, 2, 2, GpuShardMode::Sharded,
                                                DistanceMetric::L2Squared);
        CHECK(e.search({39.9f, 40.1f}, 1)[0].id == 3 && e.search({20.1f, 19.9f}, 1)[0].id == 1);
    });
    run("ddp_knn_cosine_metric_sharded_and_replicated (distributed_knn.rs:394)", [] {
        for (auto mode : {GpuShardMode::Sharded, GpuShardMode::Replicated}) {
            auto e = DistributedKnnEngine::emulator({1, 0, 0, 1, -1, 0, 0, -1}, 2, 2, mode,
                                                    DistanceMetric::CosineSimilarity);
            auto r = e.search({0.99f, 0.01f}, 2);
            CHECK(r.size() == 2 && r[0].id == 0);
        }
    });
    run("ddp_knn_more_gpus_than_vectors (distributed_knn.rs:430)", [] {
        auto e = DistributedKnnEngine::emulator({1, 1, 2, 2}, 2, 8, GpuShardMode::Sharded, DistanceMetric::L2Squared);
        CHECK(e.num_gpus() == 2 && e.num_vectors() == 2);
        auto r = e.search({1, 1}, 2);
        CHECK(r.size() == 2 && r[0].id == 0);
    });
    run("ddp_knn_getters (distributed_knn.rs:451)", [] {
        auto e = DistributedKnnEngine::emulator({1, 2, 3, 4, 5, 6}, 3, 2, GpuShardMode::Sharded,
                                                DistanceMetric::L2Squared);
        CHECK(e.num_gpus() == 2 && e.num_vectors() == 2 && e.dimension() == 3);
        CHECK(e.mode() == GpuShardMode::Sharded && e.metric() == DistanceMetric::L2Squared);
    });
    run("ddp_try_new_single_gpu routes to the GPU", [] {
        auto data = knn_rs_data(40);
        auto e = DistributedKnnEngine::try_new(data, 4, 1, GpuShardMode::Sharded, DistanceMetric::L2Squared);
        CHECK(e.num_gpus() == 1 && e.search(std::vector<float>(data.begin() + 28, data.begin() + 32), 1)[0].id == 7);
    });
    // ---- kmeans.rs:473-577 ----
    run("cuda_kmeans_clustering (kmeans.rs:474)", [] {
        std::vector<float> data;
        for (int c = 0; c < 3; ++c)
            for (int i = 0; i < 50; ++i) {
                const float b = 10.0f * c;
                for (float v : {b + 0.1f, b - 0.1f, b + 0.05f, b - 0.05f}) data.push_back(v);
            }
        CudaKMeansEngine eng;
        auto r = eng.fit(data, 4, 3, 20, 1e-4f, DistanceMetric::L2Squared);
        CHECK(r.k == 3 && r.dimension == 4 && r.iterations > 0 && r.inertia < 1.0f);
    });
    run("cuda_kmeans_single_cluster (kmeans.rs:507)", [] {
        auto r = CudaKMeansEngine().fit({1.0f, 1.0f, 1.1f, 0.9f, 0.9f, 1.1f}, 2, 1, 10, 1e-4f,
                                        DistanceMetric::L2Squared);
        CHECK(r.k == 1 && std::fabs(r.centroid(0)[0] - 1.0f) < 0.1f && std::fabs(r.centroid(0)[1] - 1.0f) < 0.1f);
    });
    run("cuda_kmeans_empty_and_zero_k (kmeans.rs:520)", [] {
        CudaKMeansEngine eng;
        CHECK(eng.fit({}, 4, 3, 10, 1e-4f, DistanceMetric::L2Squared).k == 0);
        CHECK(eng.fit({1, 2}, 2, 0, 10, 1e-4f, DistanceMetric::L2Squared).k == 0);
    });
    run("cuda_kmeans_k_greater_than_n (kmeans.rs:530)", [] {
        CHECK(CudaKMeansEngine().fit({1, 2, 3, 4}, 2, 5, 10, 1e-4f, DistanceMetric::L2Squared).k == 2);
    });
    run("cuda_kmeans_cosine_and_dot_product_metrics (kmeans.rs:540)", [] {
        std::vector<float> data{1, 0, 0, 0, 1, 0, 0, 0, 1, 0.9f, 0.1f, 0};
        CudaKMeansEngine eng;
        CHECK(eng.fit(data, 3, 3, 10, 1e-4f, DistanceMetric::CosineSimilarity).k == 3);
        CHECK(eng.fit(data, 3, 3, 10, 1e-4f, DistanceMetric::DotProduct).k == 3);
    });
    run("cuda_kmeans_high_dimension (kmeans.rs:560)", [] {
        std::vector<float> data(20 * 128);
        for (size_t i = 0; i < data.size(); ++i) data[i] = (float)i * 0.01f;
        auto r = CudaKMeansEngine().fit(data, 128, 4, 5, 1e-3f, DistanceMetric::L2Squared);
        CHECK(r.k == 4 && r.dimension == 128);
    });
    run("test_device_context (device.rs:329)", [] {
        CudaDeviceContext ctx;
        CHECK(ctx.device_id() == 0 && ctx.total_memory_bytes() > 0 && !ctx.device_name().empty());
        CHECK(ctx.is_hardware_available());
        auto w = CudaDeviceContext::with_ordinal(0);
        CHECK(w.device_name() == ctx.device_name() && w.total_memory_bytes() == ctx.total_memory_bytes());
        auto copy = ctx;
        CHECK(copy.total_memory_bytes() == ctx.total_memory_bytes());
        CudaKnnEngine e({1, 2, 3, 4}, 2, DistanceMetric::L2Squared);
        CHECK(e.context().device_id() == 0 && e.context().is_hardware_available());
    });
    run("cuda_kmeans_engine_context (kmeans.rs:573)", [] {
        CudaKMeansEngine eng;
        CHECK(eng.context().device_id() == 0 && eng.context().total_memory_bytes() > 0);
    });
    // ---- ddp/distributed_kmeans.rs:548-618 ----
    run("ddp_kmeans_multi_gpu (distributed_kmeans.rs:549)", [] {
        auto r = DistributedKMeansEngine::emulator(4).fit({0, 0, 0.1f, 0.1f, -0.1f, -0.1f, 10, 10, 10.1f, 10.1f,
                                                           9.9f, 9.9f},
                                                          2, 2, 25, 1e-5f, DistanceMetric::L2Squared);
        CHECK(r.k == 2 && r.dimension == 2 && r.iterations > 0 && r.inertia >= 0.0f);
        const float *c0 = r.centroid(0), *c1 = r.centroid(1);
        const float *n0 = c0[0] < 5.0f ? c0 : c1, *n10 = c0[0] < 5.0f ? c1 : c0;
        CHECK(std::fabs(n0[0]) < 0.5f && std::fabs(n0[1]) < 0.5f);
        CHECK(std::fabs(n10[0] - 10.0f) < 0.5f && std::fabs(n10[1] - 10.0f) < 0.5f);
    });
    run("ddp_kmeans_empty_and_zero_k (distributed_kmeans.rs:572)", [] {
        auto e = DistributedKMeansEngine::emulator(4);
        auto a = e.fit({}, 2, 2, 10, 1e-4f, DistanceMetric::L2Squared);
        CHECK(a.k == 0 && a.centroids.empty() && a.iterations == 0);
        auto b = e.fit({1, 2, 3, 4}, 2, 0, 10, 1e-4f, DistanceMetric::L2Squared);
        CHECK(b.k == 0 && b.centroids.empty());
    });
    run("ddp_kmeans_more_gpus_than_vectors (distributed_kmeans.rs:587)", [] {
        auto r = DistributedKMeansEngine::emulator(8).fit({1, 1, 2, 2, 3, 3}, 2, 2, 15, 1e-4f,
                                                          DistanceMetric::L2Squared);
        CHECK(r.k == 2 && r.centroids.size() == 4);
    });
    run("ddp_kmeans_single_cluster (distributed_kmeans.rs:597)", [] {
        auto r = DistributedKMeansEngine::emulator(2).fit({1, 1, 3, 3, 5, 5, 7, 7}, 2, 1, 10, 1e-5f,
                                                          DistanceMetric::L2Squared);
        CHECK(r.k == 1 && std::fabs(r.centroid(0)[0] - 4.0f) < 1e-3f && std::fabs(r.centroid(0)[1] - 4.0f) < 1e-3f);
    });
    run("ddp_kmeans_cosine_metric (distributed_kmeans.rs:609)", [] {
        auto r = DistributedKMeansEngine::emulator(2).fit({1, 0, 0.98f, 0.2f, 0, 1, 0.2f, 0.98f}, 2, 2, 20, 1e-4f,
                                                          DistanceMetric::CosineSimilarity);
        CHECK(r.k == 2 && r.dimension == 2);
    });
    // ---- tests/integration_tests.rs ----
    run("end_to_end_clustering_and_sharded_search (integration_tests.rs:8)", [] {
        std::vector<float> data;
        const float cl[3][4] = {{0.1f, 0.0f, -0.1f, 0.05f}, {9.9f, 10.1f, 10.0f, 9.95f}, {20.0f, 19.9f, 20.1f, 20.05f}};
        for (int c = 0; c < 3; ++c)
            for (int i = 0; i < 30; ++i) data.insert(data.end(), cl[c], cl[c] + 4);
        auto km = DistributedKMeansEngine::emulator(4).fit(data, 4, 3, 30, 1e-5f, DistanceMetric::L2Squared);
        CHECK(km.k == 3 && km.dimension == 4);
        auto knn = DistributedKnnEngine::emulator(data, 4, 3, GpuShardMode::Sharded, DistanceMetric::L2Squared);
        CHECK(knn.num_vectors() == 90);
        auto r = knn.search({10, 10, 10, 10}, 5);
        CHECK(r.size() == 5);
        for (auto &x : r) CHECK(x.id >= 30 && x.id < 60 && x.distance < 1.0f);
    });
    run("single_gpu_vs_multi_gpu_consistency (integration_tests.rs:59)", [] {
        std::vector<float> data;
        for (int i = 0; i < 60; ++i) {
            data.push_back((float)i * 0.5f);
            data.push_back((float)(i * i) * 0.05f);
            data.push_back(std::sin((float)i + 3.0f));
        }
        std::vector<float> q{1.0f, 2.0f, 0.5f, 15.0f, 45.0f, -0.5f, 25.0f, 120.0f, 0.8f};
        auto single = CudaKnnEngine(data, 3, DistanceMetric::L2Squared).search_batch(q, 5);
        for (auto mode : {GpuShardMode::Sharded, GpuShardMode::Replicated}) {
            auto other = DistributedKnnEngine::emulator(data, 3, 4, mode, DistanceMetric::L2Squared).search_batch(q, 5);
            CHECK(single.size() == 3 && other.size() == 3);
            for (int a = 0; a < 3; ++a)
                for (int b = 0; b < 5; ++b)
                    CHECK(other[a][b].id == single[a][b].id &&
                          std::fabs(other[a][b].distance - single[a][b].distance) < 1e-4f);
        }
    });
    run("all_metrics_consistency (integration_tests.rs:122)", [] {
        std::vector<float> data{0.8f, 0.6f, 0.8f, 0.0f, 0.0f, 0.6f, 0.1f, 0.1f, -1.0f, -1.0f};
        for (int m = 0; m < 10; ++m) {
            const auto metric = (DistanceMetric)m;
            auto s = CudaKnnEngine(data, 2, metric).search({0.8f, 0.6f}, 3);
            auto d = DistributedKnnEngine::emulator(data, 2, 2, GpuShardMode::Sharded, metric).search({0.8f, 0.6f}, 3);
            CHECK(s.size() == 3 && d.size() == 3);
            for (int i = 0; i < 3; ++i) CHECK(std::fabs(s[i].distance - d[i].distance) < 1e-4f);
        }
    });
    run("find_nearest_centroid_l2 / dot (vector-mpi distributed_kmeans.rs:497-520)", [] {
        IvfCoarseQuantizer q({0, 0, 10, 10}, 2);
        auto r = q.find_nearest_centroid({1, 1});
        CHECK(r.first == 0 && std::fabs(r.second - 2.0f) < 1e-5f);
        IvfCoarseQuantizer d({1, 0, 0, 1}, 2, DistanceMetric::DotProduct);
        CHECK(d.find_nearest_centroid({1, 0}).first == 0);
        auto top = q.find_top_centroids({9, 9}, 5);
        CHECK(top.size() == 2 && top[0].first == 1 && top[1].first == 0);
    });
    run("fit_cuda_aware single and multi GPU (vector-mpi distributed_kmeans.rs:522-548)", [] {
        std::vector<float> data{0.0f, 0.1f, 0.1f, 0.0f, -0.1f, 0.0f, 10.0f, 10.1f, 10.1f, 10.0f, 9.9f, 10.0f};
        for (size_t g : {1, 2}) {
            auto r = fit_cuda_aware(data, 2, 2, 30, 1e-5f, DistanceMetric::L2Squared, g);
            CHECK(r.k == 2 && r.dimension == 2 && r.iterations > 0);
        }
    });
    run("ivf_pq end-to-end search and getters (ivf/mod.rs:456-485, 633-646)", [] {
        std::vector<float> st;
        for (int i = 0; i < 50; ++i)
            for (int d = 0; d < 8; ++d) st.push_back((float)(i * 10 + d) * 0.1f);
        auto cfg = IvfPqConfig::make(4, 2, 2).with_sub_clusters(8).with_max_kmeans_iters(15);
        auto ix = IvfPqIndex::build_with_config(st, 8, cfg, DistanceMetric::L2Squared);
        CHECK(ix.len() == 50 && !ix.is_empty() && ix.config().nlist == 4);
        std::vector<float> q(st.begin() + 80, st.begin() + 88);
        auto r = ix.search(q, 5);
        bool has10 = false;
        for (auto &x : r) has10 |= x.id == 10;
        CHECK(r.size() == 5 && has10);
        CHECK(ix.coarse_centroids().size() == 4 * 8 && ix.pq().num_subvectors == 2 && ix.inverted_index().nlist() == 4);
    });
    run("ivf_pq recall vs flat (ivf/mod.rs:487-515)", [] {
        std::vector<float> st;
        for (int i = 0; i < 100; ++i)
            for (int d = 0; d < 16; ++d) st.push_back((float)((i * 7 + d) % 30));
        auto cfg = IvfPqConfig::make(8, 4, 4).with_sub_clusters(16).with_max_kmeans_iters(20);
        auto ix = IvfPqIndex::build_with_config(st, 16, cfg, DistanceMetric::L2Squared);
        std::vector<float> q(st.begin() + 42 * 16, st.begin() + 43 * 16);
        CudaKnnEngine flat(st, 16, DistanceMetric::L2Squared);
        CHECK(IvfPqIndex::evaluate_recall(flat.search(q, 10), ix.search(q, 10)) >= 0.5f);
        CHECK(IvfPqIndex::evaluate_recall({}, {}) == 0.0f);
    });
    run("ivf_pq save/load, cosine/dot, k = 0, empty storage, nprobe, dimension mismatch (ivf/mod.rs:517-631)", [] {
        const std::string p = "/tmp/vhip_facade_ivfpq_ix.bin";
        std::vector<float> st{1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12};
        auto ix = IvfPqIndex::build_with_config(st, 4, IvfPqConfig::make(2, 2, 2).with_sub_clusters(4),
                                                DistanceMetric::L2Squared);
        ix.save_to_file(p);
        auto lo = IvfPqIndex::load_from_file(4, p);
        CHECK(lo.len() == 3 && lo.inverted_index().nlist() == 2);
        std::remove(p.c_str());
        std::vector<float> cs, ds;
        for (int i = 1; i <= 20; ++i) {
            const float f = (float)i;
            cs.insert(cs.end(), {f, f + 1, f + 2, f + 3});
            ds.insert(ds.end(), {f, f * 2, f * 0.5f, f + 1});
        }
        auto cfg = IvfPqConfig::make(2, 2, 2).with_sub_clusters(4);
        CHECK(IvfPqIndex::build_with_config(cs, 4, cfg, DistanceMetric::CosineSimilarity).search({1, 2, 3, 4}, 2).size() == 2);
        CHECK(IvfPqIndex::build_with_config(ds, 4, cfg, DistanceMetric::DotProduct).search({1, 2, 0.5f, 2}, 2).size() == 2);
        bool empty_threw = false;
        try {
            IvfPqIndex::build_with_config({}, 2, IvfPqConfig::make(1, 1, 1).with_sub_clusters(1), DistanceMetric::L2Squared);
        } catch (const CudaError &e) { empty_threw = e.kind() == CudaError::Kind::EmptyIndex; }
        CHECK(empty_threw);
        auto one = IvfPqIndex::build_with_config({1, 2}, 2, IvfPqConfig::make(1, 1, 1).with_sub_clusters(1),
                                                 DistanceMetric::L2Squared);
        CHECK(one.search({1, 2}, 0).empty());
        std::vector<float> s30;
        for (int i = 0; i < 30; ++i) s30.insert(s30.end(), {(float)i, (float)i + 1, (float)i + 2, (float)i + 3});
        auto ix30 = IvfPqIndex::build_with_config(s30, 4, IvfPqConfig::make(4, 1, 2).with_sub_clusters(4),
                                                  DistanceMetric::L2Squared);
        CHECK(!ix30.search_with_nprobe({0, 1, 2, 3}, 3, 1).empty() && !ix30.search_with_nprobe({0, 1, 2, 3}, 3, 4).empty());
        bool dim_threw = false;
        try { ix30.search({1, 2}, 1); } catch (const CudaError &e) { dim_threw = e.kind() == CudaError::Kind::InvalidConfig; }
        CHECK(dim_threw);
    });
    run("pq training and encoding (ivf/pq.rs:302-346)", [] {
        std::vector<float> data;
        for (int i = 0; i < 20; ++i) {
            const float v = (float)i;
            data.insert(data.end(), {v, v + 1, v + 2, v + 3, v, v, v, v});
        }
        auto pq = ProductQuantizer::train(data, 8, 2, 4, 15, 1e-4f, DistanceMetric::L2Squared);
        CHECK(pq.dimension == 8 && pq.num_subvectors == 2 && pq.sub_dimension == 4 && pq.sub_clusters == 4);
        CHECK(pq.codebooks.size() == 32);
        auto code = pq.encode(std::vector<float>(data.begin(), data.begin() + 8), DistanceMetric::L2Squared);
        CHECK(code[0] < 4 && code[1] < 4 && pq.decode(code).size() == 8);
        auto batch = pq.encode_batch(data, DistanceMetric::L2Squared);
        CHECK(batch[0] == code[0] && batch[1] == code[1]);
        auto lut = pq.compute_adc_lut(std::vector<float>(data.begin(), data.begin() + 8), DistanceMetric::L2Squared);
        CHECK(lut.size() == 8);
    });
    run("explicit-init k-means is deterministic (extension)", [] {
        std::vector<float> data;
        for (int i = 0; i < 4000; ++i) data.push_back(std::sin(0.37f * i) * 3.0f + (i % 7));
        std::vector<float> init(data.begin(), data.begin() + 8 * 4);
        KMeansInit ini;
        ini.centroids = init.data();
        auto a = CudaKMeansEngine().fit(data, 4, 8, 6, -1.0f, DistanceMetric::L2Squared, ini);
        auto b = CudaKMeansEngine().fit(data, 4, 8, 6, -1.0f, DistanceMetric::L2Squared, ini);
        CHECK(a.iterations == 6 && a.centroids == b.centroids);
    });
}

int main(int argc, char **argv) {
    const bool host_only = argc > 1 && std::strcmp(argv[1], "--host") == 0;
    host_tests();
    if (!host_only) {
        if (CudaDeviceContext::device_count() < 1) {
            std::printf("FAIL no gfx950 GPU visible\n");
            return 1;
        }
        gpu_tests();
    }
    std::printf("%s: %d failed\n", host_only ? "host tests" : "all tests", g_failed);
    return g_failed ? 1 : 0;
}
