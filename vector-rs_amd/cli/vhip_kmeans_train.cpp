// vhip_kmeans_train -- the GPU k-means index trainer, as `mpi_kmeans --use-cuda`
// (vector-mpi/src/bin/mpi_kmeans.rs:28-65 flags, 284-364 run_cuda_aware_mode) runs it:
// reads data_dir/shard_0.bin, shard_1.bin, ... (VECRSTOR), fits k coarse centroids on the GPU
// and writes the VRSKMEAN centroid file data_dir/<output>.  Flags keep the reference's names and
// defaults; --seed (default 42) seeds the k-means++ initialisation the reference drew from an
// unseeded thread_rng.
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "vector_hip.h"

namespace {

// parse_metric (mpi_kmeans.rs:67-83): unknown names fall back to squared L2.
int parse_metric(std::string s) {
    for (char &c : s) c = (char)std::tolower((unsigned char)c);
    if (s == "l2" || s == "l2_squared" || s == "euclidean") return VHIP_METRIC_L2SQUARED;
    if (s == "dot" || s == "dot_product" || s == "inner_product") return VHIP_METRIC_DOTPRODUCT;
    if (s == "cosine" || s == "cosine_similarity" || s == "cos") return VHIP_METRIC_COSINE;
    if (s == "manhattan" || s == "l1") return VHIP_METRIC_MANHATTAN;
    if (s == "minkowski" || s == "lp") return VHIP_METRIC_MINKOWSKI;
    if (s == "chebyshev" || s == "linf") return VHIP_METRIC_CHEBYSHEV;
    if (s == "hamming" || s == "l0") return VHIP_METRIC_HAMMING;
    if (s == "mahalanobis") return VHIP_METRIC_MAHALANOBIS;
    if (s == "jaccard" || s == "tanimoto") return VHIP_METRIC_JACCARD;
    if (s == "hellinger") return VHIP_METRIC_HELLINGER;
    std::fprintf(stderr, "Unknown metric '%s', defaulting to L2Squared\n", s.c_str());
    return VHIP_METRIC_L2SQUARED;
}

const char *metric_name(int m) {
    static const char *n[] = {"L2Squared", "DotProduct", "CosineSimilarity", "Manhattan", "Minkowski",
                              "Chebyshev", "Hamming",    "Mahalanobis",      "Jaccard",   "Hellinger"};
    return (m >= 0 && m <= 9) ? n[m] : "?";
}

void usage() {
    std::printf(
        "usage: vhip_kmeans_train [-d DATA_DIR] [-k CLUSTERS] [--max-iters N] [--tolerance T] [-m METRIC]\n"
        "                         [-o OUTPUT] [-g GPUS] [--seed S]\n"
        "  -d, --data-dir   directory with shard_0.bin, shard_1.bin, ... (default: data)\n"
        "  -k, --num-clusters  number of centroids (default: 64)\n"
        "      --max-iters  Lloyd iterations (default: 30)\n"
        "      --tolerance  stop when the largest centroid shift (squared L2) <= T (default: 1e-4)\n"
        "  -m, --metric     l2 | dot | cosine | manhattan | minkowski | chebyshev | hamming |\n"
        "                   mahalanobis | jaccard | hellinger (default: l2)\n"
        "  -o, --output     centroid file name inside DATA_DIR (default: centroids_global.bin)\n"
        "  -g, --num-gpus   GPUs requested (one is used; more than present is an error) (default: 1)\n"
        "      --seed       k-means++ seed (default: 42)\n");
}

}  // namespace

int main(int argc, char **argv) {
    std::string data_dir = "data", output = "centroids_global.bin", metric_s = "l2";
    size_t k = 64, max_iters = 30, gpus = 1;
    float tol = 1e-4f;
    unsigned long long seed = 42;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto val = [&](const char *name) -> const char * {
            if (i + 1 >= argc) {
                std::fprintf(stderr, "missing value for %s\n", name);
                std::exit(2);
            }
            return argv[++i];
        };
        if (a == "-h" || a == "--help") {
            usage();
            return 0;
        } else if (a == "-d" || a == "--data-dir") {
            data_dir = val("--data-dir");
        } else if (a == "-k" || a == "--num-clusters") {
            k = std::strtoull(val("--num-clusters"), nullptr, 10);
        } else if (a == "--max-iters") {
            max_iters = std::strtoull(val("--max-iters"), nullptr, 10);
        } else if (a == "--tolerance") {
            tol = std::strtof(val("--tolerance"), nullptr);
        } else if (a == "-m" || a == "--metric") {
            metric_s = val("--metric");
        } else if (a == "-o" || a == "--output") {
            output = val("--output");
        } else if (a == "-g" || a == "--num-gpus" || a == "--gpus") {
            gpus = std::strtoull(val("--num-gpus"), nullptr, 10);
        } else if (a == "--seed") {
            seed = std::strtoull(val("--seed"), nullptr, 10);
        } else {
            std::fprintf(stderr, "unknown argument '%s'\n", a.c_str());
            usage();
            return 2;
        }
    }
    const int metric = parse_metric(metric_s);
    std::printf("=== GPU k-Means Training ===\n");
    std::printf("  Data dir:      %s\n  GPUs:          %zu\n  Clusters (k):  %zu\n  Max iters:     %zu\n"
                "  Metric:        %s\n  ---\n",
                data_dir.c_str(), gpus, k, max_iters, metric_name(metric));
    vhip_kmeans_result r;
    size_t shards = 0;
    const auto t0 = std::chrono::steady_clock::now();
    const int rc = vhip_train_from_shards(data_dir.c_str(), k, max_iters, tol, metric, gpus, output.c_str(), seed, &r,
                                          &shards);
    const double secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    if (rc != VHIP_OK) {
        std::fprintf(stderr, "Error: %s\n", vhip_last_error());
        return 1;
    }
    std::printf("  Shards read:   %zu\n  Dimension:     %zu\n  Iterations:    %zu\n  Inertia:       %.6f\n"
                "  Elapsed:       %.3fs\n  Output:        %s/%s\n=== Training Complete ===\n",
                shards, r.dimension, r.iterations, (double)r.inertia, secs, data_dir.c_str(), output.c_str());
    return 0;
}
