// coarse.hip -- IVF coarse quantizer on one GPU behind the C ABI.
//
// IvfPqIndex::build_parallel_with_config (vector-index/src/ivf/mod.rs:106-133) trains coarse
// centroids, then runs KMeans::find_nearest_centroid (ivf/kmeans.rs:262-309) for every vector in
// one serial host loop and forms the residual x - c; every search calls
// KMeans::find_top_centroids (ivf/kmeans.rs:311-356), which scores all centroids and sorts them.
// Here both run on the GPU:
//  * assign: the k-means assignment kernels (FP32 MFMA for squared L2 / dot / cosine, VALU for
//    the other metrics) pick each point's centroid -- the lowest index among equals, as the
//    reference's strict comparison in ascending order -- and k_coarse_score (kmeans.hip)
//    recomputes the chosen pair in the reference's direct form and writes the residual;
//  * probe: a kNN engine whose base rows are the centroids answers find_top_centroids for a
//    batch of queries with k = nprobe: best first, equal scores in ascending index order (the
//    reference's stable sort), similarities for dot / cosine.
#include <memory>
#include <vector>

#include "vh_runtime.h"

struct vhip_coarse {
    int dev = 0;
    size_t nlist = 0, dim = 0;
    int metric = 0;
    std::vector<float> centroids;  // nlist x dim, row-major
    vhip_knn *probe = nullptr;
    std::mutex mu;
    ~vhip_coarse() {
        if (probe) vhip_knn_destroy(probe);
    }
};

using namespace vh;

extern "C" {

int vhip_coarse_create(const float *centroids, size_t nlist, size_t dim, int metric, int ordinal, vhip_coarse **out) {
    clear_error();
    if (!out) return set_error(VHIP_ERR_INVALID_CONFIG, "out is null");
    *out = nullptr;
    if (nlist == 0 || dim == 0 || !centroids)
        return set_error(VHIP_ERR_INVALID_CONFIG, "the coarse quantizer needs at least one centroid of dimension > 0");
    if (metric < 0 || metric > 9) return set_error(VHIP_ERR_INVALID_CONFIG, "unknown metric code");
    std::unique_ptr<vhip_coarse> C(new vhip_coarse());
    C->dev = ordinal;
    C->nlist = nlist;
    C->dim = dim;
    C->metric = metric;
    C->centroids.assign(centroids, centroids + nlist * dim);
    VH_CHECK(vhip_knn_create(centroids, nlist, dim, metric, ordinal, &C->probe));
    *out = C.release();
    return VHIP_OK;
}

int vhip_coarse_assign(vhip_coarse *C, const float *points, size_t n, uint32_t *out_cluster, float *out_score,
                       float *out_residual) {
    clear_error();
    if (!C) return set_error(VHIP_ERR_INVALID_CONFIG, "null quantizer");
    if (n == 0) return VHIP_OK;
    if (!points) return set_error(VHIP_ERR_INVALID_CONFIG, "points is null");
    std::lock_guard<std::mutex> lock(C->mu);
    vhip_kmeans *K = nullptr;
    VH_CHECK(vhip_kmeans_create(C->dev, points, n, C->dim, C->metric, &K));
    std::unique_ptr<vhip_kmeans, void (*)(vhip_kmeans *)> hold(K, vhip_kmeans_destroy);
    VH_CHECK(vhip_kmeans_set_centroids(K, C->centroids.data(), C->nlist));
    return vhip_kmeans_assign_only(K, (int32_t *)out_cluster, out_score, out_residual);
}

int vhip_coarse_probe(vhip_coarse *C, const float *queries, size_t nq, size_t nprobe, uint32_t *out_ids,
                      float *out_scores, size_t *out_len) {
    clear_error();
    if (!C) return set_error(VHIP_ERR_INVALID_CONFIG, "null quantizer");
    std::lock_guard<std::mutex> lock(C->mu);
    return vhip_knn_search_batch(C->probe, queries, nq, nprobe, out_ids, out_scores, out_len);
}

size_t vhip_coarse_nlist(const vhip_coarse *C) { return C ? C->nlist : 0; }
size_t vhip_coarse_dimension(const vhip_coarse *C) { return C ? C->dim : 0; }

void vhip_coarse_destroy(vhip_coarse *C) { delete C; }

}  // extern "C"
