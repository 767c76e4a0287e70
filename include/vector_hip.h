/*
 * vector_hip.h -- C ABI of the MI355X (gfx950) kNN / k-means library.
 *
 * This is the drop-in boundary for the reference's GPU hot path (Malset2603/vector-rs,
 * crate vector-cuda).  Each entry point names the reference interface it replaces.
 * Plain pointers and sizes only; every host pointer is owned by the caller and the
 * library copies what it keeps.  All functions are thread-safe per engine (an engine
 * serialises its own calls on one HIP stream).
 *
 * Status codes mirror CudaError (vector-cuda/src/error.rs:7-29):
 *   VHIP_OK, InsufficientDevices, DeviceNotFound, DriverError, HardwareNotAvailable,
 *   InvalidConfig.  vhip_last_error() returns the calling thread's last message.
 *
 * Semantics kept from the reference (knn.rs:151-169, distributed_knn.rs:155-231):
 *   effective_k = min(k, N); empty queries, k == 0 or N == 0 give empty lists;
 *   results are best first; DotProduct / CosineSimilarity report the similarity and
 *   sort descending; cosine with a zero-norm operand is 0; squared L2 is clamped >= 0.
 * Semantics deliberately changed:
 *   k is not clamped to 128 (knn.cu:218) -- any k <= VHIP_MAX_K is exact;
 *   the Q x N distance matrix is never materialised (knn.rs:195);
 *   k-means at one GPU runs on the GPU (distributed_kmeans.rs:80 never did);
 *   empty clusters keep their centroid (as kmeans.cu:350-356, not a random reseed);
 *   k-means init is explicit or seeded (the reference used an unseeded thread_rng);
 *   there is no silent CPU fallback: a missing GPU is an error, not a slow answer.
 */
#ifndef VECTOR_HIP_H
#define VECTOR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#pragma GCC visibility push(default) /* the library hides everything but this API */
#endif

/* ---- status codes: CudaError (error.rs:7-29) -------------------------------- */
#define VHIP_OK                          0
#define VHIP_ERR_INSUFFICIENT_DEVICES  (-1) /* InsufficientDevices{requested, available} */
#define VHIP_ERR_DEVICE_NOT_FOUND      (-2) /* DeviceNotFound{ordinal} */
#define VHIP_ERR_DRIVER                (-3) /* DriverError(String) */
#define VHIP_ERR_HARDWARE_NOT_AVAILABLE (-4) /* HardwareNotAvailable */
#define VHIP_ERR_INVALID_CONFIG        (-5) /* InvalidConfig(String) */
#define VHIP_ERR_EMPTY_INDEX           (-6) /* vector-index VectorIndexError::EmptyIndex (types.rs) */

/* ---- metric codes: knn.rs:235-246 / kmeans.rs:152-163 ------------------------ */
#define VHIP_METRIC_L2SQUARED    0
#define VHIP_METRIC_DOTPRODUCT   1
#define VHIP_METRIC_COSINE       2
#define VHIP_METRIC_MANHATTAN    3
#define VHIP_METRIC_MINKOWSKI    4 /* p = 3 */
#define VHIP_METRIC_CHEBYSHEV    5
#define VHIP_METRIC_HAMMING      6 /* thresholded float mismatch count, |a-b| > 1e-6 */
#define VHIP_METRIC_MAHALANOBIS  7 /* standardised: sqrt(L2^2) */
#define VHIP_METRIC_JACCARD      8
#define VHIP_METRIC_HELLINGER    9

/* ---- GpuShardMode (distributed_knn.rs:14-19) --------------------------------- */
#define VHIP_SHARD_SHARDED    0
#define VHIP_SHARD_REPLICATED 1

#define VHIP_MAX_K 2048 /* largest k served exactly by one search call */

/* ---- errors ------------------------------------------------------------------- */
/* Message of the calling thread's last failed call ("" if none). */
const char *vhip_last_error(void);
/* requested / available of the last InsufficientDevices error of this thread. */
void vhip_last_error_devices(size_t *requested, size_t *available);
/* The ordinal of the last DeviceNotFound error of this thread (CudaError::DeviceNotFound{ordinal},
 * error.rs:13-14); -1 before any. */
int vhip_last_error_ordinal(void);

/* ---- device context: CudaDeviceContext (device.rs:110-256) ------------------- */
/* CudaDeviceContext::device_count (device.rs:112-117): number of usable gfx950 GPUs. */
int vhip_device_count(void);
/* CudaDeviceContext::with_ordinal_strict (device.rs:127-171): name / total memory of a
 * device, DeviceNotFound when ordinal >= device_count. */
int vhip_device_info(int ordinal, char *name, size_t name_len, size_t *total_memory_bytes);

/* ---- CudaKnnEngine (knn.rs:45-401) ------------------------------------------- */
typedef struct vhip_knn vhip_knn;
/* CudaKnnEngine::with_ordinal (knn.rs:90-140): uploads the row-major n x dim base once
 * and keeps it resident in HBM until vhip_knn_destroy. */
int vhip_knn_create(const float *base, size_t n, size_t dim, int metric, int ordinal, vhip_knn **out);
/* CudaKnnEngine::search_batch (knn.rs:151-169): nq row-major queries, k neighbours.
 * out_ids / out_dist are nq x k (row stride k); out_len[q] = min(k, n) valid entries
 * best first.  Host buffers; the call returns when results are in them. */
int vhip_knn_search_batch(vhip_knn *eng, const float *queries, size_t nq, size_t k, uint32_t *out_ids,
                          float *out_dist, size_t *out_len);
/* Same search with queries and outputs already in device memory of the engine's GPU
 * (no reference counterpart; it serves callers whose queries are produced on the GPU).
 * Returns after the results are written. */
int vhip_knn_search_batch_device(vhip_knn *eng, const float *d_queries, size_t nq, size_t k, uint32_t *d_ids,
                                 float *d_dist);
/* Allocation-free variant of vhip_knn_search_batch_device.  It has no counterpart in the
 * reference.  It is for callers that cannot allocate device memory: code that must not call
 * hipMalloc inside a serving loop, and harnesses that forbid it.  It returns the same results.
 * Its working memory is one fixed array of VHIP_NOALLOC_SCRATCH_BYTES per GPU inside the
 * library, in a code object of its own that a GPU loads at the first allocation-free call on it
 * and holds until the process ends (GPUs and engines that never call it reserve nothing);
 * queries are served in batches that fit it.  It calls no hipMalloc or hipFree.  Error VHIP_ERR_INVALID_CONFIG
 * when a single query at this k and engine size needs more than the array holds (about
 * 8 * max(2048, 32 k) bytes per query plus the row buffers).  Every call on one GPU shares that
 * GPU's array and leaves its contents behind: the library takes a per-GPU lock for the whole
 * call, so calls from several threads run one after another; calls that overlapped on one GPU
 * would race on the array.  Every return, errors included, comes after the call's kernels have
 * finished, so the lock is never released with work on the array still queued.  Returns after
 * the results are written. */
#define VHIP_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int vhip_knn_search_batch_device_noalloc(vhip_knn *eng, const float *d_queries, size_t nq, size_t k,
                                         uint32_t *d_ids, float *d_dist);
size_t vhip_knn_dimension(const vhip_knn *eng);    /* knn.rs:387 */
size_t vhip_knn_num_vectors(const vhip_knn *eng);  /* knn.rs:393 */
int vhip_knn_metric(const vhip_knn *eng);          /* knn.rs:399 */
int vhip_knn_device_id(const vhip_knn *eng);       /* knn.rs:381 context().device_id() */
void vhip_knn_destroy(vhip_knn *eng);              /* Drop of the CudaSlice (knn.rs:50-51) */

/* Kernel timing of the engine's distance kernel (HIP events on its stream).  Enable,
 * run searches, then read the summed kernel time, launch count and the algorithmic
 * flops (2*nq*rows*dim, or pair operations for VALU metrics) and HBM bytes (base
 * rows + queries read once per launch) of those launches. */
int vhip_knn_profile(vhip_knn *eng, int enable);
int vhip_knn_profile_read(vhip_knn *eng, double *kernel_ms, uint64_t *launches, double *work, double *bytes);

/* ---- DistributedKnnEngine (ddp/distributed_knn.rs:24-262) --------------------- */
typedef struct vhip_dknn vhip_dknn;
/* DistributedKnnEngine::try_new (:40-61): InsufficientDevices when num_gpus > device_count. */
int vhip_dknn_try_new(const float *base, size_t n, size_t dim, size_t num_gpus, int mode, int metric,
                      vhip_dknn **out);
/* DistributedKnnEngine::emulator (:64-74): num_gpus ranks without the device-count check.
 * Every rank runs on the one GPU (ordinal 0); sharded ranks hold N/G rows each and are
 * merged with top_k_reduce, so results equal the single-rank ones. */
int vhip_dknn_emulator(const float *base, size_t n, size_t dim, size_t num_gpus, int mode, int metric,
                       vhip_dknn **out);
/* DistributedKnnEngine::search_batch (:155-231); same output contract as vhip_knn_search_batch. */
int vhip_dknn_search_batch(vhip_dknn *eng, const float *queries, size_t nq, size_t k, uint32_t *out_ids,
                           float *out_dist, size_t *out_len);
size_t vhip_dknn_num_gpus(const vhip_dknn *eng);     /* :235 */
int vhip_dknn_mode(const vhip_dknn *eng);            /* :241 */
size_t vhip_dknn_dimension(const vhip_dknn *eng);    /* :247 */
size_t vhip_dknn_num_vectors(const vhip_dknn *eng);  /* :253 */
int vhip_dknn_metric(const vhip_dknn *eng);          /* :259 */
void vhip_dknn_destroy(vhip_dknn *eng);

/* CollectiveOps::top_k_reduce (ddp/collective.rs:115-159), host arrays: merges the
 * concatenated per-rank lists (total entries) into the best k, best first.  Returns
 * the number of results. */
size_t vhip_top_k_reduce(const uint32_t *ids, const float *dist, size_t total, size_t k, int metric,
                         uint32_t *out_ids, float *out_dist);

/* ---- packed-bit Hamming kNN (extension: the reference has only the thresholded float
 * Hamming of scalar.rs:143-153, which equals popcount(a ^ b) on 0/1 codes) ------- */
typedef struct vhip_hamming vhip_hamming;
/* n codes of `words` uint32 each (1..32).  The codes are also held on the device expanded to one
 * fp4 value per bit (4x the packed size) and searched on the fp4 matrix cores, when that copy
 * takes at most half of the free device memory; otherwise the popcount kernel scans the packed
 * codes.  The environment variable VHIP_HAMMING_KERNEL ("popcount" or "fp4") overrides the
 * choice at creation.  Distances are exact either way. */
int vhip_hamming_create(const uint32_t *codes, size_t n, size_t words, int ordinal, vhip_hamming **out);
int vhip_hamming_search_batch(vhip_hamming *eng, const uint32_t *queries, size_t nq, size_t k,
                              uint32_t *out_ids, uint32_t *out_dist, size_t *out_len);
int vhip_hamming_search_batch_device(vhip_hamming *eng, const uint32_t *d_queries, size_t nq, size_t k,
                                     uint32_t *d_ids, uint32_t *d_dist);
int vhip_hamming_profile(vhip_hamming *eng, int enable);
int vhip_hamming_profile_read(vhip_hamming *eng, double *kernel_ms, uint64_t *launches, double *work,
                              double *bytes);
void vhip_hamming_destroy(vhip_hamming *eng);

/* ---- k-means: CudaKMeansEngine (kmeans.rs:37-467) / DistributedKMeansEngine ---- */
/* CudaKMeansResult (kmeans.rs:15-26) without the centroid buffer (written to out_centroids). */
typedef struct {
    size_t dimension;
    size_t k;
    size_t iterations;
    float inertia;
} vhip_kmeans_result;

#define VHIP_INIT_KMEANSPP 0 /* CudaKMeansEngine::init_random (kmeans.rs:409-460), seeded */
#define VHIP_INIT_SHUFFLE  1 /* DistributedKMeansEngine::init_random (distributed_kmeans.rs:524-535), seeded */

/* CudaKMeansEngine::fit (kmeans.rs:58-97) on GPU `ordinal`: Lloyd iterations until
 * max_iters or max centroid shift <= tol (tol < 0 never stops early).  k is clamped to n
 * (effective_k); n == 0 or k == 0 gives k = 0 and writes nothing.  init_centroids
 * (effective_k x dim) gives the starting centroids; NULL seeds them with `init_mode`
 * from `seed`.  out_centroids receives effective_k x dim floats; out_assign (n, may be
 * NULL) the final assignment; inertia is the sum of per-point metric values of the last
 * assignment (kmeans.cu:110-170 conventions: L2^2, -dot, 1-cos). */
int vhip_kmeans_fit(int ordinal, const float *data, size_t n, size_t dim, size_t k, size_t max_iters, float tol,
                    int metric, const float *init_centroids, int init_mode, uint64_t seed, float *out_centroids,
                    int32_t *out_assign, vhip_kmeans_result *result);
/* DistributedKMeansEngine::try_new (distributed_kmeans.rs:28-38): validates num_gpus
 * against the device count (InsufficientDevices). */
int vhip_dkmeans_check(size_t num_gpus);

/* Resident k-means state for per-iteration use (no reference counterpart: it exposes
 * one Lloyd step for parity checks and the per-iteration benchmark).  Every state, also the
 * one vhip_kmeans_fit makes, assigns squared L2, dot product and cosine on the FP32 matrix
 * cores, except small point sets (fewer than 128 points per compute unit, at most 256
 * centroids and 1e6 point-centroid pairs), which take the direct form on the vector units;
 * the environment variable VHIP_KMEANS_ASSIGN=mfma at creation keeps those on the matrix
 * cores.  Both give the reference's assignment. */
typedef struct vhip_kmeans vhip_kmeans;
int vhip_kmeans_create(int ordinal, const float *data, size_t n, size_t dim, int metric, vhip_kmeans **out);
/* The same state from nseg host segments (segment i: counts[i] rows of dim floats) uploaded one
 * after another (no reference counterpart: it serves callers with several shards, such as the
 * trainer over mapped VECRSTOR files, which would otherwise concatenate them on the host). */
int vhip_kmeans_create_segments(int ordinal, const float *const *segments, const size_t *counts, size_t nseg,
                                size_t dim, int metric, vhip_kmeans **out);
/* CudaKMeansEngine::fit (kmeans.rs:58-237) on the points of an existing state; the same
 * arguments and results as vhip_kmeans_fit. */
int vhip_kmeans_fit_state(vhip_kmeans *km, size_t k, size_t max_iters, float tol, const float *init_centroids,
                          int init_mode, uint64_t seed, float *out_centroids, int32_t *out_assign,
                          vhip_kmeans_result *result);
/* Sets the current centroids (k x dim host floats). */
int vhip_kmeans_set_centroids(vhip_kmeans *km, const float *centroids, size_t k);
/* Runs `iters` assign+update iterations on the device without host synchronisation. */
int vhip_kmeans_run(vhip_kmeans *km, size_t iters);
/* Copies out the state after the last iteration: centroids (k x dim), assignment (n),
 * counts (k), per-cluster shift (k), max shift and inertia.  Any pointer may be NULL. */
int vhip_kmeans_read(vhip_kmeans *km, float *centroids, int32_t *assign, int64_t *counts, float *shifts,
                     float *max_shift, float *inertia);
int vhip_kmeans_profile(vhip_kmeans *km, int enable);
int vhip_kmeans_profile_read(vhip_kmeans *km, double *kernel_ms, uint64_t *launches, double *work,
                             double *bytes);
void vhip_kmeans_destroy(vhip_kmeans *km);

/* One assignment step without the centroid update: every point's nearest centroid (as
 * KMeans::find_nearest_centroid, ivf/kmeans.rs:262-309, lowest index on ties), the metric value
 * of that pair in the reference's direct form (squared L2, dot, cosine similarity, ...; NULL to
 * skip) and the residual point - centroid (n x dim, NULL to skip) as IvfPqIndex::build forms it
 * (ivf/mod.rs:119-132).  No reference counterpart as one call: it replaces that serial loop. */
int vhip_kmeans_assign_only(vhip_kmeans *km, int32_t *out_assign, float *out_score, float *out_residual);

/* ---- IVF coarse quantizer: IvfPqIndex build + search front end (ivf/mod.rs:106-133, 270-283) ---- */
typedef struct vhip_coarse vhip_coarse;
/* Holds nlist x dim coarse centroids (KMeans::fit output) on GPU `ordinal`. */
int vhip_coarse_create(const float *centroids, size_t nlist, size_t dim, int metric, int ordinal,
                       vhip_coarse **out);
/* KMeans::find_nearest_centroid (ivf/kmeans.rs:262-309) for n row-major points: cluster index,
 * its metric value (similarity for dot / cosine) and, if out_residual is not NULL, the residual
 * point - centroid (n x dim) of the IVF-PQ build loop (ivf/mod.rs:119-132).  Host buffers. */
int vhip_coarse_assign(vhip_coarse *q, const float *points, size_t n, uint32_t *out_cluster, float *out_score,
                       float *out_residual);
/* KMeans::find_top_centroids (ivf/kmeans.rs:311-356) for nq queries: min(nprobe, nlist)
 * (index, score) pairs per query, best first, ties in ascending index order; same output
 * contract as vhip_knn_search_batch (row stride nprobe). */
int vhip_coarse_probe(vhip_coarse *q, const float *queries, size_t nq, size_t nprobe, uint32_t *out_ids,
                      float *out_scores, size_t *out_len);
size_t vhip_coarse_nlist(const vhip_coarse *q);
size_t vhip_coarse_dimension(const vhip_coarse *q);
void vhip_coarse_destroy(vhip_coarse *q);

/* ---- files of the offline trainer ------------------------------------------------ */
/* MmapStorage::create_from_flat (storage/mmap.rs:128-160): VECRSTOR file (u64 magic
 * 0x5645435253544F52, u64 n, u64 dim, n x dim f32, little-endian). */
int vhip_vecrstor_write(const char *path, const float *data, size_t n, size_t dim);
/* MmapStorage::open (storage/mmap.rs:171-224): validates magic and size, returns n and dim. */
int vhip_vecrstor_open(const char *path, size_t *n, size_t *dim);
/* Copies the n x dim vectors of a VECRSTOR file (n, dim as vhip_vecrstor_open reported). */
int vhip_vecrstor_read(const char *path, float *out, size_t n, size_t dim);
/* MmapStorage::open + as_raw_slice (storage/mmap.rs:171-260) without a copy: the file mapped
 * read-only, *data pointing at its n x dim floats until vhip_vecrstor_unmap.  Every entry point
 * that takes host vectors accepts such a view; their uploads stream it from the page cache. */
typedef struct vhip_vecrstor_view vhip_vecrstor_view;
int vhip_vecrstor_map(const char *path, const float **data, size_t *n, size_t *dim, vhip_vecrstor_view **view);
void vhip_vecrstor_unmap(vhip_vecrstor_view *view);
/* CudaKnnEngine::new over MmapStorage::open(path).as_raw_slice() (knn.rs:85-140): the base is
 * uploaded straight from the mapped file. */
int vhip_knn_create_from_vecrstor(const char *path, int metric, int ordinal, vhip_knn **out);
/* A k-means state over the concatenation of npaths VECRSTOR files (mpi_kmeans.rs:307-325 loads
 * them into one Vec), uploaded from the mapped files one after another. */
int vhip_kmeans_create_from_vecrstor(int ordinal, const char *const *paths, size_t npaths, int metric,
                                     vhip_kmeans **out);
/* IvfPqSerializer::save_centroid_file (ivf/serializer.rs:264-306): VRSKMEAN file (u64 magic
 * 0x5652534B4D45414E, u32 version 1, u8 metric, u32 dim, u32 k, u32 iterations, f32 inertia,
 * k x dim f32, little-endian). */
int vhip_centroid_file_save(const char *path, const float *centroids, size_t dim, size_t k, int metric,
                            size_t iterations, float inertia);
/* IvfPqSerializer::load_centroid_file (ivf/serializer.rs:309-360), header part: validates magic,
 * version and metric code.  Any output pointer may be NULL. */
int vhip_centroid_file_info(const char *path, size_t *dim, size_t *k, int *metric, size_t *iterations,
                            float *inertia);
/* ... and the k x dim centroid data (k, dim as vhip_centroid_file_info reported). */
int vhip_centroid_file_load(const char *path, float *centroids, size_t k, size_t dim);
/* vector-mpi fit_cuda_aware (src/distributed_kmeans.rs:375-415) as mpi_kmeans --use-cuda runs it
 * (src/bin/mpi_kmeans.rs:284-364): loads data_dir/shard_0.bin, shard_1.bin, ... (VECRSTOR,
 * until the first missing index), fits k-means on GPU 0 (seeded k-means++ init) and writes the
 * VRSKMEAN file data_dir/output.  num_gpus is accepted as fit_cuda_aware does (max(1); more GPUs
 * than present fall back to the emulator there, to the one GPU here).  num_shards (may be NULL)
 * receives the number of shard files read. */
int vhip_train_from_shards(const char *data_dir, size_t k, size_t max_iters, float tol, int metric, size_t num_gpus,
                           const char *output, uint64_t seed, vhip_kmeans_result *result, size_t *num_shards);

/* ---- device memory helpers (for callers without a framework) ------------------- */
int vhip_malloc(int ordinal, size_t bytes, void **ptr);
int vhip_free(int ordinal, void *ptr);
int vhip_memcpy_htod(int ordinal, void *dst, const void *src, size_t bytes);
int vhip_memcpy_dtoh(int ordinal, void *dst, const void *src, size_t bytes);
int vhip_memcpy_dtod(int ordinal, void *dst, const void *src, size_t bytes);
int vhip_synchronize(int ordinal);

/* ---- product quantization and the IVF-PQ index (vector-index/src/ivf) ------------- */
/* IvfPqConfig (ivf/config.rs:25-44); max_train_points 0 means None (the build does not read it,
 * like ivf/mod.rs). */
typedef struct {
    size_t nlist;
    size_t nprobe;
    size_t num_subvectors;
    size_t sub_clusters;
    size_t max_kmeans_iters;
    float kmeans_tolerance;
    size_t max_train_points;
} vhip_ivfpq_config;
/* IvfPqConfig::default (config.rs:46-58) */
void vhip_ivfpq_config_default(vhip_ivfpq_config *cfg);
/* IvfPqConfig::validate (config.rs:96-147): InvalidConfig with the reference's reasons. */
int vhip_ivfpq_config_validate(const vhip_ivfpq_config *cfg, size_t dim);

/* ProductQuantizer::train (pq.rs:53-107): one k-means per sub-space on the GPU, codebooks
 * M x Ks x (dim / M) floats, zero rows past min(Ks, n) (pq.rs:84-88).  Initial sub-centroids
 * are a seeded sample without replacement (KMeans::init_centroids_random, ivf/kmeans.rs:359-371,
 * draws from an unseeded thread_rng) or, with init_codebooks != NULL, the given
 * min(Ks, n) x ds rows of each sub-space (at stride Ks rows). */
int vhip_pq_train(int ordinal, const float *data, size_t n, size_t dim, size_t num_subvectors, size_t sub_clusters,
                  size_t max_iters, float tol, int metric, const float *init_codebooks, uint64_t seed,
                  float *out_codebooks);
/* ProductQuantizer::encode_batch (pq.rs:178-214): out_codes n x M bytes. */
int vhip_pq_encode(int ordinal, const float *codebooks, size_t dim, size_t num_subvectors, size_t sub_clusters,
                   int metric, const float *data, size_t n, uint8_t *out_codes);
/* ProductQuantizer::compute_adc_lut (pq.rs:233-266) for nq queries: out_lut nq x M x Ks. */
int vhip_pq_adc_lut(int ordinal, const float *codebooks, size_t dim, size_t num_subvectors, size_t sub_clusters,
                    int metric, const float *queries, size_t nq, float *out_lut);

/* IvfPqIndex (ivf/mod.rs:63-71): coarse centroids, product quantizer and inverted lists resident
 * on one GPU.  Lists are held in CSR order: list c is entries [sum of sizes < c, + size c) of
 * ids / codes (M bytes each). */
typedef struct vhip_ivfpq vhip_ivfpq;
#define VHIP_IVFPQ_MAX_K 1024
typedef struct {
    size_t dimension;
    int metric;
    size_t nlist; /* lists held (coarse centroids actually trained) */
    size_t num_subvectors;
    size_t sub_clusters;
    size_t num_vectors; /* InvertedIndex::total_vectors */
    vhip_ivfpq_config config;
} vhip_ivfpq_desc;
/* IvfPqIndex::build_parallel_with_config (ivf/mod.rs:90-165): validate, coarse k-means (seeded
 * sample init), assignment + residuals, PQ training on the residuals, codes, inverted lists in
 * ascending id order.  EmptyIndex for n == 0. */
int vhip_ivfpq_build(int ordinal, const float *data, size_t n, size_t dim, const vhip_ivfpq_config *cfg, int metric,
                     uint64_t seed, vhip_ivfpq **out);
/* An index from its parts (IvfPqIndex::load_from_file, ivf/mod.rs:388-408, after
 * IvfPqSerializer::load_from_file): list_sizes has nlist entries, ids / codes their sum. */
int vhip_ivfpq_create(int ordinal, size_t dim, int metric, const vhip_ivfpq_config *cfg, const float *coarse,
                      size_t nlist, const float *codebooks, const uint32_t *list_sizes, const uint32_t *ids,
                      const uint8_t *codes, vhip_ivfpq **out);
/* IvfPqIndex::search_with_nprobe (ivf/mod.rs:256-345) for a batch: rows of k results (ids, ADC
 * distance, similarity for dot / cosine), best first, out_len[q] = min(k, entries in the probed
 * lists); unused slots hold UINT32_MAX / NaN.  nprobe is clamped to [1, nlist]; k <= VHIP_IVFPQ_MAX_K. */
int vhip_ivfpq_search_batch(vhip_ivfpq *ix, const float *queries, size_t nq, size_t k, size_t nprobe,
                            uint32_t *out_ids, float *out_dist, size_t *out_len);
/* Same search with queries and outputs in device memory of the index's GPU (no reference
 * counterpart; for callers whose queries live on the GPU).  Returns after the results are written. */
int vhip_ivfpq_search_batch_device(vhip_ivfpq *ix, const float *d_queries, size_t nq, size_t k, size_t nprobe,
                                   uint32_t *d_ids, float *d_dist, uint32_t *d_len);
/* The coarse probe lists the search uses (KMeans::find_top_centroids, ivf/kmeans.rs:311-356),
 * nq x min(max(nprobe, 1), nlist) list indices, best first. */
int vhip_ivfpq_probe(vhip_ivfpq *ix, const float *queries, size_t nq, size_t nprobe, uint32_t *out_lists);
/* Getters (ivf/mod.rs:411-449) and the parts for IvfPqSerializer::save_to_file. */
int vhip_ivfpq_info(const vhip_ivfpq *ix, vhip_ivfpq_desc *info);
int vhip_ivfpq_export(const vhip_ivfpq *ix, float *coarse, float *codebooks, uint32_t *list_sizes, uint32_t *ids,
                      uint8_t *codes);
/* Kernel time of the ADC scan (HIP events on the index's stream). */
int vhip_ivfpq_profile(vhip_ivfpq *ix, int enable);
int vhip_ivfpq_profile_read(vhip_ivfpq *ix, double *kernel_ms, uint64_t *launches);
void vhip_ivfpq_destroy(vhip_ivfpq *ix);
/* IvfPqSerializer::save_to_file (ivf/serializer.rs:26-99): the IVFPQVEC file of an index's
 * parts; list_sizes has nlists entries, ids / codes (num_subvectors bytes each) their sum. */
int vhip_ivfpq_file_save(const char *path, const vhip_ivfpq_config *cfg, size_t dim, int metric, const float *coarse,
                         size_t num_centroids, const float *codebooks, size_t codebooks_len,
                         const uint32_t *list_sizes, size_t nlists, const uint32_t *ids, const uint8_t *codes);
/* IvfPqSerializer::load_from_file (:102-254) in two calls: the header and sizes (InvalidConfig
 * for a bad magic, version, metric code, codebook shape or a truncated file), then the arrays. */
int vhip_ivfpq_file_info(const char *path, vhip_ivfpq_config *cfg, size_t *dim, int *metric, size_t *num_centroids,
                         size_t *codebooks_len, size_t *nlists, size_t *total_vectors);
int vhip_ivfpq_file_load(const char *path, float *coarse, float *codebooks, uint32_t *list_sizes, uint32_t *ids,
                         uint8_t *codes);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif

#endif /* VECTOR_HIP_H */
