// storage.cpp -- the file formats around the k-means trainer, and the trainer itself.
//
//  * VECRSTOR vector files: MmapStorage (vector-index/src/storage/mmap.rs:9-16, 90-224):
//      u64 magic 0x56454352_53544F52 ("VECRSTOR"), u64 n, u64 dim, then n x dim f32, all
//      little-endian.  open() validates the magic and that the file holds the declared data.
//  * VRSKMEAN centroid files: IvfPqSerializer::save/load_centroid_file
//      (vector-index/src/ivf/serializer.rs:264-360, 374-377): u64 magic 0x5652534B_4D45414E,
//      u32 version 1, u8 metric code, u32 dim, u32 k, u32 iterations, f32 inertia, then k x dim
//      f32, little-endian, no padding (29-byte header).
//  * IVFPQVEC index files: IvfPqSerializer::save_to_file / load_from_file
//      (vector-index/src/ivf/serializer.rs:16-254): u64 magic 0x49564650_51564543, u32 version 1,
//      u8 metric, u32 dim, u32 nlist, nprobe, num_subvectors, sub_clusters, max_kmeans_iters,
//      f32 tolerance, u32 centroid count + f32 coarse centroids, u32 codebook length + f32
//      codebooks, u32 list count, then per list u32 count, count x u32 ids, count x M code bytes.
//  * Zero-copy VECRSTOR views (vhip_vecrstor_map): the file mapped read-only, its data handed
//      to the engines' uploads, which stream it from the page cache through their pinned staging
//      buffers: no host copy of the vectors (the reference copies every shard into one Vec,
//      mpi_kmeans.rs:307-325, and CudaKnnEngine copies and transposes the base, knn.rs:111-122).
//  * Offline trainer: vector-mpi fit_cuda_aware (src/distributed_kmeans.rs:375-415) reached from
//      mpi_kmeans --use-cuda (src/bin/mpi_kmeans.rs:284-364): load data_dir/shard_0.bin,
//      shard_1.bin, ... (until the first missing index), fit k-means on the GPU, write the
//      centroid file data_dir/output.
// Host code only: it reads and writes files and calls the GPU k-means through the C ABI.
#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <vector>

#include "vector_hip.h"
#include "vh_error.h"

namespace {

constexpr uint64_t kVecMagic = 0x5645435253544F52ull;
constexpr uint64_t kCentroidMagic = 0x5652534B4D45414Eull;
constexpr uint32_t kCentroidVersion = 1;
constexpr size_t kVecHeader = 24;
constexpr size_t kCentroidHeader = 29;
constexpr uint64_t kIvfPqMagic = 0x4956465051564543ull;
constexpr uint32_t kIvfPqVersion = 1;

struct File {
    FILE *f = nullptr;
    explicit File(FILE *p) : f(p) {}
    ~File() {
        if (f) fclose(f);
    }
};

// Little-endian encode / decode (the formats are LE regardless of the host).
void put_u64(unsigned char *p, uint64_t v) {
    for (int i = 0; i < 8; ++i) p[i] = (unsigned char)(v >> (8 * i));
}
void put_u32(unsigned char *p, uint32_t v) {
    for (int i = 0; i < 4; ++i) p[i] = (unsigned char)(v >> (8 * i));
}
uint64_t get_u64(const unsigned char *p) {
    uint64_t v = 0;
    for (int i = 7; i >= 0; --i) v = (v << 8) | p[i];
    return v;
}
uint32_t get_u32(const unsigned char *p) {
    uint32_t v = 0;
    for (int i = 3; i >= 0; --i) v = (v << 8) | p[i];
    return v;
}
bool host_is_le() {
    const uint32_t one = 1;
    unsigned char b;
    std::memcpy(&b, &one, 1);
    return b == 1;
}

// Writes / reads count floats in little-endian order.
bool write_f32(FILE *f, const float *v, size_t count) {
    if (host_is_le()) return fwrite(v, sizeof(float), count, f) == count;
    unsigned char b[4];
    for (size_t i = 0; i < count; ++i) {
        uint32_t u;
        std::memcpy(&u, &v[i], 4);
        put_u32(b, u);
        if (fwrite(b, 1, 4, f) != 4) return false;
    }
    return true;
}
bool read_f32(FILE *f, float *v, size_t count) {
    if (fread(v, sizeof(float), count, f) != count) return false;
    if (!host_is_le()) {
        for (size_t i = 0; i < count; ++i) {
            unsigned char b[4];
            std::memcpy(b, &v[i], 4);
            const uint32_t u = get_u32(b);
            std::memcpy(&v[i], &u, 4);
        }
    }
    return true;
}

int io_error(const std::string &what, const char *path) {
    return vh::set_error(VHIP_ERR_INVALID_CONFIG, what + " '" + path + "': " + std::strerror(errno));
}

long long file_size(const char *path) {
    struct stat st;
    if (stat(path, &st) != 0) return -1;
    return (long long)st.st_size;
}

// MmapStorage::open validation (mmap.rs:171-224).
int vec_header(const char *path, size_t *n, size_t *dim) {
    const long long size = file_size(path);
    if (size < 0) return io_error("cannot open vector file", path);
    if (size < (long long)kVecHeader)
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, std::string("invalid header in '") + path +
                                                          "': file too small: " + std::to_string(size) +
                                                          " bytes (minimum 24)");
    File f(fopen(path, "rb"));
    if (!f.f) return io_error("cannot open vector file", path);
    unsigned char h[kVecHeader];
    if (fread(h, 1, kVecHeader, f.f) != kVecHeader) return io_error("cannot read vector file header", path);
    const uint64_t magic = get_u64(h);
    if (magic != kVecMagic) {
        char msg[160];
        snprintf(msg, sizeof msg, "invalid magic number: 0x%016llX (expected 0x%016llX)", (unsigned long long)magic,
                 (unsigned long long)kVecMagic);
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, std::string("invalid header in '") + path + "': " + msg);
    }
    const uint64_t nv = get_u64(h + 8), d = get_u64(h + 16);
    if (d != 0 && nv > (uint64_t)(size) / 4 / d + 1)
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, std::string("file size mismatch in '") + path + "'");
    const unsigned long long need = kVecHeader + (unsigned long long)nv * d * 4ull;
    if ((unsigned long long)size < need)
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, std::string("file size mismatch in '") + path +
                                                          "': expected " + std::to_string(need) + " bytes, got " +
                                                          std::to_string(size));
    *n = (size_t)nv;
    *dim = (size_t)d;
    return VHIP_OK;
}

int centroid_header(FILE *f, const char *path, size_t *dim, size_t *k, int *metric, size_t *iters, float *inertia) {
    unsigned char h[kCentroidHeader];
    if (fread(h, 1, kCentroidHeader, f) != kCentroidHeader)
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, std::string("truncated centroid file '") + path + "'");
    const uint64_t magic = get_u64(h);
    if (magic != kCentroidMagic) {
        char msg[160];
        snprintf(msg, sizeof msg, "expected centroid magic 0x%llX, got 0x%llX", (unsigned long long)kCentroidMagic,
                 (unsigned long long)magic);
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, std::string("invalid header in '") + path + "': " + msg);
    }
    const uint32_t version = get_u32(h + 8);
    if (version != kCentroidVersion)
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, std::string("invalid header in '") + path +
                                                          "': unsupported centroid file version: " +
                                                          std::to_string(version));
    const unsigned code = h[12];
    if (code > 9)
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, std::string("invalid header in '") + path +
                                                          "': unknown metric code " + std::to_string(code));
    uint32_t ib = get_u32(h + 25);
    float in;
    std::memcpy(&in, &ib, 4);
    if (dim) *dim = get_u32(h + 13);
    if (k) *k = get_u32(h + 17);
    if (metric) *metric = (int)code;
    if (iters) *iters = get_u32(h + 21);
    if (inertia) *inertia = in;
    return VHIP_OK;
}

}  // namespace

extern "C" {

int vhip_vecrstor_write(const char *path, const float *data, size_t n, size_t dim) {
    vh::clear_error();
    if (!path || (n * dim > 0 && !data)) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "null path or data");
    File f(fopen(path, "wb"));
    if (!f.f) return io_error("cannot create vector file", path);
    unsigned char h[kVecHeader];
    put_u64(h, kVecMagic);
    put_u64(h + 8, (uint64_t)n);
    put_u64(h + 16, (uint64_t)dim);
    if (fwrite(h, 1, kVecHeader, f.f) != kVecHeader || !write_f32(f.f, data, n * dim))
        return io_error("cannot write vector file", path);
    if (fflush(f.f) != 0) return io_error("cannot write vector file", path);
    return VHIP_OK;
}

int vhip_vecrstor_open(const char *path, size_t *n, size_t *dim) {
    vh::clear_error();
    if (!path || !n || !dim) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    return vec_header(path, n, dim);
}

int vhip_vecrstor_read(const char *path, float *out, size_t n, size_t dim) {
    vh::clear_error();
    if (!path || (n * dim > 0 && !out)) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    size_t fn = 0, fd = 0;
    const int rc = vec_header(path, &fn, &fd);
    if (rc != VHIP_OK) return rc;
    if (fn != n || fd != dim)
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, std::string("'") + path + "' holds " + std::to_string(fn) +
                                                          " x " + std::to_string(fd) + " vectors, not " +
                                                          std::to_string(n) + " x " + std::to_string(dim));
    File f(fopen(path, "rb"));
    if (!f.f) return io_error("cannot open vector file", path);
    if (fseek(f.f, (long)kVecHeader, SEEK_SET) != 0 || !read_f32(f.f, out, n * dim))
        return io_error("cannot read vector file", path);
    return VHIP_OK;
}

int vhip_centroid_file_save(const char *path, const float *centroids, size_t dim, size_t k, int metric,
                            size_t iterations, float inertia) {
    vh::clear_error();
    if (!path || (k * dim > 0 && !centroids)) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    if (metric < 0 || metric > 9) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "unknown metric code");
    if (dim > 0xffffffffull || k > 0xffffffffull || iterations > 0xffffffffull)
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, "dimension, k and iterations are stored as u32");
    File f(fopen(path, "wb"));
    if (!f.f) return io_error("cannot create centroid file", path);
    unsigned char h[kCentroidHeader];
    put_u64(h, kCentroidMagic);
    put_u32(h + 8, kCentroidVersion);
    h[12] = (unsigned char)metric;
    put_u32(h + 13, (uint32_t)dim);
    put_u32(h + 17, (uint32_t)k);
    put_u32(h + 21, (uint32_t)iterations);
    uint32_t ib;
    std::memcpy(&ib, &inertia, 4);
    put_u32(h + 25, ib);
    if (fwrite(h, 1, kCentroidHeader, f.f) != kCentroidHeader || !write_f32(f.f, centroids, k * dim))
        return io_error("cannot write centroid file", path);
    if (fflush(f.f) != 0) return io_error("cannot write centroid file", path);
    return VHIP_OK;
}

int vhip_centroid_file_info(const char *path, size_t *dim, size_t *k, int *metric, size_t *iterations,
                            float *inertia) {
    vh::clear_error();
    if (!path) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "null path");
    File f(fopen(path, "rb"));
    if (!f.f) return io_error("cannot open centroid file", path);
    return centroid_header(f.f, path, dim, k, metric, iterations, inertia);
}

int vhip_centroid_file_load(const char *path, float *centroids, size_t k, size_t dim) {
    vh::clear_error();
    if (!path || (k * dim > 0 && !centroids)) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    File f(fopen(path, "rb"));
    if (!f.f) return io_error("cannot open centroid file", path);
    size_t fd = 0, fk = 0;
    const int rc = centroid_header(f.f, path, &fd, &fk, nullptr, nullptr, nullptr);
    if (rc != VHIP_OK) return rc;
    if (fd != dim || fk != k)
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, std::string("'") + path + "' holds " + std::to_string(fk) +
                                                          " x " + std::to_string(fd) + " centroids, not " +
                                                          std::to_string(k) + " x " + std::to_string(dim));
    if (!read_f32(f.f, centroids, k * dim))
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, std::string("truncated centroid file '") + path + "'");
    return VHIP_OK;
}

namespace {

bool write_u32(FILE *f, uint32_t v) {
    unsigned char b[4];
    put_u32(b, v);
    return fwrite(b, 1, 4, f) == 4;
}
bool read_u32(FILE *f, uint32_t *v) {
    unsigned char b[4];
    if (fread(b, 1, 4, f) != 4) return false;
    *v = get_u32(b);
    return true;
}

struct IvfPqHead {
    vhip_ivfpq_config cfg{};
    size_t dim = 0, num_centroids = 0, codebooks_len = 0, nlists = 0, total = 0;
    int metric = 0;
};

// Parses an IVFPQVEC file (serializer.rs:102-254).  Arrays that are null are skipped; with all
// of them null the call only fills `h` (sizes included, so callers can allocate).
int ivfpq_read(const char *path, IvfPqHead *h, float *coarse, float *codebooks, uint32_t *sizes, uint32_t *ids,
               uint8_t *codes) {
    File f(fopen(path, "rb"));
    if (!f.f) return io_error("cannot open IVF-PQ index file", path);
    auto truncated = [&] {
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, std::string("truncated IVF-PQ index file '") + path + "'");
    };
    auto bad = [&](const std::string &why) {
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, std::string("invalid header in '") + path + "': " + why);
    };
    unsigned char b8[8];
    if (fread(b8, 1, 8, f.f) != 8) return truncated();
    const uint64_t magic = get_u64(b8);
    if (magic != kIvfPqMagic) {
        char msg[96];
        snprintf(msg, sizeof msg, "expected magic %#llX, got %#llX", (unsigned long long)kIvfPqMagic,
                 (unsigned long long)magic);
        return bad(msg);
    }
    uint32_t v = 0;
    if (!read_u32(f.f, &v)) return truncated();
    if (v != kIvfPqVersion) return bad("unsupported version: " + std::to_string(v));
    unsigned char mc;
    if (fread(&mc, 1, 1, f.f) != 1) return truncated();
    if (mc > 9) return bad("invalid metric code: " + std::to_string(mc));
    h->metric = mc;
    uint32_t u[6];
    for (int j = 0; j < 6; ++j)
        if (!read_u32(f.f, &u[j])) return truncated();
    h->dim = u[0];
    h->cfg.nlist = u[1];
    h->cfg.nprobe = u[2];
    h->cfg.num_subvectors = u[3];
    h->cfg.sub_clusters = u[4];
    h->cfg.max_kmeans_iters = u[5];
    if (!read_f32(f.f, &h->cfg.kmeans_tolerance, 1)) return truncated();
    h->cfg.max_train_points = 0;
    const size_t m_sub = h->cfg.num_subvectors;
    if (!read_u32(f.f, &v)) return truncated();
    h->num_centroids = v;
    if (coarse) {
        if (!read_f32(f.f, coarse, h->num_centroids * h->dim)) return truncated();
    } else if (fseek(f.f, (long)(h->num_centroids * h->dim * 4), SEEK_CUR) != 0) {
        return truncated();
    }
    if (!read_u32(f.f, &v)) return truncated();
    h->codebooks_len = v;
    // ProductQuantizer::new (pq.rs:30-50) asserts these; here they are errors
    if (m_sub == 0 || h->dim % m_sub != 0)
        return bad("dimension " + std::to_string(h->dim) + " is not divisible by num_subvectors " +
                   std::to_string(m_sub));
    if (h->codebooks_len != m_sub * h->cfg.sub_clusters * (h->dim / m_sub))
        return bad("codebook length " + std::to_string(h->codebooks_len) + " is not num_subvectors x sub_clusters x " +
                   "sub_dimension");
    if (codebooks) {
        if (!read_f32(f.f, codebooks, h->codebooks_len)) return truncated();
    } else if (fseek(f.f, (long)(h->codebooks_len * 4), SEEK_CUR) != 0) {
        return truncated();
    }
    if (!read_u32(f.f, &v)) return truncated();
    h->nlists = v;
    size_t total = 0;
    for (size_t c = 0; c < h->nlists; ++c) {
        uint32_t cnt = 0;
        if (!read_u32(f.f, &cnt)) return truncated();
        if (sizes) sizes[c] = cnt;
        if (ids) {
            for (uint32_t j = 0; j < cnt; ++j)
                if (!read_u32(f.f, &ids[total + j])) return truncated();
        } else if (fseek(f.f, (long)cnt * 4, SEEK_CUR) != 0) {
            return truncated();
        }
        const size_t nb = (size_t)cnt * m_sub;
        if (codes) {
            if (fread(codes + total * m_sub, 1, nb, f.f) != nb) return truncated();
        } else if (fseek(f.f, (long)nb, SEEK_CUR) != 0) {
            return truncated();
        }
        total += cnt;
    }
    // fseek past the end succeeds: confirm that the last list really is in the file
    const long pos = ftell(f.f);
    if (pos < 0 || file_size(path) < pos) return truncated();
    h->total = total;
    return VHIP_OK;
}

}  // namespace

int vhip_ivfpq_file_save(const char *path, const vhip_ivfpq_config *cfg, size_t dim, int metric, const float *coarse,
                         size_t num_centroids, const float *codebooks, size_t codebooks_len,
                         const uint32_t *list_sizes, size_t nlists, const uint32_t *ids, const uint8_t *codes) {
    vh::clear_error();
    if (!path || !cfg) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    if (metric < 0 || metric > 9) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "unknown metric code");
    size_t total = 0;
    for (size_t c = 0; c < nlists; ++c) total += list_sizes ? list_sizes[c] : 0;
    if ((num_centroids * dim != 0 && !coarse) || (codebooks_len && !codebooks) || (nlists && !list_sizes) ||
        (total && (!ids || !codes)))
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    const size_t u32s[] = {dim, cfg->nlist, cfg->nprobe, cfg->num_subvectors, cfg->sub_clusters,
                           cfg->max_kmeans_iters, num_centroids, codebooks_len, nlists};
    for (size_t x : u32s)
        if (x > 0xffffffffull) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "a stored size exceeds u32");
    File f(fopen(path, "wb"));
    if (!f.f) return io_error("cannot create IVF-PQ index file", path);
    unsigned char b8[8];
    put_u64(b8, kIvfPqMagic);
    const unsigned char mc = (unsigned char)metric;
    bool ok = fwrite(b8, 1, 8, f.f) == 8 && write_u32(f.f, kIvfPqVersion) && fwrite(&mc, 1, 1, f.f) == 1 &&
              write_u32(f.f, (uint32_t)dim) && write_u32(f.f, (uint32_t)cfg->nlist) &&
              write_u32(f.f, (uint32_t)cfg->nprobe) && write_u32(f.f, (uint32_t)cfg->num_subvectors) &&
              write_u32(f.f, (uint32_t)cfg->sub_clusters) && write_u32(f.f, (uint32_t)cfg->max_kmeans_iters) &&
              write_f32(f.f, &cfg->kmeans_tolerance, 1) && write_u32(f.f, (uint32_t)num_centroids) &&
              write_f32(f.f, coarse, num_centroids * dim) && write_u32(f.f, (uint32_t)codebooks_len) &&
              write_f32(f.f, codebooks, codebooks_len) && write_u32(f.f, (uint32_t)nlists);
    size_t off = 0;
    for (size_t c = 0; ok && c < nlists; ++c) {
        const uint32_t cnt = list_sizes[c];
        ok = write_u32(f.f, cnt);
        for (uint32_t j = 0; ok && j < cnt; ++j) ok = write_u32(f.f, ids[off + j]);
        const size_t nb = (size_t)cnt * cfg->num_subvectors;
        ok = ok && fwrite(codes + off * cfg->num_subvectors, 1, nb, f.f) == nb;
        off += cnt;
    }
    if (!ok || fflush(f.f) != 0) return io_error("cannot write IVF-PQ index file", path);
    return VHIP_OK;
}

int vhip_ivfpq_file_info(const char *path, vhip_ivfpq_config *cfg, size_t *dim, int *metric, size_t *num_centroids,
                         size_t *codebooks_len, size_t *nlists, size_t *total_vectors) {
    vh::clear_error();
    if (!path) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "null path");
    IvfPqHead h;
    const int rc = ivfpq_read(path, &h, nullptr, nullptr, nullptr, nullptr, nullptr);
    if (rc != VHIP_OK) return rc;
    if (cfg) *cfg = h.cfg;
    if (dim) *dim = h.dim;
    if (metric) *metric = h.metric;
    if (num_centroids) *num_centroids = h.num_centroids;
    if (codebooks_len) *codebooks_len = h.codebooks_len;
    if (nlists) *nlists = h.nlists;
    if (total_vectors) *total_vectors = h.total;
    return VHIP_OK;
}

int vhip_ivfpq_file_load(const char *path, float *coarse, float *codebooks, uint32_t *list_sizes, uint32_t *ids,
                         uint8_t *codes) {
    vh::clear_error();
    if (!path || !coarse || !codebooks || !list_sizes || !ids || !codes)
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    IvfPqHead h;
    return ivfpq_read(path, &h, coarse, codebooks, list_sizes, ids, codes);
}

struct vhip_vecrstor_view {
    void *base = nullptr;
    size_t bytes = 0;
    size_t n = 0, dim = 0;
    ~vhip_vecrstor_view() {
        if (base) munmap(base, bytes);
    }
};

int vhip_vecrstor_map(const char *path, const float **data, size_t *n, size_t *dim, vhip_vecrstor_view **view) {
    vh::clear_error();
    if (!path || !data || !n || !dim || !view) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    *view = nullptr;
    *data = nullptr;
    size_t fn = 0, fd = 0;
    const int rc = vec_header(path, &fn, &fd);
    if (rc != VHIP_OK) return rc;
    std::unique_ptr<vhip_vecrstor_view> v(new vhip_vecrstor_view());
    v->n = fn;
    v->dim = fd;
    v->bytes = kVecHeader + fn * fd * sizeof(float);
    const int fdesc = open(path, O_RDONLY);
    if (fdesc < 0) return io_error("cannot open vector file", path);
    void *m = mmap(nullptr, v->bytes, PROT_READ, MAP_PRIVATE, fdesc, 0);
    close(fdesc);
    if (m == MAP_FAILED) return io_error("cannot map vector file", path);
    v->base = m;
    (void)madvise(m, v->bytes, MADV_SEQUENTIAL);
    // the format is little-endian; a big-endian host would need a converting read instead
    if (!host_is_le()) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "mapped VECRSTOR views need a little-endian host");
    *data = reinterpret_cast<const float *>(static_cast<const unsigned char *>(m) + kVecHeader);
    *n = fn;
    *dim = fd;
    *view = v.release();
    return VHIP_OK;
}

void vhip_vecrstor_unmap(vhip_vecrstor_view *view) { delete view; }

int vhip_knn_create_from_vecrstor(const char *path, int metric, int ordinal, vhip_knn **out) {
    vh::clear_error();
    if (!out) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "out is null");
    *out = nullptr;
    const float *data = nullptr;
    size_t n = 0, dim = 0;
    vhip_vecrstor_view *v = nullptr;
    int rc = vhip_vecrstor_map(path, &data, &n, &dim, &v);
    if (rc != VHIP_OK) return rc;
    std::unique_ptr<vhip_vecrstor_view> hold(v);
    return vhip_knn_create(data, n, dim, metric, ordinal, out);
}

int vhip_kmeans_create_from_vecrstor(int ordinal, const char *const *paths, size_t npaths, int metric,
                                     vhip_kmeans **out) {
    vh::clear_error();
    if (!out || (npaths && !paths)) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    *out = nullptr;
    std::vector<std::unique_ptr<vhip_vecrstor_view>> views;
    std::vector<const float *> segs;
    std::vector<size_t> counts;
    size_t dim = 0;
    for (size_t i = 0; i < npaths; ++i) {
        const float *data = nullptr;
        size_t n = 0, d = 0;
        vhip_vecrstor_view *v = nullptr;
        const int rc = vhip_vecrstor_map(paths[i], &data, &n, &d, &v);
        if (rc != VHIP_OK) return rc;
        views.emplace_back(v);
        if (i == 0) dim = d;
        else if (d != dim) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "dimension mismatch across shard files");
        segs.push_back(data);
        counts.push_back(n);
    }
    return vhip_kmeans_create_segments(ordinal, segs.data(), counts.data(), segs.size(), dim, metric, out);
}

int vhip_train_from_shards(const char *data_dir, size_t k, size_t max_iters, float tol, int metric, size_t num_gpus,
                           const char *output, uint64_t seed, vhip_kmeans_result *result, size_t *num_shards) {
    vh::clear_error();
    if (!data_dir || !output || !result) return vh::set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    *result = vhip_kmeans_result{0, 0, 0, 0.0f};
    if (num_shards) *num_shards = 0;
    // fit_cuda_aware takes num_gpus.max(1) and, when more GPUs are requested than exist, runs
    // the DDP engine's emulator (distributed_kmeans.rs:385-392); here one GPU runs every request.
    (void)num_gpus;
    std::vector<std::string> shards;
    for (size_t i = 0;; ++i) {
        std::string p = std::string(data_dir) + "/shard_" + std::to_string(i) + ".bin";
        if (file_size(p.c_str()) < 0) break;
        shards.push_back(p);
    }
    if (shards.empty())
        return vh::set_error(VHIP_ERR_INVALID_CONFIG, std::string("no shard files (shard_0.bin, shard_1.bin, ...) "
                                                                  "found in ") + data_dir);
    // shards are mapped and uploaded one after another: no concatenated host copy
    std::vector<const char *> paths;
    for (const std::string &p : shards) paths.push_back(p.c_str());
    vhip_kmeans *K = nullptr;
    int rc = vhip_kmeans_create_from_vecrstor(0, paths.data(), paths.size(), metric, &K);
    if (rc != VHIP_OK) return rc;
    std::unique_ptr<vhip_kmeans, void (*)(vhip_kmeans *)> hold(K, vhip_kmeans_destroy);
    size_t dim = 0, n = 0;
    for (const std::string &p : shards) {
        size_t sn = 0;
        (void)vhip_vecrstor_open(p.c_str(), &sn, &dim);
        n += sn;
    }
    std::vector<float> cent(std::min(k, n) * dim);
    rc = vhip_kmeans_fit_state(K, k, max_iters, tol, nullptr, VHIP_INIT_KMEANSPP, seed, cent.data(), nullptr, result);
    if (rc != VHIP_OK) return rc;
    const std::string out = std::string(data_dir) + "/" + output;
    rc = vhip_centroid_file_save(out.c_str(), cent.data(), result->dimension, result->k, metric, result->iterations,
                                 result->inertia);
    if (rc != VHIP_OK) return rc;
    if (num_shards) *num_shards = shards.size();
    return VHIP_OK;
}

}  // extern "C"
