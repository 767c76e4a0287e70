// runtime.hip -- error state, device context, staging, timing, memory helpers and the
// host-side top_k_reduce of the C ABI.
#include <algorithm>
#include <cmath>
#include <condition_variable>
#include <mutex>
#include <thread>

#include "vh_runtime.h"

namespace vh {

namespace {
thread_local std::string t_err;
thread_local size_t t_req = 0, t_avail = 0;
thread_local int t_ordinal = -1;
}  // namespace

int set_error(int code, const std::string &msg) {
    t_err = msg;
    return code;
}
void set_insufficient(size_t requested, size_t available) {
    t_req = requested;
    t_avail = available;
    t_err = "Insufficient hardware GPUs: requested " + std::to_string(requested) + " device(s), but only " +
            std::to_string(available) + " physical GPU(s) found";
}
int set_device_not_found(int ordinal, const std::string &msg) {
    t_ordinal = ordinal;
    t_err = msg;
    return VHIP_ERR_DEVICE_NOT_FOUND;
}
void clear_error() { t_err.clear(); }

int device_count() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    int c = 0;
    for (int i = 0; i < n; ++i) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, i) == hipSuccess && std::strncmp(p.gcnArchName, "gfx950", 6) == 0) ++c;
    }
    return c;
}

int open_device(int ordinal) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
        (void)hipGetLastError();
        return set_error(VHIP_ERR_HARDWARE_NOT_AVAILABLE, "No HIP-capable GPU hardware devices found on this system");
    }
    if (ordinal < 0 || ordinal >= n) {
        return set_device_not_found(ordinal, "HIP device with ordinal " + std::to_string(ordinal) + " was not found");
    }
    hipDeviceProp_t p;
    VH_HIP(hipGetDeviceProperties(&p, ordinal));
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0) {
        return set_device_not_found(ordinal, "HIP device " + std::to_string(ordinal) + " is " +
                                                       p.gcnArchName + ", this library is built for gfx950");
    }
    VH_HIP(hipSetDevice(ordinal));
    return VHIP_OK;
}

int device_grid_cap(int ordinal) {
    int cus = 256;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ordinal) != hipSuccess) {
        (void)hipGetLastError();
        cus = 256;
    }
    return 2 * cus;
}

// ---- pinned staging ---------------------------------------------------------------------
namespace {
// Host copy into a pinned block, split over a few threads for large blocks: a single thread
// copying from pageable (or freshly mapped, page-cache backed) memory reaches only a fraction of
// what the PCIe DMA drains.  The helper threads are started once per process and kept (spawning
// them per 32 MiB block cost more than the copy gained); one copy runs at a time, the caller
// taking the first part itself.
class CopyPool {
public:
    static CopyPool &get() {
        static CopyPool *p = new CopyPool();  // never destroyed: its threads block until exit
        return *p;
    }
    void copy(void *dst, const void *src, size_t bytes) {
        constexpr size_t kPart = 4u << 20;
        const unsigned nt = (unsigned)std::min<size_t>(helpers_ + 1, (bytes + kPart - 1) / kPart);
        if (nt <= 1) {
            std::memcpy(dst, src, bytes);
            return;
        }
        std::lock_guard<std::mutex> one(job_mu_);
        const size_t per = (bytes + nt - 1) / nt;
        {
            std::lock_guard<std::mutex> g(mu_);
            dst_ = (char *)dst;
            src_ = (const char *)src;
            bytes_ = bytes;
            per_ = per;
            next_ = 1;
            parts_ = nt;
            left_ = nt - 1;
            ++gen_;
        }
        cv_.notify_all();
        std::memcpy(dst, src, std::min(per, bytes));
        std::unique_lock<std::mutex> g(mu_);
        done_cv_.wait(g, [&] { return left_ == 0; });
    }

private:
    CopyPool() {
        const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
        helpers_ = std::min(7u, hw - 1);
        for (unsigned t = 0; t < helpers_; ++t) std::thread([this] { run(); }).detach();
    }
    void run() {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> g(mu_);
        for (;;) {
            cv_.wait(g, [&] { return gen_ != seen && next_ < parts_; });
            seen = gen_;
            while (next_ < parts_) {
                const size_t o = (size_t)next_++ * per_;
                char *d = dst_;
                const char *s = src_;
                const size_t n = o < bytes_ ? std::min(per_, bytes_ - o) : 0;
                g.unlock();
                if (n) std::memcpy(d + o, s + o, n);
                g.lock();
                if (--left_ == 0) done_cv_.notify_all();
            }
        }
    }
    unsigned helpers_ = 0;
    std::mutex job_mu_, mu_;
    std::condition_variable cv_, done_cv_;
    char *dst_ = nullptr;
    const char *src_ = nullptr;
    size_t bytes_ = 0, per_ = 0;
    unsigned next_ = 0, parts_ = 0, left_ = 0;
    uint64_t gen_ = 0;
};

void staged_copy(void *dst, const void *src, size_t bytes) { CopyPool::get().copy(dst, src, bytes); }
}  // namespace

PinnedStager::~PinnedStager() {
    if (dev >= 0) (void)hipSetDevice(dev);
    for (int i = 0; i < 2; ++i) {
        if (ev[i]) (void)hipEventDestroy(ev[i]);
        if (buf[i]) (void)hipHostFree(buf[i]);
    }
}

int PinnedStager::init(int device) {
    if (buf[0]) return VHIP_OK;
    dev = device;
    for (int i = 0; i < 2; ++i) {
        VH_HIP(hipHostMalloc(&buf[i], kBlock, hipHostMallocDefault));
        VH_HIP(hipEventCreateWithFlags(&ev[i], hipEventDisableTiming));
    }
    return VHIP_OK;
}

int PinnedStager::h2d(void *dst, const void *src, size_t bytes, hipStream_t s) {
    VH_CHECK(init(dev < 0 ? 0 : dev));
    size_t off = 0;
    int i = 0;
    bool pending[2] = {false, false};
    while (off < bytes) {
        const size_t b = std::min(kBlock, bytes - off);
        if (pending[i]) VH_HIP(hipEventSynchronize(ev[i]));
        staged_copy(buf[i], (const char *)src + off, b);
        VH_HIP(hipMemcpyAsync((char *)dst + off, buf[i], b, hipMemcpyHostToDevice, s));
        VH_HIP(hipEventRecord(ev[i], s));
        pending[i] = true;
        off += b;
        i ^= 1;
    }
    VH_HIP(hipStreamSynchronize(s));
    return VHIP_OK;
}

int PinnedStager::d2h(void *dst, const void *src, size_t bytes, hipStream_t s) {
    VH_CHECK(init(dev < 0 ? 0 : dev));
    size_t off = 0;
    while (off < bytes) {
        const size_t b = std::min(kBlock, bytes - off);
        VH_HIP(hipMemcpyAsync(buf[0], (const char *)src + off, b, hipMemcpyDeviceToHost, s));
        VH_HIP(hipStreamSynchronize(s));
        std::memcpy((char *)dst + off, buf[0], b);
        off += b;
    }
    return VHIP_OK;
}

int PinnedStager::d2h_pair(void *dst0, const void *src0, size_t b0, void *dst1, const void *src1, size_t b1,
                           hipStream_t s) {
    if (b0 > kBlock || b1 > kBlock) {
        VH_CHECK(d2h(dst0, src0, b0, s));
        return d2h(dst1, src1, b1, s);
    }
    VH_CHECK(init(dev < 0 ? 0 : dev));
    VH_HIP(hipMemcpyAsync(buf[0], src0, b0, hipMemcpyDeviceToHost, s));
    VH_HIP(hipMemcpyAsync(buf[1], src1, b1, hipMemcpyDeviceToHost, s));
    VH_HIP(hipStreamSynchronize(s));
    std::memcpy(dst0, buf[0], b0);
    std::memcpy(dst1, buf[1], b1);
    return VHIP_OK;
}

// ---- kernel timer -------------------------------------------------------------------------
KernelTimer::~KernelTimer() {
    for (auto &p : pool) {
        (void)hipEventDestroy(p.first);
        (void)hipEventDestroy(p.second);
    }
}

TimedLaunch &timed_launch_slot() {
    thread_local TimedLaunch t;
    return t;
}

// The pair goes to the region's scan launches (scan_launch), which record it on their own
// dispatches; a region that launched none records it here, empty.
int KernelTimer::begin(hipStream_t) {
    if (!enabled) return -1;
    if (used == pool.size()) {
        hipEvent_t a, b;
        if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) {
            (void)hipGetLastError();
            return -1;
        }
        pool.emplace_back(a, b);
    }
    const int idx = (int)used++;
    TimedLaunch &t = timed_launch_slot();
    t.start = pool[idx].first;
    t.stop = pool[idx].second;
    t.used = false;
    return idx;
}

void KernelTimer::end(int idx, hipStream_t s, double w, double b) {
    if (idx < 0) return;
    TimedLaunch &t = timed_launch_slot();
    if (!t.used) {
        (void)hipEventRecord(pool[idx].first, s);
        (void)hipEventRecord(pool[idx].second, s);
    }
    t = TimedLaunch{};
    if ((size_t)idx >= meta.size()) meta.resize(idx + 1);
    meta[idx] = {w, b};
}

void KernelTimer::collect() {
    for (size_t i = 0; i < used; ++i) {
        float t = 0.0f;
        if (hipEventElapsedTime(&t, pool[i].first, pool[i].second) == hipSuccess) {
            ms += t;
            ++launches;
            if (i < meta.size()) {
                work += meta[i].first;
                bytes += meta[i].second;
            }
        } else {
            (void)hipGetLastError();
        }
    }
    used = 0;
}

// ---- permutation ---------------------------------------------------------------------------
uint64_t splitmix64(uint64_t &state) {
    uint64_t z = (state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

std::vector<uint32_t> row_permutation(size_t n, uint64_t seed) {
    std::vector<uint32_t> p(n);
    for (size_t i = 0; i < n; ++i) p[i] = (uint32_t)i;
    uint64_t st = seed;
    for (size_t i = n; i > 1; --i) {
        const size_t j = (size_t)(splitmix64(st) % i);
        std::swap(p[i - 1], p[j]);
    }
    return p;
}

// ---- CollectiveOps::top_k_reduce restated with std BinaryHeap rules ------------------------
namespace {
struct HeapCand {
    float score, dist;
    uint32_t id;
};
inline bool le(float a, float b) { return !(a > b); }
void sift_up(std::vector<HeapCand> &h, size_t start, size_t pos) {
    HeapCand e = h[pos];
    while (pos > start) {
        const size_t parent = (pos - 1) / 2;
        if (le(e.score, h[parent].score)) break;
        h[pos] = h[parent];
        pos = parent;
    }
    h[pos] = e;
}
HeapCand heap_pop(std::vector<HeapCand> &h) {
    HeapCand item = h.back();
    h.pop_back();
    if (!h.empty()) {
        std::swap(item, h[0]);
        const size_t end = h.size();
        size_t pos = 0;
        HeapCand e = h[0];
        size_t child = 1;
        while (end >= 2 && child <= end - 2) {
            child += le(h[child].score, h[child + 1].score) ? 1 : 0;
            h[pos] = h[child];
            pos = child;
            child = 2 * pos + 1;
        }
        if (child == end - 1) {
            h[pos] = h[child];
            pos = child;
        }
        h[pos] = e;
        sift_up(h, 0, pos);
    }
    return item;
}
}  // namespace

size_t top_k_reduce_host(const uint32_t *ids, const float *dist, size_t total, size_t k, bool hib,
                         uint32_t *out_ids, float *out_dist) {
    if (k == 0 || total == 0) return 0;
    std::vector<HeapCand> h;
    h.reserve(k + 1);
    for (size_t i = 0; i < total; ++i) {
        HeapCand c{hib ? -dist[i] : dist[i], dist[i], ids[i]};
        if (h.size() < k) {
            h.push_back(c);
            sift_up(h, 0, h.size() - 1);
        } else if (c.score < h[0].score) {
            (void)heap_pop(h);
            h.push_back(c);
            sift_up(h, 0, h.size() - 1);
        }
    }
    const size_t m = h.size();
    for (size_t j = 0; j < m; ++j) {
        HeapCand c = heap_pop(h);
        out_ids[m - 1 - j] = c.id;
        out_dist[m - 1 - j] = c.dist;
    }
    return m;
}

}  // namespace vh

// ======================= C ABI: errors, devices, memory, top_k_reduce ======================
using namespace vh;

extern "C" {

const char *vhip_last_error(void) { return t_err.c_str(); }

int vhip_last_error_ordinal(void) { return t_ordinal; }

void vhip_last_error_devices(size_t *requested, size_t *available) {
    if (requested) *requested = t_req;
    if (available) *available = t_avail;
}

int vhip_device_count(void) { return device_count(); }

int vhip_device_info(int ordinal, char *name, size_t name_len, size_t *total_memory_bytes) {
    const int avail = device_count();
    if (ordinal < 0 || ordinal >= avail)
        return set_device_not_found(
            ordinal, "HIP device with ordinal " + std::to_string(ordinal) + " was not found or could not be initialized");
    hipDeviceProp_t p;
    VH_HIP(hipGetDeviceProperties(&p, ordinal));
    if (name && name_len) {
        std::string arch(p.gcnArchName);
        arch = arch.substr(0, arch.find(':'));
        std::string s = std::string("AMD ") + (p.name[0] ? p.name : "Instinct") + " " + arch + " (GPU " +
                        std::to_string(ordinal) + ", " + std::to_string(p.multiProcessorCount) + " CUs)";
        std::strncpy(name, s.c_str(), name_len - 1);
        name[name_len - 1] = 0;
    }
    if (total_memory_bytes) *total_memory_bytes = p.totalGlobalMem;
    return VHIP_OK;
}

int vhip_malloc(int ordinal, size_t bytes, void **ptr) {
    VH_CHECK(open_device(ordinal));
    VH_HIP(hipMalloc(ptr, bytes ? bytes : 256));
    return VHIP_OK;
}
int vhip_free(int ordinal, void *ptr) {
    VH_CHECK(open_device(ordinal));
    VH_HIP(hipFree(ptr));
    return VHIP_OK;
}
int vhip_memcpy_htod(int ordinal, void *dst, const void *src, size_t bytes) {
    VH_CHECK(open_device(ordinal));
    VH_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return VHIP_OK;
}
int vhip_memcpy_dtoh(int ordinal, void *dst, const void *src, size_t bytes) {
    VH_CHECK(open_device(ordinal));
    VH_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return VHIP_OK;
}
int vhip_memcpy_dtod(int ordinal, void *dst, const void *src, size_t bytes) {
    VH_CHECK(open_device(ordinal));
    VH_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
    return VHIP_OK;
}
int vhip_synchronize(int ordinal) {
    VH_CHECK(open_device(ordinal));
    VH_HIP(hipDeviceSynchronize());
    return VHIP_OK;
}

size_t vhip_top_k_reduce(const uint32_t *ids, const float *dist, size_t total, size_t k, int metric,
                         uint32_t *out_ids, float *out_dist) {
    return top_k_reduce_host(ids, dist, total, k, metric == DOT || metric == COS, out_ids, out_dist);
}

}  // extern "C"
