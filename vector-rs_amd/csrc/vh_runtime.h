// vh_runtime.h -- host-side runtime pieces shared by the engines: error state,
// device context, RAII device buffers, pinned staging and kernel timing.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "vector_hip.h"
#include "vh_common.h"
#include "vh_error.h"

namespace vh {


#define VH_HIP(expr)                                                                              \
    do {                                                                                          \
        hipError_t e_ = (expr);                                                                   \
        if (e_ != hipSuccess) {                                                                   \
            (void)hipGetLastError();                                                              \
            return ::vh::set_error(VHIP_ERR_DRIVER, std::string(#expr) + ": " + hipGetErrorString(e_)); \
        }                                                                                         \
    } while (0)

#define VH_CHECK(status)             \
    do {                                 \
        int s_ = (status);               \
        if (s_ != VHIP_OK) return s_;    \
    } while (0)

// ---- devices ---------------------------------------------------------------------
int device_count();                // usable gfx950 devices
int open_device(int ordinal);      // DeviceNotFound / HardwareNotAvailable / OK, sets current device
int device_grid_cap(int ordinal);  // persistent-grid size: 2 workgroups per CU

// ---- device buffer -----------------------------------------------------------------
struct DevBuf {
    void *p = nullptr;
    size_t bytes = 0;
    int dev = 0;
    DevBuf() = default;
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    ~DevBuf() { release(); }
    void release() {
        if (p) {
            (void)hipSetDevice(dev);
            (void)hipFree(p);
            p = nullptr;
            bytes = 0;
        }
    }
    // Grows to at least `b` bytes (contents are not preserved).
    int ensure(int device, size_t b) {
        if (b <= bytes && p) return VHIP_OK;
        release();
        dev = device;
        if (b == 0) b = 256;
        hipError_t e = hipMalloc(&p, b);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            p = nullptr;
            return set_error(VHIP_ERR_DRIVER, std::string("hipMalloc(") + std::to_string(b) +
                                                  " bytes): " + hipGetErrorString(e));
        }
        bytes = b;
        return VHIP_OK;
    }
    template <class T>
    T *as() const { return static_cast<T *>(p); }
};

// ---- pinned staging: host <-> device copies through two pinned buffers so the
// host-side memcpy of one block overlaps the DMA of the other ---------------------------
struct PinnedStager {
    static constexpr size_t kBlock = 32u << 20;
    void *buf[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    int dev = -1;
    ~PinnedStager();
    int init(int device);
    int h2d(void *dst, const void *src, size_t bytes, hipStream_t s);
    int d2h(void *dst, const void *src, size_t bytes, hipStream_t s);
    // Two device ranges to host with one wait when each fits a staging buffer.
    int d2h_pair(void *dst0, const void *src0, size_t b0, void *dst1, const void *src1, size_t b1, hipStream_t s);
};

// ---- kernel timing with events on the engine's stream ----------------------------------
struct KernelTimer {
    bool enabled = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> pool;
    std::vector<std::pair<double, double>> meta;  // (work, bytes) of each recorded pair
    size_t used = 0;
    double ms = 0.0, work = 0.0, bytes = 0.0;
    uint64_t launches = 0;
    ~KernelTimer();
    // Records the start event (returns the pair index, or -1 when disabled).
    int begin(hipStream_t s);
    void end(int idx, hipStream_t s, double w, double b);
    // Call after the stream is synchronised: folds recorded pairs into the totals.
    void collect();
    void reset() { ms = work = bytes = 0.0; launches = 0; used = 0; }
};

// The allocation-free search's working memory on device dev (VHIP_NOALLOC_SCRATCH_BYTES): takes
// that device's lock into `lock`, held until the caller releases it, and returns the array's
// device address (looked up once per device).
int noalloc_scratch_acquire(int dev, std::unique_lock<std::mutex> &lock, void **ptr);

uint64_t splitmix64(uint64_t &state);
// Fisher-Yates permutation of [0, n) from a seed (the seeded shuffle init of k-means).
std::vector<uint32_t> row_permutation(size_t n, uint64_t seed);

// Rust BinaryHeap-based bounded top-k merge: CollectiveOps::top_k_reduce
// (ddp/collective.rs:115-159).  Returns the merged count.
size_t top_k_reduce_host(const uint32_t *ids, const float *dist, size_t total, size_t k, bool higher_is_better,
                         uint32_t *out_ids, float *out_dist);

}  // namespace vh
