// noalloc_scratch.hip -- the fixed working memory of the allocation-free kNN search
// (vhip_knn_search_batch_device_noalloc).
//
// One array in this library's device code, of which every device that uses it holds its own
// copy until the process ends.  This translation unit holds no kernel: its code object, and with
// it the array, is loaded onto a device only when hipGetSymbolAddress asks for the array there,
// i.e. at the first allocation-free call on that device.  Engines that never make such a call
// reserve nothing for it.  On the host the array's name is only a stand-in, never a device
// address: each device's address comes from hipGetSymbolAddress, taken once per device with that
// device current, and only that address reaches kernels.
#include "vh_runtime.h"

namespace vh {

static __device__ __align__(256) unsigned char scratch[VHIP_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
struct ScratchSlot {
    std::mutex mu;        // held for a whole call: calls on one device run one after another
    void *ptr = nullptr;  // this device's copy of `scratch`
};
ScratchSlot g_scratch[kMaxScratchDevices];
}  // namespace

int noalloc_scratch_acquire(int dev, std::unique_lock<std::mutex> &lock, void **ptr) {
    *ptr = nullptr;
    if (dev < 0 || dev >= kMaxScratchDevices)
        return set_error(VHIP_ERR_INVALID_CONFIG, "device ordinal " + std::to_string(dev) +
                                                      " is beyond the allocation-free search's device table");
    ScratchSlot &S = g_scratch[dev];
    lock = std::unique_lock<std::mutex>(S.mu);
    if (!S.ptr) {
        VH_CHECK(open_device(dev));
        void *p = nullptr;
        VH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return set_error(VHIP_ERR_DRIVER, "hipGetSymbolAddress(scratch) returned a null address");
        S.ptr = p;
    }
    *ptr = S.ptr;
    return VHIP_OK;
}

}  // namespace vh
