// pq_scan_mem.hip -- IVF-PQ scan kernels that build the ADC tables from codebooks read through
// the caches, for every metric (k_ivfpq_scan in pq_scan.h).
#include "pq_scan.h"

namespace vh {

void launch_ivfpq_scan_mem(const ScanArgs &A, int nv, int cus, size_t lds, hipStream_t s) {
#define VH_MEM(MT) launch_scan_nv<MT, 0>(A, nv, cus, lds, s)
    VH_METRIC_SWITCH(A.metric, VH_MEM)
#undef VH_MEM
}

}  // namespace vh
