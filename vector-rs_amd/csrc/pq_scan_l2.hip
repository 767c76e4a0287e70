// pq_scan_l2.hip -- IVF-PQ scan kernels for squared L2 with the register-held codebook
// (k_ivfpq_scan in pq_scan.h; one file per metric family so they compile in parallel).
#include "pq_scan.h"

namespace vh {

void launch_ivfpq_scan_l2(const ScanArgs &A, int ds, int nv, int cus, size_t lds, hipStream_t s) {
    launch_scan_reg<L2>(A, ds, nv, cus, lds, s);
}

}  // namespace vh
