// pq_scan_l2.hip -- IVF-PQ scan kernels for squared L2 with the register-held codebook
// (k_ivfpq_scan in pq_scan.h; one file per metric family so they compile in parallel).
#include "pq_scan.h"

namespace vh {

void launch_ivfpq_scan_l2(const ScanArgs &A, int ds, int nv, int cus, size_t lds, hipStream_t s) {
    launch_scan_reg<L2>(A, ds, nv, cus, lds, s);
}

void launch_ivfpq_lists_l2(const ListArgs &L, int ds, int cus, hipStream_t s) { launch_lists_mt<L2>(L, ds, cus, s); }

void launch_ivfpq_list_merge(const ListArgs &L, int cus, hipStream_t s) {
    if (hib_metric(L.s.metric))
        launch_lists_merge<true>(L, cus, s);
    else
        launch_lists_merge<false>(L, cus, s);
}

}  // namespace vh
