// pq_scan_ip.hip -- IVF-PQ scan kernels for dot product and cosine similarity with the
// register-held codebook (k_ivfpq_scan in pq_scan.h).
#include "pq_scan.h"

namespace vh {

void launch_ivfpq_scan_ip(const ScanArgs &A, int ds, int nv, int cus, size_t lds, hipStream_t s) {
    if (A.metric == DOT)
        launch_scan_reg<DOT>(A, ds, nv, cus, lds, s);
    else
        launch_scan_reg<COS>(A, ds, nv, cus, lds, s);
}

void launch_ivfpq_lists_ip(const ListArgs &L, int ds, int cus, hipStream_t s) {
    if (L.s.metric == DOT)
        launch_lists_mt<DOT>(L, ds, cus, s);
    else
        launch_lists_mt<COS>(L, ds, cus, s);
}

}  // namespace vh
