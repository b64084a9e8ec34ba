// Fused scan instantiations for codec C_Q1P (see bv_scan.h).
#include "bv_scan.h"

namespace bvk {

hipError_t scan_codec_q1p(int lpr, int upl, const ScanArgs &a, uint32_t nq, hipStream_t s) {
    return dispatch_layout<C_Q1P>(Layout{lpr, upl}, a, nq, s);
}

}  // namespace bvk
