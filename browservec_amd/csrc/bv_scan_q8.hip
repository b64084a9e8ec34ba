// Fused scan instantiations for codec C_Q8 (see bv_scan.h).
#include "bv_scan.h"

namespace bvk {

hipError_t scan_codec_q8(int lpr, int upl, const ScanArgs &a, uint32_t nq, hipStream_t s) {
    return dispatch_layout<C_Q8>(Layout{lpr, upl}, a, nq, s);
}

}  // namespace bvk
