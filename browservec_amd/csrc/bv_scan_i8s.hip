// Fused scan instantiations for codec C_I8S (see bv_scan.h).
#include "bv_scan.h"

namespace bvk {

hipError_t scan_codec_i8s(int lpr, int upl, const ScanArgs &a, uint32_t nq, hipStream_t s) {
    return dispatch_layout<C_I8S>(Layout{lpr, upl}, a, nq, s);
}

}  // namespace bvk
