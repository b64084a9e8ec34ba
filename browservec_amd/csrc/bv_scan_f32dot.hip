// Fused scan instantiations for codec C_F32DOT (see bv_scan.h).
#include "bv_scan.h"

namespace bvk {

hipError_t scan_codec_f32dot(int lpr, int upl, const ScanArgs &a, uint32_t nq, hipStream_t s) {
    return dispatch_layout<C_F32DOT>(Layout{lpr, upl}, a, nq, s);
}

}  // namespace bvk
