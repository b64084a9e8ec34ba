// Fused scan instantiations for codec C_Q1P (see bv_scan.h).
#include "bv_scan.h"

namespace bvk {

hipError_t scan_codec_q1p(int lpr, int upl, const ScanArgs &a, uint32_t nq, hipStream_t s) {
    return dispatch_layout<C_Q1P>(Layout{lpr, upl}, a, nq, s);
}

namespace {
template <int LPR, int UPL>
hipError_t exact_rows(const Q1pRowsArgs &a, uint32_t nq, uint32_t gx, hipStream_t s) {
    const size_t lds = q1p_lut_bytes(a.P);
    if (lds > 160 * 1024 || a.units == 0 || a.P != a.units * 128) return hipErrorInvalidValue;
    hipLaunchKernelGGL((q1p_exact_rows<LPR, UPL>), dim3(gx, nq), dim3(SCAN_WG), lds, s, a);
    return hipGetLastError();
}
template <int LPR, int UPL>
hipError_t tau_exact(const Q1pRowsArgs &a, const uint64_t *merged, const uint32_t *merged_n, uint32_t kk,
                     uint64_t *tau, uint32_t nq, hipStream_t s) {
    const size_t lds = q1p_lut_bytes(a.P) + (size_t)kk * 4;
    if (lds > 160 * 1024 || a.units == 0 || a.P != a.units * 128 || kk > 4096) return hipErrorInvalidValue;
    hipLaunchKernelGGL((q1p_tau_exact<LPR, UPL>), dim3(1, nq), dim3(SCAN_WG), lds, s, a, merged, merged_n, kk, tau);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_q1p_tau_exact(const Q1pRowsArgs &a, const uint64_t *merged, const uint32_t *merged_n, uint32_t kk,
                                uint64_t *tau, uint32_t nq, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    Layout L;
    if (nq > 65535 || !pick_layout(a.units, L) || L.upl != 1) return hipErrorInvalidValue;
    switch (L.lpr) {  // the batch path's dimensions (P <= 1024)
    case 4: return tau_exact<4, 1>(a, merged, merged_n, kk, tau, nq, s);
    case 8: return tau_exact<8, 1>(a, merged, merged_n, kk, tau, nq, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_q1p_exact_rows(const Q1pRowsArgs &a, uint32_t nq, uint32_t gx, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    Layout L;
    if (gx == 0 || nq > 65535 || !pick_layout(a.units, L) || L.upl != 1) return hipErrorInvalidValue;
    switch (L.lpr) {  // the fused scan's layout, so the sums run in its order (P <= 1024)
    case 4: return exact_rows<4, 1>(a, nq, gx, s);
    case 8: return exact_rows<8, 1>(a, nq, gx, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace bvk
