// gfx950 (CDNA4) kernels for BrowserVec's search path: launchers of the
// row encoder, the query level split and the explicit re-rank, and the
// codec switch of the fused scan (whose instantiations live in one
// translation unit per codec, bv_scan_*.hip, so they compile in parallel).
#include "bv_scan.h"

namespace bvk {
namespace {

// ---------------------------------------------------------------- rerank --
// Re-rank of an explicit candidate list: one wave per candidate computes
// Store.dotRow exactly (exact_key_wave); the last wave of each query ranks
// the re-ranked keys and writes the top-k_out.  Dynamic LDS: 8 * (dim & ~3).
__global__ __launch_bounds__(64) void rerank_topk(RerankArgs a) {
    extern __shared__ __align__(16) double prod[];
    __shared__ uint64_t keys[MAX_KPRIME];
    __shared__ uint32_t last_s;
    const uint32_t qi = blockIdx.y, c = blockIdx.x;
    const int lane = threadIdx.x;
    uint32_t m;
    uint32_t row = 0;
    bool have = false;
    if (a.merged) {
        m = a.merged_n[qi];
        if (c < m) {
            row = key_row(a.merged[(uint64_t)qi * a.kprime + c]);
            have = true;
        }
    } else {
        m = a.cand_n[qi];
        if (c < m) {
            row = a.cand_rows[(uint64_t)qi * a.kprime + c];
            have = true;
        }
    }
    if (have) {
        const uint64_t ek = exact_key_wave(a.rows + (uint64_t)row * a.dim, a.q + (uint64_t)qi * a.q_stride, a.dim, row,
                                           prod, lane);
        if (lane == 0) store_shared(&a.rr_keys[(uint64_t)qi * a.kprime + c], ek);
    }
    wait_stores_done();
    __syncthreads();
    if (lane == 0) last_s = atomicAdd(&a.tickets[qi], 1u) == gridDim.x - 1;
    __syncthreads();
    if (!last_s) return;
    for (uint32_t j = lane; j < m; j += 64) keys[j] = load_shared(&a.rr_keys[(uint64_t)qi * a.kprime + j]);
    __syncthreads();
    const uint32_t ko = m < a.k_out ? m : a.k_out;
    if (m <= 256) {
        // rank by counting (keys are unique): key j goes to slot #{greater}
        for (uint32_t j = lane; j < m; j += 64) {
            const uint64_t kj = keys[j];
            const uint32_t r = count_greater(keys, m, kj);
            if (r < ko) {
                a.out_rows[(uint64_t)qi * a.k_out + r] = key_row(kj);
                a.out_scores[(uint64_t)qi * a.k_out + r] = f32_from_ord((uint32_t)(kj >> 32));
            }
        }
    } else {
        const uint32_t npow = pow2_at_least(m);
        for (uint32_t j = m + lane; j < npow; j += 64) keys[j] = 0;
        __syncthreads();
        bitonic_desc(keys, npow);
        for (uint32_t j = lane; j < ko; j += 64) {
            a.out_rows[(uint64_t)qi * a.k_out + j] = key_row(keys[j]);
            a.out_scores[(uint64_t)qi * a.k_out + j] = f32_from_ord((uint32_t)(keys[j] >> 32));
        }
    }
    if (lane == 0) {
        a.out_n[qi] = ko;
        a.tickets[qi] = 0;
    }
}

__global__ __launch_bounds__(256) void zero_words(uint32_t *p, uint64_t words) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += stride) p[i] = 0u;
}

}  // namespace

hipError_t launch_zero(void *p, size_t bytes, hipStream_t s) {
    if (bytes == 0) return hipSuccess;
    if (bytes & 3) return hipErrorInvalidValue;
    const uint64_t words = bytes / 4;
    uint64_t blocks = (words + 255) / 256;
    if (blocks > 2048) blocks = 2048;
    hipLaunchKernelGGL(zero_words, dim3((uint32_t)blocks), dim3(256), 0, s, (uint32_t *)p, words);
    return hipGetLastError();
}


bool scan_supported(int codec, uint32_t units) {
    Layout L;
    if (!pick_layout(units, L)) return false;
    // register budget: at most 64 query values per lane
    static const int qn[C_COUNT] = {4, 4, 12, 24, 32, 4, 4, 1, 1, Codec<C_Q1P>::QN};
    return codec >= 0 && codec < C_COUNT && L.upl * qn[codec] <= 64;
}

hipError_t launch_scan(int codec, uint32_t units, const ScanArgs &a, uint32_t nq, hipStream_t s) {
    Layout L;
    if (!pick_layout(units, L) || !scan_supported(codec, units)) return hipErrorInvalidValue;
    switch (codec) {
    case C_F32DOT: return scan_codec_f32dot(L.lpr, L.upl, a, nq, s);
    case C_F32L2: return scan_codec_f32l2(L.lpr, L.upl, a, nq, s);
    case C_Q8: return scan_codec_q8(L.lpr, L.upl, a, nq, s);
    case C_Q4: return scan_codec_q4(L.lpr, L.upl, a, nq, s);
    case C_Q1A: return scan_codec_q1a(L.lpr, L.upl, a, nq, s);
    case C_Q1P: return scan_codec_q1p(L.lpr, L.upl, a, nq, s);
    case C_HAM: return scan_codec_ham(L.lpr, L.upl, a, nq, s);
    case C_I8S: return scan_codec_i8s(L.lpr, L.upl, a, nq, s);
    case C_F32DOT_S: return scan_codec_f32dot_s(L.lpr, L.upl, a, nq, s);
    case C_F32L2_S: return scan_codec_f32l2_s(L.lpr, L.upl, a, nq, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_encode(const EncodeArgs &a, hipStream_t s) {
    if (a.rows == 0) return hipSuccess;
    const uint32_t E = a.P >= 64 ? a.P / 64 : 1;
    const int waves = 2;
    const size_t lds = (size_t)waves * (a.P + 4 * (size_t)a.P);
    uint64_t blocks = (a.rows + waves - 1) / waves;
    if (blocks > 65536) blocks = 65536;
    dim3 grid((uint32_t)blocks), block(64 * waves);
    switch (E) {
    case 1: hipLaunchKernelGGL(encode_rows<1>, grid, block, lds, s, a); break;
    case 2: hipLaunchKernelGGL(encode_rows<2>, grid, block, lds, s, a); break;
    case 4: hipLaunchKernelGGL(encode_rows<4>, grid, block, lds, s, a); break;
    case 8: hipLaunchKernelGGL(encode_rows<8>, grid, block, lds, s, a); break;
    case 16: hipLaunchKernelGGL(encode_rows<16>, grid, block, lds, s, a); break;
    case 32: hipLaunchKernelGGL(encode_rows<32>, grid, block, lds, s, a); break;
    case 64: hipLaunchKernelGGL(encode_rows<64>, grid, block, lds, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_levels(const LevelArgs &a, uint32_t nq, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    const size_t lds = 3 * (size_t)a.P;
    switch (a.P >= 64 ? a.P / 64 : 1) {
    case 1: hipLaunchKernelGGL(query_levels<1>, dim3(nq), dim3(64), lds, s, a); break;
    case 2: hipLaunchKernelGGL(query_levels<2>, dim3(nq), dim3(64), lds, s, a); break;
    case 4: hipLaunchKernelGGL(query_levels<4>, dim3(nq), dim3(64), lds, s, a); break;
    case 8: hipLaunchKernelGGL(query_levels<8>, dim3(nq), dim3(64), lds, s, a); break;
    case 16: hipLaunchKernelGGL(query_levels<16>, dim3(nq), dim3(64), lds, s, a); break;
    case 32: hipLaunchKernelGGL(query_levels<32>, dim3(nq), dim3(64), lds, s, a); break;
    case 64: hipLaunchKernelGGL(query_levels<64>, dim3(nq), dim3(64), lds, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

size_t level_stride(int codec, uint32_t P) { return query_layout_bytes(codec, P); }

hipError_t launch_q1p_layout(const LevelArgs &a, uint32_t nq, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    const size_t lds = 2 * (size_t)a.P;
    switch (a.P / 64) {
    case 2: hipLaunchKernelGGL(query_q1p<2>, dim3(nq), dim3(64), lds, s, a); break;
    case 4: hipLaunchKernelGGL(query_q1p<4>, dim3(nq), dim3(64), lds, s, a); break;
    case 8: hipLaunchKernelGGL(query_q1p<8>, dim3(nq), dim3(64), lds, s, a); break;
    case 16: hipLaunchKernelGGL(query_q1p<16>, dim3(nq), dim3(64), lds, s, a); break;
    case 32: hipLaunchKernelGGL(query_q1p<32>, dim3(nq), dim3(64), lds, s, a); break;
    case 64: hipLaunchKernelGGL(query_q1p<64>, dim3(nq), dim3(64), lds, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool scan_prep_supported(int codec, uint32_t units, uint32_t P) {
    Layout L;
    if (!pick_layout(units, L)) return false;
    int upc = 0;
    switch (codec) {
    case C_Q8: case C_I8S: upc = 16; break;
    case C_Q4: case C_Q1A: upc = 32; break;
    case C_HAM: case C_Q1P: upc = 128; break;
    default: return false;
    }
    const uint32_t full = (uint32_t)upc * L.lpr * L.upl;
    return P == full && P >= 64 && P / 64 <= 16;
}
size_t scan_query_lds(int codec, uint32_t P) { return query_prep_lds(codec, P); }
size_t scan_lds_bytes(int codec, uint32_t P, uint32_t wstride) {
    size_t lds = (size_t)(SCAN_WG / 64) * wstride * sizeof(uint64_t);
    if (lds < sizeof(TopkLds)) lds = sizeof(TopkLds);
    const size_t prep = (query_prep_lds(codec, P) + 15) & ~(size_t)15;
    if (lds < prep) lds = prep;
    if (codec == C_Q1P) lds = ((lds + 15) & ~(size_t)15) + q1p_lut_bytes(P);
    return lds;
}

hipError_t launch_rerank(const RerankArgs &a, uint32_t nq, hipStream_t s) {
    const size_t lds = sizeof(double) * (size_t)(a.dim & ~3u) + 16;
    hipLaunchKernelGGL(rerank_topk, dim3(a.kprime, nq), dim3(64), lds, s, a);
    return hipGetLastError();
}

}  // namespace bvk
