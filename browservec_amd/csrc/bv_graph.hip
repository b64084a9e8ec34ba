// Graph beam search over a flat fixed-degree adjacency (HNSW's layer 0), one
// wave per query: the searcher of src/index/hnswGpu.ts:134-206 with the
// best-first beam of src/engine/wgsl/graphSearch.ts:62-259.
//
// The wave keeps the whole beam in registers (lane t holds slots t, t + 64,
// t + 128, t + 192), so the argmin / argmax reductions are cross-lane
// shuffles in the shader's own order: each lane keeps the first strict best
// of its slots, then a halving tree of strict compares.  The visited set is
// the shader's 2048-slot open-addressed table in LDS; a staged batch of ids
// is inserted in lane order (one LDS read by 16 lanes finds the first slot of
// the probe run that holds the id or is empty; a run of 16 full slots sheds
// the id, reported unseen).  Distances run in f32, element order, each
// multiply and add rounded (`acc = acc + c * q`), one lane per row, with the
// query in LDS.  The end of the kernel dedups the beam (first slot of an id),
// sorts it by score (-distance) with ties in slot order, and writes the top k.
#include <hip/hip_runtime.h>

#include "bv_kernels.h"

namespace bvk {
namespace {

constexpr uint32_t GS_WG = 64;
constexpr uint32_t GS_SLOTS = GRAPH_EF_CAP / GS_WG;  // beam slots per lane
constexpr uint32_t GS_HASH = 2048;
constexpr uint32_t GS_PROBES = 16;
constexpr float GS_INF = 3.4e38f;
constexpr uint32_t GS_EMPTY = 0xffffffffu;

__device__ __forceinline__ float rdlane(float v, uint32_t l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)l));
}
__device__ __forceinline__ uint32_t rdlane(uint32_t v, uint32_t l) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)l);
}

// f32 distance of one row, element order, no contraction (smaller = closer:
// -dot for dot / cosine, the squared difference for l2).
template <bool L2>
__device__ float row_dist(const float *__restrict__ row, const float *qv, uint32_t dim, bool vec4) {
#pragma clang fp contract(off)
    float acc = 0.0f;
    uint32_t i = 0;
    if (vec4) {
        const float4 *r4 = (const float4 *)row;
        const float4 *q4 = (const float4 *)qv;
        for (; i + 32 <= dim; i += 32) {
            float4 x[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) x[u] = r4[i / 4 + u];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float4 y = q4[i / 4 + u];
                if (L2) {
                    float d = x[u].x - y.x;
                    acc = acc + d * d;
                    d = x[u].y - y.y;
                    acc = acc + d * d;
                    d = x[u].z - y.z;
                    acc = acc + d * d;
                    d = x[u].w - y.w;
                    acc = acc + d * d;
                } else {
                    acc = acc + x[u].x * y.x;
                    acc = acc + x[u].y * y.y;
                    acc = acc + x[u].z * y.z;
                    acc = acc + x[u].w * y.w;
                }
            }
        }
    }
    for (; i < dim; ++i) {
        if (L2) {
            const float d = row[i] - qv[i];
            acc = acc + d * d;
        } else {
            acc = acc + row[i] * qv[i];
        }
    }
    return L2 ? acc : -acc;
}

// The lanes in `want` insert their id into the visited set in lane order;
// returns true on a lane whose id was not there before (inserted or shed).
__device__ bool mark_batch(uint32_t *vis, uint32_t id, bool want, uint32_t t) {
    uint64_t m = __ballot(want);
    bool fresh = false;
    while (m) {
        const uint32_t j = (uint32_t)__builtin_ctzll(m);
        m &= m - 1;
        const uint32_t x = rdlane(id, j);
        const uint32_t h = (x * 2654435761u) & (GS_HASH - 1u);
        const uint32_t pos = (h + t) & (GS_HASH - 1u);
        const uint32_t cur = t < GS_PROBES ? vis[pos] : 0xfffffffeu;
        const uint64_t hit = __ballot(t < GS_PROBES && (cur == x + 1u || cur == 0u));
        bool seen = false;
        if (hit) {
            const uint32_t p = (uint32_t)__builtin_ctzll(hit);
            const uint32_t c = rdlane(cur, p);
            seen = c == x + 1u;
            if (!seen && t == p) vis[pos] = x + 1u;  // the first empty slot of the run
        }
        if (t == j) fresh = !seen;
    }
    return fresh;
}

// Argmax over the active slots (foldStaged's worst) or argmin over the
// unexpanded ones, in the shader's order.
template <bool MAX>
__device__ __forceinline__ void beam_arg(const float (&cd)[GS_SLOTS], const uint32_t (&ce)[GS_SLOTS], uint32_t efA,
                                         uint32_t t, float &val, uint32_t &slot) {
    float v = MAX ? -GS_INF : GS_INF;
    uint32_t ix = 0;
#pragma unroll
    for (uint32_t m = 0; m < GS_SLOTS; ++m) {
        const uint32_t s = t + GS_WG * m;
        if (s < efA) {
            if (MAX ? cd[m] > v : (ce[m] == 0u && cd[m] < v)) {
                v = cd[m];
                ix = s;
            }
        }
    }
#pragma unroll
    for (uint32_t stride = GS_WG / 2; stride; stride >>= 1) {
        const float ov = __shfl_down(v, stride);
        const uint32_t oi = __shfl_down(ix, stride);
        if (t < stride && (MAX ? ov > v : ov < v)) {
            v = ov;
            ix = oi;
        }
    }
    val = rdlane(v, 0);
    slot = rdlane(ix, 0);
}

// foldStaged: lane j's staged (dist, id), j < count in order, replaces the
// worst active slot when it is better.
__device__ void fold(float (&cd)[GS_SLOTS], uint32_t (&ci)[GS_SLOTS], uint32_t (&ce)[GS_SLOTS], uint32_t efA,
                     float sd, uint32_t si, uint32_t count, uint32_t t) {
    uint64_t live = __ballot(t < count && sd < GS_INF);  // an INF entry never replaces anything
    while (live) {
        const uint32_t j = (uint32_t)__builtin_ctzll(live);
        live &= live - 1;
        const float d = rdlane(sd, j);
        const uint32_t id = rdlane(si, j);
        float worst;
        uint32_t slot;
        beam_arg<true>(cd, ce, efA, t, worst, slot);
        if (d < worst && (slot & (GS_WG - 1)) == t) {
#pragma unroll
            for (uint32_t m = 0; m < GS_SLOTS; ++m)
                if (slot == t + GS_WG * m) {
                    cd[m] = d;
                    ci[m] = id;
                    ce[m] = 0u;
                }
        }
    }
}

template <bool L2>
__global__ __launch_bounds__(GS_WG) void graph_beam(GraphArgs a) {
    __shared__ uint32_t vis[GS_HASH];
    __shared__ float hd[GRAPH_EF_CAP];
    __shared__ uint32_t hi[GRAPH_EF_CAP];
    extern __shared__ float qv[];
    const uint32_t q = blockIdx.x, t = threadIdx.x;
    const uint32_t dim = a.dim;
    for (uint32_t i = t; i < dim; i += GS_WG) qv[i] = a.queries[(uint64_t)q * dim + i];
    for (uint32_t i = t; i < GS_HASH; i += GS_WG) vis[i] = 0u;
    __syncthreads();
    const bool vec4 = (dim & 3u) == 0 && (((uintptr_t)a.corpus) & 15u) == 0;
    const uint32_t efA = a.efA;
    float cd[GS_SLOTS];
    uint32_t ci[GS_SLOTS], ce[GS_SLOTS];
#pragma unroll
    for (uint32_t m = 0; m < GS_SLOTS; ++m) {
        cd[m] = GS_INF;
        ci[m] = GS_EMPTY;
        ce[m] = 1u;
    }
    // seeds, staged like a neighbour batch
    const uint32_t ne = a.n_entries < GS_WG ? a.n_entries : GS_WG;
    uint32_t id = t < ne ? a.entries[t] : GS_EMPTY;
    bool ok = t < ne && id < a.corpus_rows;
    bool fresh = mark_batch(vis, id, ok, t);
    float sd = GS_INF;
    uint32_t si = GS_EMPTY;
    if (ok && fresh) {
        sd = row_dist<L2>(a.corpus + (uint64_t)id * dim, qv, dim, vec4);
        si = id;
    }
    fold(cd, ci, ce, efA, sd, si, ne, t);
    for (uint32_t iter = 0; iter < a.iter_cap; ++iter) {
        float best;
        uint32_t slot;
        beam_arg<false>(cd, ce, efA, t, best, slot);
        if (best >= GS_INF) break;
        uint32_t node = 0;
#pragma unroll
        for (uint32_t m = 0; m < GS_SLOTS; ++m)
            if (slot == t + GS_WG * m) {
                ce[m] = 1u;
                node = ci[m];
            }
        node = rdlane(node, slot & (GS_WG - 1));
        id = (t < a.K && node < a.graph_rows) ? a.graph[(uint64_t)node * a.K + t] : GS_EMPTY;
        ok = id < a.corpus_rows;
        fresh = mark_batch(vis, id, ok, t);
        sd = GS_INF;
        si = GS_EMPTY;
        if (ok && fresh) {
            sd = row_dist<L2>(a.corpus + (uint64_t)id * dim, qv, dim, vec4);
            si = id;
        }
        fold(cd, ci, ce, efA, sd, si, a.K, t);
    }
    // the raw beam (parity export) and the searcher's hits
#pragma unroll
    for (uint32_t m = 0; m < GS_SLOTS; ++m) {
        hd[t + GS_WG * m] = cd[m];
        hi[t + GS_WG * m] = ci[m];
        if (a.beam_dist) {
            a.beam_dist[(uint64_t)q * GRAPH_EF_CAP + t + GS_WG * m] = cd[m];
            a.beam_id[(uint64_t)q * GRAPH_EF_CAP + t + GS_WG * m] = ci[m];
        }
    }
    __syncthreads();
    if (!a.out_rows) return;
    // live slot: below efA, not empty, its id's first slot (flags in the
    // visited table's space, no longer needed)
    uint32_t *live = vis;
    bool lv[GS_SLOTS];
    uint32_t nlive = 0;
#pragma unroll
    for (uint32_t m = 0; m < GS_SLOTS; ++m) {
        const uint32_t s = t + GS_WG * m;
        bool l = s < efA && hi[s] != GS_EMPTY;
        for (uint32_t s2 = 0; l && s2 < s; ++s2) l = hi[s2] != hi[s];
        lv[m] = l;
        nlive += (uint32_t)__popcll(__ballot(l));
    }
    __syncthreads();  // every lane is past its last visited-set read
#pragma unroll
    for (uint32_t m = 0; m < GS_SLOTS; ++m) live[t + GS_WG * m] = lv[m] ? 1u : 0u;
    __syncthreads();
    // rank = live slots with a higher score, or the same score at a lower slot
#pragma unroll
    for (uint32_t m = 0; m < GS_SLOTS; ++m) {
        const uint32_t s = t + GS_WG * m;
        if (!lv[m]) continue;
        const float sc = -hd[s];
        uint32_t r = 0;
        for (uint32_t s2 = 0; s2 < efA; ++s2) {
            const float o = -hd[s2];
            r += (live[s2] && s2 != s && (o > sc || (o == sc && s2 < s))) ? 1u : 0u;
        }
        if (r < a.k) {
            a.out_rows[(uint64_t)q * a.out_stride + r] = hi[s];
            a.out_scores[(uint64_t)q * a.out_stride + r] = sc;
        }
    }
    if (t == 0) a.out_n[q] = nlive < a.k ? nlive : a.k;
}

}  // namespace

hipError_t launch_graph_beam(const GraphArgs &a, uint32_t nq, bool l2, hipStream_t s) {
    if (nq == 0) return hipSuccess;
    if (a.K == 0 || a.K > GS_WG || a.efA == 0 || a.efA > GRAPH_EF_CAP || a.k > GRAPH_EF_CAP || a.dim == 0 ||
        (size_t)a.dim * 4 > 64 * 1024)
        return hipErrorInvalidValue;
    const size_t lds = (size_t)a.dim * 4;
    if (l2)
        hipLaunchKernelGGL(graph_beam<true>, dim3(nq), dim3(GS_WG), lds, s, a);
    else
        hipLaunchKernelGGL(graph_beam<false>, dim3(nq), dim3(GS_WG), lds, s, a);
    return hipGetLastError();
}

}  // namespace bvk
