// Ragged token -> expert packing on gfx950 (moe_route_workspace_bytes, moe_group_routes): per-expert counts,
// exclusive-scan offsets and the slot permutation, stable (ascending slot order inside an expert's bucket), plus the
// tile tables the grouped expert kernels walk.
//
// Work is split into chunks of kChunk slots, one wave64 per chunk. Inside a wave, the lanes holding the same bucket
// find each other with ballots over the bucket's bits (an exact "match any"), so each lane knows its rank among
// equal buckets in lane order and one leader lane updates the bucket's count - no atomics, so the placement is the
// stable order by construction. Small S (<= 16 chunks) runs as one 1024-thread block with everything in LDS; larger S
// as three launches (chunk histograms, scan, placement) through the workspace.
#include "route_small.hpp"

#include <type_traits>

namespace strix::kernels {

namespace {

using namespace route;


// ---- S <= kFusedSlots: one block, everything in LDS until the final stores (route_small.hpp) ------------------------
__global__ void __launch_bounds__(1024) route_small_kernel(const int32_t *ids, Layout L, int nbits, int32_t *ws,
                                                           uint32_t *err) {
    extern __shared__ int lds[];
    pack_small_body<1, false>(nullptr, 0, ids, 0, (int)L.E, 0, nullptr, nullptr, L, nbits, ws, nullptr, err, lds);
}

// ---- larger S: chunk histograms, one scan block, placement ----------------------------------------------------------
constexpr int kWavesPerBlock = 4;

__global__ void __launch_bounds__(kWavesPerBlock * kWave) route_hist_kernel(const int32_t *ids, Layout L, int nbits,
                                                                           int32_t *ws) {
    extern __shared__ int lds[];  // [kWavesPerBlock][E + 1]
    const int E = (int)L.E, wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int64_t ch = (int64_t)blockIdx.x * kWavesPerBlock + wave;
    if (ch >= L.nch) return;  // whole wave; no barrier in this kernel
    int *h = lds + wave * (E + 1);
    for (int b = lane; b <= E; b += kWave) h[b] = 0;
    const int64_t s0 = ch * kChunk, s1 = s0 + kChunk < L.S ? s0 + kChunk : L.S;
    const int fb = chunk_hist(ids, s0, s1, E, nbits, h);
    int32_t *gh = ws + L.hist() + ch * (E + 1);
    for (int b = lane; b <= E; b += kWave) gh[b] = h[b];
    if (lane == 0) ws[L.bad() + ch] = fb;
}

__global__ void __launch_bounds__(1024) route_scan_kernel(const int32_t *ids, Layout L, int32_t *ws, uint32_t *err) {
    __shared__ int wsum[48];
    __shared__ int bad_lds;
    const int E = (int)L.E, t = threadIdx.x;
    if (t == 0) bad_lds = INT_MAX;
    __syncthreads();
    int fb = INT_MAX;
    for (int64_t c = t; c < L.nch; c += blockDim.x) fb = min(fb, ws[L.bad() + c]);
    if (fb != INT_MAX) atomicMin(&bad_lds, fb);
    // the chunk histograms are read 16 at a time (independent loads in flight together: a round trip per 16 chunks
    // instead of one per chunk)
    constexpr int B = 16;
    int cnt = 0;
    if (t <= E)
        for (int64_t c0 = 0; c0 < L.nch; c0 += B) {
            int h[B];
#pragma unroll
            for (int b = 0; b < B; ++b) h[b] = c0 + b < L.nch ? ws[L.hist() + (c0 + b) * (E + 1) + t] : 0;
#pragma unroll
            for (int b = 0; b < B; ++b) cnt += h[b];
        }
    int v[3] = {cnt, (cnt + kTileRows - 1) / kTileRows, (cnt + kWideRows - 1) / kWideRows}, tot[3];
    block_scan3(v, wsum, tot);
    if (t <= E) {
        write_bucket(t, cnt, v, ws, L);
        int run = v[0];
        for (int64_t c0 = 0; c0 < L.nch; c0 += B) {
            int h[B];
#pragma unroll
            for (int b = 0; b < B; ++b) h[b] = c0 + b < L.nch ? ws[L.hist() + (c0 + b) * (E + 1) + t] : 0;
#pragma unroll
            for (int b = 0; b < B; ++b)
                if (c0 + b < L.nch) {
                    ws[L.hist() + (c0 + b) * (E + 1) + t] = run;
                    run += h[b];
                }
        }
    }
    if (t == 0) {
        write_header(ws, L, tot);
        report_bad(ids, bad_lds, err);
    }
}

__global__ void __launch_bounds__(kWavesPerBlock * kWave) route_place_kernel(const int32_t *ids, Layout L, int nbits,
                                                                            int32_t *ws) {
    extern __shared__ int lds[];
    const int E = (int)L.E, wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int64_t ch = (int64_t)blockIdx.x * kWavesPerBlock + wave;
    if (ch >= L.nch) return;
    int *c = lds + wave * (E + 1);
    const int32_t *gh = ws + L.hist() + ch * (E + 1);
    for (int b = lane; b <= E; b += kWave) c[b] = gh[b];
    const int64_t s0 = ch * kChunk, s1 = s0 + kChunk < L.S ? s0 + kChunk : L.S;
    chunk_place(ids, s0, s1, E, nbits, c, ws + L.slots());
}

__global__ void __launch_bounds__(256) route_tiles_kernel(Layout L, int32_t *ws) {
    fill_tile_slots(ws, L, ws[0], (int64_t)blockIdx.x * blockDim.x + threadIdx.x, (int64_t)gridDim.x * blockDim.x);
}


template <int NV>
__global__ void __launch_bounds__(1024)
    topk_route_small_kernel(const float *logits, int64_t ld, int M, int E, int k, int32_t *ids_out, float *coef_out,
                            Layout L, int nbits, int32_t *ws, uint32_t *err_router, uint32_t *err_route,
                            bool shared_slot) {
    extern __shared__ int lds[];
    topk_route_small_body<NV>(logits, ld, M, E, k, ids_out, coef_out, L, nbits, ws, err_router, err_route, lds,
                              shared_slot);
}


}  // namespace

size_t moe_route_workspace_bytes(int64_t M, int64_t A, int64_t E) {
    STRIX_CHECK(M >= 1 && A >= 1 && E >= 1 && E <= kMoeMaxExperts && M * A <= kMoeMaxSlots,
                "moe_route_workspace_bytes: M = ", M, ", A = ", A, ", E = ", E, " (E <= ", kMoeMaxExperts,
                ", M*A <= ", kMoeMaxSlots, ")");
    return (size_t)route::layout(M, A, E).ints() * 4;
}

void moe_group_routes(const int32_t *ids, int64_t M, int64_t A, int64_t E, void *ws, size_t ws_bytes, uint32_t *err,
                      hipStream_t stream) {
    const char *fn = "moe_group_routes";
    STRIX_CHECK(ids != nullptr && ws != nullptr && err != nullptr, fn, ": null pointer (ids=", (const void *)ids,
                ", ws=", ws, ", err=", (const void *)err, ")");
    STRIX_CHECK(M >= 1 && A >= 1 && A <= 64 && E >= 1 && E <= kMoeMaxExperts && M * A <= kMoeMaxSlots, fn, ": M = ",
                M, ", A = ", A, ", E = ", E, " (A 1..64, E 1..", kMoeMaxExperts, ", M*A <= ", kMoeMaxSlots, ")");
    STRIX_CHECK(ws_bytes >= moe_route_workspace_bytes(M, A, E), fn, ": workspace of ", ws_bytes, " bytes, needs ",
                moe_route_workspace_bytes(M, A, E));
    STRIX_CHECK(disjoint(ids, M * A * 4, ws, (int64_t)ws_bytes), fn, ": ids overlaps the workspace");
    STRIX_CHECK(reinterpret_cast<uintptr_t>(ws) % 16 == 0, fn, ": workspace must be 16-byte aligned");
    const Layout L = route::layout(M, A, E);
    int nbits = 0;
    while ((1ll << nbits) <= E) ++nbits;  // buckets 0..E
    int32_t *w = static_cast<int32_t *>(ws);
    if (L.S <= kFusedSlots) {
        route_small_kernel<<<1, 1024, topk_route_small_lds(L), stream>>>(ids, L, nbits, w, err);
    } else {
        const unsigned blocks = (unsigned)((L.nch + kWavesPerBlock - 1) / kWavesPerBlock);
        const size_t lds = (size_t)kWavesPerBlock * (E + 1) * 4;
        route_hist_kernel<<<blocks, kWavesPerBlock * kWave, lds, stream>>>(ids, L, nbits, w);
        route_scan_kernel<<<1, 1024, 0, stream>>>(ids, L, w, err);
        route_place_kernel<<<blocks, kWavesPerBlock * kWave, lds, stream>>>(ids, L, nbits, w);
        const int64_t tb = (L.T16 * kTileRows + 255) / 256;
        route_tiles_kernel<<<(unsigned)(tb < 4096 ? tb : 4096), 256, 0, stream>>>(L, w);
    }
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " A=", A, " E=", E);
}


void moe_topk_group_routes_small(const float *logits, int64_t ld, int64_t M, int64_t E, int64_t k, int32_t *ids,
                                 float *coef, void *ws, size_t ws_bytes, uint32_t *err_router, uint32_t *err_route,
                                 hipStream_t stream, bool shared_slot) {
    const char *fn = "moe_topk_group_routes_small";
    const int64_t A = k + (shared_slot ? 1 : 0), Es = E + (shared_slot ? 1 : 0);  // slots; experts packed
    STRIX_CHECK(M >= 1 && k >= 1 && A <= 64 && k <= E && Es <= kMoeMaxExperts && M * A <= kFusedSlots, fn,
                ": M = ", M, ", E = ", E, ", k = ", k, shared_slot ? " + the shared slot" : "", " (M A <= ",
                kFusedSlots, ")");
    STRIX_CHECK(ws_bytes >= moe_route_workspace_bytes(M, A, Es) && reinterpret_cast<uintptr_t>(ws) % 16 == 0, fn,
                ": workspace of ", ws_bytes, " bytes, needs ", moe_route_workspace_bytes(M, A, Es), ", 16-byte aligned");
    const route::Layout L = route::layout(M, A, Es);
    int nbits = 0;
    while ((1ll << nbits) <= Es) ++nbits;
    const size_t lds = route::topk_route_small_lds(L);
    const int nv = E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : 16;
    auto go = [&](auto nvc) {
        topk_route_small_kernel<decltype(nvc)::value><<<1, 1024, lds, stream>>>(
            logits, ld, (int)M, (int)Es, (int)k, ids, coef, L, nbits, static_cast<int32_t *>(ws), err_router, err_route,
            shared_slot);
    };
    switch (nv) {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        case 4: go(std::integral_constant<int, 4>{}); break;
        case 8: go(std::integral_constant<int, 8>{}); break;
        default: go(std::integral_constant<int, 16>{}); break;
    }
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " E=", E, " k=", k);
}

}  // namespace strix::kernels
