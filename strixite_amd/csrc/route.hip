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

// ---- larger S: range histograms, one scan block, placement ------------------------------------------------------------
// A histogram block takes a range of kRangeChunks chunks, a wave each: the chunk counts meet in LDS, and the block
// writes each chunk's position within the range and the range's bucket counts. The scan block then has only the
// ranges' counts to read (the chunks' would be a long chain of round trips on one CU at prefill sizes); it turns
// them into each range's first position; a chunk's cursor is its range's first position plus its position in the
// range.
constexpr int kRangeChunks = Layout::kRangeChunks;

__global__ void __launch_bounds__(kRangeChunks * kWave) route_hist_kernel(const int32_t *ids, Layout L, int nbits,
                                                                          int32_t *ws) {
    extern __shared__ int lds[];  // [kRangeChunks][E + 1]
    const int E = (int)L.E, nb = E + 1, wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int64_t r = blockIdx.x, ch0 = r * kRangeChunks;
    const int64_t ch = ch0 + wave, s0 = ch * kChunk, s1 = s0 + kChunk < L.S ? s0 + kChunk : L.S;
    ChunkIds ci{};
    if (ch < L.nch) ci = chunk_ids(ids, s0, s1);  // in flight while the counters are cleared
    for (int i = threadIdx.x; i < kRangeChunks * nb; i += blockDim.x) lds[i] = 0;
    __syncthreads();
    if (ch < L.nch) {
        const int fb = chunk_hist(ci, s0, s1, E, nbits, lds + wave * nb);
        if (lane == 0) ws[L.bad() + ch] = fb;
    }
    __syncthreads();
    const int nc = (int)(L.nch - ch0 < kRangeChunks ? L.nch - ch0 : kRangeChunks);
    for (int t = threadIdx.x; t < nb; t += blockDim.x) {
        int run = 0;
#pragma unroll
        for (int w = 0; w < kRangeChunks; ++w)
            if (w < nc) {
                ws[L.hist() + (ch0 + w) * nb + t] = run;
                run += lds[w * nb + t];
            }
        ws[L.rsum() + r * nb + t] = run;
    }
}

__global__ void __launch_bounds__(1024) route_scan_kernel(const int32_t *ids, Layout L, int32_t *ws, uint32_t *err) {
    __shared__ int wsum[scan_lds_ints(7)];
    __shared__ int bad_lds;
    const int E = (int)L.E, t = threadIdx.x;
    const int64_t R = L.nrange();
    if (t == 0) bad_lds = INT_MAX;
    __syncthreads();
    int fb = INT_MAX;
    for (int64_t c = t; c < L.nch; c += blockDim.x) fb = min(fb, ws[L.bad() + c]);
    if (fb != INT_MAX) atomicMin(&bad_lds, fb);
    // the ranges' counts are read 16 at a time (independent loads in flight together)
    constexpr int B = 16;
    int cnt = 0, h0[B];  // h0: the first B ranges' counts, kept for the second pass
    if (t <= E)
        for (int64_t r0 = 0; r0 < R; r0 += B) {
            int h[B];
#pragma unroll
            for (int b = 0; b < B; ++b) h[b] = r0 + b < R ? ws[L.rsum() + (r0 + b) * (E + 1) + t] : 0;
#pragma unroll
            for (int b = 0; b < B; ++b) cnt += h[b];
            if (r0 == 0)
#pragma unroll
                for (int b = 0; b < B; ++b) h0[b] = h[b];
        }
    int v[7], tot[7];
    bucket_scan_values(cnt, v);
    block_scan<7>(v, wsum, tot);
    if (t <= E) {
        int pos_full, pos_part;
        pair_starts(v, tot, pos_full, pos_part, cnt);
        ws[L.offsets() + t] = v[0];
        ws[L.tstart() + t] = v[1];
        ws[L.tstart() + (E + 2) + t] = v[2];
        ws[L.pstart() + t] = pos_full;
        ws[L.pstart() + (E + 2) + t] = pos_part;
        int run = v[0];
        for (int64_t r0 = 0; r0 < R; r0 += B) {
            int h[B];
#pragma unroll
            for (int b = 0; b < B; ++b)
                h[b] = r0 == 0 ? h0[b] : r0 + b < R ? ws[L.rsum() + (r0 + b) * (E + 1) + t] : 0;
#pragma unroll
            for (int b = 0; b < B; ++b)
                if (r0 + b < R) {
                    ws[L.rsum() + (r0 + b) * (E + 1) + t] = run;
                    run += h[b];
                }
        }
    }
    if (t == 0) {
        write_header(ws, L, tot);
        ws[L.tstart() + E + 1] = tot[1];
        ws[L.tstart() + (E + 2) + E + 1] = tot[2];
        ws[L.npairs()] = tot[3] + tot[4] + tot[5] + tot[6];
        report_bad(ids, bad_lds, err);
    }
}

constexpr int kWavesPerBlock = 4;

__global__ void __launch_bounds__(kWavesPerBlock * kWave) route_place_kernel(const int32_t *ids, Layout L, int nbits,
                                                                            int32_t *ws) {
    extern __shared__ int lds[];
    const int E = (int)L.E, wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int64_t ch = (int64_t)blockIdx.x * kWavesPerBlock + wave;
    if (ch >= L.nch) return;
    int *c = lds + wave * (E + 1);
    const int64_t s0 = ch * kChunk, s1 = s0 + kChunk < L.S ? s0 + kChunk : L.S;
    const ChunkIds ci = chunk_ids(ids, s0, s1);  // in flight with the cursors' loads
    const int32_t *gh = ws + L.hist() + ch * (E + 1), *rs = ws + L.rsum() + (ch / kRangeChunks) * (E + 1);
    // the cursors 8 a lane at a time (their loads in flight together)
    for (int b0 = 0; b0 <= E; b0 += 8 * kWave) {
        int g[8], q[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int b = b0 + u * kWave + lane;
            g[u] = b <= E ? gh[b] : 0, q[u] = b <= E ? rs[b] : 0;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (b0 + u * kWave + lane <= E) c[b0 + u * kWave + lane] = g[u] + q[u];
    }
    chunk_place(ci, s0, s1, E, nbits, c, ws + L.slots());
}

// The tile records, after placement, a thread per (16-slot tile, entry) and per 64-slot tile: a tile's bucket is the
// last whose first tile is at or before it (binary search over the buckets' first tiles, staged in LDS; empty buckets
// share their successor's first tile and are passed over). The thread of a bucket's even 64-slot tile 2 q also writes
// pair q's record at its place in the pair order.
__global__ void __launch_bounds__(256) route_tiles_kernel(Layout L, int32_t *ws) {
    extern __shared__ int tl[];  // [3][E + 2]: first 16-slot tiles, first 64-slot tiles, bucket offsets
    const int nb = (int)L.E + 2;
    for (int i = threadIdx.x; i < nb; i += blockDim.x) {
        tl[i] = ws[L.tstart() + i];
        tl[nb + i] = ws[L.tstart() + nb + i];
        tl[2 * nb + i] = ws[L.offsets() + i];
    }
    __syncthreads();
    auto bucket_of_tile = [&](const int *st, int ti) {
        int lo = 0, hi = nb - 1;  // st[lo] <= ti < st[hi]
        while (hi - lo > 1) {
            const int mid = (lo + hi) / 2;
            if (st[mid] <= ti) lo = mid;
            else hi = mid;
        }
        return lo;
    };
    const int n16 = tl[nb - 1], n64 = tl[2 * nb - 1];
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (int64_t)n16 * kTileRows; i += stride) {
        const int ti = (int)(i / kTileRows), jj = (int)(i % kTileRows);
        const int b = bucket_of_tile(tl, ti), r = ti - tl[b];
        const int first = tl[2 * nb + b] + r * kTileRows;
        const int rows = min(kTileRows, tl[2 * nb + b + 1] - first);
        int32_t *rec = ws + L.t16_rec() + kRec16 * ti;
        if (jj == 0) *reinterpret_cast<int4 *>(rec) = make_int4(b, first, rows, 0);
        rec[4 + jj] = jj < rows ? ws[L.slots() + first + jj] : -1;
    }
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n64; i += stride) {
        const int ti = (int)i, b = bucket_of_tile(tl + nb, ti), r = ti - tl[nb + b];
        const int first = tl[2 * nb + b] + r * kWideRows, c = tl[2 * nb + b + 1] - tl[2 * nb + b];
        *reinterpret_cast<int4 *>(ws + L.t64_rec() + 4 * ti) =
            make_int4(b, first, min(kWideRows, tl[2 * nb + b + 1] - first), 0);
        if (r % 2 == 0) {
            const int q = r / 2;
            const int pos = pair_pos(q, c, ws[L.pstart() + b], ws[L.pstart() + nb + b]);
            *reinterpret_cast<int4 *>(ws + L.pair_rec() + 4 * pos) =
                make_int4(b, first, min(kPairRows, c - q * kPairRows), 0);
        }
    }
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
        route_hist_kernel<<<(unsigned)L.nrange(), kRangeChunks * kWave, (size_t)kRangeChunks * (E + 1) * 4, stream>>>(
            ids, L, nbits, w);
        route_scan_kernel<<<1, 1024, 0, stream>>>(ids, L, w, err);
        route_place_kernel<<<blocks, kWavesPerBlock * kWave, lds, stream>>>(ids, L, nbits, w);
        const int64_t tb = (L.T16 * kTileRows + 255) / 256;
        route_tiles_kernel<<<(unsigned)(tb < 4096 ? tb : 4096), 256, (size_t)3 * (E + 2) * 4, stream>>>(L, w);
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
