// Packing pieces shared by the routing kernels (route.hip) and the fused decode launches (experts.hip): the
// grouping workspace layout, the wave64 ballot-match histogram / stable placement, the block scan, and the top-k +
// packing body of the one-block small-batch path.
#pragma once

#include "common.hpp"
#include "topk.hpp"

#include <algorithm>
#include <climits>

namespace strix::kernels::route {

constexpr int kWave = 64;
constexpr int kChunk = 256;          // slots per wave chunk
constexpr int kSmallWaves = 16;      // the one-block path: 1024 threads
constexpr int kTileRows = 16;        // slots per tile of the grouped expert kernels
constexpr int kWideRows = 64;        // slots per wide tile (kept for the large-M kernels)
constexpr int kRec16 = 4 + kTileRows; // ints per 16-slot tile record

struct Layout {
    int64_t S, E, T16, T64, nch;
    __host__ __device__ int64_t offsets() const { return 4; }
    __host__ __device__ int64_t slots() const { return offsets() + E + 2; }
    // 16-slot tile records {bucket, first index into slots, rows, 0, slot[16] (-1 past rows)}: everything an
    // expert kernel needs about a tile in independent loads; 64-slot tiles {bucket, first index, rows, 0}
    __host__ __device__ int64_t t16_rec() const { return (slots() + S + 3) / 4 * 4; }
    __host__ __device__ int64_t t64_rec() const { return t16_rec() + kRec16 * T16; }
    // 128-slot pairs (a bucket's 64-slot tiles 2 q and 2 q + 1) {bucket, first index, rows, 0}, the F16 GEMM's blocks,
    // ordered by their 32-slot sub-tiles, most first (full pairs, then the buckets' last pairs by size): the longest
    // blocks start first. At most one pair a 64-slot tile; then the pair count.
    __host__ __device__ int64_t pair_rec() const { return t64_rec() + 4 * T64; }
    __host__ __device__ int64_t npairs() const { return pair_rec() + 4 * T64; }
    // the large-S path: chunk positions within their range of kRangeChunks chunks [nch][E + 1], the ranges' bucket
    // counts and then their first positions [nrange][E + 1], each chunk's first invalid slot [nch]
    __host__ __device__ int64_t hist() const { return npairs() + 1; }
    __host__ __device__ int64_t rsum() const { return hist() + nch * (E + 1); }
    __host__ __device__ int64_t bad() const { return rsum() + nrange() * (E + 1); }
    // each bucket's first 16-slot and 64-slot tile, with the totals at E + 1: [2][E + 2]
    __host__ __device__ int64_t tstart() const { return bad() + nch; }
    // each bucket's first full pair's position and its last (partial) pair's position in the pair order: [2][E + 2]
    __host__ __device__ int64_t pstart() const { return tstart() + 2 * (E + 2); }
    __host__ __device__ int64_t ints() const { return pstart() + 2 * (E + 2); }
    __host__ __device__ int64_t nrange() const { return (nch + kRangeChunks - 1) / kRangeChunks; }
    static constexpr int kRangeChunks = 16;  // chunks a histogram block (a wave each)
};

inline Layout layout(int64_t M, int64_t A, int64_t E) {
    const int64_t S = M * A;
    // sum over buckets of ceil(count / R) <= min(S, S / R + (E + 1)): a tile holds at least one slot
    const int64_t t16 = std::min(S, S / kTileRows + E + 2), t64 = std::min(S, S / kWideRows + E + 2);
    return {S, E, t16, t64, (S + kChunk - 1) / kChunk};
}


__device__ __forceinline__ int bucket_of(int32_t id, int E) { return (id < 0 || id >= E) ? E : id; }

constexpr int kPairRows = 2 * kWideRows;  // slots a pair
// a bucket of c slots: its pairs' counts by 32-slot sub-tiles, n[0] = 4 (the full ones and a last of > 96 slots),
// n[1] = 3, n[2] = 2, n[3] = 1
__host__ __device__ inline void pair_classes(int c, int (&n)[4]) {
    const int rem = c % kPairRows, cls = (rem + 31) / 32;  // the last pair's sub-tiles (0: none)
    n[0] = c / kPairRows + (cls == 4);
    n[1] = cls == 3, n[2] = cls == 2, n[3] = cls == 1;
}
// pair q of a bucket of c slots whose full pairs start at pos_full and whose partial pair sits at pos_part
__host__ __device__ inline int pair_pos(int q, int c, int pos_full, int pos_part) {
    return (q < c / kPairRows || c % kPairRows > 96) ? pos_full + q : pos_part;
}

// Lanes of the wave whose (valid) bucket equals this lane's: a ballot per bucket bit.
__device__ __forceinline__ uint64_t match_bucket(int b, bool valid, int nbits) {
    uint64_t m = __ballot(valid);
    for (int bit = 0; bit < nbits; ++bit) {
        const bool one = (b >> bit) & 1;
        const uint64_t bb = __ballot(one);
        m &= one ? bb : ~bb;
    }
    return m;
}

__device__ __forceinline__ uint64_t lanes_below() { return (1ull << (threadIdx.x % kWave)) - 1ull; }

// A chunk's ids from global memory, all loaded before any is used (one round trip instead of one a 64-slot step).
struct ChunkIds {
    int32_t v[kChunk / kWave];
};
__device__ __forceinline__ ChunkIds chunk_ids(const int32_t *ids, int64_t s0, int64_t s1) {
    const int lane = threadIdx.x % kWave;
    ChunkIds c;
#pragma unroll
    for (int u = 0; u < kChunk / kWave; ++u) {
        const int64_t s = s0 + u * kWave + lane;
        c.v[u] = s < s1 ? ids[s] : 0;
    }
    return c;
}

// Histogram of chunk [s0, s1) into the wave-private counters h[E + 1] (zeroed by the caller); returns the chunk's
// smallest invalid slot (INT_MAX if none) on every lane.
__device__ inline int chunk_hist(const ChunkIds &ci, int64_t s0, int64_t s1, int E, int nbits, int *h) {
    const int lane = threadIdx.x % kWave;
    int first_bad = INT_MAX;
#pragma unroll
    for (int u = 0; u < kChunk / kWave; ++u) {
        const int64_t s = s0 + u * kWave + lane;
        const bool valid = s < s1;
        const int32_t id = ci.v[u];
        const int b = bucket_of(id, E);
        const uint64_t same = match_bucket(b, valid, nbits);
        if (valid && (same & lanes_below()) == 0) h[b] += __popcll(same);
        if (valid && b == E && (int)s < first_bad) first_bad = (int)s;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) first_bad = min(first_bad, __shfl_xor(first_bad, off, kWave));
    return first_bad;
}
// (ids in LDS: a 64-slot step at a time, only the steps the chunk has)
__device__ inline int chunk_hist(const int32_t *ids, int64_t s0, int64_t s1, int E, int nbits, int *h) {
    const int lane = threadIdx.x % kWave;
    int first_bad = INT_MAX;
    for (int64_t base = s0; base < s1; base += kWave) {
        const int64_t s = base + lane;
        const bool valid = s < s1;
        const int32_t id = valid ? ids[s] : 0;
        const int b = bucket_of(id, E);
        const uint64_t same = match_bucket(b, valid, nbits);
        if (valid && (same & lanes_below()) == 0) h[b] += __popcll(same);
        if (valid && b == E && (int)s < first_bad) first_bad = (int)s;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) first_bad = min(first_bad, __shfl_xor(first_bad, off, kWave));
    return first_bad;
}

// Stable placement of chunk [s0, s1) through the wave-private cursors c[E + 1] (each at the bucket's first free
// position for this chunk).
__device__ inline void chunk_place(const ChunkIds &ci, int64_t s0, int64_t s1, int E, int nbits, int *c,
                                   int32_t *slots) {
    const int lane = threadIdx.x % kWave;
#pragma unroll
    for (int u = 0; u < kChunk / kWave; ++u) {
        const int64_t s = s0 + u * kWave + lane;
        const bool valid = s < s1;
        const int32_t id = ci.v[u];
        const int b = bucket_of(id, E);
        const uint64_t same = match_bucket(b, valid, nbits);
        const int rank = __popcll(same & lanes_below());
        int cur = 0;
        if (valid) cur = c[b];
        if (valid) slots[cur + rank] = (int32_t)s;
        if (valid && rank == 0) c[b] = cur + __popcll(same);
    }
}
__device__ inline void chunk_place(const int32_t *ids, int64_t s0, int64_t s1, int E, int nbits, int *c, int32_t *slots) {
    const int lane = threadIdx.x % kWave;
    for (int64_t base = s0; base < s1; base += kWave) {
        const int64_t s = base + lane;
        const bool valid = s < s1;
        const int32_t id = valid ? ids[s] : 0;
        const int b = bucket_of(id, E);
        const uint64_t same = match_bucket(b, valid, nbits);
        const int rank = __popcll(same & lanes_below());
        int cur = 0;
        if (valid) cur = c[b];
        if (valid) slots[cur + rank] = (int32_t)s;
        if (valid && rank == 0) c[b] = cur + __popcll(same);
    }
}

// Inclusive sum over the wave's lanes in lane order: Kogge-Stone inside each 16-lane row (DPP row shifts), then the
// rows' totals carried across by the row broadcasts.
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1 and 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2 and 3
    return v;
}

// Exclusive scan of N ints over the threads of a block (at most 16 waves); totals returned through tot[N]. Each wave
// scans in registers; wave 0 scans the waves' totals; two barriers. wsum: scan_lds_ints(N) ints of LDS.
__host__ __device__ constexpr int scan_lds_ints(int N) { return 33 * N; }
template <int N>
__device__ inline void block_scan(int (&v)[N], int *wsum /* [16][N] totals, [16][N] prefixes, [N] */, int (&tot)[N]) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, nw = (int)(blockDim.x / kWave);
    int inc[N];
#pragma unroll
    for (int j = 0; j < N; ++j) inc[j] = wave_incl_scan(v[j]);
    if (lane == kWave - 1)
#pragma unroll
        for (int j = 0; j < N; ++j) wsum[wave * N + j] = inc[j];
    __syncthreads();
    if (wave == 0) {  // lanes 0..nw-1: the waves' totals, scanned; exclusive prefixes and the totals after them
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int t = lane < nw ? wsum[lane * N + j] : 0;
            const int p = wave_incl_scan(t);
            if (lane < nw) wsum[16 * N + lane * N + j] = p - t;
            if (lane == kWave - 1) wsum[32 * N + j] = p;
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < N; ++j) {
        v[j] = wsum[16 * N + wave * N + j] + inc[j] - v[j];
        tot[j] = wsum[32 * N + j];
    }
}

// The scan's 7 ints of a bucket of c slots (t <= E, else 0): slots, 16-slot tiles, 64-slot tiles, pairs by class
__device__ inline void bucket_scan_values(int c, int (&v)[7]) {
    int n[4];
    pair_classes(c, n);
    v[0] = c, v[1] = (c + kTileRows - 1) / kTileRows, v[2] = (c + kWideRows - 1) / kWideRows;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[3 + j] = n[j];
}
// After the scan: this bucket's full-pair and partial-pair positions (the classes one after another, 4 first)
__device__ inline void pair_starts(const int (&v)[7], const int (&tot)[7], int &pos_full, int &pos_part, int c) {
    int base[4] = {0, tot[3], tot[3] + tot[4], tot[3] + tot[4] + tot[5]};
    int n[4];
    pair_classes(c, n);
    pos_full = base[0] + v[3];
    pos_part = n[1] ? base[1] + v[4] : n[2] ? base[2] + v[5] : n[3] ? base[3] + v[6] : 0;
}

template <int N> __device__ inline void write_header(int32_t *ws, const Layout &L, const int (&tot)[N]) {
    ws[0] = tot[1];
    ws[1] = (int32_t)L.S;
    ws[2] = (int32_t)L.E;
    ws[3] = tot[2];
    ws[L.offsets() + L.E + 1] = tot[0];
}

__device__ inline void report_bad(const int32_t *ids, int first_bad, uint32_t *err) {
    if (first_bad != INT_MAX && atomicCAS(&err[0], 0u, 1u) == 0u) {
        err[1] = (uint32_t)ids[first_bad];
        err[2] = (uint32_t)first_bad;
    }
}

// ---- top-k + packing for small batches (S = M k <= 1024): one 1024-thread block --------------------------------------
// Everything stays in LDS until the last phase, which only stores (ids, coefficients, the workspace tables): a
// barrier after a global store or before a dependent global load costs a memory round trip, and a one-block launch
// is a chain of them otherwise.
// Phase A: TOPK - wave w takes tokens w, w + 16, ...: top-k of the logits into LDS; else the ids are read into LDS.
// B: wave w takes slots [64 w, 64 w + 64): histogram. C: block scan of the bucket counts. D: stable placement.
// E: the stores. The workspace layout and contents are those of moe_group_routes.
constexpr int kFusedSlots = 1024;

// TOPK with shared_slot: each token's slot k is the shared expert (id E_top, coefficient sigmoid(its gate logit at
// column E_top of the logits); a non-finite one is bad index E_top, strixite kernels/moe_router.hip:108-111), and the
// packing runs over L.E = E_top + 1 experts. E: the packing's expert count (L.E).
// PAIRS: also the F16 GEMM's 128-slot pair table (the layer's own decode launches, whose routes no GEMM reads, skip it
// and leave a pair count of 0).
template <int NV, bool TOPK, bool PAIRS = true>
__device__ inline void pack_small_body(const float *logits, int64_t ld, const int32_t *ids_in, int M, int E, int k,
                                       int32_t *ids_out, float *coef_out, Layout L, int nbits, int32_t *ws,
                                       uint32_t *err_router, uint32_t *err_route, int *lds, bool shared_slot = false) {
    const int S = (int)L.S, nb = E + 1, wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, t = threadIdx.x;
    const int Etop = shared_slot ? E - 1 : E, A = k + (shared_slot ? 1 : 0);
    const int nthr = (int)blockDim.x;
    int *sids = lds;                          // [S] ids by slot
    float *scoef = reinterpret_cast<float *>(sids + kFusedSlots);  // [S] coefficients by slot (TOPK)
    int *sl = sids + 2 * kFusedSlots;         // [S] slots by position
    int *cnt = sl + kFusedSlots;              // [16][E + 1] wave counts, then cursors
    int *bstart = cnt + kSmallWaves * nb;     // [E + 1] bucket start
    int *btile = bstart + nb;                 // [E + 1] bucket's first 16-slot tile
    int *bcount = btile + nb;                 // [E + 1]
    int *b64 = bcount + nb;                   // [E + 1] bucket's first 64-slot tile
    int *tile_b = b64 + nb;                   // [T16] bucket of a tile
    int *wsum = tile_b + L.T16;               // [scan_lds_ints(7)]
    int *bad = wsum + scan_lds_ints(7);       // [1]
    // [16][kCandScratch] the waves' top-k candidates (8-byte aligned)
    uint2 *cand = reinterpret_cast<uint2 *>(
        lds + ((3 * kFusedSlots + kSmallWaves * nb + 4 * nb + L.T16 + scan_lds_ints(7) + 1 + 1) & ~1));
    // only the waves that hold slots (chunks of 64) count: their counters are the only ones cleared and summed
    const int nw = (S + kWave - 1) / kWave;
    for (int i = t; i < nw * nb; i += nthr) cnt[i] = 0;
    if (t == 0) *bad = INT_MAX;
    // A
    if constexpr (TOPK) {
        for (int m = wave; m < M; m += kSmallWaves) {
            int id;
            float cf;
            // the shared gate logit is loaded with the row (one memory round trip), checked after the top-k
            const float gl = shared_slot ? logits[(int64_t)m * ld + Etop] : 0.f;
            int rb = topk::wave_topk<float, NV>(logits + (int64_t)m * ld, Etop, k, id, cf,
                                                cand + wave * topk::kCandScratch);
            if (shared_slot && !isfinite(gl) && Etop < rb) rb = Etop;
            if (rb != INT_MAX) {
                if (lane == 0 && atomicCAS(&err_router[0], 0u, 1u) == 0u) {
                    err_router[1] = (uint32_t)m;
                    err_router[2] = (uint32_t)rb;
                }
                id = -1, cf = dev::qnan();
            }
            if (lane < k) sids[m * A + lane] = id, scoef[m * A + lane] = cf;
            if (shared_slot && lane == k)
                sids[m * A + k] = rb != INT_MAX ? -1 : Etop,
                scoef[m * A + k] = rb != INT_MAX ? dev::qnan() : 1.0f / (1.0f + expf(-gl));
        }
    } else {
        for (int i = t; i < S; i += nthr) sids[i] = ids_in[i];
    }
    __syncthreads();
    // B
    const int s0 = wave * kWave, s1 = min(s0 + kWave, S);
    if (s0 < S) {
        const int fb = chunk_hist(sids, s0, s1, E, nbits, cnt + wave * nb);
        if (lane == 0 && fb != INT_MAX) atomicMin(bad, fb);
    }
    __syncthreads();
    // C
    int c = 0;
    if (t <= E)
        for (int w = 0; w < nw; ++w) c += cnt[w * nb + t];
    constexpr int NSC = PAIRS ? 7 : 3;
    int v7[7], v[NSC], tot[NSC];
    bucket_scan_values(c, v7);
#pragma unroll
    for (int i = 0; i < NSC; ++i) v[i] = v7[i];
    block_scan<NSC>(v, wsum, tot);
    int pos_full = 0, pos_part = 0;
    if constexpr (PAIRS) pair_starts(v, tot, pos_full, pos_part, c);
    if (t <= E) {
        bstart[t] = v[0], btile[t] = v[1], bcount[t] = c, b64[t] = v[2];
        for (int i = 0; i < (c + kTileRows - 1) / kTileRows; ++i) tile_b[v[1] + i] = t;
        int run = v[0];
        for (int w = 0; w < nw; ++w) {
            const int x = cnt[w * nb + t];
            cnt[w * nb + t] = run;
            run += x;
        }
    }
    __syncthreads();
    // D
    if (s0 < S) chunk_place(sids, s0, s1, E, nbits, cnt + wave * nb, sl);
    __syncthreads();
    // E: stores only
    if constexpr (TOPK)
        for (int i = t; i < S; i += nthr) ids_out[i] = sids[i], coef_out[i] = scoef[i];
    for (int i = t; i < S; i += nthr) ws[L.slots() + i] = sl[i];
    if (t <= E) {
        ws[L.offsets() + t] = bstart[t];
        const int n64 = (bcount[t] + kWideRows - 1) / kWideRows;
        for (int i = 0; i < n64; ++i)
            *reinterpret_cast<int4 *>(ws + L.t64_rec() + 4 * (b64[t] + i)) =
                make_int4(t, bstart[t] + i * kWideRows, min(kWideRows, bcount[t] - i * kWideRows), 0);
        if constexpr (PAIRS)
            for (int q = 0; q < (bcount[t] + kPairRows - 1) / kPairRows; ++q)
                *reinterpret_cast<int4 *>(ws + L.pair_rec() + 4 * pair_pos(q, bcount[t], pos_full, pos_part)) =
                    make_int4(t, bstart[t] + q * kPairRows, min(kPairRows, bcount[t] - q * kPairRows), 0);
    }
    // 16-slot tile records {bucket, first, rows, 0, slot[16]}: a thread per (tile, slot entry)
    for (int i = t; i < tot[1] * kTileRows; i += nthr) {
        const int ti = i / kTileRows, jj = i % kTileRows, b = tile_b[ti], r = ti - btile[b];
        const int rows = min(kTileRows, bcount[b] - r * kTileRows);
        int32_t *rec = ws + L.t16_rec() + kRec16 * ti;
        if (jj == 0) *reinterpret_cast<int4 *>(rec) = make_int4(b, bstart[b] + r * kTileRows, rows, 0);
        rec[4 + jj] = jj < rows ? sl[bstart[b] + r * kTileRows + jj] : -1;
    }
    if (t == 0) {
        write_header(ws, L, tot);
        if constexpr (PAIRS) ws[L.npairs()] = tot[3] + tot[4] + tot[5] + tot[6];
        else ws[L.npairs()] = 0;
        report_bad(sids, *bad, err_route);  // the ids live in LDS here: report_bad reads them through this pointer
    }
}

template <int NV, bool PAIRS = true>
__device__ inline void topk_route_small_body(const float *logits, int64_t ld, int M, int E, int k, int32_t *ids_out,
                                             float *coef_out, Layout L, int nbits, int32_t *ws, uint32_t *err_router,
                                             uint32_t *err_route, int *lds, bool shared_slot = false) {
    pack_small_body<NV, true, PAIRS>(logits, ld, nullptr, M, E, k, ids_out, coef_out, L, nbits, ws, err_router, err_route,
                              lds, shared_slot);
}

// LDS bytes pack_small_body needs
inline size_t topk_route_small_lds(const Layout &L) {
    const size_t ints = ((size_t)3 * kFusedSlots + (size_t)kSmallWaves * (L.E + 1) + 4 * (size_t)(L.E + 1) +
                         (size_t)L.T16 + scan_lds_ints(7) + 1 + 1) & ~(size_t)1;
    return ints * 4 + (size_t)kSmallWaves * topk::kCandScratch * 8;  // + the top-k candidates
}
// ballot bits a bucket index 0..E takes
inline int bucket_bits(int64_t E) {
    int nbits = 0;
    while ((1ll << nbits) <= E) ++nbits;
    return nbits;
}

}  // namespace strix::kernels::route
