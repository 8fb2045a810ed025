// Wave64 top-k over one row of router logits (strixite kernels/moe_router.hip:36-84 semantics: softmax over the k
// selected logits, ties to the lower expert index), shared by the standalone top-k kernel and the fused small-batch
// top-k + packing kernel.
//
// A round is one wave max over order-preserving integer keys: four DPP max steps leave every lane with its 16-lane
// row's maximum (quad swaps, then the half-row and row mirrors), and the four row maxima meet through readlane; a
// ballot names the lane that holds it. No LDS round trips and no value/index pair compares.
#pragma once

#include "common.hpp"

#include <climits>

namespace strix::kernels::topk {

constexpr int kWave = 64;

template <typename T> __device__ __forceinline__ float load_logit(const T *p, int64_t i);
template <> __device__ __forceinline__ float load_logit<float>(const float *p, int64_t i) { return p[i]; }
template <> __device__ __forceinline__ float load_logit<uint16_t>(const uint16_t *p, int64_t i) {
    return dev::bf16_to_f32(p[i]);
}

// Order-preserving key of a finite float: larger value <-> larger unsigned key; -0 and +0 share a key (they compare
// equal, so they tie and the lower index wins); 0 is below every finite value's key and marks a taken expert or the
// padding past E.
__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t b = f == 0.0f ? 0u : __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : b | 0x80000000u;
}
__device__ __forceinline__ float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? k & 0x7fffffffu : ~k);
}

// every lane gets the wave's largest (MIN: smallest) unsigned value: four DPP steps leave each 16-lane row's result in
// all of its lanes, two row broadcasts carry it to lane 63 (rows 1 and 3 take lane 15 of the row before, then rows 2
// and 3 take lane 31), one readlane
template <bool MIN> __device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v) {
    auto op = [](uint32_t a, uint32_t b) __attribute__((always_inline)) { return MIN ? (a < b ? a : b) : (a > b ? a : b); };
    v = op(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true));   // quad_perm [1, 0, 3, 2]
    v = op(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true));   // quad_perm [2, 3, 0, 1]
    v = op(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, true));  // row_half_mirror
    v = op(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, true));  // row_mirror
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xA, 0xF, false));  // row_bcast:15
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xC, 0xF, false));  // row_bcast:31
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Inclusive sum over the wave's lanes in lane order: Kogge-Stone inside each 16-lane row (DPP row shifts), then the
// rows' totals carried across by the row broadcasts.
__device__ __forceinline__ int wave_incl_sum(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1 and 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2 and 3
    return v;
}

// The sum of the 64 lanes' values in the butterfly order (lane i adds lane i ^ 1, then i ^ 2, ... i ^ 32; every lane
// ends with the same bits), through DPP: after the xor-1 and xor-2 steps (quad permutes) a quad holds one value, so
// the half-row and row mirrors pair the same operands as xor 4 and xor 8 (the float add commutes), and the four
// rows' sums meet as (r0 + r1) + (r2 + r3), which is what xor 16 then xor 32 compute.
__device__ __forceinline__ float wave_butterfly_sum(float v) {
#define STRIX_DPP_F(x, ctrl) __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), ctrl, 0xF, 0xF, true))
    v = v + STRIX_DPP_F(v, 0xB1);   // quad_perm [1, 0, 3, 2]: xor 1
    v = v + STRIX_DPP_F(v, 0x4E);   // quad_perm [2, 3, 0, 1]: xor 2
    v = v + STRIX_DPP_F(v, 0x141);  // row_half_mirror: the other quad of the 8
    v = v + STRIX_DPP_F(v, 0x140);  // row_mirror: the other 8 of the row
#undef STRIX_DPP_F
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// LDS a wave's candidate top-k needs (uint2 entries): the candidates, then the k picks
constexpr int kCandScratch = kWave + kWave;

// The k largest of the wave's keys (key[j] of lane l is expert l + 64 j; 0 = not eligible), larger key first, on an
// exact tie the lower expert index: lane r < k ends with the r-th pick's expert (id) and key (my_k), every lane with
// the first pick's key (top). key is clobbered. With scratch (kCandScratch uint2 of LDS for this wave): the
// candidates are the keys >= T, T the k-th largest of the 64 lanes' maxima (the k lanes holding those maxima hold k
// keys >= T, so no key below T is among the top k); a 32-step bitwise search with ballot counts finds T, the
// candidates (usually k to k + a few) are packed into LDS by a wave prefix sum and ranked exactly across lanes, and
// pick r goes to lane r. More than 64 candidates (many equal keys), or no scratch: k rounds, each the wave max of the
// lanes' best keys, its holder (the lowest index on an exact tie) marking it taken and rescanning its NV keys. Both
// give the same picks.
template <int NV>
__device__ __forceinline__ void wave_picks(uint32_t (&key)[NV], int k, uint2 *scratch, int &id, uint32_t &my_k,
                                           uint32_t &top) {
    const int lane = threadIdx.x % kWave;
    my_k = 0, top = 0;
    id = -1;
    bool done = false;
    if (scratch != nullptr) {
        uint32_t lmax = 0;
#pragma unroll
        for (int j = 0; j < NV; ++j) lmax = key[j] > lmax ? key[j] : lmax;
        // T, bit by bit from the top: the largest t with at least k lanes' maxima >= t (one compare and a ballot
        // count a bit)
        uint32_t thr = 0;
        for (int b = 31; b >= 0; --b) {
            const uint32_t t = thr | (1u << b);
            if (__popcll(__ballot(lmax >= t)) >= k) thr = t;
        }
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < NV; ++j) cnt += key[j] >= thr && key[j] != 0u;
        const int incl = wave_incl_sum(cnt);
        const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
        if (total <= kWave && total >= k) {
            int pos = incl - cnt;
#pragma unroll
            for (int j = 0; j < NV; ++j)
                if (key[j] >= thr && key[j] != 0u) scratch[pos++] = make_uint2(key[j], (uint32_t)(lane + j * kWave));
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // lane i ranks candidate i against all of them (read across lanes, no LDS round trip a candidate):
            // (key desc, index asc); ranks are distinct
            const uint2 c = lane < total ? scratch[lane] : make_uint2(0u, 0u);
            int rank = 0;
            for (int jj = 0; jj < total; ++jj) {
                const uint32_t ox = (uint32_t)__builtin_amdgcn_readlane((int)c.x, jj);
                const uint32_t oy = (uint32_t)__builtin_amdgcn_readlane((int)c.y, jj);
                rank += ox > c.x || (ox == c.x && oy < c.y);
            }
            if (lane < total && rank < k) scratch[kWave + rank] = c;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (lane < k) {
                const uint2 pk = scratch[kWave + lane];
                my_k = pk.x, id = (int)pk.y;
            }
            top = (uint32_t)__builtin_amdgcn_readlane((int)my_k, 0);
            done = true;
        }
    }
    if (!done) {
        uint32_t lk = 0;
        int lj = 0;
        auto lane_best = [&]() __attribute__((always_inline)) {
            lk = 0, lj = 0;
#pragma unroll
            for (int j = 0; j < NV; ++j)
                if (key[j] > lk) lk = key[j], lj = j;  // ascending scan, strict >: lower index on ties
        };
        lane_best();
        for (int r = 0; r < k; ++r) {
            const uint32_t best = wave_reduce_u32<false>(lk);
            const uint64_t holders = __ballot(lk == best);
            int win;
            if ((holders & (holders - 1)) == 0) {
                win = __builtin_ctzll(holders);
            } else {  // several lanes hold the best value: the lowest expert index wins
                const uint32_t mine = lk == best ? (uint32_t)(lane + lj * kWave) : 0xffffffffu;
                win = (int)(wave_reduce_u32<true>(mine) % kWave);
            }
            const int wj = __builtin_amdgcn_readlane(lj, win);
            if (r == 0) top = best;
            if (lane == r) my_k = best, id = win + wj * kWave;
            if (lane == win) {
#pragma unroll
                for (int j = 0; j < NV; ++j)
                    if (j == wj) key[j] = 0u;
                lane_best();
            }
        }
    }
}

// Top-k of row[0, E) (E <= 64 NV). Returns the smallest index of a non-finite logit, or INT_MAX; when none, lanes
// a < k hold the a-th pick (id) and its softmax weight over the k picks (coef). Order: larger logit first, on an exact
// tie the lower expert index (wave_picks; scratch as there).
template <typename T, int NV>
__device__ __forceinline__ int wave_topk(const T *row, int E, int k, int &id, float &coef, uint2 *scratch = nullptr) {
    const int lane = threadIdx.x % kWave;
    uint32_t key[NV];
    bool fin = true;
    int bad = INT_MAX;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e = lane + j * kWave;
        const float xv = e < E ? load_logit(row, e) : 0.0f;
        const bool f = isfinite(xv);
        if (e < E && !f && e < bad) bad = e;
        fin = fin && f;
        key[j] = e < E && f ? order_key(xv) : 0u;
    }
    if (__ballot(!fin) != 0) {  // rare: the smallest bad index
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1) bad = min(bad, __shfl_xor(bad, off, kWave));
        return bad;
    }
    uint32_t my_k, top;
    wave_picks<NV>(key, k, scratch, id, my_k, top);
    const float ex = lane < k ? expf(key_value(my_k) - key_value(top)) : 0.f;
    coef = ex / wave_butterfly_sum(ex);
    return INT_MAX;
}

}  // namespace strix::kernels::topk
