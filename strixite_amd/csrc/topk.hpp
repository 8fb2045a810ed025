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

// Top-k of row[0, E) (E <= 64 NV). Returns the smallest index of a non-finite logit, or INT_MAX; when none, lanes
// a < k hold the a-th pick (id) and its softmax weight over the k picks (coef).
// A round: the wave max of the lanes' best keys; the lanes holding it (a ballot) - one, or on an exact tie the one
// whose best index is lowest; that lane marks its pick taken and rescans its NV keys (ascending, strict: the lowest
// index among its equal keys).
template <typename T, int NV>
__device__ __forceinline__ int wave_topk(const T *row, int E, int k, int &id, float &coef) {
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
    uint32_t lk = 0;
    int lj = 0;
    auto lane_best = [&]() __attribute__((always_inline)) {
        lk = 0, lj = 0;
#pragma unroll
        for (int j = 0; j < NV; ++j)
            if (key[j] > lk) lk = key[j], lj = j;  // ascending scan, strict >: lower index on ties
    };
    lane_best();
    uint32_t my_k = 0, top = 0;
    id = -1;
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
    const float ex = lane < k ? expf(key_value(my_k) - key_value(top)) : 0.f;
    float sum = ex;
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) sum = sum + __shfl_xor(sum, off, kWave);
    coef = ex / sum;
    return INT_MAX;
}

}  // namespace strix::kernels::topk
