// Wave64 top-k over one row of router logits (strixite kernels/moe_router.hip:36-84 semantics: softmax over the k
// selected logits, ties to the lower expert index), shared by the standalone top-k kernel and the fused small-batch
// top-k + packing kernel.
//
// A round is one wave argmax of (value, index): four DPP steps leave every lane with its 16-lane row's winner
// (quad swaps, then the half-row and row mirrors), and the four row winners meet through readlane. No LDS round trips,
// so k rounds cost a few hundred cycles each instead of the microseconds of a shuffle butterfly.
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

__device__ __forceinline__ bool better(float ov, int oi, float v, int i) { return ov > v || (ov == v && oi < i); }

template <int CTRL> __device__ __forceinline__ void dpp_step(float &v, int &i) {
    const float ov = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
    const int oi = __builtin_amdgcn_update_dpp(0, i, CTRL, 0xF, 0xF, false);
    if (better(ov, oi, v, i)) v = ov, i = oi;
}

// every lane gets the wave's best (value, index)
__device__ __forceinline__ void wave_argmax(float &v, int &i) {
    dpp_step<0xB1>(v, i);   // quad_perm [1, 0, 3, 2]
    dpp_step<0x4E>(v, i);   // quad_perm [2, 3, 0, 1]
    dpp_step<0x141>(v, i);  // row_half_mirror
    dpp_step<0x140>(v, i);  // row_mirror
    float bv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
    for (int r = 1; r < 4; ++r) {
        const float ov = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16 * r));
        const int oi = __builtin_amdgcn_readlane(i, 16 * r);
        if (better(ov, oi, bv, bi)) bv = ov, bi = oi;
    }
    v = bv, i = bi;
}

// Top-k of row[0, E) (E <= 64 NV). Returns the smallest index of a non-finite logit, or INT_MAX; when none, lanes
// a < k hold the a-th pick (id) and its softmax weight over the k picks (coef).
template <typename T, int NV>
__device__ __forceinline__ int wave_topk(const T *row, int E, int k, int &id, float &coef) {
    const int lane = threadIdx.x % kWave;
    float v[NV];
    int bad = INT_MAX;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e = lane + j * kWave;
        const float xv = e < E ? load_logit(row, e) : -INFINITY;
        v[j] = xv;
        if (e < E && !isfinite(xv) && e < bad) bad = e;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) bad = min(bad, __shfl_xor(bad, off, kWave));
    if (bad != INT_MAX) return bad;
    // finite from here: -inf marks a taken expert and the padding past E
    float lv = -INFINITY;
    int li = INT_MAX;
    auto lane_best = [&]() __attribute__((always_inline)) {
        lv = -INFINITY, li = INT_MAX;
#pragma unroll
        for (int j = 0; j < NV; ++j)
            if (v[j] > lv) lv = v[j], li = lane + j * kWave;  // ascending scan, strict >: lower index on ties
    };
    lane_best();
    float my_v = -INFINITY, top = 0.f;
    id = -1;
    for (int r = 0; r < k; ++r) {
        float bv = lv;
        int bi = li;
        wave_argmax(bv, bi);
        if (r == 0) top = bv;
        if (lane == r) my_v = bv, id = bi;
        if (bi == li) {  // the pick is this lane's best (an index lives in one lane only)
#pragma unroll
            for (int j = 0; j < NV; ++j)
                if (lane + j * kWave == bi) v[j] = -INFINITY;
            lane_best();
        }
    }
    const float ex = lane < k ? expf(my_v - top) : 0.f;
    float sum = ex;
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) sum = sum + __shfl_xor(sum, off, kWave);
    coef = ex / sum;
    return INT_MAX;
}

}  // namespace strix::kernels::topk
