// FP32 activations (Act::F32) for the expert and dense projections: the reference's FP32-activation semantics
// (strixite kernels/linear_q4.hpp:32-41, moe_grouped.hpp:3-16: FP32 x against the Q4 / Q8 codes, per 32-code chunk
// acc = fma(s, sum(x * code), fma(m, sum(x), acc)), FP32 accumulation) for engines that run FP32 activations.
// Included by experts.hip (it uses QV, route::slots_at, the bf16 helpers). The BF16 path keeps its streaming and
// matrix-core kernels; this one is a compatibility path: one wave per output element (a lane per 32-code chunk,
// chunks l, l + 64, ..., then a butterfly), x and weight rows read through L2.
#pragma once

namespace f32a {

enum Mode { DENSE_ROWS = 0, GROUPED_POS = 1, PERSLOT_IDS = 2 };

struct Args {
    const float *x;                       // activation rows [*, K] FP32
    const uint8_t *q;
    const uint16_t *scale, *minv;
    int64_t N, K, G;                      // N: weight rows an expert (DENSE: all)
    int64_t E, A, S;                      // S: output rows (DENSE: M tokens; slots otherwise)
    const int32_t *ws, *ids;              // GROUPED: the grouping workspace; PERSLOT: ids [M, A]
    uint32_t *err;                        // PERSLOT: the expert error word
    void *y;                              // output [S, ldy] in the output dtype
    int64_t ldy;
    int64_t ncol;                         // output columns (SwiGLU: I = N / 2)
};

// the dot of activation row xr with weight row wrow (FP32, the reference's per-chunk form), every lane holding it
template <int BITS>
__device__ __forceinline__ float row_dot(const Args &a, const float *xr, int64_t wrow, int lane) {
    const int64_t nc = a.K / 32, gpr = a.K / a.G;
    float acc = 0.f;
    for (int64_t c = lane; c < nc; c += 64) {
        const uint4 *qp = reinterpret_cast<const uint4 *>(a.q + (wrow * nc + c) * (32 * BITS / 8));
        uint32_t w[BITS];
#pragma unroll
        for (int i = 0; i < BITS / 4; ++i) {
            const uint4 u = qp[i];
            w[4 * i] = u.x, w[4 * i + 1] = u.y, w[4 * i + 2] = u.z, w[4 * i + 3] = u.w;
        }
        const int64_t gi = wrow * gpr + c * 32 / a.G;
        const float s = strix::dev::bf16_to_f32(a.scale[gi]), m = strix::dev::bf16_to_f32(a.minv[gi]);
        const float4 *xp = reinterpret_cast<const float4 *>(xr + c * 32);
        float dot = 0.f, xs = 0.f;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const float4 v = xp[p];
            const float xv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int i = 4 * p + k;
                constexpr int per = 32 / BITS;
                const float code = (float)((w[i / per] >> (BITS * (i % per))) & ((1u << BITS) - 1u));
                dot = fmaf(xv[k], code, dot);
                xs += xv[k];
            }
        }
        acc = fmaf(s, dot, fmaf(m, xs, acc));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    return acc;
}

// the expert of grouped position p: the bucket b with offsets[b] <= p < offsets[b + 1] (offsets at ws + 4)
__device__ __forceinline__ int32_t bucket_of(const int32_t *ws, int64_t E, int64_t p) {
    int64_t lo = 0, hi = E;  // buckets 0 .. E (E: invalid ids)
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) / 2;
        if (ws[4 + mid] <= p) lo = mid;
        else hi = mid - 1;
    }
    return (int32_t)lo;
}

// one wave per (output row r, column j): MODE picks where r's activation row and expert come from; SWI: h = silu(g) u
// from the gate row j and up row ncol + j of the expert
template <int BITS, int MODE, bool SWI, typename TY>
__global__ void __launch_bounds__(256) f32act_kernel(Args a) {
    const int lane = threadIdx.x % 64;
    const int64_t item = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
    if (item >= a.S * a.ncol) return;  // whole wave; no barrier in this kernel
    const int64_t r0 = item / a.ncol, j = item % a.ncol;
    int64_t xrow = r0, orow = r0, expert = 0;
    bool nan = false;
    if constexpr (MODE == GROUPED_POS) {
        const int32_t b = bucket_of(a.ws, a.E, r0);
        const int32_t slot = a.ws[strix::kernels::route::slots_at(a.E) + r0];
        orow = slot, xrow = slot / a.A, expert = b, nan = b >= a.E;
    } else if constexpr (MODE == PERSLOT_IDS) {
        const int32_t id = a.ids[r0];
        nan = id < 0 || id >= a.E;
        expert = nan ? 0 : id, xrow = r0 / a.A;
        if (nan && j == 0 && lane == 0 && atomicCAS(&a.err[0], 0u, 1u) == 0u) {
            a.err[1] = (uint32_t)id;
            a.err[2] = (uint32_t)r0;
        }
    }
    const float *xr = a.x + xrow * a.K;
    float v;
    if constexpr (SWI) {
        const float g = row_dot<BITS>(a, xr, expert * a.N + j, lane);
        const float u = row_dot<BITS>(a, xr, expert * a.N + a.ncol + j, lane);
        v = strix::dev::silu(g) * u;
    } else {
        v = row_dot<BITS>(a, xr, expert * a.N + j, lane);
    }
    if (nan) v = strix::dev::qnan();
    if (lane == 0) {
        TY *y = static_cast<TY *>(a.y) + orow * a.ldy + j;
        if constexpr (std::is_same_v<TY, float>) *y = v;
        else *y = strix::dev::f32_to_bf16(v);
    }
}

// y[m, n] = sum_a coef[m, a] partial[m A + a, n] in slot order (fmaf), FP32; an invalid id of the token: NaN
__global__ void __launch_bounds__(256) f32_combine_kernel(const float *partial, const int32_t *ids, const float *coef,
                                                          int64_t M, int64_t A, int64_t E, int64_t N, float *y) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= M * N) return;
    const int64_t m = i / N, n = i % N;
    float acc = 0.f;
    bool bad = false;
    for (int64_t s = 0; s < A; ++s) {
        const int32_t id = ids[m * A + s];
        bad = bad || id < 0 || id >= E;
        acc = fmaf(coef[m * A + s], partial[(m * A + s) * N + n], acc);
    }
    y[i] = bad ? strix::dev::qnan() : acc;
}

template <int BITS, int MODE, bool SWI, typename TY> void launch(const Args &a, hipStream_t stream) {
    const int64_t blocks = (a.S * a.ncol + 3) / 4;
    STRIX_CHECK(blocks < (1ll << 31), "FP32-activation path: ", a.S, " x ", a.ncol, " outputs, too many");
    f32act_kernel<BITS, MODE, SWI, TY><<<(unsigned)blocks, 256, 0, stream>>>(a);
}

template <int MODE, bool SWI, typename TY> void launch_bits(int bits, const Args &a, hipStream_t stream) {
    if (bits == 4) launch<4, MODE, SWI, TY>(a, stream);
    else launch<8, MODE, SWI, TY>(a, stream);
}

}  // namespace f32a

namespace f32a {
// per-slot combine: y[m, n] = sum_a coef[m, a] (h[m A + a] . W[ids[m, a] N + n]) (fmaf in slot order), FP32; an
// invalid id: NaN and the error word
template <int BITS>
__global__ void __launch_bounds__(256) f32_perslot_combine_kernel(Args a, const float *coef, int64_t M) {
    const int lane = threadIdx.x % 64;
    const int64_t item = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
    if (item >= M * a.ncol) return;  // whole wave; no barrier in this kernel
    const int64_t m = item / a.ncol, n = item % a.ncol;
    float acc = 0.f;
    bool bad = false;
    for (int64_t s = 0; s < a.A; ++s) {
        const int32_t id = a.ids[m * a.A + s];
        const bool nan = id < 0 || id >= a.E;
        if (nan && n == 0 && lane == 0 && atomicCAS(&a.err[0], 0u, 1u) == 0u) {
            a.err[1] = (uint32_t)id;
            a.err[2] = (uint32_t)(m * a.A + s);
        }
        bad = bad || nan;
        const float d = row_dot<BITS>(a, a.x + (m * a.A + s) * a.K, (nan ? 0 : id) * a.N + n, lane);
        acc = fmaf(coef[m * a.A + s], d, acc);
    }
    if (lane == 0) static_cast<float *>(a.y)[m * a.ldy + n] = bad ? strix::dev::qnan() : acc;
}
}  // namespace f32a
