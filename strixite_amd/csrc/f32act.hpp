// The compatibility path of the expert and dense projections: FP32 activations (Act::F32) with Q4 / Q8 weights, and
// the Q5 experts (strixite formats/q5.hpp) with either activation dtype. The reference's semantics (strixite
// kernels/linear_q4.hpp:32-41, moe_grouped.hpp:3-16: x against the exact codes, per 32-code chunk
// acc = fma(s, sum(x * code), fma(m, sum(x), acc)), FP32 accumulation). Included by experts.hip (it uses QV,
// route::slots_at, the bf16 helpers). The BF16 Q4 / Q8 path keeps its streaming and matrix-core kernels; this one is
// one wave per output element (a lane per 32-code chunk, chunks l, l + 64, ..., then a butterfly), x and weight rows
// read through L2. FMT: 4, 8 (one plane, row-major) or 5 (per row a low plane [K/2] of 4-bit codes and a high plane
// [K/8] of bit 4, code k at bit k % 8 of byte k / 8).
#pragma once

namespace f32a {

enum Mode { DENSE_ROWS = 0, GROUPED_POS = 1, PERSLOT_IDS = 2 };

struct Args {
    const void *x;                        // activation rows [*, K] (FP32 or BF16)
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

// 8 activations of a chunk (FP32 or BF16 bits) at element offset i
__device__ __forceinline__ void ld8x(const float *p, int64_t i, float (&v)[8]) {
    const float4 a = *reinterpret_cast<const float4 *>(p + i), b = *reinterpret_cast<const float4 *>(p + i + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}
__device__ __forceinline__ void ld8x(const uint16_t *p, int64_t i, float (&v)[8]) {
    const uint4 u = *reinterpret_cast<const uint4 *>(p + i);
    const uint32_t d[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) v[2 * k] = __uint_as_float(d[k] << 16), v[2 * k + 1] = __uint_as_float(d[k] & 0xffff0000u);
}

// the 32 codes of chunk c of weight row wrow: code i = (w[i / per] >> (BITS (i % per))) & mask (FMT 4, 8), or the low
// nibble of lo[] with bit i of hi (FMT 5)
template <int FMT> struct ChunkCodes {
    static constexpr int W = FMT == 5 ? 4 : FMT;
    uint32_t w[W], hi = 0;
    __device__ __forceinline__ void load(const uint8_t *q, int64_t K, int64_t wrow, int64_t c) {
        const uint8_t *p = FMT == 5 ? q + wrow * (K / 2 + K / 8) + c * 16 : q + (wrow * (K / 32) + c) * (4 * FMT);
#pragma unroll
        for (int i = 0; i < W / 4; ++i) {
            const uint4 u = reinterpret_cast<const uint4 *>(p)[i];
            w[4 * i] = u.x, w[4 * i + 1] = u.y, w[4 * i + 2] = u.z, w[4 * i + 3] = u.w;
        }
        if constexpr (FMT == 5) hi = *reinterpret_cast<const uint32_t *>(q + wrow * (K / 2 + K / 8) + K / 2 + c * 4);
    }
    __device__ __forceinline__ float code(int i) const {
        if constexpr (FMT == 5) return (float)(((w[i / 8] >> (4 * (i % 8))) & 0xFu) | (((hi >> i) & 1u) << 4));
        else {
            constexpr int per = 32 / FMT;
            return (float)((w[i / per] >> (FMT * (i % per))) & ((1u << FMT) - 1u));
        }
    }
};

// the dot of activation row xr with weight row wrow (FP32, the reference's per-chunk form), every lane holding it
template <int BITS, typename TX>
__device__ __forceinline__ float row_dot(const Args &a, const TX *xr, int64_t wrow, int lane) {
    const int64_t nc = a.K / 32, gpr = a.K / a.G;
    float acc = 0.f;
    for (int64_t c = lane; c < nc; c += 64) {
        ChunkCodes<BITS> cc;
        cc.load(a.q, a.K, wrow, c);
        const int64_t gi = wrow * gpr + c * 32 / a.G;
        const float s = strix::dev::bf16_to_f32(a.scale[gi]), m = strix::dev::bf16_to_f32(a.minv[gi]);
        float dot = 0.f, xs = 0.f;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            float xv[8];
            ld8x(xr, c * 32 + 8 * p, xv);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                dot = fmaf(xv[k], cc.code(8 * p + k), dot);
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
template <int BITS, int MODE, bool SWI, typename TY, typename TX>
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
    const TX *xr = static_cast<const TX *>(a.x) + xrow * a.K;
    float v;
    if constexpr (SWI) {
        const float g = row_dot<BITS, TX>(a, xr, expert * a.N + j, lane);
        const float u = row_dot<BITS, TX>(a, xr, expert * a.N + a.ncol + j, lane);
        v = strix::dev::silu(g) * u;
    } else {
        v = row_dot<BITS, TX>(a, xr, expert * a.N + j, lane);
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

template <int BITS, int MODE, bool SWI, typename TY, typename TX> void launch(const Args &a, hipStream_t stream) {
    const int64_t blocks = (a.S * a.ncol + 3) / 4;
    STRIX_CHECK(blocks < (1ll << 31), "compatibility projection path: ", a.S, " x ", a.ncol, " outputs, too many");
    f32act_kernel<BITS, MODE, SWI, TY, TX><<<(unsigned)blocks, 256, 0, stream>>>(a);
}

// TX: the activations' type (float: FP32, uint16_t: BF16 bits)
template <int MODE, bool SWI, typename TY, typename TX = float>
void launch_bits(int bits, const Args &a, hipStream_t stream) {
    if (bits == 4) launch<4, MODE, SWI, TY, TX>(a, stream);
    else if (bits == 5) launch<5, MODE, SWI, TY, TX>(a, stream);
    else launch<8, MODE, SWI, TY, TX>(a, stream);
}

}  // namespace f32a

namespace f32a {
// per-slot combine: y[m, n] = sum_a coef[m, a] (h[m A + a] . W[ids[m, a] N + n]) (fmaf in slot order), FP32; an
// invalid id: NaN and the error word
template <int BITS, typename TY, typename TX>
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
        const float d = row_dot<BITS, TX>(a, static_cast<const TX *>(a.x) + (m * a.A + s) * a.K, (nan ? 0 : id) * a.N + n,
                                          lane);
        acc = fmaf(coef[m * a.A + s], d, acc);
    }
    if (lane == 0) {
        const float v = bad ? strix::dev::qnan() : acc;
        if constexpr (std::is_same_v<TY, float>) static_cast<float *>(a.y)[m * a.ldy + n] = v;
        else static_cast<TY *>(a.y)[m * a.ldy + n] = strix::dev::f32_to_bf16(v);
    }
}
}  // namespace f32a
