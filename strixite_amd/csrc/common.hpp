// Shared host + device pieces of the gfx950 MoE library: precondition errors, HIP launch checks, bf16 / f16 bit
// helpers, and the wave64 MFMA operand decoders for the Q4 / Q8 block layout.
#pragma once

#include "strixite_moe.hpp"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <sstream>
#include <string>

namespace strix {

// Internal entry (route.hip), used by the layer forward for small batches: top-k of FP32 logits (shared_slot: plus
// the shared expert as slot k, id E, its gate logit at column E) and the packing of moe_group_routes (over E + 1
// experts with the shared slot) in one launch, M A <= 1024.
namespace kernels {
// "F32" / "BF16" for messages (strixite's act_name lives in its kernels/norm.hip; this library does not export one)
const char *act_str(Act a);
void moe_topk_group_routes_small(const float *logits, int64_t ld, int64_t M, int64_t E, int64_t k, int32_t *ids,
                                 float *coef, void *ws, size_t ws_bytes, uint32_t *err_router, uint32_t *err_route,
                                 hipStream_t stream, bool shared_slot = false);
// Internal entry (router_prefill.hip), used by the layer forward for prefill-size batches: router projection (+ the
// optional FP32 bias) and top-k with the canonical order's exact routing via bf16 MFMA plus exact recomputation of the
// candidates. logits: [4][M][E (+1)] floats (the layer's logits are part 0); norms: 4 (M + E (+1)) floats of
// scratch. shared_slot (with shared): the shared expert routed as slot k of every token (id E, coefficient
// sigmoid(its gate logit)): ids / coef [M, k + 1]. x16 (optional): x [M, H] also written as F16 (toward zero) in the
// paired k order of every 8 elements, the prefill expert GEMM's input. Returns false (nothing launched) for shapes it
// does not take.
bool moe_router_prefill(const void *x, const uint16_t *w, const float *bias, int64_t M, int64_t H, int64_t E,
                        int64_t k, bool shared, float *logits, float *norms, int32_t *ids, float *coef, uint32_t *err,
                        hipStream_t stream, bool shared_slot = false, void *x16 = nullptr);
// The same in its two passes, so a caller can start other work between them: the approximate projection (false,
// nothing launched, for shapes it does not take) and the selection (after a successful approximate pass only).
bool moe_router_prefill_approx(const void *x, const uint16_t *w, int64_t M, int64_t H, int64_t E, int64_t k,
                               bool shared, float *logits, float *norms, hipStream_t stream);
void moe_router_prefill_select(const void *x, const uint16_t *w, const float *bias, int64_t M, int64_t H, int64_t E,
                               int64_t k, bool shared, float *logits, float *norms, int32_t *ids, float *coef,
                               uint32_t *err, hipStream_t stream, bool shared_slot = false, void *x16 = nullptr);
}  // namespace kernels

// ---- host-side checks -----------------------------------------------------------------------------------------
// A failed precondition throws strix::Error carrying "fn (file:line): check `cond` failed: message", the form of
// strixite common/check.hpp:59-79.
namespace detail {
template <typename... Ts> std::string cat(const Ts &...xs) {
    std::ostringstream os;
    (os << ... << xs);
    return os.str();
}
}  // namespace detail

#define STRIX_CHECK(cond, ...)                                                                                        \
    do {                                                                                                              \
        if (!(cond))                                                                                                  \
            throw ::strix::Error(::strix::detail::cat(__func__, " (", __FILE__, ":", __LINE__, "): check `", #cond, \
                                                      "` failed: ", __VA_ARGS__));                                    \
    } while (0)

#define STRIX_HIP_CHECK(expr, ...)                                                                                   \
    do {                                                                                                             \
        const hipError_t e_ = (expr);                                                                                \
        if (e_ != hipSuccess)                                                                                        \
            throw ::strix::GpuFatalError(::strix::detail::cat(__func__, ": ", #expr, " -> ", hipGetErrorString(e_), " ", \
                                                         __VA_ARGS__));                                             \
    } while (0)

// After every launch: a bad configuration shows up here; a fault shows up at the next synchronizing call.
#define STRIX_HIP_CHECK_LAUNCH(...) STRIX_HIP_CHECK(hipGetLastError(), "launching ", __VA_ARGS__)

inline bool disjoint(const void *a, int64_t an, const void *b, int64_t bn) {
    const auto x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x + (uintptr_t)an <= y || y + (uintptr_t)bn <= x;
}

// ---- device bit helpers ---------------------------------------------------------------------------------------
namespace dev {

typedef float float4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
// RNE, NaN kept quiet (strixite common/bf16.hpp:19-26): gfx950's v_cvt_pk_bf16_f32, which gives the bits of the
// integer form (u + 0x7fff + lsb) >> 16 for every finite or infinite input and the quieted top half of a NaN (checked
// on the device against that form through strix_calib_bf16_round), in one instruction for two values.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
typedef float float2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
// two values in one dword (a low, b high)
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((float2v{a, b}), bf16x2v));
}
__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }
__device__ __forceinline__ float qnan() { return __uint_as_float(0x7fc00000u); }


// ---- MFMA operand decoders ------------------------------------------------------------------------------------
// The expert kernels use v_mfma_f32_16x16x32_bf16 with A = activations (16 token rows) and B = weights (16 weight
// rows as columns): a lane supplies 8 bf16 of a token row and 8 of a weight row for the same 8 k positions. Which
// 8 k a lane's slots stand for is chosen identically for A and B, so the product is the plain dot product.
//
// Weights enter as their exact integer codes ("scaled codes"): D = sum_k code_k * x_k over one quantization group,
// then w . x = s * D + m * sum_k x_k on the FP32 accumulator (code * s + m per formats/q4.hpp:3-6). Nothing is
// rounded on the weight side; activations stay bf16 (full range).
//
// Q4: the bf16 bits 0x4300 | n are exactly 128 + n (n < 16), so a byte shuffle with the constant 0x43 turns a
// masked dword into bf16 pairs; the offset is folded into the min: m' = m - 128 s. Two more shuffles interleave the
// even (low) and odd (high) nibbles first, so the 8 codes of a dword come out in natural k order.
// Q8: codes 0..255 are exact in bf16 (8 significant bits): byte -> f32 (v_cvt_f32_ubyte) -> high half; natural order.

typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

struct Frag {  // 8 bf16 as 4 dwords
    uint32_t d[4];
};
__device__ __forceinline__ bf16x8v as_bf16x8(const Frag &f) { return __builtin_bit_cast(bf16x8v, f); }

__device__ __forceinline__ Frag q4_codes_to_bf16(uint32_t w) {
    const uint32_t t = w & 0x0F0F0F0Fu, u = (w >> 4) & 0x0F0F0F0Fu, c = 0x43434343u;
    // perm(S0, S1, sel): selector bytes 0..3 pick S1's bytes, 4..7 S0's. t holds the even k of the 4 bytes, u the odd:
    // interleave them to k0..k3 and k4..k7, then widen each code byte n to the bf16 0x43nn = 128 + n
    const uint32_t m0 = __builtin_amdgcn_perm(u, t, 0x05010400u), m1 = __builtin_amdgcn_perm(u, t, 0x07030602u);
    return Frag{{__builtin_amdgcn_perm(c, m0, 0x04010400u), __builtin_amdgcn_perm(c, m0, 0x04030402u),
                 __builtin_amdgcn_perm(c, m1, 0x04010400u), __builtin_amdgcn_perm(c, m1, 0x04030402u)}};
}

__device__ __forceinline__ uint32_t hi16_pair(float a, float b) {
    return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
}
// Q8: two dwords = codes k0..k7 -> bf16 in natural order
__device__ __forceinline__ Frag q8_codes_to_bf16(uint32_t lo, uint32_t hi) {
    return Frag{{hi16_pair((float)(lo & 0xFF), (float)((lo >> 8) & 0xFF)),
                 hi16_pair((float)((lo >> 16) & 0xFF), (float)(lo >> 24)),
                 hi16_pair((float)(hi & 0xFF), (float)((hi >> 8) & 0xFF)),
                 hi16_pair((float)((hi >> 16) & 0xFF), (float)(hi >> 24))}};
}

// sum of the 8 bf16 activations of a fragment, FP32 (v_dot2_f32_bf16 against (1, 1))
__device__ __forceinline__ float frag_sum(const uint4 &v, float acc) {
    const bf16x2v one = __builtin_bit_cast(bf16x2v, 0x3F803F80u);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, v.x), one, acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, v.y), one, acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, v.z), one, acc, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, v.w), one, acc, false);
}

__device__ __forceinline__ float4v mfma_bf16(const Frag &a, const Frag &b, float4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }  // strixite kernels/swiglu.hip:22

}  // namespace dev
}  // namespace strix
