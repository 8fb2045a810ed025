// Shared host + device pieces of the gfx950 MoE library: precondition errors, HIP launch checks, bf16 / f16 bit
// helpers, the weight views the launchers take, and the wave64 MFMA operand decoders for the Q4 / Q8 block layout.
#pragma once

#include "strixite_moe.hpp"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <sstream>
#include <string>

namespace strix {

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
            throw ::strix::GpuError(::strix::detail::cat(__func__, ": ", #expr, " -> ", hipGetErrorString(e_), " ", \
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

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
// RNE, NaN kept quiet (strixite common/bf16.hpp:19-26).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0x007fffffu) ? 0x0040u : 0u));
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }
__device__ __forceinline__ float qnan() { return __uint_as_float(0x7fc00000u); }

__device__ __forceinline__ half2v as_h2(uint32_t u) { return __builtin_bit_cast(half2v, u); }
__device__ __forceinline__ uint32_t h2_bits(half2v h) { return __builtin_bit_cast(uint32_t, h); }

// A bf16 scale or min as a splatted f16 pair (exact for values in f16's normal range).
__device__ __forceinline__ half2v bf16_splat_h2(uint16_t b) {
    const _Float16 h = (_Float16)bf16_to_f32(b);
    return half2v{h, h};
}

// ---- MFMA operand decoders ------------------------------------------------------------------------------------
// Every MFMA here is v_mfma_f32_16x16x32_f16: a lane supplies 8 f16 of an A row and 8 of a B column for the same
// 8 k positions. Which 8 k a lane's slots stand for is this file's choice, made identically for A (weights) and B
// (activations), so the product is the plain dot product. For 8 consecutive codes k0..k7 the slot order is
//   [k0, k4, k1, k5, k2, k6, k3, k7]
// - the order in which a Q4 dword's nibbles fall out of (w >> 4j) & 0x000F000F without any byte shuffling.
//
// Dequantization: w = f16(code * s + m), one rounding (strixite kernels/wmma_gemm.hpp:120-141 uses the same
// one-rounding F16 form). code -> f16 by the exponent trick: the f16 bits 0x6400 | c are 1024 + c exactly for
// c < 1024, so subtracting 1024 is exact; then one packed fma with (s, m).

__device__ __forceinline__ half2v dq_pair(uint32_t bits_1024, half2v s, half2v m) {
    const half2v c = as_h2(bits_1024) - half2v{(_Float16)1024.0f, (_Float16)1024.0f};
    return __builtin_elementwise_fma(c, s, m);
}

// Q4: one dword = codes k0..k7 (low nibble = even k, formats/q4.hpp:4) -> A slots [k0,k4,k1,k5,k2,k6,k3,k7].
__device__ __forceinline__ half8v dq4_dword(uint32_t w, half2v s, half2v m) {
    const half2v p0 = dq_pair((w & 0x000F000Fu) | 0x64006400u, s, m);
    const half2v p1 = dq_pair(((w >> 4) & 0x000F000Fu) | 0x64006400u, s, m);
    const half2v p2 = dq_pair(((w >> 8) & 0x000F000Fu) | 0x64006400u, s, m);
    const half2v p3 = dq_pair(((w >> 12) & 0x000F000Fu) | 0x64006400u, s, m);
    return half8v{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// Q8: two dwords = codes k0..k3, k4..k7 (one byte each) -> the same slot order, bytes paired by v_perm_b32.
__device__ __forceinline__ half8v dq8_dwords(uint32_t lo, uint32_t hi, half2v s, half2v m) {
    // perm(S0 = hi, S1 = lo, sel): byte selector 0..3 picks lo's bytes, 4..7 hi's, 0x0C gives 0x00.
    const half2v p0 = dq_pair(__builtin_amdgcn_perm(hi, lo, 0x0C040C00u) | 0x64006400u, s, m);
    const half2v p1 = dq_pair(__builtin_amdgcn_perm(hi, lo, 0x0C050C01u) | 0x64006400u, s, m);
    const half2v p2 = dq_pair(__builtin_amdgcn_perm(hi, lo, 0x0C060C02u) | 0x64006400u, s, m);
    const half2v p3 = dq_pair(__builtin_amdgcn_perm(hi, lo, 0x0C070C03u) | 0x64006400u, s, m);
    return half8v{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// B operand: 8 consecutive bf16 activations (16 bytes) -> f16 in the slot order above. bf16 -> f16 rounds toward
// zero (v_cvt_pkrtz): exact for values in f16's normal range, which the activations must lie in.
__device__ __forceinline__ half2v pkrtz(float a, float b) {
    return __builtin_bit_cast(half2v, __builtin_amdgcn_cvt_pkrtz(a, b));
}
__device__ __forceinline__ half8v bf16x8_to_b(uint4 v) {
    const half2v p0 = pkrtz(__uint_as_float(v.x << 16), __uint_as_float(v.z << 16));
    const half2v p1 = pkrtz(__uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.z & 0xffff0000u));
    const half2v p2 = pkrtz(__uint_as_float(v.y << 16), __uint_as_float(v.w << 16));
    const half2v p3 = pkrtz(__uint_as_float(v.y & 0xffff0000u), __uint_as_float(v.w & 0xffff0000u));
    return half8v{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

__device__ __forceinline__ float4v mfma16(half8v a, half8v b, float4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }  // strixite kernels/swiglu.hip:22

}  // namespace dev
}  // namespace strix
