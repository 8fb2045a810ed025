// C++ launch interface of the gfx950 MoE FFN library, self-contained: the boundary types
// (strixite_moe_types.hpp), the launchers under the reference's own signatures (namespace strix::kernels, C++
// linkage, default arguments - each declaration cites the reference declaration it replaces), and this library's
// additions (strixite_moe_extras.hpp). For a build that has no strixite headers: this library, its C-ABI
// (strixite_moe.h) and tests. Inside the strixite tree keep strixite's own kernel headers - they declare the same
// functions with the same types, and this library exports exactly those symbols - and include only
// strixite_moe_extras.hpp with STRIXITE_MOE_DROPIN defined.
//
// Numerics shared by the expert kernels: activations BF16; under the exact MoeMath kinds (and for Q8 experts and the
// shared expert) the weights enter the matrix cores as their exact integer codes in BF16 with the group's scale and
// min applied to the FP32 accumulator (v_mfma_f32_16x16x32_bf16), so no weight is rounded; the grouped Q4 entry points
// under the F16 MoeMath kinds use the reference's F16 math (v_mfma_f32_32x32x16_f16) at every batch size, and the
// sublayer call (moe_layer_forward) uses it at prefill sizes, exact weights at decode sizes. Every stored value is
// rounded once (RNE) to BF16. Router logits are FP32 in one fixed summation order (linear_bf16w below).
#pragma once

#include <hip/hip_runtime.h>

#include "strixite_moe_types.hpp"

namespace strix {
namespace kernels {

// ---- router: strixite kernels/linear.hpp:20-26 ----------------------------------------------------------------
// y[M, N] = x[M, K] * W^T, W [N, K] BF16 bits. FP32 accumulation in one fixed order at every M: lane l of a wave64
// accumulates the 8-element chunks l, l + 64, ... with fmaf (elements in order), then a butterfly over the lanes
// (offsets 32 .. 1). out_act F32 stores the sum unrounded (the router logits). x BF16, or F32 (each
// product fmaf(x, w) in FP32 in the same order: F32 x holding BF16 values gives the BF16 bits).
void linear_bf16w(const void *x, const uint16_t *w, void *y, int64_t M, int64_t N, int64_t K, Act act,
                  hipStream_t stream);
void linear_bf16w(const void *x, const uint16_t *w, void *y, int64_t M, int64_t N, int64_t K, Act act, Act out_act,
                  hipStream_t stream);

// ---- top-k: strixite kernels/moe_router.hpp:38-43 -------------------------------------------------------------
void moe_router(const void *logits, int64_t ld, int64_t M, int64_t E, int64_t k, const void *shared_logit,
                int64_t shared_ld, int32_t shared_id, int32_t *ids, float *coef, Act act, uint32_t *err,
                hipStream_t stream);
void check_router_error(const uint32_t *err, const char *what);
void report_router_error(const uint32_t e[3], const char *what);

// ---- shared expert add: strixite kernels/moe_router.hpp:45-63 --------------------------------------------------
void moe_shared_add(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M, int64_t N,
                    uint32_t gate_index, Act act, uint32_t *err, hipStream_t stream);
void moe_shared_add_inject(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M, int64_t N,
                           uint32_t gate_index, void *x, const float *w_in, int64_t H, Act act, uint32_t *err,
                           hipStream_t stream);

// ---- residual injection: strixite kernels/hc.hpp:51-55 -----------------------------------------------------------
// In place: x[t, s d + j] = stored(fma(w_in[t, s], y[t, j], x[t, s d + j])), one rounding per element; y must not
// overlap x.
void hc_inject(void *x, const float *w_in, const void *y, int64_t T, int64_t H, int64_t d, Act act,
               hipStream_t stream);

// ---- Q5 experts: strixite kernels/moe_grouped.hpp:93-104, kernels/linear_q4.hpp:47-58 --------------------------
// The Q4 entry points' meaning with formats/q5.hpp weights (K % 128 == 0), either activation dtype. Every MoeMath
// kind computes with the exact weights (FP32 accumulation); the F16 h form (h_f16) is refused.
void linear_q5_experts_gather_grouped(const void *x, const Q5DeviceView &w, int64_t E, const void *ws,
                                      size_t ws_bytes, int64_t M, int64_t A, void *y, Act act, MoeMath math,
                                      hipStream_t stream);
void linear_q5_experts_gather_grouped_swiglu(const void *x, const Q5DeviceView &w, int64_t E, const void *ws,
                                             size_t ws_bytes, int64_t M, int64_t A, void *h, Act act, MoeMath math,
                                             hipStream_t stream, bool h_f16 = false);
void linear_q5_experts_combine_grouped(const void *h, const Q5DeviceView &w, int64_t E, const int32_t *ids,
                                       const float *coef, const void *ws, size_t ws_bytes, float *partial, int64_t M,
                                       int64_t A, void *y, Act act, MoeMath math, hipStream_t stream,
                                       const MoeSharedAdd *shared = nullptr, bool h_f16 = false);
void linear_q5_experts_gather(const void *x, const Q5DeviceView &w, int64_t E, const int32_t *ids, int64_t M,
                              int64_t A, void *y, Act act, uint32_t *err, hipStream_t stream);
void linear_q5_experts_gather_swiglu(const void *x, const Q5DeviceView &w, int64_t E, const int32_t *ids, int64_t M,
                                     int64_t A, void *h, Act act, uint32_t *err, hipStream_t stream);
void linear_q5_experts_combine(const void *h, const Q5DeviceView &w, int64_t E, const int32_t *ids,
                               const float *coef, int64_t M, int64_t A, void *y, Act act, uint32_t *err,
                               hipStream_t stream);

// ---- hyper-connection mix, the step that produces the sublayer's input: strixite kernels/hc.hpp:31-50 -----------
// X [T, H d] (H = 4 streams) -> inv [T, H] = 1 / sqrt(mean(X_s^2) + eps), a = sum_s inv_s (W_s . X_s) for the rows of
// the folded w [r (+ H), H d], h [T, r] = silu(a / H), w_in [T, H] = 2 sigmoid(a / H) for the H injection rows (when
// inject; w_in null iff !inject). FP32 inside; d % 32 == 0; x 16-byte aligned.
void hc_mix_down(const void *x, const Q4DeviceView &w, int64_t T, int64_t H, int64_t d, int64_t r, bool inject,
                 float eps, float *h, float *w_in, float *inv, Act act, hipStream_t stream);
void hc_mix_down(const void *x, const Q8DeviceView &w, int64_t T, int64_t H, int64_t d, int64_t r, bool inject,
                 float eps, float *h, float *w_in, float *inv, Act act, hipStream_t stream);
// u[t, j] = (1/H) sum_s sigmoid(W_up[s d + j] . h[t]) * (X[t, s d + j] * inv[t, s] * (1 + norm_w[s d + j])), W_up
// [H d, r] chunk-major, r % 32 == 0, r <= 1024; u [T, d] in the activation dtype, rounded once.
void hc_mix_up(const float *h, const Q4ChunkMajorView &w_up, const void *x, const float *norm_w, const float *inv,
               int64_t T, int64_t H, int64_t d, void *u, Act act, hipStream_t stream);
void hc_mix_up(const float *h, const Q8ChunkMajorView &w_up, const void *x, const float *norm_w, const float *inv,
               int64_t T, int64_t H, int64_t d, void *u, Act act, hipStream_t stream);

// ---- grouping: strixite kernels/moe_grouped.hpp:46-54 ----------------------------------------------------------
// ws (int32): [n_tiles, S, E, n_wide_tiles], offsets [E + 2] at ws + 4 (bucket b's slots at slots[offsets[b] ..
// offsets[b + 1]); bucket E = invalid ids; offsets[E + 1] = S), slots [S] after them - the reference's prefix
// layout. Inside a bucket the slots are in ascending order (deterministic). Private tables follow.
size_t moe_route_workspace_bytes(int64_t M, int64_t A, int64_t E);
void moe_group_routes(const int32_t *ids, int64_t M, int64_t A, int64_t E, void *ws, size_t ws_bytes, uint32_t *err,
                      hipStream_t stream);

// ---- grouped experts: strixite kernels/moe_grouped.hpp:56-91 ---------------------------------------------------
void linear_q4_experts_gather_grouped(const void *x, const Q4DeviceView &w, int64_t E, const void *ws,
                                      size_t ws_bytes, int64_t M, int64_t A, void *y, Act act, MoeMath math,
                                      hipStream_t stream);
void linear_q4_experts_gather_grouped_swiglu(const void *x, const Q4DeviceView &w, int64_t E, const void *ws,
                                             size_t ws_bytes, int64_t M, int64_t A, void *h, Act act, MoeMath math,
                                             hipStream_t stream, bool h_f16 = false);

// partial: M*A*N FP32 scratch; y = sum over a (slot order) of coef * partial, rounded once; NaN rows for tokens
// with an invalid id. h_f16: h holds f16 bits (the swiglu gather's h_f16 output).
void linear_q4_experts_combine_grouped(const void *h, const Q4DeviceView &w, int64_t E, const int32_t *ids,
                                       const float *coef, const void *ws, size_t ws_bytes, float *partial, int64_t M,
                                       int64_t A, void *y, Act act, MoeMath math, hipStream_t stream,
                                       const MoeSharedAdd *shared = nullptr, bool h_f16 = false);

// ---- per-slot experts: strixite kernels/linear_q4.hpp:42-61 ----------------------------------------------------
void linear_q4_experts_gather(const void *x, const Q4DeviceView &w, int64_t E, const int32_t *ids, int64_t M,
                              int64_t A, void *y, Act act, uint32_t *err, hipStream_t stream);
void linear_q4_experts_gather_swiglu(const void *x, const Q4DeviceView &w, int64_t E, const int32_t *ids, int64_t M,
                                     int64_t A, void *h, Act act, uint32_t *err, hipStream_t stream);
void linear_q4_experts_combine(const void *h, const Q4DeviceView &w, int64_t E, const int32_t *ids,
                               const float *coef, int64_t M, int64_t A, void *y, Act act, uint32_t *err,
                               hipStream_t stream);
void check_expert_error(const uint32_t *err, const char *what);
void report_expert_error(const uint32_t e[3], const char *what);

// ---- swiglu: strixite kernels/swiglu.hpp:21 -------------------------------------------------------------------
void swiglu(const void *gu, void *h, int64_t rows, int64_t I, Act act, hipStream_t stream);

// ---- Q4 dense projection: strixite kernels/linear_q4.hpp:23-31 --------------------------------------------------
// y [M, N] = x [M, K] . dequant(W)^T, FP32 accumulation; out_act == act, or BF16 x -> F32 y (stored unrounded).
void linear_q4(const void *x, const Q4DeviceView &w, void *y, int64_t M, Act act, hipStream_t stream);
void linear_q4(const void *x, const Q4DeviceView &w, void *y, int64_t M, Act act, Act out_act, hipStream_t stream);

// ---- Q8 dense projection: strixite kernels/linear_q8.hpp:13-14 (the shared expert) ------------------------------
void linear_q8(const void *x, const Q8DeviceView &w, void *y, int64_t M, Act act, hipStream_t stream);
void linear_q8(const void *x, const Q8DeviceView &w, void *y, int64_t M, Act act, Act out_act, hipStream_t stream);

}  // namespace kernels
}  // namespace strix

#include "strixite_moe_extras.hpp"
