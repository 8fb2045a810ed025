// C++ launch interface of the gfx950 MoE FFN library: the reference's own signatures (namespace strix::kernels,
// C++ linkage, default arguments), so the calls in strixite runtime/qwen4exp.cpp:3143-3217 compile against it
// unchanged. Each declaration cites the reference declaration it replaces. The C-ABI over the same functions is
// include/strixite_moe.h.
//
// Numerics shared by every expert kernel here: activations BF16; weights dequantized to f16 as code * s + m (one
// rounding, codes exact); v_mfma_f32_16x16x32_f16 products with FP32 accumulation over the whole K; every stored
// value rounded once (RNE) to BF16. Router logits are FP32 in one fixed summation order (linear_bf16w below).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>

namespace strix {

// strixite common/check.hpp:21-33: a failed host-side precondition; a HIP runtime failure.
class Error : public std::runtime_error {
public:
    using std::runtime_error::runtime_error;
};
class GpuError : public Error {
public:
    using Error::Error;
};

// strixite runtime/q4_device.hpp:13-18, runtime/q8_device.hpp:12-17: non-owning device views of the formats/q4.hpp
// and formats/q8.hpp layouts (q [N, K/2] or [N, K] bytes, scale / min [N, K/G] BF16 bits, w = q * scale + min).
struct Q4DeviceView {
    const uint8_t *q = nullptr;
    const uint16_t *scale = nullptr;
    const uint16_t *minv = nullptr;
    int64_t N = 0, K = 0, G = 0;
};
struct Q8DeviceView {
    const uint8_t *q = nullptr;
    const uint16_t *scale = nullptr;
    const uint16_t *minv = nullptr;
    int64_t N = 0, K = 0, G = 0;
};

namespace kernels {

// strixite kernels/norm.hpp:20
enum class Act { F32, BF16 };
const char *act_name(Act a);

// strixite kernels/moe_grouped.hpp:38. The F16 kinds (WmmaF16, Narrow, Wide, Wide256: one math, tiles picked by
// shape) run Q4 experts' prefill-size grouped GEMMs in the reference's F16 math (x rounded to F16 toward zero, each
// weight one F16 rounding of code * s + m, FP32 accumulation); F32 and WmmaBf16 keep the weights exact (scaled
// codes, FP32 accumulation). Q8 experts and decode-size calls use the exact weights under every kind.
enum class MoeMath { F32, WmmaBf16, WmmaF16, WmmaF16Narrow, WmmaF16Wide, WmmaF16Wide256 };

constexpr int64_t kMoeMaxExperts = 1023;  // strixite kernels/moe_grouped.hpp:43: E + 1 buckets
constexpr int64_t kMoeMaxSlots = 1 << 20;  // strixite kernels/moe_grouped.hpp:44

// ---- router: strixite kernels/linear.hpp:20-26 ----------------------------------------------------------------
// y[M, N] = x[M, K] * W^T, W [N, K] BF16 bits. FP32 accumulation in one fixed order at every M: lane l of a wave64
// accumulates the 8-element chunks l, l + 64, ... with fmaf (elements in order), then a butterfly over the lanes
// (offsets 32 .. 1). out_act F32 stores the sum unrounded (the router logits). x BF16 only.
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

// strixite kernels/moe_grouped.hpp:75-81
struct MoeSharedAdd {
    const void *s = nullptr;
    const float *gate_logit = nullptr;
    int64_t gate_ld = 0;
    uint32_t gate_index = 0;
    uint32_t *err = nullptr;
};

// partial: M*A*N FP32 scratch; y = sum over a (slot order) of coef * partial, rounded once; NaN rows for tokens
// with an invalid id. h_f16: h holds f16 bits (the swiglu gather's h_f16 output).
void linear_q4_experts_combine_grouped(const void *h, const Q4DeviceView &w, int64_t E, const int32_t *ids,
                                       const float *coef, const void *ws, size_t ws_bytes, float *partial, int64_t M,
                                       int64_t A, void *y, Act act, MoeMath math, hipStream_t stream,
                                       const MoeSharedAdd *shared = nullptr, bool h_f16 = false);

// The Q8 expert family (BITS = 8), for 8-bit routed experts; same semantics.
void linear_q8_experts_gather_grouped_swiglu(const void *x, const Q8DeviceView &w, int64_t E, const void *ws,
                                             size_t ws_bytes, int64_t M, int64_t A, void *h, Act act, MoeMath math,
                                             hipStream_t stream, bool h_f16 = false);
void linear_q8_experts_combine_grouped(const void *h, const Q8DeviceView &w, int64_t E, const int32_t *ids,
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

// ---- Q8 dense projection: strixite kernels/linear_q8.hpp:13-14 (the shared expert) ------------------------------
void linear_q8(const void *x, const Q8DeviceView &w, void *y, int64_t M, Act act, hipStream_t stream);
void linear_q8(const void *x, const Q8DeviceView &w, void *y, int64_t M, Act act, Act out_act, hipStream_t stream);

}  // namespace kernels

// ---- the whole MoE sublayer, the sequence of strixite runtime/qwen4exp.cpp:3143-3217 --------------------------
// router projection -> moe_router -> moe_group_routes -> gate_up + SwiGLU -> down -> ordered combine with the
// shared expert's gated add folded in -> residual write x_out = x + y. BF16 activations.
struct MoeLayerWeights {
    int64_t H = 0, E = 0, k = 0, I = 0;
    const uint16_t *router = nullptr;    // [E + (shared ? 1 : 0), H] BF16; row E = the shared expert's gate
    const float *router_bias = nullptr;  // optional [E], added once in FP32 (a harness-side routing bias)
    int gate_up_bits = 4, down_bits = 4; // routed experts: Q4 or Q8 (both projections use one format per view)
    Q4DeviceView gate_up, down;          // stacked [E * 2I, H], [E * H, I]; a Q8 view uses the same fields
    bool has_shared = false;
    Q8DeviceView sh_gate_up, sh_down;    // [2I, H], [H, I]
};

// Bytes of caller-owned device scratch for moe_layer_forward at up to M tokens.
size_t moe_layer_workspace_bytes(const MoeLayerWeights &w, int64_t M);

// x [M, H] BF16 in; y [M, H] BF16 (the MoE output), x_out [M, H] (x + y, may be null). logits_in (optional, FP32
// [M, E (+1)]) bypasses the router projection. ids / coef (optional, [M, k]) receive the routing. err: 6 zeroed
// uint32 (router word, then expert word). Asynchronous on stream; allocates nothing.
void moe_layer_forward(const MoeLayerWeights &w, const void *x, int64_t M, const float *logits_in, void *y,
                       void *x_out, int32_t *ids, float *coef, void *ws, size_t ws_bytes, uint32_t *err,
                       hipStream_t stream);

}  // namespace strix
