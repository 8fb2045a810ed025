// This library's additions to the reference's MoE launch interface: the Q8 routed-expert family, the whole
// sublayer in one call, and its workspace size. Defines no boundary type: inside the strixite tree (compile with
// STRIXITE_MOE_DROPIN defined) Act, MoeMath, MoeSharedAdd, Q4DeviceView, Q8DeviceView and strix::Error come from
// strixite's own headers, included here; elsewhere from strixite_moe_types.hpp.
#pragma once

#include <hip/hip_runtime.h>

#ifdef STRIXITE_MOE_DROPIN
#include "kernels/moe_grouped.hpp"  // Act (kernels/norm.hpp), MoeMath, MoeSharedAdd, Q4DeviceView
#include "runtime/q8_device.hpp"    // Q8DeviceView
#else
#include "strixite_moe_types.hpp"
#endif

#include <cstddef>
#include <cstdint>

namespace strix {
namespace kernels {

// The Q8 expert family (BITS = 8), for 8-bit routed experts; same semantics.
void linear_q8_experts_gather_grouped_swiglu(const void *x, const Q8DeviceView &w, int64_t E, const void *ws,
                                             size_t ws_bytes, int64_t M, int64_t A, void *h, Act act, MoeMath math,
                                             hipStream_t stream, bool h_f16 = false);
void linear_q8_experts_combine_grouped(const void *h, const Q8DeviceView &w, int64_t E, const int32_t *ids,
                                       const float *coef, const void *ws, size_t ws_bytes, float *partial, int64_t M,
                                       int64_t A, void *y, Act act, MoeMath math, hipStream_t stream,
                                       const MoeSharedAdd *shared = nullptr, bool h_f16 = false);

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
    // The shared expert stacked as expert E of gate_up / down (the converter's default layout, strixite
    // formats/merge_plan.cpp:31-41; has_shared false): the views then hold E + 1 experts, and every token routes to
    // it as slot k (id E, coefficient sigmoid(its gate logit, router row E)), so ids / coef are [M, k + 1].
    bool shared_stacked = false;
};

// Bytes of caller-owned device scratch for moe_layer_forward at up to M tokens.
size_t moe_layer_workspace_bytes(const MoeLayerWeights &w, int64_t M);

// A layer context: a helper stream and its fork / join events, on which moe_layer_forward runs the shared expert
// beside the routing kernels at prefill sizes (M > 16 tokens). Create it on the device it serves, before any graph
// capture; use it from one host thread at a time (like a stream). Without a context the shared expert runs on the
// caller's stream.
struct MoeLayerContext;
MoeLayerContext *moe_layer_context_create();  // on the current device
void moe_layer_context_destroy(MoeLayerContext *ctx);

// The residual end of a layer with hyper-connections (strixite runtime/qwen4exp.cpp:3206-3216): the layer's stored
// y injected into `streams` residual streams in place, xs[m, st H + n] = stored(fma(w_in[m, st], y[m, n], xs[..]))
// (strixite kernels/hc.hpp:51-55), folded into the combine's epilogue.
struct MoeLayerInject {
    void *xs = nullptr;            // [M, streams * H] BF16, 16-byte aligned
    const float *w_in = nullptr;   // [M, streams]
    int64_t streams = 4;
};

// x [M, H] BF16 in; y [M, H] BF16 (the MoE output), x_out [M, H] (x + y, may be null, may be x). x, y, x_out 16-byte
// aligned. logits_in (optional, FP32 [M, E (+1)]) bypasses the router projection. ids / coef (optional, [M, k])
// receive the routing. err: 6 zeroed uint32 (router word, then expert word). inject (optional, with x_out null): the
// hyper-connection injection instead of the residual write. Asynchronous on stream; allocates nothing.
void moe_layer_forward(const MoeLayerWeights &w, const void *x, int64_t M, const float *logits_in, void *y,
                       void *x_out, int32_t *ids, float *coef, void *ws, size_t ws_bytes, uint32_t *err,
                       hipStream_t stream, MoeLayerContext *ctx = nullptr, const MoeLayerInject *inject = nullptr);

// No counterpart in the reference: moe_layer_forward for callers that cannot allocate (code under HIP graph capture,
// serving loops, harnesses that forbid hipMalloc). The scratch is a fixed device array of moe_layer_noalloc_max_bytes()
// (16 MiB) that the library holds on every device it runs on until the process ends; a call whose
// moe_layer_workspace_bytes(w, M) exceeds it is refused (strix::Error). Every call on one device shares that array:
// calls that overlap on a device (other streams, other threads) race. Nothing is allocated; the shared expert runs on
// the caller's stream.
size_t moe_layer_noalloc_max_bytes();
void moe_layer_forward_noalloc(const MoeLayerWeights &w, const void *x, int64_t M, const float *logits_in, void *y,
                               void *x_out, int32_t *ids, float *coef, uint32_t *err, hipStream_t stream);

}  // namespace strix
