// extern "C" wrappers over the C++ launchers: exceptions become return codes plus a thread-local message.
#include "strixite_moe.h"

#include "common.hpp"

#include <string>

namespace strix::synth {
uint64_t tensor_key(uint64_t seed, uint32_t tensor, uint32_t layer);
void bf16_normal(uint64_t key, float sigma, uint16_t *out, int64_t n, hipStream_t stream);
void q_weight(int bits, uint64_t key_codes, uint64_t key_scales, int64_t rows, int64_t K, int64_t G, uint8_t *q,
              uint16_t *scale, uint16_t *minv, hipStream_t stream);
void uniform_pm1(uint64_t key, float *out, int64_t n, hipStream_t stream);
}  // namespace strix::synth

namespace {

thread_local std::string g_last_error;

template <typename F> int guard(F &&f) {
    try {
        f();
        g_last_error.clear();
        return 0;
    } catch (const strix::GpuFatalError &e) {
        g_last_error = e.what();
        return STRIX_E_GPU;
    } catch (const strix::Error &e) {
        g_last_error = e.what();
        return STRIX_E_PRECONDITION;
    } catch (const std::exception &e) {
        g_last_error = e.what();
        return STRIX_E_OTHER;
    }
}

using strix::kernels::Act;
using strix::kernels::MoeMath;

Act act_of(int a) {
    STRIX_CHECK(a == 0 || a == 1, "activation dtype code ", a, " (0 = F32, 1 = BF16)");
    return a == 0 ? Act::F32 : Act::BF16;
}
MoeMath math_of(int m) {
    STRIX_CHECK(m >= 0 && m <= 5, "MoeMath code ", m, " (0..5)");
    return static_cast<MoeMath>(m);
}
hipStream_t st(void *s) { return static_cast<hipStream_t>(s); }
strix::Q4DeviceView q4(const strix_qview *w) {
    STRIX_CHECK(w != nullptr, "null weight view");
    return {w->q, w->scale, w->minv, w->N, w->K, w->G};
}
strix::Q8DeviceView q8(const strix_qview *w) {
    STRIX_CHECK(w != nullptr, "null weight view");
    return {w->q, w->scale, w->minv, w->N, w->K, w->G};
}
strix::kernels::MoeSharedAdd shared_of(const strix_moe_shared_add_t *s) {
    return {s->s, s->gate_logit, s->gate_ld, s->gate_index, s->err};
}

}  // namespace

namespace {
strix::MoeLayerWeights layer_of(const strix_moe_layer_weights *w) {
    STRIX_CHECK(w != nullptr, "null layer weights");
    strix::MoeLayerWeights L;
    L.H = w->H, L.E = w->E, L.k = w->k, L.I = w->I;
    L.router = w->router, L.router_bias = w->router_bias;
    L.gate_up_bits = L.down_bits = w->routed_bits;
    L.gate_up = q4(&w->gate_up), L.down = q4(&w->down);
    L.has_shared = w->has_shared != 0;
    if (L.has_shared) L.sh_gate_up = q8(&w->sh_gate_up), L.sh_down = q8(&w->sh_down);
    L.shared_stacked = w->shared_stacked != 0;
    return L;
}
}  // namespace

extern "C" {

int strix_moe_abi_version(void) { return STRIX_MOE_ABI_VERSION; }
const char *strix_moe_last_error(void) { return g_last_error.c_str(); }

int strix_linear_bf16w(const void *x, const uint16_t *w, void *y, int64_t M, int64_t N, int64_t K, int act,
                       int out_act, void *stream) {
    return guard([&] { strix::kernels::linear_bf16w(x, w, y, M, N, K, act_of(act), act_of(out_act), st(stream)); });
}

int strix_moe_router(const void *logits, int64_t ld, int64_t M, int64_t E, int64_t k, const void *shared_logit,
                     int64_t shared_ld, int32_t shared_id, int32_t *ids, float *coef, int act, uint32_t *err,
                     void *stream) {
    return guard([&] {
        strix::kernels::moe_router(logits, ld, M, E, k, shared_logit, shared_ld, shared_id, ids, coef, act_of(act), err,
                                   st(stream));
    });
}

int strix_check_router_error(const uint32_t *err, const char *what) {
    return guard([&] { strix::kernels::check_router_error(err, what ? what : "moe_router"); });
}
int strix_report_router_error(const uint32_t *e, const char *what) {
    return guard([&] {
        STRIX_CHECK(e != nullptr, "null error words");
        strix::kernels::report_router_error(e, what ? what : "moe_router");
    });
}

int strix_moe_shared_add(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M, int64_t N,
                         uint32_t gate_index, int act, uint32_t *err, void *stream) {
    return guard([&] {
        strix::kernels::moe_shared_add(y, s, gate_logit, gate_ld, M, N, gate_index, act_of(act), err, st(stream));
    });
}

int strix_moe_shared_add_inject(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M,
                                int64_t N, uint32_t gate_index, void *x, const float *w_in, int64_t H, int act,
                                uint32_t *err, void *stream) {
    return guard([&] {
        strix::kernels::moe_shared_add_inject(y, s, gate_logit, gate_ld, M, N, gate_index, x, w_in, H, act_of(act), err,
                                              st(stream));
    });
}

int64_t strix_moe_route_workspace_bytes(int64_t M, int64_t A, int64_t E) {
    int64_t r = -1;
    guard([&] { r = (int64_t)strix::kernels::moe_route_workspace_bytes(M, A, E); });
    return r;
}

int strix_moe_group_routes(const int32_t *ids, int64_t M, int64_t A, int64_t E, void *ws, size_t ws_bytes,
                           uint32_t *err, void *stream) {
    return guard([&] { strix::kernels::moe_group_routes(ids, M, A, E, ws, ws_bytes, err, st(stream)); });
}

int strix_linear_q4_experts_gather_grouped(const void *x, const strix_qview *w, int64_t E, const void *ws,
                                           size_t ws_bytes, int64_t M, int64_t A, void *y, int act, int math,
                                           void *stream) {
    return guard([&] {
        strix::kernels::linear_q4_experts_gather_grouped(x, q4(w), E, ws, ws_bytes, M, A, y, act_of(act), math_of(math),
                                                         st(stream));
    });
}

int strix_linear_q4_experts_gather_grouped_swiglu(const void *x, const strix_qview *w, int64_t E, const void *ws,
                                                  size_t ws_bytes, int64_t M, int64_t A, void *h, int act, int math,
                                                  void *stream, int h_f16) {
    return guard([&] {
        strix::kernels::linear_q4_experts_gather_grouped_swiglu(x, q4(w), E, ws, ws_bytes, M, A, h, act_of(act),
                                                                math_of(math), st(stream), h_f16 != 0);
    });
}

int strix_linear_q4_experts_combine_grouped(const void *h, const strix_qview *w, int64_t E, const int32_t *ids,
                                            const float *coef, const void *ws, size_t ws_bytes, float *partial,
                                            int64_t M, int64_t A, void *y, int act, int math, void *stream,
                                            const strix_moe_shared_add_t *shared, int h_f16) {
    return guard([&] {
        const strix::kernels::MoeSharedAdd sh = shared ? shared_of(shared) : strix::kernels::MoeSharedAdd{};
        strix::kernels::linear_q4_experts_combine_grouped(h, q4(w), E, ids, coef, ws, ws_bytes, partial, M, A, y,
                                                          act_of(act), math_of(math), st(stream),
                                                          shared ? &sh : nullptr, h_f16 != 0);
    });
}

int strix_linear_q8_experts_gather_grouped_swiglu(const void *x, const strix_qview *w, int64_t E, const void *ws,
                                                  size_t ws_bytes, int64_t M, int64_t A, void *h, int act, int math,
                                                  void *stream, int h_f16) {
    return guard([&] {
        strix::kernels::linear_q8_experts_gather_grouped_swiglu(x, q8(w), E, ws, ws_bytes, M, A, h, act_of(act),
                                                                math_of(math), st(stream), h_f16 != 0);
    });
}

int strix_linear_q8_experts_combine_grouped(const void *h, const strix_qview *w, int64_t E, const int32_t *ids,
                                            const float *coef, const void *ws, size_t ws_bytes, float *partial,
                                            int64_t M, int64_t A, void *y, int act, int math, void *stream,
                                            const strix_moe_shared_add_t *shared, int h_f16) {
    return guard([&] {
        const strix::kernels::MoeSharedAdd sh = shared ? shared_of(shared) : strix::kernels::MoeSharedAdd{};
        strix::kernels::linear_q8_experts_combine_grouped(h, q8(w), E, ids, coef, ws, ws_bytes, partial, M, A, y,
                                                          act_of(act), math_of(math), st(stream),
                                                          shared ? &sh : nullptr, h_f16 != 0);
    });
}

int strix_linear_q4_experts_gather(const void *x, const strix_qview *w, int64_t E, const int32_t *ids, int64_t M,
                                   int64_t A, void *y, int act, uint32_t *err, void *stream) {
    return guard([&] {
        strix::kernels::linear_q4_experts_gather(x, q4(w), E, ids, M, A, y, act_of(act), err, st(stream));
    });
}

int strix_linear_q4_experts_gather_swiglu(const void *x, const strix_qview *w, int64_t E, const int32_t *ids,
                                          int64_t M, int64_t A, void *h, int act, uint32_t *err, void *stream) {
    return guard([&] {
        strix::kernels::linear_q4_experts_gather_swiglu(x, q4(w), E, ids, M, A, h, act_of(act), err, st(stream));
    });
}

int strix_linear_q4_experts_combine(const void *h, const strix_qview *w, int64_t E, const int32_t *ids,
                                    const float *coef, int64_t M, int64_t A, void *y, int act, uint32_t *err,
                                    void *stream) {
    return guard([&] {
        strix::kernels::linear_q4_experts_combine(h, q4(w), E, ids, coef, M, A, y, act_of(act), err, st(stream));
    });
}

int strix_check_expert_error(const uint32_t *err, const char *what) {
    return guard([&] { strix::kernels::check_expert_error(err, what ? what : "experts"); });
}
int strix_report_expert_error(const uint32_t *e, const char *what) {
    return guard([&] {
        STRIX_CHECK(e != nullptr, "null error words");
        strix::kernels::report_expert_error(e, what ? what : "experts");
    });
}

int strix_swiglu(const void *gu, void *h, int64_t rows, int64_t I, int act, void *stream) {
    return guard([&] { strix::kernels::swiglu(gu, h, rows, I, act_of(act), st(stream)); });
}

int strix_linear_q4(const void *x, const strix_qview *w, void *y, int64_t M, int act, int out_act, void *stream) {
    return guard([&] { strix::kernels::linear_q4(x, q4(w), y, M, act_of(act), act_of(out_act), st(stream)); });
}
int strix_linear_q8(const void *x, const strix_qview *w, void *y, int64_t M, int act, int out_act, void *stream) {
    return guard([&] { strix::kernels::linear_q8(x, q8(w), y, M, act_of(act), act_of(out_act), st(stream)); });
}


int64_t strix_moe_layer_workspace_bytes(const strix_moe_layer_weights *w, int64_t M) {
    int64_t r = -1;
    guard([&] { r = (int64_t)strix::moe_layer_workspace_bytes(layer_of(w), M); });
    return r;
}

int strix_moe_layer_context_create(void **ctx) {
    return guard([&] {
        STRIX_CHECK(ctx != nullptr, "strix_moe_layer_context_create: null ctx");
        *ctx = strix::moe_layer_context_create();
    });
}
int strix_moe_layer_context_destroy(void *ctx) {
    return guard([&] { strix::moe_layer_context_destroy(static_cast<strix::MoeLayerContext *>(ctx)); });
}

int strix_moe_layer_forward(const strix_moe_layer_weights *w, const void *x, int64_t M, const float *logits_in,
                            void *y, void *x_out, int32_t *ids, float *coef, void *ws, size_t ws_bytes, uint32_t *err,
                            void *stream, void *ctx, const strix_moe_inject_t *inject) {
    return guard([&] {
        strix::MoeLayerInject inj;
        if (inject != nullptr) inj.xs = inject->xs, inj.w_in = inject->w_in, inj.streams = inject->streams;
        strix::moe_layer_forward(layer_of(w), x, M, logits_in, y, x_out, ids, coef, ws, ws_bytes, err, st(stream),
                                 static_cast<strix::MoeLayerContext *>(ctx), inject ? &inj : nullptr);
    });
}

int strix_hc_inject(void *x, const float *w_in, const void *y, int64_t T, int64_t H, int64_t d, int act,
                    void *stream) {
    return guard([&] { strix::kernels::hc_inject(x, w_in, y, T, H, d, act_of(act), st(stream)); });
}

int64_t strix_moe_layer_noalloc_max_bytes(void) { return (int64_t)strix::moe_layer_noalloc_max_bytes(); }
int strix_moe_layer_forward_noalloc(const strix_moe_layer_weights *w, const void *x, int64_t M,
                                    const float *logits_in, void *y, void *x_out, int32_t *ids, float *coef,
                                    uint32_t *err, void *stream) {
    return guard([&] {
        strix::moe_layer_forward_noalloc(layer_of(w), x, M, logits_in, y, x_out, ids, coef, err, st(stream));
    });
}

uint64_t strix_synth_tensor_key(uint64_t seed, uint32_t tensor, uint32_t layer) {
    return strix::synth::tensor_key(seed, tensor, layer);
}
int strix_synth_bf16_normal(uint64_t key, float sigma, uint16_t *out, int64_t n, void *stream) {
    return guard([&] { strix::synth::bf16_normal(key, sigma, out, n, st(stream)); });
}
int strix_synth_q_weight(int bits, uint64_t key_codes, uint64_t key_scales, int64_t rows, int64_t K, int64_t G,
                         uint8_t *q, uint16_t *scale, uint16_t *minv, void *stream) {
    return guard([&] { strix::synth::q_weight(bits, key_codes, key_scales, rows, K, G, q, scale, minv, st(stream)); });
}
int strix_synth_uniform_pm1(uint64_t key, float *out, int64_t n, void *stream) {
    return guard([&] { strix::synth::uniform_pm1(key, out, n, st(stream)); });
}

}  // extern "C"
