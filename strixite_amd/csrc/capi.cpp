// extern "C" wrappers over the C++ launchers: exceptions become return codes plus a thread-local message.
#include "strixite_moe.h"

#include "common.hpp"
#include "strixite_strixw.hpp"

#include <iterator>
#include <map>
#include <string>
#include <vector>

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
strix::Q5DeviceView q5(const strix_qview *w) {
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

int strix_linear_q5_experts_gather_grouped(const void *x, const strix_qview *w, int64_t E, const void *ws,
                                           size_t ws_bytes, int64_t M, int64_t A, void *y, int act, int math,
                                           void *stream) {
    return guard([&] {
        strix::kernels::linear_q5_experts_gather_grouped(x, q5(w), E, ws, ws_bytes, M, A, y, act_of(act), math_of(math),
                                                         st(stream));
    });
}

int strix_linear_q5_experts_gather_grouped_swiglu(const void *x, const strix_qview *w, int64_t E, const void *ws,
                                                  size_t ws_bytes, int64_t M, int64_t A, void *h, int act, int math,
                                                  void *stream, int h_f16) {
    return guard([&] {
        strix::kernels::linear_q5_experts_gather_grouped_swiglu(x, q5(w), E, ws, ws_bytes, M, A, h, act_of(act),
                                                                math_of(math), st(stream), h_f16 != 0);
    });
}

int strix_linear_q5_experts_combine_grouped(const void *h, const strix_qview *w, int64_t E, const int32_t *ids,
                                            const float *coef, const void *ws, size_t ws_bytes, float *partial,
                                            int64_t M, int64_t A, void *y, int act, int math, void *stream,
                                            const strix_moe_shared_add_t *shared, int h_f16) {
    return guard([&] {
        const strix::kernels::MoeSharedAdd sh = shared ? shared_of(shared) : strix::kernels::MoeSharedAdd{};
        strix::kernels::linear_q5_experts_combine_grouped(h, q5(w), E, ids, coef, ws, ws_bytes, partial, M, A, y,
                                                          act_of(act), math_of(math), st(stream),
                                                          shared ? &sh : nullptr, h_f16 != 0);
    });
}

int strix_linear_q5_experts_gather(const void *x, const strix_qview *w, int64_t E, const int32_t *ids, int64_t M,
                                   int64_t A, void *y, int act, uint32_t *err, void *stream) {
    return guard([&] {
        strix::kernels::linear_q5_experts_gather(x, q5(w), E, ids, M, A, y, act_of(act), err, st(stream));
    });
}

int strix_linear_q5_experts_gather_swiglu(const void *x, const strix_qview *w, int64_t E, const int32_t *ids,
                                          int64_t M, int64_t A, void *h, int act, uint32_t *err, void *stream) {
    return guard([&] {
        strix::kernels::linear_q5_experts_gather_swiglu(x, q5(w), E, ids, M, A, h, act_of(act), err, st(stream));
    });
}

int strix_linear_q5_experts_combine(const void *h, const strix_qview *w, int64_t E, const int32_t *ids,
                                    const float *coef, int64_t M, int64_t A, void *y, int act, uint32_t *err,
                                    void *stream) {
    return guard([&] {
        strix::kernels::linear_q5_experts_combine(h, q5(w), E, ids, coef, M, A, y, act_of(act), err, st(stream));
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

int strix_hc_mix_down(const void *x, const strix_qview *w, int bits, int64_t T, int64_t H, int64_t d, int64_t r,
                      int inject, float eps, float *h, float *w_in, float *inv, int act, void *stream) {
    return guard([&] {
        STRIX_CHECK(w != nullptr && (bits == 4 || bits == 8), "strix_hc_mix_down: null view or bits = ", bits);
        if (bits == 4)
            strix::kernels::hc_mix_down(x, q4(w), T, H, d, r, inject != 0, eps, h, w_in, inv, act_of(act), st(stream));
        else
            strix::kernels::hc_mix_down(x, q8(w), T, H, d, r, inject != 0, eps, h, w_in, inv, act_of(act), st(stream));
    });
}
int strix_hc_mix_up(const float *h, const strix_qview *w_up, int bits, const void *x, const float *norm_w,
                    const float *inv, int64_t T, int64_t H, int64_t d, void *u, int act, void *stream) {
    return guard([&] {
        STRIX_CHECK(w_up != nullptr && (bits == 4 || bits == 8), "strix_hc_mix_up: null view or bits = ", bits);
        if (bits == 4) {
            const strix::Q4ChunkMajorView v{w_up->q, w_up->scale, w_up->minv, w_up->N, w_up->K, w_up->G};
            strix::kernels::hc_mix_up(h, v, x, norm_w, inv, T, H, d, u, act_of(act), st(stream));
        } else {
            const strix::Q8ChunkMajorView v{w_up->q, w_up->scale, w_up->minv, w_up->N, w_up->K, w_up->G};
            strix::kernels::hc_mix_up(h, v, x, norm_w, inv, T, H, d, u, act_of(act), st(stream));
        }
    });
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

// ---- strixw ---------------------------------------------------------------------------------------------------
namespace {
strix::StrixwFile *file_of(void *f) {
    STRIX_CHECK(f != nullptr, "null strixw file handle");
    return static_cast<strix::StrixwFile *>(f);
}
strix::StrixwDevice *device_of(void *d) {
    STRIX_CHECK(d != nullptr, "null strixw device handle");
    return static_cast<strix::StrixwDevice *>(d);
}
strix::StrixwRole role_of(int r) {
    STRIX_CHECK(r >= 0 && r <= 3, "strixw role code ", r, " (0 data, 1 q, 2 scale, 3 min)");
    return static_cast<strix::StrixwRole>(r);
}
strix_moe_layer_weights c_layer(const strix::MoeLayerWeights &L) {
    strix_moe_layer_weights w{};
    w.H = L.H, w.E = L.E, w.k = L.k, w.I = L.I;
    w.router = L.router, w.router_bias = L.router_bias;
    w.routed_bits = L.gate_up_bits;
    w.gate_up = {L.gate_up.q, L.gate_up.scale, L.gate_up.minv, L.gate_up.N, L.gate_up.K, L.gate_up.G};
    w.down = {L.down.q, L.down.scale, L.down.minv, L.down.N, L.down.K, L.down.G};
    w.has_shared = L.has_shared ? 1 : 0;
    if (L.has_shared) {
        w.sh_gate_up = {L.sh_gate_up.q, L.sh_gate_up.scale, L.sh_gate_up.minv, L.sh_gate_up.N, L.sh_gate_up.K,
                        L.sh_gate_up.G};
        w.sh_down = {L.sh_down.q, L.sh_down.scale, L.sh_down.minv, L.sh_down.N, L.sh_down.K, L.sh_down.G};
    }
    w.shared_stacked = L.shared_stacked ? 1 : 0;
    return w;
}
}  // namespace

extern "C" {

uint64_t strix_strixw_hash64(const void *p, size_t n) { return strix::strix_hash64(p, n); }

int strix_strixw_open(const char *path, void **file) {
    return guard([&] {
        STRIX_CHECK(path != nullptr && file != nullptr, "strix_strixw_open: null argument");
        *file = nullptr;
        *file = new strix::StrixwFile(path);
    });
}
int strix_strixw_close(void *file) {
    return guard([&] { delete file_of(file); });
}
int strix_strixw_info(void *file, uint64_t *file_bytes, uint64_t *data_offset, uint32_t *version, int64_t *ntensors,
                      int64_t *nmeta) {
    return guard([&] {
        const strix::StrixwFile *f = file_of(file);
        if (file_bytes) *file_bytes = f->file_bytes();
        if (data_offset) *data_offset = f->data_offset();
        if (version) *version = f->version();
        if (ntensors) *ntensors = (int64_t)f->tensors().size();
        if (nmeta) *nmeta = (int64_t)f->meta().size();
    });
}
int strix_strixw_tensor(void *file, int64_t i, strix_strixw_tensor_info *out) {
    return guard([&] {
        const strix::StrixwFile *f = file_of(file);
        STRIX_CHECK(out != nullptr && i >= 0 && i < (int64_t)f->tensors().size(), "strix_strixw_tensor: index ", i,
                    " of ", f->tensors().size());
        const strix::StrixwTensor &t = f->tensors()[(size_t)i];
        *out = strix_strixw_tensor_info{};
        out->name = t.name.c_str();
        out->encoding = (int)t.encoding;
        out->ndim = (int)t.shape.size();
        for (size_t d = 0; d < t.shape.size(); ++d) out->shape[d] = t.shape[d];
        out->group_size = t.group_size, out->experts = t.experts, out->nparts = (int64_t)t.parts.size();
        out->ncomponents = (int)t.components.size();
        for (size_t c = 0; c < t.components.size() && c < 4; ++c) {
            out->role[c] = (int)t.components[c].role;
            out->offset[c] = t.components[c].offset, out->bytes[c] = t.components[c].bytes;
            out->hash[c] = t.components[c].hash;
        }
    });
}
int strix_strixw_find(void *file, const char *name, int64_t *index) {
    return guard([&] {
        const strix::StrixwFile *f = file_of(file);
        STRIX_CHECK(name != nullptr && index != nullptr, "strix_strixw_find: null argument");
        const strix::StrixwTensor *t = f->find(name);
        *index = t ? (int64_t)(t - f->tensors().data()) : -1;
    });
}
int strix_strixw_part(void *file, int64_t tensor, int64_t part, const char **source, int64_t *row_offset,
                      int64_t *rows) {
    return guard([&] {
        const strix::StrixwFile *f = file_of(file);
        STRIX_CHECK(tensor >= 0 && tensor < (int64_t)f->tensors().size(), "strix_strixw_part: tensor ", tensor);
        const auto &ps = f->tensors()[(size_t)tensor].parts;
        STRIX_CHECK(part >= 0 && part < (int64_t)ps.size(), "strix_strixw_part: part ", part, " of ", ps.size());
        if (source) *source = ps[(size_t)part].source.c_str();
        if (row_offset) *row_offset = ps[(size_t)part].row_offset;
        if (rows) *rows = ps[(size_t)part].rows;
    });
}
int strix_strixw_meta(void *file, int64_t i, const char **key, const char **value) {
    return guard([&] {
        const strix::StrixwFile *f = file_of(file);
        STRIX_CHECK(i >= 0 && i < (int64_t)f->meta().size(), "strix_strixw_meta: index ", i, " of ", f->meta().size());
        auto it = f->meta().begin();
        std::advance(it, i);
        if (key) *key = it->first.c_str();
        if (value) *value = it->second.c_str();
    });
}
int strix_strixw_verify(void *file, int threads) {
    return guard([&] { file_of(file)->verify_hashes(threads); });
}

int strix_strixw_writer_create(const char *path, int64_t nmeta, const char *const *keys, const char *const *values,
                               int64_t ntensors, const strix_strixw_plan_t *plan, void **writer) {
    return guard([&] {
        STRIX_CHECK(path != nullptr && writer != nullptr && nmeta >= 0 && ntensors >= 1 && plan != nullptr &&
                        (nmeta == 0 || (keys != nullptr && values != nullptr)),
                    "strix_strixw_writer_create: bad arguments");
        *writer = nullptr;
        std::map<std::string, std::string> meta;
        for (int64_t i = 0; i < nmeta; ++i) meta[keys[i]] = values[i];
        std::vector<strix::StrixwTensor> ts((size_t)ntensors);
        for (int64_t i = 0; i < ntensors; ++i) {
            const strix_strixw_plan_t &p = plan[i];
            STRIX_CHECK(p.name != nullptr && p.ndim >= 1 && p.ndim <= 8 && p.encoding >= 1 && p.encoding <= 9,
                        "strix_strixw_writer_create: plan ", i, " (ndim ", p.ndim, ", encoding ", p.encoding, ")");
            strix::StrixwTensor &t = ts[(size_t)i];
            t.name = p.name;
            t.encoding = static_cast<strix::StrixwEncoding>(p.encoding);
            t.shape.assign(p.shape, p.shape + p.ndim);
            t.group_size = p.group_size, t.experts = p.experts;
            STRIX_CHECK(p.nparts >= 0 && (p.nparts == 0 || (p.part_sources != nullptr && p.part_rows != nullptr)),
                        "strix_strixw_writer_create: plan ", i, " parts");
            for (int64_t j = 0, row = 0; j < p.nparts; row += p.part_rows[j], ++j) {
                STRIX_CHECK(p.part_sources[j] != nullptr, "strix_strixw_writer_create: plan ", i, " part ", j);
                t.parts.push_back({p.part_sources[j], row, p.part_rows[j]});
            }
        }
        *writer = new strix::StrixwWriter(path, std::move(meta), std::move(ts));
    });
}
int strix_strixw_writer_write(void *writer, int64_t tensor, int role, const void *data, size_t bytes) {
    return guard([&] {
        STRIX_CHECK(writer != nullptr && tensor >= 0, "strix_strixw_writer_write: bad arguments");
        static_cast<strix::StrixwWriter *>(writer)->write((size_t)tensor, role_of(role), data, bytes);
    });
}
int strix_strixw_writer_finish(void *writer) {
    return guard([&] {
        STRIX_CHECK(writer != nullptr, "strix_strixw_writer_finish: null writer");
        static_cast<strix::StrixwWriter *>(writer)->finish();
    });
}
int strix_strixw_writer_destroy(void *writer) {
    return guard([&] { delete static_cast<strix::StrixwWriter *>(writer); });
}

int strix_strixw_device_load(const char *path, int read_threads, void **dev) {
    return guard([&] {
        STRIX_CHECK(path != nullptr && dev != nullptr, "strix_strixw_device_load: null argument");
        *dev = nullptr;
        *dev = new strix::StrixwDevice(path, read_threads);
    });
}
int strix_strixw_device_free(void *dev) {
    return guard([&] { delete static_cast<strix::StrixwDevice *>(dev); });
}
int strix_strixw_device_info(void *dev, uint64_t *device_bytes, double *load_seconds) {
    return guard([&] {
        const strix::StrixwDevice *d = device_of(dev);
        if (device_bytes) *device_bytes = d->device_bytes();
        if (load_seconds) *load_seconds = d->load_seconds();
    });
}
int strix_strixw_device_ptr(void *dev, const char *name, int role, const void **ptr) {
    return guard([&] {
        const strix::StrixwDevice *d = device_of(dev);
        STRIX_CHECK(name != nullptr && ptr != nullptr, "strix_strixw_device_ptr: null argument");
        *ptr = d->ptr(d->file().get(name), role_of(role));
    });
}
int strix_strixw_moe_layer(void *dev, const char *prefix, int64_t top_k, strix_moe_layer_weights *out) {
    return guard([&] {
        STRIX_CHECK(prefix != nullptr && out != nullptr, "strix_strixw_moe_layer: null argument");
        *out = c_layer(strix::strixw_moe_layer(*device_of(dev), prefix, top_k));
    });
}

}  // extern "C"
