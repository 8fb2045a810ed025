/*
 * C-ABI of the gfx950 MoE FFN library (libstrixite_moe.so): the drop-in boundary for strixite's quantized MoE
 * sublayer. Plain pointers and sizes; no C++ or torch types. Each entry point wraps the C++ launcher of the same name
 * in include/strixite_moe.hpp and cites the reference declaration it replaces.
 *
 * Conventions (strixite kernels/ headers): every buffer is caller-owned device memory; launches are asynchronous on
 * `stream` (a hipStream_t, NULL = the default stream); nothing is allocated or freed. Return value: 0 on success,
 * STRIX_E_PRECONDITION when a host-detectable precondition fails (the reference throws strix::Error),
 * STRIX_E_GPU when the HIP runtime reports an error; strix_moe_last_error() then holds the message (thread-local).
 * Device-detected data errors (non-finite logits, invalid expert ids) never trap: they set the caller-zeroed
 * uint32_t err[3] word ({1, token or id, expert or slot}, first flag wins) and make the affected rows NaN.
 * act / out_act: 0 = F32, 1 = BF16 (strixite kernels/norm.hpp:20 Act). math: strixite MoeMath (0..5; 2..5 = the F16 math for Q4 experts' grouped projections).
 */
#ifndef STRIXITE_MOE_H
#define STRIXITE_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STRIX_MOE_ABI_VERSION 4
#define STRIX_E_PRECONDITION 1
#define STRIX_E_GPU 2
#define STRIX_E_OTHER 3

/* strixite runtime/q4_device.hpp:13-18 Q4DeviceView / runtime/q8_device.hpp:12-17 Q8DeviceView */
typedef struct {
    const uint8_t *q;
    const uint16_t *scale;
    const uint16_t *minv;
    int64_t N, K, G;
} strix_qview;

/* strixite kernels/moe_grouped.hpp:75-81 MoeSharedAdd */
typedef struct {
    const void *s;
    const float *gate_logit;
    int64_t gate_ld;
    uint32_t gate_index;
    uint32_t *err;
} strix_moe_shared_add_t;

int strix_moe_abi_version(void);
const char *strix_moe_last_error(void);

/* strixite kernels/linear.hpp:23-26 linear_bf16w (router logits; the fixed FP32 summation order) */
int strix_linear_bf16w(const void *x, const uint16_t *w, void *y, int64_t M, int64_t N, int64_t K, int act,
                       int out_act, void *stream);

/* strixite kernels/moe_router.hpp:38-40 moe_router */
int strix_moe_router(const void *logits, int64_t ld, int64_t M, int64_t E, int64_t k, const void *shared_logit,
                     int64_t shared_ld, int32_t shared_id, int32_t *ids, float *coef, int act, uint32_t *err,
                     void *stream);
/* strixite kernels/moe_router.hpp:41-43 check_router_error / report_router_error (host words) */
int strix_check_router_error(const uint32_t *err, const char *what);
int strix_report_router_error(const uint32_t *err_host, const char *what);

/* strixite kernels/moe_router.hpp:52-53 moe_shared_add, :61-63 moe_shared_add_inject */
int strix_moe_shared_add(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M, int64_t N,
                         uint32_t gate_index, int act, uint32_t *err, void *stream);
int strix_moe_shared_add_inject(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M,
                                int64_t N, uint32_t gate_index, void *x, const float *w_in, int64_t H, int act,
                                uint32_t *err, void *stream);

/* strixite kernels/moe_grouped.hpp:47 moe_route_workspace_bytes (-1 on bad arguments), :52-53 moe_group_routes */
int64_t strix_moe_route_workspace_bytes(int64_t M, int64_t A, int64_t E);
int strix_moe_group_routes(const int32_t *ids, int64_t M, int64_t A, int64_t E, void *ws, size_t ws_bytes,
                           uint32_t *err, void *stream);

/* strixite kernels/moe_grouped.hpp:56-58, :66-69, :88-91 (Q4 experts); the Q8 family (BITS = 8) has no reference
 * GPU counterpart - the reference's converter refuses Q8 experts (formats/convert_qwen4exp.cpp:347-349) - and serves
 * 8-bit routed experts behind the same signatures. */
int strix_linear_q4_experts_gather_grouped(const void *x, const strix_qview *w, int64_t E, const void *ws,
                                           size_t ws_bytes, int64_t M, int64_t A, void *y, int act, int math,
                                           void *stream);
int strix_linear_q4_experts_gather_grouped_swiglu(const void *x, const strix_qview *w, int64_t E, const void *ws,
                                                  size_t ws_bytes, int64_t M, int64_t A, void *h, int act, int math,
                                                  void *stream, int h_f16);
int strix_linear_q4_experts_combine_grouped(const void *h, const strix_qview *w, int64_t E, const int32_t *ids,
                                            const float *coef, const void *ws, size_t ws_bytes, float *partial,
                                            int64_t M, int64_t A, void *y, int act, int math, void *stream,
                                            const strix_moe_shared_add_t *shared, int h_f16);
int strix_linear_q8_experts_gather_grouped_swiglu(const void *x, const strix_qview *w, int64_t E, const void *ws,
                                                  size_t ws_bytes, int64_t M, int64_t A, void *h, int act, int math,
                                                  void *stream, int h_f16);
int strix_linear_q8_experts_combine_grouped(const void *h, const strix_qview *w, int64_t E, const int32_t *ids,
                                            const float *coef, const void *ws, size_t ws_bytes, float *partial,
                                            int64_t M, int64_t A, void *y, int act, int math, void *stream,
                                            const strix_moe_shared_add_t *shared, int h_f16);

/* strixite kernels/linear_q4.hpp:42-43, :44-46, :55-56 (per-slot decode forms), :59-61 check / report */
int strix_linear_q4_experts_gather(const void *x, const strix_qview *w, int64_t E, const int32_t *ids, int64_t M,
                                   int64_t A, void *y, int act, uint32_t *err, void *stream);
int strix_linear_q4_experts_gather_swiglu(const void *x, const strix_qview *w, int64_t E, const int32_t *ids,
                                          int64_t M, int64_t A, void *h, int act, uint32_t *err, void *stream);
int strix_linear_q4_experts_combine(const void *h, const strix_qview *w, int64_t E, const int32_t *ids,
                                    const float *coef, int64_t M, int64_t A, void *y, int act, uint32_t *err,
                                    void *stream);
/* strixite kernels/moe_grouped.hpp:93-104, kernels/linear_q4.hpp:47-58: the same with Q5 experts (formats/q5.hpp,
 * K % 128 == 0; the view's q holds each row's low and high planes). Either activation dtype; exact weights under
 * every MoeMath; h_f16 refused. */
int strix_linear_q5_experts_gather_grouped(const void *x, const strix_qview *w, int64_t E, const void *ws,
                                           size_t ws_bytes, int64_t M, int64_t A, void *y, int act, int math,
                                           void *stream);
int strix_linear_q5_experts_gather_grouped_swiglu(const void *x, const strix_qview *w, int64_t E, const void *ws,
                                                  size_t ws_bytes, int64_t M, int64_t A, void *h, int act, int math,
                                                  void *stream, int h_f16);
int strix_linear_q5_experts_combine_grouped(const void *h, const strix_qview *w, int64_t E, const int32_t *ids,
                                            const float *coef, const void *ws, size_t ws_bytes, float *partial,
                                            int64_t M, int64_t A, void *y, int act, int math, void *stream,
                                            const strix_moe_shared_add_t *shared, int h_f16);
int strix_linear_q5_experts_gather(const void *x, const strix_qview *w, int64_t E, const int32_t *ids, int64_t M,
                                   int64_t A, void *y, int act, uint32_t *err, void *stream);
int strix_linear_q5_experts_gather_swiglu(const void *x, const strix_qview *w, int64_t E, const int32_t *ids,
                                          int64_t M, int64_t A, void *h, int act, uint32_t *err, void *stream);
int strix_linear_q5_experts_combine(const void *h, const strix_qview *w, int64_t E, const int32_t *ids,
                                    const float *coef, int64_t M, int64_t A, void *y, int act, uint32_t *err,
                                    void *stream);
int strix_check_expert_error(const uint32_t *err, const char *what);
int strix_report_expert_error(const uint32_t *err_host, const char *what);

/* strixite kernels/swiglu.hpp:21 swiglu */
int strix_swiglu(const void *gu, void *h, int64_t rows, int64_t I, int act, void *stream);

/* strixite kernels/linear_q4.hpp:23-31 linear_q4 (a dense Q4 projection) */
int strix_linear_q4(const void *x, const strix_qview *w, void *y, int64_t M, int act, int out_act, void *stream);

/* strixite kernels/linear_q8.hpp:13-14 linear_q8 (the shared expert's projections) */
int strix_linear_q8(const void *x, const strix_qview *w, void *y, int64_t M, int act, int out_act, void *stream);

/* The MoE sublayer in the order of strixite runtime/qwen4exp.cpp:3143-3217 (its caller), as one entry point:
 * router projection, moe_router, moe_group_routes, gate_up + SwiGLU, down, ordered combine with the shared expert's
 * gated add folded in, residual write. routed_bits: 4 or 8 (gate_up and down alike). router_bias (optional, [E]) is a
 * harness-side routing bias added once in FP32; logits_in (optional, [M, E + has_shared] FP32) bypasses the
 * router projection. err: 6 caller-zeroed words (router word, expert word). */
typedef struct {
    int64_t H, E, k, I;
    const uint16_t *router;
    const float *router_bias;
    int routed_bits;
    strix_qview gate_up, down;
    int has_shared;
    strix_qview sh_gate_up, sh_down;
    int shared_stacked; /* the shared expert is expert E of gate_up / down, routed as slot k (ids / coef [M, k + 1]) */
} strix_moe_layer_weights;

int64_t strix_moe_layer_workspace_bytes(const strix_moe_layer_weights *w, int64_t M);
/* ctx (optional, from strix_moe_layer_context_create): the helper stream for the shared expert at M > 16 tokens;
 * created before any graph capture, used by one host thread at a time; null: the shared expert runs on stream. */
int strix_moe_layer_context_create(void **ctx);
int strix_moe_layer_context_destroy(void *ctx);
/* inject (optional, with x_out null): the hyper-connection residual end, xs[m, s H + n] = stored(fma(w_in[m, s],
 * y[m, n], xs[..])) in place over `streams` residual streams (strixite kernels/hc.hpp:51-55), in the combine. */
typedef struct {
    void *xs;
    const float *w_in;
    int64_t streams;
} strix_moe_inject_t;
int strix_moe_layer_forward(const strix_moe_layer_weights *w, const void *x, int64_t M, const float *logits_in,
                            void *y, void *x_out, int32_t *ids, float *coef, void *ws, size_t ws_bytes, uint32_t *err,
                            void *stream, void *ctx, const strix_moe_inject_t *inject);

/* strixite kernels/hc.hpp:51-55 hc_inject: x[t, s d + j] = stored(fma(w_in[t, s], y[t, j], x[...])) in place */
int strix_hc_inject(void *x, const float *w_in, const void *y, int64_t T, int64_t H, int64_t d, int act,
                    void *stream);
/* strixite kernels/hc.hpp:31-36 hc_mix_down (bits 4 or 8: the Q4 / Q8 overload; w row-major, folded): inv [T, H],
 * h [T, r] = silu(a / H), w_in [T, H] = 2 sigmoid(a / H) when inject (w_in null iff !inject) */
int strix_hc_mix_down(const void *x, const strix_qview *w, int bits, int64_t T, int64_t H, int64_t d, int64_t r,
                      int inject, float eps, float *h, float *w_in, float *inv, int act, void *stream);
/* strixite kernels/hc.hpp:38-50 hc_mix_up (bits 4 or 8; w_up chunk-major [H d, r]): u [T, d] */
int strix_hc_mix_up(const float *h, const strix_qview *w_up, int bits, const void *x, const float *norm_w,
                    const float *inv, int64_t T, int64_t H, int64_t d, void *u, int act, void *stream);

/* No counterpart in the reference: strix_moe_layer_forward for callers that cannot allocate (graph capture, serving
 * loops, harnesses that forbid hipMalloc). Its scratch is a fixed 16 MiB device array per device, held until the
 * process ends (strix_moe_layer_noalloc_max_bytes); a call needing more is refused with STRIX_E_PRECONDITION. Calls
 * that overlap on one device share the array and race. */
int64_t strix_moe_layer_noalloc_max_bytes(void);
int strix_moe_layer_forward_noalloc(const strix_moe_layer_weights *w, const void *x, int64_t M,
                                    const float *logits_in, void *y, void *x_out, int32_t *ids, float *coef,
                                    uint32_t *err, void *stream);

/* strixw, the converted-weights file (strixite formats/strixw.hpp) and its load into HBM (strixite
 * runtime/strixw_loader.hpp:36-88, Device placement). Handles are opaque; names are NUL-terminated. The file, its
 * tensors and metadata stay valid until strix_strixw_close. role: 0 data, 1 q, 2 scale, 3 min (StrixwRole);
 * encoding: StrixwEncoding's values (1 q4 ... 9 q5). */
/* strixite formats/strixw.hpp:58 strix_hash64 */
uint64_t strix_strixw_hash64(const void *p, size_t n);
typedef struct {
    const char *name;
    int encoding, ndim;
    int64_t shape[8];
    int64_t group_size, experts, nparts;
    int ncomponents;
    int role[4];
    uint64_t offset[4], bytes[4], hash[4];
} strix_strixw_tensor_info;
/* strixite formats/strixw.hpp:111-130 StrixwFile */
int strix_strixw_open(const char *path, void **file);
int strix_strixw_close(void *file);
int strix_strixw_info(void *file, uint64_t *file_bytes, uint64_t *data_offset, uint32_t *version, int64_t *ntensors,
                      int64_t *nmeta);
int strix_strixw_tensor(void *file, int64_t i, strix_strixw_tensor_info *out);
int strix_strixw_find(void *file, const char *name, int64_t *index); /* index -1 when absent */
int strix_strixw_part(void *file, int64_t tensor, int64_t part, const char **source, int64_t *row_offset,
                      int64_t *rows);
int strix_strixw_meta(void *file, int64_t i, const char **key, const char **value);
int strix_strixw_verify(void *file, int threads);
/* strixite formats/strixw.hpp:82-109 StrixwWriter: plan (name, encoding, shape, group size, experts, and the
 * checkpoint tensors its rows came from: nparts sources of part_rows[i] rows each, consecutive), write each
 * component once, finish. */
typedef struct {
    const char *name;
    int encoding, ndim;
    int64_t shape[8];
    int64_t group_size, experts;
    int64_t nparts;
    const char *const *part_sources;
    const int64_t *part_rows;
} strix_strixw_plan_t;
int strix_strixw_writer_create(const char *path, int64_t nmeta, const char *const *keys, const char *const *values,
                               int64_t ntensors, const strix_strixw_plan_t *plan, void **writer);
int strix_strixw_writer_write(void *writer, int64_t tensor, int role, const void *data, size_t bytes);
int strix_strixw_writer_finish(void *writer);
int strix_strixw_writer_destroy(void *writer);
/* strixite runtime/strixw_loader.hpp:42-60 StrixwDevice (the data region in one HBM allocation on the current
 * device); ptr: the device address of a tensor's component. */
int strix_strixw_device_load(const char *path, int read_threads, void **dev);
int strix_strixw_device_free(void *dev);
int strix_strixw_device_info(void *dev, uint64_t *device_bytes, double *load_seconds);
int strix_strixw_device_ptr(void *dev, const char *name, int role, const void **ptr);
/* the MoE sublayer's weights of one decoder layer (strixite runtime/qwen4exp.cpp:147-156): prefix
 * "model.language_model.layers.N."; the views point into dev's allocation. */
int strix_strixw_moe_layer(void *dev, const char *prefix, int64_t top_k, strix_moe_layer_weights *out);

/* Calibration kernels for the bench (no reference counterpart): dense f16 MFMA chains on `blocks` blocks of 4 waves
 * for `iters` iterations (returns the flops launched, -1 on error), and a plain streaming read of `bytes` bytes.
 * Asynchronous on stream; out: one float of device scratch. */
int64_t strix_calib_mfma_peak(int64_t blocks, int iters, float *out, void *stream);
int strix_calib_read_peak(const void *p, int64_t bytes, int64_t blocks, float *out, void *stream);
/* The FP32 -> BF16 rounding every kernel of this library stores with (no reference counterpart; the tests pin it
 * against the reference's integer RNE, strixite common/bf16.hpp:19-26): y[i] = bf16(x[i]), n elements. */
int strix_calib_bf16_round(const float *x, uint16_t *y, int64_t n, void *stream);

/* Seeded synthetic tensors on the device (no reference counterpart: the bench's input generator). Element i of a
 * tensor is a function of (key, i) only; key = strix_synth_tensor_key(seed, tensor id, layer). */
uint64_t strix_synth_tensor_key(uint64_t seed, uint32_t tensor, uint32_t layer);
int strix_synth_bf16_normal(uint64_t key, float sigma, uint16_t *out, int64_t n, void *stream);
int strix_synth_q_weight(int bits, uint64_t key_codes, uint64_t key_scales, int64_t rows, int64_t K, int64_t G,
                         uint8_t *q, uint16_t *scale, uint16_t *minv, void *stream);
int strix_synth_uniform_pm1(uint64_t key, float *out, int64_t n, void *stream);

#ifdef __cplusplus
}
#endif
#endif
