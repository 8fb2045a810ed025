/*
 * CPU oracle for the quantized MoE FFN path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference algorithm (strixite: kernels/moe_router.hip, kernels/moe_grouped.hip,
 * kernels/linear_q4.hip, kernels/swiglu.hip, formats/q4.cpp, formats/q8.cpp). Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it, and there only as the checker or the timed CPU baseline; the product
 * path (strixite_amd/) never calls it.
 *
 * Every function names the reference file:line it follows. How each one is pinned (golden vectors from the
 * reference's own quantizer, closed forms, brute force, invariants) is written beside it; a function with no
 * such check says "parity unpinned".
 *
 * Arithmetic is IEEE binary32 with FP contraction off (built with -ffp-contract=off); fmaf() is written where a
 * fused multiply-add is meant.
 */
#ifndef STRIX_MOE_ORACLE_H
#define STRIX_MOE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 bits (strixite common/bf16.hpp:19-26: RNE, NaN kept quiet) ---- */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t b);

/* ---- seeded synthetic data: counter-based SplitMix64, identical bytes on the CPU and the GPU ---- */
uint64_t orc_splitmix64(uint64_t z);
uint64_t orc_tensor_key(uint64_t seed, uint32_t tensor, uint32_t layer);
/* approximately N(0, sigma): Irwin-Hall sum of four 16-bit uniforms, standardized, one float multiply,
 * rounded RNE to bf16. No transcendental function, so CPU and GPU produce the same bits. */
float orc_gen_normal(uint64_t key, uint64_t i, float sigma);
void orc_gen_bf16_normal(uint64_t key, float sigma, uint16_t *out, int64_t n);
/* Q4 experts: codes uniform 0..15, scale bf16(|N(0,0.02)|), min bf16(-8 s).  Q8: signed c uniform in
 * [-127, 127] stored u = c + 128, min bf16(-128 s). rows x K codes, groups of G. */
void orc_gen_q4(uint64_t key_codes, uint64_t key_scales, int64_t rows, int64_t K, int64_t G, uint8_t *q,
                uint16_t *scale, uint16_t *minv);
void orc_gen_q8(uint64_t key_codes, uint64_t key_scales, int64_t rows, int64_t K, int64_t G, uint8_t *q,
                uint16_t *scale, uint16_t *minv);
/* f32 uniform in [-1, 1): 24-bit integer times 2^-23 minus 1, exact. */
void orc_gen_uniform_pm1(uint64_t key, float *out, int64_t n);

/* ---- formats (strixite formats/q4.hpp:3-6, formats/q4.cpp:44-134, formats/q8.hpp:3-10, formats/q8.cpp:43-127) ---- */
/* returns 0, or -1 on bad shape / non-finite input (the reference throws). */
int orc_quantize_q4(const float *w, int64_t N, int64_t K, int64_t G, uint8_t *q, uint16_t *scale, uint16_t *minv);
int orc_quantize_q8(const float *w, int64_t N, int64_t K, int64_t G, uint8_t *q, uint16_t *scale, uint16_t *minv);
void orc_dequantize(int bits, const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t N, int64_t K,
                    int64_t G, float *w);
void orc_dequantize_row(int bits, const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t row,
                        int64_t K, int64_t G, float *w);

/* ---- router ---- */
/* y[m, n] = x[m, :] . w[n, :] in the canonical order every product of this build uses (bf16 in, f32 out):
 * lane l of 64 accumulates the 8-element chunks c = l, l + 64, ... with fmaf, element order inside a chunk,
 * then a butterfly over the lanes (offsets 32, 16, 8, 4, 2, 1). Follows linear_bf16w's FP32 semantics
 * (strixite kernels/linear.hpp:1-26, kernels/linear.hip:83-147); its order is the one this build specifies.
 * bias (optional, E entries) is added once in FP32 to columns < n_bias. */
void orc_router_logits(const uint16_t *x, const uint16_t *w, int64_t M, int64_t N, int64_t K, const float *bias,
                       int64_t n_bias, float *y, int threads);
/* one dot in that order (the unit the GPU's canonical re-check computes) */
float orc_canonical_dot(const uint16_t *x, const uint16_t *w, int64_t K);

/* strixite kernels/moe_router.hpp:3-23, moe_router.hip:32-112: top-k (larger first, ties -> lower index),
 * softmax over the k picks, shared slot sigmoid; a non-finite logit fails that token (ids -1, coef NaN,
 * err = {1, m, smallest bad expert (E = shared)}, first token in token order). Returns 0 or -1 on bad args. */
int orc_topk(const float *logits, int64_t ld, int64_t M, int64_t E, int64_t k, const float *shared,
             int64_t shared_ld, int32_t shared_id, int32_t *ids, float *coef, uint32_t *err);

/* ---- ragged packing (strixite kernels/moe_grouped.hip:89-188) ----
 * counts per bucket (E experts, bucket E = invalid ids), offsets[E + 2] exclusive scan (offsets[E + 1] = S),
 * slots[S] grouped by bucket, ascending slot order inside a bucket (the stable order); err = first invalid slot
 * {1, id, slot}. */
void orc_group_routes(const int32_t *ids, int64_t M, int64_t A, int64_t E, int32_t *offsets, int32_t *slots,
                      uint32_t *err);

/* ---- expert math (FP32 reference semantics, strixite kernels/linear_q4.hpp:32-58, moe_grouped.hpp:3-16) ---- */
typedef struct {
    int bits; /* 4 or 8 */
    const uint8_t *q;
    const uint16_t *scale, *minv;
    int64_t N, K, G; /* the stacked [E * N_expert, K] matrix */
} orc_qview;

float orc_silu(float v); /* v / (1 + expf(-v)), strixite kernels/swiglu.hip:22 */
/* h[s, j] = bf16(silu(g) * u) for every slot s = m * A + a, g / u the FP32 dots of x[m] with expert ids[s]'s gate
 * row j and up row I + j (I = N_expert / 2) of the exact dequantized weights. Invalid id -> NaN row. */
void orc_experts_gate_up_swiglu(const uint16_t *x, const orc_qview *w, int64_t E, const int32_t *ids, int64_t M,
                                int64_t A, uint16_t *h, int threads);
/* partial[s, n] = h[s, :] . Wd[ids[s]] row n, FP32 (invalid id -> NaN row). */
void orc_experts_down(const uint16_t *h, const orc_qview *w, int64_t E, const int32_t *ids, int64_t M, int64_t A,
                      float *partial, int threads);
/* dense: y[m, n] = x[m, :] . W row n (FP32), the shared expert's projections. */
void orc_dense(const uint16_t *x, const orc_qview *w, int64_t M, float *y, int threads);
/* strixite kernels/swiglu.hip:31-36, the bf16 form: h = bf16(bf16(silu(g)) * u) on bf16 g, u */
void orc_swiglu_bf16(const uint16_t *gu, uint16_t *h, int64_t rows, int64_t I);

/* strixite kernels/moe_grouped.hip:948-985 (combine_reduce_kernel): y[m, n] = sum_a coef * partial in slot order
 * (fmaf), NaN if any id of the token is invalid; with s (shared expert output, bf16) and gate logits:
 * y = bf16(bf16(sum) + sigmoid(gl) * s) (moe_shared_add's arithmetic, moe_router.hip:129-146); then, with
 * resid, out[m, n] = bf16(resid + y) (the residual write). */
void orc_combine(const float *partial, const int32_t *ids, const float *coef, int64_t M, int64_t A, int64_t E,
                 int64_t N, const uint16_t *s, const float *gate_logit, int64_t gate_ld, uint16_t *y,
                 const uint16_t *resid, uint16_t *out);

/* ---- the whole MoE sublayer (strixite runtime/qwen4exp.cpp:3143-3217 order) ---- */
typedef struct {
    int64_t M, H, E, k, I;
    const uint16_t *x;          /* [M, H] bf16 */
    const uint16_t *router;     /* [E + has_shared, H] bf16; row E = shared gate */
    const float *router_bias;   /* optional [E] */
    const float *logits_in;     /* optional [M, ld_in]: bypasses the router GEMV (uniform-logit configs) */
    int64_t ld_in;
    orc_qview gate_up, down;    /* routed experts, stacked */
    int has_shared;
    orc_qview sh_gate_up, sh_down;
    /* the shared expert stacked as expert E of gate_up / down (strixite formats/merge_plan.cpp:31-41; has_shared
     * 0): routed as slot k of every token, id E, coef sigmoid(logit E) (moe_router's shared slot,
     * kernels/moe_router.hip:108-111), so A = k + 1 and the expert views hold E + 1 experts */
    int shared_stacked;
} orc_layer;

typedef struct {
    float *logits;      /* [M, E + (has_shared or shared_stacked)] */
    int32_t *ids;       /* [M, A], A = k (+ 1 stacked) */
    float *coef;        /* [M, A] */
    int32_t *offsets;   /* [E' + 2], E' = E (+ 1 stacked) */
    int32_t *slots;     /* [M * A] */
    uint16_t *h;        /* [M * A, I] */
    float *partial;     /* [M * A, H] */
    uint16_t *sh_h;     /* [M, I] (has_shared) */
    uint16_t *sh_s;     /* [M, H] (has_shared) */
    uint16_t *y;        /* [M, H] MoE output */
    uint16_t *out;      /* [M, H] x + y */
    uint32_t err_router[3], err_route[3];
} orc_layer_out;

int orc_moe_layer(const orc_layer *L, orc_layer_out *o, int threads);

/* strixw's component / header / index hash, one shot (strixite formats/strixw.cpp:204-246: four lanes seeded by the
 * length, 32-byte blocks, the tail's 8-byte words then its last bytes tagged with their count, a fold and a finish). */
uint64_t orc_strixw_hash64(const void *p, uint64_t n);

#ifdef __cplusplus
}
#endif
#endif
