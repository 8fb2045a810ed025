/*
 * CPU oracle for the quantized MoE FFN path — TEST INFRASTRUCTURE ONLY (see moe_oracle.h).
 *
 * Pinning (what checks each part; tests/test_oracle.py runs them):
 *   bf16 RNE ............ closed form + the reference's own f32_to_bf16 via oracle/_ref golden vectors
 *   quantize/dequantize . golden vectors written by the reference's formats/q4.cpp, q8.cpp (tests/golden/)
 *   router logits ....... brute-force double dot (error bound) + order-exactness against a per-lane restatement
 *   top-k / softmax ..... brute-force sort on tiny E, special cases (ties, all-equal, k = E, NaN / inf)
 *   packing ............. textbook counting sort invariants + brute force
 *   expert math ......... closed form via dequantize-then-matmul in float64 (numpy)
 *   combine ............. closed form in float64
 *   generator ........... no reference counterpart (harness-side); pinned by the GPU generator producing the same bytes
 */
#include "moe_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------------------------ */
/* bf16: strixite common/bf16.hpp:19-26 (round to nearest even, NaN payload kept quiet) */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0x007fffffu) ? 0x0040u : 0u));
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* parallel for over [0, n) in contiguous blocks */
typedef void (*orc_body)(void *ctx, int64_t lo, int64_t hi);
typedef struct {
    orc_body fn;
    void *ctx;
    int64_t lo, hi;
} orc_task;

static void *orc_run_task(void *p) {
    orc_task *t = (orc_task *)p;
    if (t->lo < t->hi) t->fn(t->ctx, t->lo, t->hi);
    return NULL;
}

static void orc_parallel_for(int64_t n, int threads, orc_body fn, void *ctx) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    if (threads == 1 || n < 2) {
        fn(ctx, 0, n);
        return;
    }
    if (threads > n) threads = (int)n;
    pthread_t th[256];
    orc_task task[256];
    for (int i = 0; i < threads; ++i) {
        task[i].fn = fn, task[i].ctx = ctx;
        task[i].lo = n * i / threads, task[i].hi = n * (i + 1) / threads;
    }
    for (int i = 1; i < threads; ++i) pthread_create(&th[i], NULL, orc_run_task, &task[i]);
    orc_run_task(&task[0]);
    for (int i = 1; i < threads; ++i) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* generator: SplitMix64 (Steele, Lea, Flood 2014) as a counter-based hash */
uint64_t orc_splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t orc_tensor_key(uint64_t seed, uint32_t tensor, uint32_t layer) {
    return orc_splitmix64(orc_splitmix64(seed) ^ ((uint64_t)tensor << 32) ^ (uint64_t)layer);
}

static uint64_t orc_hash(uint64_t key, uint64_t i) { return orc_splitmix64(key ^ (i * 0xD1B54A32D192ED03ull)); }

/* 1 / standard deviation of the sum of four uniforms on {0..65535}: sqrt((65536^2 - 1) / 3) = 37837.2265... */
#define ORC_IH_INV_SD 2.6428722e-05f
#define ORC_IH_MEAN 131070

float orc_gen_normal(uint64_t key, uint64_t i, float sigma) {
    const uint64_t h = orc_hash(key, i);
    const int32_t n = (int32_t)(h & 0xFFFF) + (int32_t)((h >> 16) & 0xFFFF) + (int32_t)((h >> 32) & 0xFFFF) +
                      (int32_t)(h >> 48);
    const float sf = sigma * ORC_IH_INV_SD;
    return (float)(n - ORC_IH_MEAN) * sf;
}

void orc_gen_bf16_normal(uint64_t key, float sigma, uint16_t *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(orc_gen_normal(key, (uint64_t)i, sigma));
}

static void gen_scales(uint64_t key_scales, int64_t n_groups, float min_mul, uint16_t *scale, uint16_t *minv) {
    for (int64_t g = 0; g < n_groups; ++g) {
        const float z = orc_gen_normal(key_scales, (uint64_t)g, 0.02f);
        const uint16_t sb = orc_f32_to_bf16(fabsf(z));
        scale[g] = sb;
        minv[g] = orc_f32_to_bf16(min_mul * orc_bf16_to_f32(sb));
    }
}

void orc_gen_q4(uint64_t key_codes, uint64_t key_scales, int64_t rows, int64_t K, int64_t G, uint8_t *q,
                uint16_t *scale, uint16_t *minv) {
    const int64_t nbytes = rows * K / 2;
    for (int64_t i = 0; i < nbytes; ++i) q[i] = (uint8_t)(orc_hash(key_codes, (uint64_t)(i >> 3)) >> (8 * (i & 7)));
    gen_scales(key_scales, rows * (K / G), -8.0f, scale, minv);
}

void orc_gen_q8(uint64_t key_codes, uint64_t key_scales, int64_t rows, int64_t K, int64_t G, uint8_t *q,
                uint16_t *scale, uint16_t *minv) {
    const int64_t n = rows * K;
    for (int64_t i = 0; i < n; ++i) {
        const uint32_t f = (uint32_t)(orc_hash(key_codes, (uint64_t)(i >> 2)) >> (16 * (i & 3))) & 0xFFFFu;
        q[i] = (uint8_t)(f % 255u + 1u); /* c = f % 255 - 127 in [-127, 127], stored c + 128 */
    }
    gen_scales(key_scales, rows * (K / G), -128.0f, scale, minv);
}

void orc_gen_uniform_pm1(uint64_t key, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const uint32_t v = (uint32_t)(orc_hash(key, (uint64_t)i) >> 40); /* 24 bits */
        out[i] = (float)v * 1.1920928955078125e-07f - 1.0f;               /* v * 2^-23 - 1, exact */
    }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* formats: strixite formats/q4.cpp:44-86 (quantize_q4), :121-134 (dequantize_q4); formats/q8.cpp:43-80, :117-127 */
static int group_ok(int64_t N, int64_t K, int64_t G) {
    return N >= 1 && K >= 1 && (G == 32 || G == 64 || G == 128) && K % G == 0;
}

static int quantize(int levels, const float *w, int64_t N, int64_t K, int64_t G, uint8_t *q, uint16_t *scale,
                    uint16_t *minv) {
    if (!w || !group_ok(N, K, G)) return -1;
    if (levels == 15) memset(q, 0, (size_t)(N * K / 2));
    for (int64_t n = 0; n < N; ++n)
        for (int64_t g = 0; g < K / G; ++g) {
            const float *grp = w + n * K + g * G;
            float lo = grp[0], hi = grp[0];
            for (int64_t i = 0; i < G; ++i) {
                if (!isfinite(grp[i])) return -1;
                lo = fminf(lo, grp[i]);
                hi = fmaxf(hi, grp[i]);
            }
            const uint16_t sb = orc_f32_to_bf16((hi - lo) / (float)levels), mb = orc_f32_to_bf16(lo);
            const float s = orc_bf16_to_f32(sb), m = orc_bf16_to_f32(mb);
            scale[n * (K / G) + g] = sb;
            minv[n * (K / G) + g] = mb;
            for (int64_t i = 0; i < G; ++i) {
                int code = 0;
                if (s > 0.0f) {
                    const float r = nearbyintf((grp[i] - m) / s); /* round half to even */
                    code = (int)fminf(fmaxf(r, 0.0f), (float)levels);
                }
                const int64_t k = g * G + i;
                if (levels == 15) q[(n * K + k) / 2] |= (uint8_t)(code << ((k & 1) ? 4 : 0));
                else q[n * K + k] = (uint8_t)code;
            }
        }
    return 0;
}

int orc_quantize_q4(const float *w, int64_t N, int64_t K, int64_t G, uint8_t *q, uint16_t *scale, uint16_t *minv) {
    return quantize(15, w, N, K, G, q, scale, minv);
}

int orc_quantize_q8(const float *w, int64_t N, int64_t K, int64_t G, uint8_t *q, uint16_t *scale, uint16_t *minv) {
    return quantize(255, w, N, K, G, q, scale, minv);
}

void orc_dequantize_row(int bits, const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t row,
                        int64_t K, int64_t G, float *w) {
    const uint16_t *sr = scale + row * (K / G), *mr = minv + row * (K / G);
    for (int64_t g = 0; g < K / G; ++g) {
        const float s = orc_bf16_to_f32(sr[g]), m = orc_bf16_to_f32(mr[g]);
        for (int64_t i = 0; i < G; ++i) {
            const int64_t k = g * G + i;
            int code;
            if (bits == 4) code = (q[(row * K + k) / 2] >> ((k & 1) ? 4 : 0)) & 0xF;
            else code = q[row * K + k];
            const float t = (float)code * s; /* two roundings, no FMA: formats/q4.cpp:121-134 */
            w[k] = t + m;
        }
    }
}

void orc_dequantize(int bits, const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t N, int64_t K,
                    int64_t G, float *w) {
    for (int64_t n = 0; n < N; ++n) orc_dequantize_row(bits, q, scale, minv, n, K, G, w + n * K);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* router logits in the canonical order (see moe_oracle.h) */
float orc_canonical_dot(const uint16_t *x, const uint16_t *w, int64_t K) {
    float lane[64];
    const int64_t chunks = (K + 7) / 8;
    for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int64_t c = l; c < chunks; c += 64)
            for (int i = 0; i < 8; ++i) {
                const int64_t k = c * 8 + i;
                if (k < K) acc = fmaf(orc_bf16_to_f32(x[k]), orc_bf16_to_f32(w[k]), acc);
            }
        lane[l] = acc;
    }
    for (int off = 32; off > 0; off >>= 1)
        for (int l = 0; l < off; ++l) lane[l] = lane[l] + lane[l + off];
    return lane[0];
}

typedef struct {
    const uint16_t *x, *w;
    int64_t M, N, K, n_bias;
    const float *bias;
    float *y;
} router_ctx;

static void router_body(void *p, int64_t lo, int64_t hi) {
    router_ctx *c = (router_ctx *)p;
    for (int64_t i = lo; i < hi; ++i) {
        const int64_t m = i / c->N, n = i % c->N;
        float v = orc_canonical_dot(c->x + m * c->K, c->w + n * c->K, c->K);
        if (c->bias && n < c->n_bias) v = v + c->bias[n];
        c->y[m * c->N + n] = v;
    }
}

void orc_router_logits(const uint16_t *x, const uint16_t *w, int64_t M, int64_t N, int64_t K, const float *bias,
                       int64_t n_bias, float *y, int threads) {
    router_ctx c = {x, w, M, N, K, n_bias, bias, y};
    orc_parallel_for(M * N, threads, router_body, &c);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* top-k: strixite kernels/moe_router.hip:32-112 */
int orc_topk(const float *logits, int64_t ld, int64_t M, int64_t E, int64_t k, const float *shared,
             int64_t shared_ld, int32_t shared_id, int32_t *ids, float *coef, uint32_t *err) {
    if (!logits || !ids || !coef || !err || M < 1 || E < 1 || E > 1024 || k < 1 || k > E || k > 32 || ld < E)
        return -1;
    const int64_t A = k + (shared ? 1 : 0);
    uint8_t *taken = (uint8_t *)malloc((size_t)E);
    for (int64_t m = 0; m < M; ++m) {
        const float *row = logits + m * ld;
        int64_t bad = -1;
        for (int64_t e = 0; e < E && bad < 0; ++e)
            if (!isfinite(row[e])) bad = e;
        const float sl = shared ? shared[m * shared_ld] : 0.0f;
        if (bad < 0 && shared && !isfinite(sl)) bad = E;
        if (bad >= 0) {
            if (err[0] == 0) err[0] = 1, err[1] = (uint32_t)m, err[2] = (uint32_t)bad;
            for (int64_t a = 0; a < A; ++a) ids[m * A + a] = -1, coef[m * A + a] = bits_f32(0x7fc00000u);
            continue;
        }
        memset(taken, 0, (size_t)E);
        float v[32];
        for (int64_t r = 0; r < k; ++r) {
            int64_t bi = -1;
            for (int64_t e = 0; e < E; ++e)
                if (!taken[e] && (bi < 0 || row[e] > row[bi])) bi = e; /* strict >: ties keep the lower index */
            taken[bi] = 1;
            ids[m * A + r] = (int32_t)bi;
            v[r] = row[bi];
        }
        float ex[32], sum = 0.0f;
        for (int64_t r = 0; r < k; ++r) ex[r] = expf(v[r] - v[0]), sum += ex[r];
        for (int64_t r = 0; r < k; ++r) coef[m * A + r] = ex[r] / sum;
        if (shared) {
            ids[m * A + k] = shared_id;
            coef[m * A + k] = 1.0f / (1.0f + expf(-sl));
        }
    }
    free(taken);
    return 0;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* packing: strixite kernels/moe_grouped.hip:136-188, with the stable order inside a bucket */
void orc_group_routes(const int32_t *ids, int64_t M, int64_t A, int64_t E, int32_t *offsets, int32_t *slots,
                      uint32_t *err) {
    const int64_t S = M * A;
    int32_t *cnt = (int32_t *)calloc((size_t)(E + 1), 4);
    for (int64_t s = 0; s < S; ++s) {
        const int32_t id = ids[s];
        const int bad = id < 0 || id >= E;
        cnt[bad ? E : id]++;
        if (bad && err[0] == 0) err[0] = 1, err[1] = (uint32_t)id, err[2] = (uint32_t)s;
    }
    int32_t run = 0;
    for (int64_t b = 0; b <= E; ++b) offsets[b] = run, run += cnt[b];
    offsets[E + 1] = run;
    for (int64_t b = 0; b <= E; ++b) cnt[b] = offsets[b];
    for (int64_t s = 0; s < S; ++s) {
        const int32_t id = ids[s];
        slots[cnt[(id < 0 || id >= E) ? E : id]++] = (int32_t)s;
    }
    free(cnt);
}

/* ------------------------------------------------------------------------------------------------------------ */
/* expert math */
float orc_silu(float v) { return v / (1.0f + expf(-v)); }

/* sixteen interleaved fmaf partial sums then a pairwise tree: one fixed order, vectorizable */
static float dotf(const float *a, const float *b, int64_t K) {
    float acc[16] = {0};
    int64_t k = 0;
    for (; k + 16 <= K; k += 16)
        for (int i = 0; i < 16; ++i) acc[i] = fmaf(a[k + i], b[k + i], acc[i]);
    for (int i = 0; k < K; ++k, ++i) acc[i] = fmaf(a[k], b[k], acc[i]);
    for (int off = 8; off > 0; off >>= 1)
        for (int i = 0; i < off; ++i) acc[i] = acc[i] + acc[i + off];
    return acc[0];
}

static void widen(const uint16_t *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_bf16_to_f32(src[i]);
}

/* grouping of slots by expert, shared by the expert functions */
typedef struct {
    int32_t *offsets, *slots;
} orc_groups;

static orc_groups make_groups(const int32_t *ids, int64_t M, int64_t A, int64_t E) {
    orc_groups g;
    uint32_t err[3] = {0, 0, 0};
    g.offsets = (int32_t *)malloc((size_t)(E + 2) * 4);
    g.slots = (int32_t *)malloc((size_t)(M * A) * 4);
    orc_group_routes(ids, M, A, E, g.offsets, g.slots, err);
    return g;
}

typedef struct {
    const float *xf; /* [rows_in, K] widened inputs */
    int64_t A;       /* slot -> input row: slot / A (gate_up) or slot (down) */
    const orc_qview *w;
    int64_t E, Ne, K;
    orc_groups g;
    int64_t row_chunks; /* per expert */
    int mode;           /* 0: gate_up + swiglu -> h (bf16), 1: down -> partial (f32) */
    uint16_t *h;
    float *partial;
} expert_ctx;

#define ORC_ROW_CHUNK 64

static void expert_body(void *p, int64_t lo, int64_t hi) {
    expert_ctx *c = (expert_ctx *)p;
    const int64_t K = c->K, G = c->w->G;
    float *wa = (float *)malloc((size_t)K * 4), *wb = (float *)malloc((size_t)K * 4);
    for (int64_t t = lo; t < hi; ++t) {
        const int64_t e = t / c->row_chunks, rc = t % c->row_chunks;
        const int32_t b0 = c->g.offsets[e], b1 = c->g.offsets[e + 1];
        if (b0 == b1) continue;
        if (c->mode == 0) {
            const int64_t I = c->Ne / 2;
            for (int64_t j = rc * ORC_ROW_CHUNK; j < (rc + 1) * ORC_ROW_CHUNK && j < I; ++j) {
                orc_dequantize_row(c->w->bits, c->w->q, c->w->scale, c->w->minv, e * c->Ne + j, K, G, wa);
                orc_dequantize_row(c->w->bits, c->w->q, c->w->scale, c->w->minv, e * c->Ne + I + j, K, G, wb);
                for (int32_t i = b0; i < b1; ++i) {
                    const int64_t s = c->g.slots[i];
                    const float *xr = c->xf + (s / c->A) * K;
                    const float gv = dotf(xr, wa, K), uv = dotf(xr, wb, K);
                    c->h[s * I + j] = orc_f32_to_bf16(orc_silu(gv) * uv);
                }
            }
        } else {
            for (int64_t n = rc * ORC_ROW_CHUNK; n < (rc + 1) * ORC_ROW_CHUNK && n < c->Ne; ++n) {
                orc_dequantize_row(c->w->bits, c->w->q, c->w->scale, c->w->minv, e * c->Ne + n, K, G, wa);
                for (int32_t i = b0; i < b1; ++i) {
                    const int64_t s = c->g.slots[i];
                    c->partial[s * c->Ne + n] = dotf(c->xf + s * K, wa, K);
                }
            }
        }
    }
    free(wa);
    free(wb);
}

static void nan_invalid_rows(const orc_groups *g, int64_t E, int64_t width, uint16_t *h, float *partial) {
    for (int32_t i = g->offsets[E]; i < g->offsets[E + 1]; ++i) {
        const int64_t s = g->slots[i];
        for (int64_t j = 0; j < width; ++j) {
            if (h) h[s * width + j] = 0x7fc0;
            if (partial) partial[s * width + j] = bits_f32(0x7fc00000u);
        }
    }
}

void orc_experts_gate_up_swiglu(const uint16_t *x, const orc_qview *w, int64_t E, const int32_t *ids, int64_t M,
                                int64_t A, uint16_t *h, int threads) {
    const int64_t K = w->K, Ne = w->N / E, I = Ne / 2;
    float *xf = (float *)malloc((size_t)(M * K) * 4);
    widen(x, xf, M * K);
    expert_ctx c;
    memset(&c, 0, sizeof c);
    c.xf = xf, c.A = A, c.w = w, c.E = E, c.Ne = Ne, c.K = K, c.mode = 0, c.h = h;
    c.g = make_groups(ids, M, A, E);
    c.row_chunks = (I + ORC_ROW_CHUNK - 1) / ORC_ROW_CHUNK;
    orc_parallel_for(E * c.row_chunks, threads, expert_body, &c);
    nan_invalid_rows(&c.g, E, I, h, NULL);
    free(c.g.offsets);
    free(c.g.slots);
    free(xf);
}

void orc_experts_down(const uint16_t *h, const orc_qview *w, int64_t E, const int32_t *ids, int64_t M, int64_t A,
                      float *partial, int threads) {
    const int64_t K = w->K, Ne = w->N / E;
    float *hf = (float *)malloc((size_t)(M * A * K) * 4);
    widen(h, hf, M * A * K);
    expert_ctx c;
    memset(&c, 0, sizeof c);
    c.xf = hf, c.A = 1, c.w = w, c.E = E, c.Ne = Ne, c.K = K, c.mode = 1, c.partial = partial;
    c.g = make_groups(ids, M, A, E);
    c.row_chunks = (Ne + ORC_ROW_CHUNK - 1) / ORC_ROW_CHUNK;
    orc_parallel_for(E * c.row_chunks, threads, expert_body, &c);
    nan_invalid_rows(&c.g, E, Ne, NULL, partial);
    free(c.g.offsets);
    free(c.g.slots);
    free(hf);
}

typedef struct {
    const float *xf;
    const orc_qview *w;
    int64_t M;
    float *y;
} dense_ctx;

static void dense_body(void *p, int64_t lo, int64_t hi) {
    dense_ctx *c = (dense_ctx *)p;
    const int64_t K = c->w->K, N = c->w->N;
    float *wr = (float *)malloc((size_t)K * 4);
    for (int64_t n = lo; n < hi; ++n) {
        orc_dequantize_row(c->w->bits, c->w->q, c->w->scale, c->w->minv, n, K, c->w->G, wr);
        for (int64_t m = 0; m < c->M; ++m) c->y[m * N + n] = dotf(c->xf + m * K, wr, K);
    }
    free(wr);
}

void orc_dense(const uint16_t *x, const orc_qview *w, int64_t M, float *y, int threads) {
    float *xf = (float *)malloc((size_t)(M * w->K) * 4);
    widen(x, xf, M * w->K);
    dense_ctx c = {xf, w, M, y};
    orc_parallel_for(w->N, threads, dense_body, &c);
    free(xf);
}

void orc_swiglu_bf16(const uint16_t *gu, uint16_t *h, int64_t rows, int64_t I) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t j = 0; j < I; ++j) {
            const float g = orc_bf16_to_f32(gu[r * 2 * I + j]), u = orc_bf16_to_f32(gu[r * 2 * I + I + j]);
            const float s = orc_bf16_to_f32(orc_f32_to_bf16(orc_silu(g)));
            h[r * I + j] = orc_f32_to_bf16(s * u);
        }
}

void orc_combine(const float *partial, const int32_t *ids, const float *coef, int64_t M, int64_t A, int64_t E,
                 int64_t N, const uint16_t *s, const float *gate_logit, int64_t gate_ld, uint16_t *y,
                 const uint16_t *resid, uint16_t *out) {
    for (int64_t m = 0; m < M; ++m) {
        int ok = 1;
        for (int64_t a = 0; a < A; ++a) ok = ok && ids[m * A + a] >= 0 && ids[m * A + a] < E;
        float g = 0.0f;
        if (s) {
            const float gl = gate_logit[m * gate_ld];
            g = isfinite(gl) ? 1.0f / (1.0f + expf(-gl)) : bits_f32(0x7fc00000u);
        }
        for (int64_t n = 0; n < N; ++n) {
            float v = 0.0f;
            for (int64_t a = 0; a < A; ++a) v = fmaf(coef[m * A + a], partial[(m * A + a) * N + n], v);
            if (!ok) v = bits_f32(0x7fc00000u);
            if (s) {
                const float t = g * orc_bf16_to_f32(s[m * N + n]);
                v = orc_bf16_to_f32(orc_f32_to_bf16(v)) + t;
            }
            const uint16_t yb = orc_f32_to_bf16(v);
            y[m * N + n] = yb;
            if (resid && out) out[m * N + n] = orc_f32_to_bf16(orc_bf16_to_f32(resid[m * N + n]) + orc_bf16_to_f32(yb));
        }
    }
}

/* ------------------------------------------------------------------------------------------------------------ */
/* the sublayer, strixite runtime/qwen4exp.cpp:3143-3217: router projection, moe_router, grouping, gate_up +
 * SwiGLU, down + ordered combine, shared expert (dense projections, its gated add folded into the combine),
 * then the residual write */
int orc_moe_layer(const orc_layer *L, orc_layer_out *o, int threads) {
    const int stacked = L->shared_stacked && !L->has_shared;
    const int64_t M = L->M, H = L->H, E = L->E, k = L->k, I = L->I, A = k + (stacked ? 1 : 0);
    const int64_t ld = E + (L->has_shared || stacked ? 1 : 0), Es = E + (stacked ? 1 : 0);
    const orc_qview *views[4] = {&L->gate_up, &L->down, &L->sh_gate_up, &L->sh_down};
    for (int i = 0; i < (L->has_shared ? 4 : 2); ++i)
        if (!group_ok(views[i]->N, views[i]->K, views[i]->G) || views[i]->K < views[i]->G) return -1;
    memset(o->err_router, 0, sizeof o->err_router);
    memset(o->err_route, 0, sizeof o->err_route);
    if (L->logits_in) {
        for (int64_t m = 0; m < M; ++m) memcpy(o->logits + m * ld, L->logits_in + m * L->ld_in, (size_t)ld * 4);
    } else {
        orc_router_logits(L->x, L->router, M, ld, H, L->router_bias, L->router_bias ? E : 0, o->logits, threads);
    }
    if (orc_topk(o->logits, ld, M, E, k, stacked ? o->logits + E : NULL, ld, (int32_t)E, o->ids, o->coef,
                 o->err_router) != 0)
        return -1;
    /* the shared gate logit is checked as the router does (moe_shared_add's error) */
    if (L->has_shared)
        for (int64_t m = 0; m < M && o->err_router[0] == 0; ++m)
            if (!isfinite(o->logits[m * ld + E])) o->err_router[0] = 1, o->err_router[1] = (uint32_t)m, o->err_router[2] = (uint32_t)E;
    orc_group_routes(o->ids, M, A, Es, o->offsets, o->slots, o->err_route);
    orc_experts_gate_up_swiglu(L->x, &L->gate_up, Es, o->ids, M, A, o->h, threads);
    orc_experts_down(o->h, &L->down, Es, o->ids, M, A, o->partial, threads);
    if (L->has_shared) {
        float *gu = (float *)malloc((size_t)(M * 2 * I) * 4);
        orc_dense(L->x, &L->sh_gate_up, M, gu, threads);
        for (int64_t m = 0; m < M; ++m)
            for (int64_t j = 0; j < I; ++j)
                o->sh_h[m * I + j] = orc_f32_to_bf16(orc_silu(gu[m * 2 * I + j]) * gu[m * 2 * I + I + j]);
        free(gu);
        float *sf = (float *)malloc((size_t)(M * H) * 4);
        orc_dense(o->sh_h, &L->sh_down, M, sf, threads);
        for (int64_t i = 0; i < M * H; ++i) o->sh_s[i] = orc_f32_to_bf16(sf[i]);
        free(sf);
    }
    orc_combine(o->partial, o->ids, o->coef, M, A, Es, H, L->has_shared ? o->sh_s : NULL,
                L->has_shared ? o->logits + E : NULL, ld, o->y, L->x, o->out);
    return 0;
}

/* ------------------------------------------------------------------------------------------------------------ */
/* strixw hash (strixite formats/strixw.cpp:24-38 mix, :204-246 StrixHasher / strix_hash64), restated one shot */
static uint64_t orc_hmix(uint64_t h, uint64_t w) {
    h ^= w * 0x9e3779b97f4a7c15ull;
    return (h ^ (h >> 31)) * 0xd6e8feb86659fd93ull;
}

uint64_t orc_strixw_hash64(const void *data, uint64_t n) {
    const uint8_t *p = (const uint8_t *)data;
    const uint64_t a = 0x9e3779b97f4a7c15ull, b = 0xd6e8feb86659fd93ull;
    uint64_t h[4] = {n ^ a, n ^ b, ~n ^ a, ~n ^ b}, w;
    uint64_t blocks = n / 32, i;
    for (i = 0; i < blocks; ++i)
        for (int l = 0; l < 4; ++l) {
            memcpy(&w, p + 32 * i + 8 * l, 8);
            h[l] = orc_hmix(h[l], w);
        }
    const uint8_t *t = p + 32 * blocks;
    const uint64_t rest = n - 32 * blocks;
    uint64_t j = 0;
    for (int l = 0; j + 8 <= rest; j += 8, ++l) {
        memcpy(&w, t + j, 8);
        h[l] = orc_hmix(h[l], w);
    }
    if (j < rest) {
        w = 0;
        memcpy(&w, t + j, rest - j);
        h[0] = orc_hmix(h[0], w ^ ((rest - j) << 56));
    }
    uint64_t r = orc_hmix(orc_hmix(orc_hmix(h[0], h[1]), h[2]), h[3]);
    r = (r ^ (r >> 33)) * a;
    return r ^ (r >> 29);
}
