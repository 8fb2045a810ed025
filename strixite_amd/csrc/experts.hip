// Expert projections on gfx950's matrix cores: the grouped gather (+ fused SwiGLU) and combine over Q4 / Q8
// experts, the per-slot decode forms, the dense Q8 projection (the shared expert), the ordered combine reduce
// (the routing-weighted un-permute) and the standalone SwiGLU.
//
// One kernel family does every projection. A wave64 owns a 16-slot token tile (the MFMA's A rows: the slots of one
// expert's bucket, 16 dense tokens, or one slot) and two 16-row weight tiles (B columns; SwiGLU: gate rows j0..j0+15
// and the matching up rows, else 32 consecutive rows). Each K step ("span", one quantization group or half of one)
// a lane loads 16 bytes of codes per weight tile - 64 contiguous bytes per row across the lane's 4 lane groups -,
// its row's scale and min, and 8 activations per MFMA; the codes go to bf16 exactly (common.hpp), one
// v_mfma_f32_16x16x32_bf16 per 32 k, and each span's sum is rescaled on the FP32 accumulator:
//   acc += s * D_span + m' * sum(x over the span)
// D layout: lane (j, g) holds tokens 4g..4g+3 of weight column j, so a lane's outputs share one row's (s, m).
// A span (Q4: 128 codes, Q8: 64) never crosses a group: Q4 needs G = 128, Q8 G = 64 or 128 (the reference's
// served layout: q4g128, q8g64).
#include "common.hpp"

#include <type_traits>

namespace strix::kernels {

namespace route {
// route.hip's workspace layout, as the expert kernels read it (header, offsets, slots, 16-slot tile tables)
__device__ __forceinline__ int64_t t16_bucket_at(int64_t S, int64_t E) { return 4 + E + 2 + S; }
__device__ __forceinline__ int64_t t16_start_at(int64_t S, int64_t E) { return t16_bucket_at(S, E) + S / 16 + E + 2; }
}  // namespace route

namespace {

using namespace strix::dev;

constexpr int kWave = 64, kWaves = 4, kThreads = kWave * kWaves;

enum Mode { GROUPED = 0, DENSE = 1, PERSLOT = 2 };
enum Epi { EPI_SWIGLU = 0, EPI_BF16 = 1, EPI_F32 = 2 };

template <int BITS> struct QFmt {
    static constexpr int CPL = BITS == 4 ? 32 : 16;  // codes per lane per 16-byte load
    static constexpr int SPAN = 4 * CPL;             // codes per row per K step
    static constexpr int NT = CPL / 8;               // MFMAs per K step
};

struct GemmArgs {
    const uint16_t *x;  // A rows (bf16, or f16 bits when XF16), row stride K
    const uint8_t *q;
    const uint16_t *scale, *minv;
    int64_t N;          // weight rows per expert
    int64_t K, G, E, A, M;
    const int32_t *ws;  // GROUPED: the grouping workspace
    const int32_t *ids; // PERSLOT: ids [M, A]
    void *y;            // output rows, stride ldy elements
    int64_t ldy;
    uint32_t *err;      // PERSLOT: the expert error word
};

__device__ __forceinline__ uint4 ld16(const void *p) { return *reinterpret_cast<const uint4 *>(p); }

// f16 activations (the h_f16 form) -> bf16 bits, 8 at a time
__device__ __forceinline__ uint4 f16x8_to_bf16x8(const uint4 &v) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float lo = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xFFFF));
        const float hi = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
        o[i] = (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

template <int BITS> __device__ __forceinline__ Frag b_frag(const uint4 &c, int u) {
    if constexpr (BITS == 4) return q4_codes_to_bf16(u == 0 ? c.x : u == 1 ? c.y : u == 2 ? c.z : c.w);
    else return u == 0 ? q8_codes_to_bf16(c.x, c.y) : q8_codes_to_bf16(c.z, c.w);
}
template <int BITS> __device__ __forceinline__ Frag a_frag(const uint4 &v) {
    if constexpr (BITS == 4) return q4_order(v);
    else return Frag{{v.x, v.y, v.z, v.w}};
}

// The token tile of this block and its expert. Token j of the tile (j < 16) is slot(j), -1 past the tile's rows.
struct Tile {
    int64_t expert;
    bool nan;   // invalid ids: outputs are NaN
    int rows;
    int64_t st;  // GROUPED: first index into slots[]; DENSE: first token; PERSLOT: the slot
};

template <int MODE>
__device__ __forceinline__ bool get_tile(const GemmArgs &a, Tile &t) {
    if constexpr (MODE == GROUPED) {
        const int64_t S = a.ws[1], E = a.ws[2];
        const int64_t tile = blockIdx.y;
        if (tile >= a.ws[0]) return false;
        const int32_t bucket = a.ws[route::t16_bucket_at(S, E) + tile], st = a.ws[route::t16_start_at(S, E) + tile];
        const int32_t end = a.ws[4 + bucket + 1];
        t.rows = end - st < 16 ? end - st : 16;
        t.expert = bucket;
        t.nan = bucket >= a.E;
        t.st = st;
    } else if constexpr (MODE == DENSE) {
        const int64_t m0 = (int64_t)blockIdx.y * 16;
        t.expert = 0;
        t.nan = false;
        t.rows = a.M - m0 < 16 ? (int)(a.M - m0) : 16;
        t.st = m0;
    } else {
        const int64_t slot = blockIdx.y;
        const int32_t id = a.ids[slot];
        t.nan = id < 0 || id >= a.E;
        t.expert = t.nan ? 0 : id;
        t.rows = 1;
        t.st = slot;
        if (t.nan && blockIdx.x == 0 && threadIdx.x == 0 && atomicCAS(&a.err[0], 0u, 1u) == 0u) {
            a.err[1] = (uint32_t)id;
            a.err[2] = (uint32_t)slot;
        }
    }
    return true;
}

template <int MODE> __device__ __forceinline__ int64_t slot_of(const GemmArgs &a, const Tile &t, int j) {
    if (j >= t.rows) return -1;
    if constexpr (MODE == GROUPED) return a.ws[4 + a.ws[2] + 2 + t.st + j];
    else return t.st + j;
}

template <typename T> __device__ __forceinline__ void store1(T *p, float v);
template <> __device__ __forceinline__ void store1<uint16_t>(uint16_t *p, float v) { *p = f32_to_bf16(v); }
template <> __device__ __forceinline__ void store1<float>(float *p, float v) { *p = v; }
// h as f16 bits of its bf16 rounding (the reference's h_f16 form)
__device__ __forceinline__ void store1_hf16(uint16_t *p, float v) {
    *p = __builtin_bit_cast(uint16_t, (_Float16)bf16_round(v));
}

// One 16-token x (2 x 16)-row wave tile over all of K: returns acc[rt][r] = token 4g + r, weight column (lane % 16)
// of tile rt.
template <int BITS, bool XF16>
__device__ __forceinline__ void wave_gemm(const GemmArgs &a, const uint16_t *xrow, const int64_t (&tile_row)[2],
                                          float4v (&acc)[2]) {
    using F = QFmt<BITS>;
    const int lane = threadIdx.x % kWave, g = lane / 16, j = lane % 16;
    const int64_t row_bytes = a.K * BITS / 8, groups = a.K / a.G;
    const uint8_t *qp[2];
    const uint16_t *sp[2], *mp[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const int64_t r = tile_row[rt] + j;
        qp[rt] = a.q + r * row_bytes + g * 16;
        sp[rt] = a.scale + r * groups;
        mp[rt] = a.minv + r * groups;
    }
    const uint16_t *xp = xrow ? xrow + g * F::CPL : nullptr;
    acc[0] = float4v{0, 0, 0, 0};
    acc[1] = float4v{0, 0, 0, 0};
    const int64_t spans = a.K / F::SPAN;
    // software pipeline: span s + 1's loads are in flight during span s's math
    uint4 cq[2], xv[F::NT];
    uint16_t cs[2], cm[2];
    auto fetch = [&](int64_t s) {
        const int64_t gi = s * F::SPAN / a.G;
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            cq[rt] = ld16(qp[rt] + s * 64);
            cs[rt] = sp[rt][gi];
            cm[rt] = mp[rt][gi];
        }
#pragma unroll
        for (int u = 0; u < F::NT; ++u) xv[u] = xp ? ld16(xp + s * F::SPAN + 8 * u) : make_uint4(0, 0, 0, 0);
    };
    fetch(0);
    for (int64_t s = 0; s < spans; ++s) {
        const uint4 q0 = cq[0], q1 = cq[1];
        float sc[2], mn[2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            sc[rt] = bf16_to_f32(cs[rt]);
            mn[rt] = BITS == 4 ? bf16_to_f32(cm[rt]) - 128.0f * sc[rt] : bf16_to_f32(cm[rt]);
        }
        Frag af[F::NT];
        float xs = 0.f;
#pragma unroll
        for (int u = 0; u < F::NT; ++u) {
            const uint4 v = XF16 ? f16x8_to_bf16x8(xv[u]) : xv[u];
            af[u] = a_frag<BITS>(v);
            xs = frag_sum(v, xs);
        }
        if (s + 1 < spans) fetch(s + 1);
        float4v d0 = {0, 0, 0, 0}, d1 = {0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < F::NT; ++u) {
            d0 = mfma_bf16(af[u], b_frag<BITS>(q0, u), d0);
            d1 = mfma_bf16(af[u], b_frag<BITS>(q1, u), d1);
        }
        // the span's activation sum per token: over the 4 lane groups, then to the lanes holding tokens 4g..4g+3
        xs += __shfl_xor(xs, 16, kWave);
        xs += __shfl_xor(xs, 32, kWave);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float xr = __shfl(xs, 4 * g + r, kWave);
            acc[0][r] = fmaf(sc[0], d0[r], fmaf(mn[0], xr, acc[0][r]));
            acc[1][r] = fmaf(sc[1], d1[r], fmaf(mn[1], xr, acc[1][r]));
        }
    }
}

// Grid: x over weight-row blocks (kWaves waves x 32 rows, or x 16 SwiGLU columns), y over token tiles.
template <int BITS, int MODE, int EPI, bool XF16, bool XROW_DIV, bool HF16>
__global__ void __launch_bounds__(kThreads) expert_gemm_kernel(GemmArgs a) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int g = lane / 16, j = lane % 16;
    Tile t;
    if (!get_tile<MODE>(a, t)) return;  // uniform per block; no barrier in this kernel
    const int64_t I = a.N / 2;
    int64_t tile_row[2];
    int64_t c0;  // SwiGLU: first h column; else first output row (within the expert)
    if constexpr (EPI == EPI_SWIGLU) {
        c0 = ((int64_t)blockIdx.x * kWaves + wave) * 16;
        if (c0 >= I) return;
        tile_row[0] = t.expert * a.N + c0;
        tile_row[1] = t.expert * a.N + I + c0;
    } else {
        c0 = ((int64_t)blockIdx.x * kWaves + wave) * 32;
        if (c0 >= a.N) return;
        tile_row[0] = t.expert * a.N + c0;
        tile_row[1] = t.expert * a.N + (c0 + 16 < a.N ? c0 + 16 : c0);  // a.N % 16 == 0: the tile exists or is skipped
    }
    // output rows of this lane's tokens 4g + r
    int64_t orow[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) orow[r] = slot_of<MODE>(a, t, 4 * g + r);
    float4v acc[2];
    if (t.nan) {
        acc[0] = acc[1] = float4v{qnan(), qnan(), qnan(), qnan()};
    } else {
        const int64_t my = slot_of<MODE>(a, t, j);  // this lane's A row (token j)
        const uint16_t *xrow = my < 0 ? nullptr : a.x + (XROW_DIV ? my / a.A : my) * a.K;
        wave_gemm<BITS, XF16>(a, xrow, tile_row, acc);
    }
    if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (orow[r] >= 0) {
                uint16_t *h = static_cast<uint16_t *>(a.y) + orow[r] * a.ldy + c0 + j;
                const float v = t.nan ? qnan() : silu(acc[0][r]) * acc[1][r];
                if constexpr (HF16) store1_hf16(h, v);
                else store1(h, v);
            }
    } else {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const int64_t n = c0 + 16 * rt + j;
            if (rt == 1 && c0 + 16 >= a.N) break;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (orow[r] >= 0) {
                    if constexpr (EPI == EPI_F32) store1(static_cast<float *>(a.y) + orow[r] * a.ldy + n, acc[rt][r]);
                    else store1(static_cast<uint16_t *>(a.y) + orow[r] * a.ldy + n, acc[rt][r]);
                }
        }
    }
}

// Per-slot combine (strixite kernels/linear_q4.hip:283-322): y[m, n] = sum_a coef[m, a] * (h[m, a, :] . Wd[id] row n),
// the slot dots in FP32 from the MFMA (token row 0 of the tile), summed over a in order with fmaf, rounded once.
// Two 16-row tiles a wave. Any invalid id of the token: NaN row, err.
template <int BITS, bool XF16>
__global__ void __launch_bounds__(kThreads) perslot_combine_kernel(GemmArgs a, const float *coef) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int g = lane / 16, j = lane % 16;
    const int64_t m = blockIdx.y;
    const int64_t c0 = ((int64_t)blockIdx.x * kWaves + wave) * 32;
    if (c0 >= a.N) return;
    bool ok = true;
    for (int64_t s = 0; s < a.A; ++s) {
        const int32_t id = a.ids[m * a.A + s];
        if (id < 0 || id >= a.E) {
            ok = false;
            if (blockIdx.x == 0 && threadIdx.x == 0 && atomicCAS(&a.err[0], 0u, 1u) == 0u) {
                a.err[1] = (uint32_t)id;
                a.err[2] = (uint32_t)(m * a.A + s);
            }
            break;
        }
    }
    float out[2] = {0.f, 0.f};
    if (ok) {
        for (int64_t s = 0; s < a.A; ++s) {
            const int64_t e = a.ids[m * a.A + s];
            const int64_t tile_row[2] = {e * a.N + c0, e * a.N + (c0 + 16 < a.N ? c0 + 16 : c0)};
            float4v acc[2];
            wave_gemm<BITS, XF16>(a, j == 0 ? a.x + (m * a.A + s) * a.K : nullptr, tile_row, acc);
            const float c = coef[m * a.A + s];
            out[0] = fmaf(c, acc[0][0], out[0]);
            out[1] = fmaf(c, acc[1][0], out[1]);
        }
    } else {
        out[0] = out[1] = qnan();
    }
    uint16_t *yrow = static_cast<uint16_t *>(a.y) + m * a.ldy;
    if (g == 0) {  // token 0 of the tile: lanes 0..15, r = 0
        store1(yrow + c0 + j, out[0]);
        if (c0 + 16 < a.N) store1(yrow + c0 + 16 + j, out[1]);
    }
}

// y[m, n] = sum_a coef[m, a] * partial[m * A + a, n] in slot order (fmaf), rounded once; NaN for a token with an
// invalid id. SH: y = stored(sum) + sigmoid(gl) * s (strixite kernels/moe_grouped.hip:948-985). RES: x_out = stored(x + y).
// 8 columns a thread (N % 8 == 0).
template <bool SH, bool RES>
__global__ void __launch_bounds__(kThreads)
    combine_reduce_kernel(const float *partial, const int32_t *ids, const float *coef, int64_t M, int64_t A, int64_t E,
                          int64_t N, uint16_t *y, const uint16_t *s, const float *gate_logit, int64_t gate_ld,
                          uint32_t gate_index, uint32_t *err, const uint16_t *resid, uint16_t *out) {
    const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 8;
    if (i >= M * N) return;
    const int64_t m = i / N, n = i % N;
    bool ok = true;
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t s_ = 0; s_ < A; ++s_) {
        const int32_t id = ids[m * A + s_];
        ok = ok && id >= 0 && id < E;
        const float c = coef[m * A + s_];
        const float4 p0 = *reinterpret_cast<const float4 *>(partial + (m * A + s_) * N + n);
        const float4 p1 = *reinterpret_cast<const float4 *>(partial + (m * A + s_) * N + n + 4);
        const float p[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = fmaf(c, p[k], v[k]);
    }
    if (!ok)
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = qnan();
    if constexpr (SH) {
        const float gl = gate_logit[m * gate_ld];
        const bool gok = isfinite(gl);
        if (!gok && n == 0 && atomicCAS(&err[0], 0u, 1u) == 0u) {
            err[1] = (uint32_t)m;
            err[2] = gate_index;
        }
        const float gv = gok ? 1.f / (1.f + expf(-gl)) : qnan();
        const uint4 su = *reinterpret_cast<const uint4 *>(s + i);
        const uint32_t sw[4] = {su.x, su.y, su.z, su.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float sv = __uint_as_float(k % 2 ? sw[k / 2] & 0xffff0000u : sw[k / 2] << 16);
            const float tv = gv * sv;
            v[k] = bf16_round(v[k]) + tv;
        }
    }
    uint32_t yw[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) yw[k] = (uint32_t)f32_to_bf16(v[2 * k]) | ((uint32_t)f32_to_bf16(v[2 * k + 1]) << 16);
    *reinterpret_cast<uint4 *>(y + i) = make_uint4(yw[0], yw[1], yw[2], yw[3]);
    if constexpr (RES) {
        const uint4 xu = *reinterpret_cast<const uint4 *>(resid + i);
        const uint32_t xw[4] = {xu.x, xu.y, xu.z, xu.w};
        uint32_t ow[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float a0 = __uint_as_float(xw[k] << 16) + __uint_as_float(yw[k] << 16);
            const float a1 = __uint_as_float(xw[k] & 0xffff0000u) + __uint_as_float(yw[k] & 0xffff0000u);
            ow[k] = (uint32_t)f32_to_bf16(a0) | ((uint32_t)f32_to_bf16(a1) << 16);
        }
        *reinterpret_cast<uint4 *>(out + i) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    }
}

// strixite kernels/swiglu.hip:24-38: h = silu(g) * u; BF16 rounds where the reference does, bf16(bf16(silu(g)) * u).
template <typename T>
__global__ void __launch_bounds__(kThreads) swiglu_kernel(const T *gu, T *h, int64_t n, int64_t I) {
    for (int64_t k = (int64_t)blockIdx.x * kThreads + threadIdx.x; k < n; k += (int64_t)gridDim.x * kThreads) {
        const int64_t r = k / I, j = k % I;
        if constexpr (std::is_same_v<T, float>) {
            h[k] = silu(gu[r * 2 * I + j]) * gu[r * 2 * I + I + j];
        } else {
            const float s = bf16_round(silu(bf16_to_f32(gu[r * 2 * I + j])));
            h[k] = f32_to_bf16(s * bf16_to_f32(gu[r * 2 * I + I + j]));
        }
    }
}

__global__ void __launch_bounds__(kThreads) add_bias_kernel(float *logits, int64_t ld, int64_t M, int64_t E,
                                                            const float *bias) {
    for (int64_t k = (int64_t)blockIdx.x * kThreads + threadIdx.x; k < M * E; k += (int64_t)gridDim.x * kThreads) {
        const int64_t m = k / E, e = k % E;
        logits[m * ld + e] = logits[m * ld + e] + bias[e];
    }
}

// ---- host side --------------------------------------------------------------------------------------------------
struct QV {
    const uint8_t *q;
    const uint16_t *scale, *minv;
    int64_t N, K, G;
    int bits;
};
QV qv(const Q4DeviceView &w) { return {w.q, w.scale, w.minv, w.N, w.K, w.G, 4}; }
QV qv(const Q8DeviceView &w) { return {w.q, w.scale, w.minv, w.N, w.K, w.G, 8}; }

void check_view(const char *fn, const QV &w, int64_t E) {
    STRIX_CHECK(w.q != nullptr && w.scale != nullptr && w.minv != nullptr, fn, ": null weight pointer (q=",
                (const void *)w.q, ", scale=", (const void *)w.scale, ", min=", (const void *)w.minv, ")");
    const int span = w.bits == 4 ? 128 : 64;
    STRIX_CHECK(w.G == 32 || w.G == 64 || w.G == 128, fn, ": group size ", w.G, " unsupported (32, 64 or 128)");
    STRIX_CHECK(w.G % span == 0, fn, ": Q", w.bits, " group size ", w.G, " is below this path's K step of ", span,
                " codes (supported: Q4 G = 128; Q8 G = 64 or 128)");
    STRIX_CHECK(w.K >= w.G && w.K % w.G == 0 && w.K <= (1 << 24), fn, ": K = ", w.K,
                " must be a positive multiple of G = ", w.G, " and <= 2^24");
    STRIX_CHECK(E >= 1 && w.N % E == 0 && (w.N / E) % 16 == 0, fn, ": ", w.N, " weight rows for E = ", E,
                " experts (each expert's rows must be a multiple of 16)");
    STRIX_CHECK(reinterpret_cast<uintptr_t>(w.q) % 16 == 0, fn, ": code array must be 16-byte aligned");
}

template <int BITS, int MODE, int EPI, bool XF16, bool XROW_DIV, bool HF16>
void launch_gemm(const GemmArgs &a, int64_t tiles, hipStream_t stream) {
    const int64_t cols = EPI == EPI_SWIGLU ? a.N / 2 : a.N, per_block = EPI == EPI_SWIGLU ? 16 * kWaves : 32 * kWaves;
    STRIX_CHECK(tiles <= 65535 * 64, "expert kernels: ", tiles, " token tiles exceed the grid");
    dim3 grid((unsigned)((cols + per_block - 1) / per_block), (unsigned)tiles), block(kThreads);
    expert_gemm_kernel<BITS, MODE, EPI, XF16, XROW_DIV, HF16><<<grid, block, 0, stream>>>(a);
}

template <int MODE, int EPI, bool XF16, bool XROW_DIV, bool HF16>
void launch_bits(int bits, const GemmArgs &a, int64_t tiles, hipStream_t stream) {
    if (bits == 4) launch_gemm<4, MODE, EPI, XF16, XROW_DIV, HF16>(a, tiles, stream);
    else launch_gemm<8, MODE, EPI, XF16, XROW_DIV, HF16>(a, tiles, stream);
}

GemmArgs make_args(const QV &w, int64_t E, const void *x, void *y, int64_t ldy) {
    GemmArgs a{};
    a.x = static_cast<const uint16_t *>(x);
    a.q = w.q, a.scale = w.scale, a.minv = w.minv;
    a.N = w.N / E, a.K = w.K, a.G = w.G, a.E = E;
    a.y = y, a.ldy = ldy;
    return a;
}

void check_grouped(const char *fn, const void *x, const QV &w, int64_t E, const void *ws, size_t ws_bytes, int64_t M,
                   int64_t A, const void *y, Act act, int64_t y_bytes, int64_t x_rows) {
    STRIX_CHECK(x != nullptr && y != nullptr && ws != nullptr, fn, ": null pointer (x=", x, ", y=", y, ", ws=", ws, ")");
    STRIX_CHECK(act == Act::BF16, fn, ": activations must be BF16 on this path, got ", act_name(act));
    check_view(fn, w, E);
    STRIX_CHECK(E <= kMoeMaxExperts, fn, ": E = ", E, " > ", kMoeMaxExperts);
    STRIX_CHECK(M >= 1 && A >= 1 && A <= 64 && A <= E && M * A <= kMoeMaxSlots, fn, ": M = ", M, " tokens x A = ", A,
                " slots (A 1..min(64, E = ", E, "), M*A <= ", kMoeMaxSlots, ")");
    STRIX_CHECK(ws_bytes >= moe_route_workspace_bytes(M, A, E), fn, ": workspace of ", ws_bytes, " bytes, needs ",
                moe_route_workspace_bytes(M, A, E), " for M = ", M, ", A = ", A, ", E = ", E);
    STRIX_CHECK(reinterpret_cast<uintptr_t>(x) % 16 == 0, fn, ": input must be 16-byte aligned");
    STRIX_CHECK(disjoint(y, y_bytes, x, x_rows * w.K * 2), fn, ": output overlaps the input");
}

int64_t grouped_tiles(int64_t M, int64_t A, int64_t E) { return M * A / 16 + E + 2; }

template <typename V>
void gather_grouped_swiglu(const char *fn, const void *x, const V &wv, int64_t E, const void *ws, size_t ws_bytes,
                           int64_t M, int64_t A, void *h, Act act, bool h_f16, hipStream_t stream) {
    const QV w = qv(wv);
    const int64_t N = w.N / E, I = N / 2;
    check_grouped(fn, x, w, E, ws, ws_bytes, M, A, h, act, M * A * I * 2, M);
    STRIX_CHECK(I % 16 == 0, fn, ": gate_up has ", N, " rows an expert; I = N / 2 must be a multiple of 16");
    STRIX_CHECK(reinterpret_cast<uintptr_t>(h) % 8 == 0, fn, ": h must be 8-byte aligned");
    GemmArgs a = make_args(w, E, x, h, I);
    a.A = A, a.ws = static_cast<const int32_t *>(ws);
    const int64_t tiles = grouped_tiles(M, A, E);
    if (h_f16) launch_bits<GROUPED, EPI_SWIGLU, false, true, true>(w.bits, a, tiles, stream);
    else launch_bits<GROUPED, EPI_SWIGLU, false, true, false>(w.bits, a, tiles, stream);
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " A=", A, " E=", E, " N=", N, " K=", w.K, " G=", w.G, h_f16 ? " (F16 h)" : "");
}

void combine_reduce(const float *partial, const int32_t *ids, const float *coef, int64_t M, int64_t A, int64_t E,
                    int64_t N, uint16_t *y, const MoeSharedAdd *sh, const uint16_t *resid, uint16_t *out,
                    hipStream_t stream) {
    const unsigned blocks = (unsigned)((M * N / 8 + kThreads - 1) / kThreads);
    const uint16_t *s = sh ? static_cast<const uint16_t *>(sh->s) : nullptr;
    const float *gl = sh ? sh->gate_logit : nullptr;
    const int64_t gld = sh ? sh->gate_ld : 0;
    const uint32_t gi = sh ? sh->gate_index : 0;
    uint32_t *err = sh ? sh->err : nullptr;
    auto go = [&](auto shc, auto resc) {
        combine_reduce_kernel<decltype(shc)::value, decltype(resc)::value><<<blocks, kThreads, 0, stream>>>(
            partial, ids, coef, M, A, E, N, y, s, gl, gld, gi, err, resid, out);
    };
    if (sh && out) go(std::true_type{}, std::true_type{});
    else if (sh) go(std::true_type{}, std::false_type{});
    else if (out) go(std::false_type{}, std::true_type{});
    else go(std::false_type{}, std::false_type{});
}

template <typename V>
void combine_grouped(const char *fn, const void *h, const V &wv, int64_t E, const int32_t *ids, const float *coef,
                     const void *ws, size_t ws_bytes, float *partial, int64_t M, int64_t A, void *y, Act act,
                     const MoeSharedAdd *shared, bool h_f16, hipStream_t stream) {
    const QV w = qv(wv);
    const int64_t N = w.N / E;
    check_grouped(fn, h, w, E, ws, ws_bytes, M, A, y, act, M * N * 2, M * A);
    STRIX_CHECK(ids != nullptr && coef != nullptr && partial != nullptr, fn, ": null pointer (ids=", (const void *)ids,
                ", coef=", (const void *)coef, ", partial=", (const void *)partial, ")");
    STRIX_CHECK(N % 8 == 0 && reinterpret_cast<uintptr_t>(partial) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0,
                fn, ": N = ", N, " must be a multiple of 8, partial and y 16-byte aligned");
    STRIX_CHECK(disjoint(y, M * N * 2, partial, M * A * N * 4) && disjoint(partial, M * A * N * 4, h, M * A * w.K * 2),
                fn, ": partial overlaps y or h");
    if (shared != nullptr) {
        STRIX_CHECK(shared->s != nullptr && shared->gate_logit != nullptr && shared->err != nullptr, fn,
                    ": shared add with a null pointer");
        STRIX_CHECK(shared->gate_ld >= 1, fn, ": shared add gate_ld = ", shared->gate_ld);
        STRIX_CHECK(reinterpret_cast<uintptr_t>(shared->s) % 16 == 0, fn, ": shared s must be 16-byte aligned");
        STRIX_CHECK(disjoint(y, M * N * 2, shared->s, M * N * 2), fn, ": shared s overlaps y");
    }
    GemmArgs a = make_args(w, E, h, partial, N);
    a.A = A, a.ws = static_cast<const int32_t *>(ws);
    const int64_t tiles = grouped_tiles(M, A, E);
    if (h_f16) launch_bits<GROUPED, EPI_F32, true, false, false>(w.bits, a, tiles, stream);
    else launch_bits<GROUPED, EPI_F32, false, false, false>(w.bits, a, tiles, stream);
    combine_reduce(partial, ids, coef, M, A, E, N, static_cast<uint16_t *>(y), shared, nullptr, nullptr, stream);
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " A=", A, " E=", E, " N=", N, " K=", w.K, " G=", w.G,
                           shared ? " +shared" : "");
}

void check_perslot(const char *fn, const void *x, const QV &w, int64_t E, const int32_t *ids, int64_t M, int64_t A,
                   const void *y, Act act, uint32_t *err) {
    STRIX_CHECK(x != nullptr && y != nullptr && ids != nullptr && err != nullptr, fn, ": null pointer");
    STRIX_CHECK(act == Act::BF16, fn, ": activations must be BF16 on this path, got ", act_name(act));
    check_view(fn, w, E);
    STRIX_CHECK(M >= 1 && A >= 1 && M * A <= 65535ll * 64, fn, ": M = ", M, ", A = ", A, " out of range");
    STRIX_CHECK(reinterpret_cast<uintptr_t>(x) % 16 == 0, fn, ": input must be 16-byte aligned");
}

}  // namespace

// ---- grouped -------------------------------------------------------------------------------------------------------
void linear_q4_experts_gather_grouped(const void *x, const Q4DeviceView &w, int64_t E, const void *ws,
                                      size_t ws_bytes, int64_t M, int64_t A, void *y, Act act, MoeMath, hipStream_t stream) {
    const char *fn = "linear_q4_experts_gather_grouped";
    const QV v = qv(w);
    const int64_t N = v.N / E;
    check_grouped(fn, x, v, E, ws, ws_bytes, M, A, y, act, M * A * N * 2, M);
    STRIX_CHECK(reinterpret_cast<uintptr_t>(y) % 8 == 0, fn, ": y must be 8-byte aligned");
    GemmArgs a = make_args(v, E, x, y, N);
    a.A = A, a.ws = static_cast<const int32_t *>(ws);
    launch_gemm<4, GROUPED, EPI_BF16, false, true, false>(a, grouped_tiles(M, A, E), stream);
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " A=", A, " E=", E);
}

void linear_q4_experts_gather_grouped_swiglu(const void *x, const Q4DeviceView &w, int64_t E, const void *ws,
                                             size_t ws_bytes, int64_t M, int64_t A, void *h, Act act, MoeMath,
                                             hipStream_t stream, bool h_f16) {
    gather_grouped_swiglu("linear_q4_experts_gather_grouped_swiglu", x, w, E, ws, ws_bytes, M, A, h, act, h_f16, stream);
}

void linear_q8_experts_gather_grouped_swiglu(const void *x, const Q8DeviceView &w, int64_t E, const void *ws,
                                             size_t ws_bytes, int64_t M, int64_t A, void *h, Act act, MoeMath,
                                             hipStream_t stream, bool h_f16) {
    gather_grouped_swiglu("linear_q8_experts_gather_grouped_swiglu", x, w, E, ws, ws_bytes, M, A, h, act, h_f16, stream);
}

void linear_q4_experts_combine_grouped(const void *h, const Q4DeviceView &w, int64_t E, const int32_t *ids,
                                       const float *coef, const void *ws, size_t ws_bytes, float *partial, int64_t M,
                                       int64_t A, void *y, Act act, MoeMath, hipStream_t stream,
                                       const MoeSharedAdd *shared, bool h_f16) {
    combine_grouped("linear_q4_experts_combine_grouped", h, w, E, ids, coef, ws, ws_bytes, partial, M, A, y, act,
                    shared, h_f16, stream);
}

void linear_q8_experts_combine_grouped(const void *h, const Q8DeviceView &w, int64_t E, const int32_t *ids,
                                       const float *coef, const void *ws, size_t ws_bytes, float *partial, int64_t M,
                                       int64_t A, void *y, Act act, MoeMath, hipStream_t stream,
                                       const MoeSharedAdd *shared, bool h_f16) {
    combine_grouped("linear_q8_experts_combine_grouped", h, w, E, ids, coef, ws, ws_bytes, partial, M, A, y, act,
                    shared, h_f16, stream);
}

// ---- per-slot (strixite kernels/linear_q4.hpp:42-61) ----------------------------------------------------------------
void linear_q4_experts_gather(const void *x, const Q4DeviceView &w, int64_t E, const int32_t *ids, int64_t M,
                              int64_t A, void *y, Act act, uint32_t *err, hipStream_t stream) {
    const char *fn = "linear_q4_experts_gather";
    const QV v = qv(w);
    check_perslot(fn, x, v, E, ids, M, A, y, act, err);
    const int64_t N = v.N / E;
    STRIX_CHECK(disjoint(y, M * A * N * 2, x, M * v.K * 2), fn, ": y overlaps x");
    GemmArgs a = make_args(v, E, x, y, N);
    a.A = A, a.M = M, a.ids = ids, a.err = err;
    launch_gemm<4, PERSLOT, EPI_BF16, false, true, false>(a, M * A, stream);
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " A=", A, " E=", E);
}

void linear_q4_experts_gather_swiglu(const void *x, const Q4DeviceView &w, int64_t E, const int32_t *ids, int64_t M,
                                     int64_t A, void *h, Act act, uint32_t *err, hipStream_t stream) {
    const char *fn = "linear_q4_experts_gather_swiglu";
    const QV v = qv(w);
    check_perslot(fn, x, v, E, ids, M, A, h, act, err);
    const int64_t I = v.N / E / 2;
    STRIX_CHECK(I % 16 == 0, fn, ": I = ", I, " must be a multiple of 16");
    STRIX_CHECK(disjoint(h, M * A * I * 2, x, M * v.K * 2), fn, ": h overlaps x");
    GemmArgs a = make_args(v, E, x, h, I);
    a.A = A, a.M = M, a.ids = ids, a.err = err;
    launch_gemm<4, PERSLOT, EPI_SWIGLU, false, true, false>(a, M * A, stream);
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " A=", A, " E=", E);
}

void linear_q4_experts_combine(const void *h, const Q4DeviceView &w, int64_t E, const int32_t *ids,
                               const float *coef, int64_t M, int64_t A, void *y, Act act, uint32_t *err,
                               hipStream_t stream) {
    const char *fn = "linear_q4_experts_combine";
    const QV v = qv(w);
    check_perslot(fn, h, v, E, ids, M, A, y, act, err);
    STRIX_CHECK(coef != nullptr, fn, ": null coef");
    const int64_t N = v.N / E;
    STRIX_CHECK(M <= 65535, fn, ": M = ", M, " tokens, at most 65535");
    STRIX_CHECK(disjoint(y, M * N * 2, h, M * A * v.K * 2), fn, ": y overlaps h");
    GemmArgs a = make_args(v, E, h, y, N);
    a.A = A, a.M = M, a.ids = ids, a.err = err;
    dim3 grid((unsigned)((N + 32 * kWaves - 1) / (32 * kWaves)), (unsigned)M), block(kThreads);
    perslot_combine_kernel<4, false><<<grid, block, 0, stream>>>(a, coef);
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " A=", A, " E=", E);
}

void check_expert_error(const uint32_t *err, const char *what) {
    STRIX_CHECK(err != nullptr, "check_expert_error(", what, "): null err");
    uint32_t e[3];
    STRIX_HIP_CHECK(hipMemcpy(e, err, sizeof(e), hipMemcpyDeviceToHost), "reading the expert error word for ", what);
    report_expert_error(e, what);
}

void report_expert_error(const uint32_t e[3], const char *what) {
    STRIX_CHECK(e[0] == 0, what, ": expert id ", (int32_t)e[1], " at slot ", e[2],
                " (token * A + a) is out of range; outputs for that token are NaN");
}

// ---- swiglu, dense Q8 -------------------------------------------------------------------------------------------------
void swiglu(const void *gu, void *h, int64_t rows, int64_t I, Act act, hipStream_t stream) {
    STRIX_CHECK(gu != nullptr && h != nullptr, "swiglu: null pointer (gu=", gu, ", h=", h, ")");
    STRIX_CHECK(rows >= 1 && I >= 1 && rows <= (1ll << 40) / I, "swiglu: rows = ", rows, ", I = ", I, " out of range");
    STRIX_CHECK(act == Act::F32 || act == Act::BF16, "swiglu: unsupported activation dtype ", (int)act);
    const int64_t es = act == Act::F32 ? 4 : 2, n = rows * I;
    STRIX_CHECK(disjoint(h, n * es, gu, 2 * n * es), "swiglu: output h overlaps input gu");
    const int64_t b = (n + kThreads - 1) / kThreads;
    const unsigned blocks = (unsigned)(b < 65536 ? b : 65536);
    if (act == Act::F32)
        swiglu_kernel<float><<<blocks, kThreads, 0, stream>>>(static_cast<const float *>(gu), static_cast<float *>(h), n, I);
    else
        swiglu_kernel<uint16_t><<<blocks, kThreads, 0, stream>>>(static_cast<const uint16_t *>(gu),
                                                                 static_cast<uint16_t *>(h), n, I);
    STRIX_HIP_CHECK_LAUNCH("swiglu ", act_name(act), " rows=", rows, " I=", I);
}

void linear_q8(const void *x, const Q8DeviceView &w, void *y, int64_t M, Act act, hipStream_t stream) {
    linear_q8(x, w, y, M, act, act, stream);
}

void linear_q8(const void *x, const Q8DeviceView &w, void *y, int64_t M, Act act, Act out_act, hipStream_t stream) {
    const char *fn = "linear_q8";
    const QV v = qv(w);
    STRIX_CHECK(x != nullptr && y != nullptr, fn, ": null pointer (x=", x, ", y=", y, ")");
    STRIX_CHECK(act == Act::BF16, fn, ": activations must be BF16 on this path, got ", act_name(act));
    STRIX_CHECK(out_act == Act::BF16 || out_act == Act::F32, fn, ": output dtype ", (int)out_act);
    check_view(fn, v, 1);
    STRIX_CHECK(M >= 1 && (M + 15) / 16 <= 65535ll * 64, fn, ": M = ", M);
    STRIX_CHECK(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0, fn,
                ": x and y must be 16-byte aligned");
    const int64_t oes = out_act == Act::F32 ? 4 : 2;
    STRIX_CHECK(disjoint(y, M * v.N * oes, x, M * v.K * 2), fn, ": y overlaps x");
    GemmArgs a = make_args(v, 1, x, y, v.N);
    a.M = M;
    if (out_act == Act::F32) launch_gemm<8, DENSE, EPI_F32, false, false, false>(a, (M + 15) / 16, stream);
    else launch_gemm<8, DENSE, EPI_BF16, false, false, false>(a, (M + 15) / 16, stream);
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " N=", v.N, " K=", v.K, " G=", v.G);
}

}  // namespace strix::kernels

// ---- the sublayer ------------------------------------------------------------------------------------------------------
namespace strix {

namespace {
struct LayerWs {
    int64_t logits, ids, coef, route, h, partial, sh_h, sh_s, total;
    size_t route_bytes;
};
int64_t al(int64_t b) { return (b + 255) / 256 * 256; }
LayerWs layer_ws(const MoeLayerWeights &w, int64_t M) {
    LayerWs L{};
    const int64_t E = w.E, k = w.k, H = w.H, I = w.I, ld = E + (w.has_shared ? 1 : 0);
    int64_t o = 0;
    L.logits = o, o += al(M * ld * 4);
    L.ids = o, o += al(M * k * 4);
    L.coef = o, o += al(M * k * 4);
    L.route_bytes = kernels::moe_route_workspace_bytes(M, k, E);
    L.route = o, o += al((int64_t)L.route_bytes);
    L.h = o, o += al(M * k * I * 2);
    L.partial = o, o += al(M * k * H * 4);
    L.sh_h = o, o += al(w.has_shared ? M * I * 2 : 0);
    L.sh_s = o, o += al(w.has_shared ? M * H * 2 : 0);
    L.total = o;
    return L;
}
}  // namespace

size_t moe_layer_workspace_bytes(const MoeLayerWeights &w, int64_t M) {
    STRIX_CHECK(M >= 1 && w.E >= 1 && w.k >= 1 && w.H >= 1 && w.I >= 1, "moe_layer_workspace_bytes: M = ", M,
                ", E = ", w.E, ", k = ", w.k, ", H = ", w.H, ", I = ", w.I);
    return (size_t)layer_ws(w, M).total;
}

void moe_layer_forward(const MoeLayerWeights &w, const void *x, int64_t M, const float *logits_in, void *y,
                       void *x_out, int32_t *ids_out, float *coef_out, void *ws, size_t ws_bytes, uint32_t *err,
                       hipStream_t stream) {
    using namespace kernels;
    const char *fn = "moe_layer_forward";
    STRIX_CHECK(x != nullptr && y != nullptr && ws != nullptr && err != nullptr, fn, ": null pointer");
    STRIX_CHECK(logits_in != nullptr || w.router != nullptr, fn, ": no router weight and no logits");
    STRIX_CHECK(w.gate_up_bits == 4 || w.gate_up_bits == 8, fn, ": routed expert bits ", w.gate_up_bits);
    STRIX_CHECK(w.down_bits == w.gate_up_bits, fn, ": gate_up and down must share a format");
    STRIX_CHECK(w.gate_up.N == w.E * 2 * w.I && w.gate_up.K == w.H && w.down.N == w.E * w.H && w.down.K == w.I, fn,
                ": weight shapes [", w.gate_up.N, ", ", w.gate_up.K, "] / [", w.down.N, ", ", w.down.K,
                "] do not match E = ", w.E, ", H = ", w.H, ", I = ", w.I);
    if (w.has_shared)
        STRIX_CHECK(w.sh_gate_up.N == 2 * w.I && w.sh_gate_up.K == w.H && w.sh_down.N == w.H && w.sh_down.K == w.I, fn,
                    ": shared expert shapes do not match H = ", w.H, ", I = ", w.I);
    const LayerWs L = layer_ws(w, M);
    STRIX_CHECK(ws_bytes >= (size_t)L.total, fn, ": workspace of ", ws_bytes, " bytes, needs ", L.total);
    STRIX_CHECK(reinterpret_cast<uintptr_t>(ws) % 256 == 0, fn, ": workspace must be 256-byte aligned");
    char *base = static_cast<char *>(ws);
    const int64_t E = w.E, k = w.k, H = w.H, I = w.I, ld = E + (w.has_shared ? 1 : 0);
    float *logits = reinterpret_cast<float *>(base + L.logits);
    int32_t *ids = ids_out ? ids_out : reinterpret_cast<int32_t *>(base + L.ids);
    float *coef = coef_out ? coef_out : reinterpret_cast<float *>(base + L.coef);
    void *route = base + L.route;
    uint16_t *h = reinterpret_cast<uint16_t *>(base + L.h);
    float *partial = reinterpret_cast<float *>(base + L.partial);
    uint16_t *sh_h = reinterpret_cast<uint16_t *>(base + L.sh_h);
    uint16_t *sh_s = reinterpret_cast<uint16_t *>(base + L.sh_s);
    uint32_t *err_router = err, *err_expert = err + 3;

    // router projection (+ harness bias) and top-k
    const float *lg = logits_in;
    if (!lg) {
        linear_bf16w(x, w.router, logits, M, ld, H, Act::BF16, Act::F32, stream);
        if (w.router_bias) {
            const int64_t b = (M * E + 255) / 256;
            add_bias_kernel<<<(unsigned)(b < 65536 ? b : 65536), 256, 0, stream>>>(logits, ld, M, E, w.router_bias);
            STRIX_HIP_CHECK_LAUNCH(fn, " router bias");
        }
        lg = logits;
    }
    moe_router(lg, ld, M, E, k, nullptr, 0, 0, ids, coef, Act::F32, err_router, stream);
    moe_group_routes(ids, M, k, E, route, L.route_bytes, err_expert, stream);
    // routed experts: gate_up + SwiGLU -> h, down -> partial
    const bool q8 = w.gate_up_bits == 8;
    const Q8DeviceView gu8{w.gate_up.q, w.gate_up.scale, w.gate_up.minv, w.gate_up.N, w.gate_up.K, w.gate_up.G};
    const Q8DeviceView dn8{w.down.q, w.down.scale, w.down.minv, w.down.N, w.down.K, w.down.G};
    if (q8) linear_q8_experts_gather_grouped_swiglu(x, gu8, E, route, L.route_bytes, M, k, h, Act::BF16, MoeMath::WmmaF16, stream, true);
    else linear_q4_experts_gather_grouped_swiglu(x, w.gate_up, E, route, L.route_bytes, M, k, h, Act::BF16, MoeMath::WmmaF16, stream, true);
    // shared expert (dense Q8): gate_up + SwiGLU -> sh_h, down -> sh_s
    if (w.has_shared) {
        const QV gv = qv(w.sh_gate_up), dv = qv(w.sh_down);
        check_view(fn, gv, 1);
        check_view(fn, dv, 1);
        GemmArgs a = make_args(gv, 1, x, sh_h, I);
        a.M = M;
        launch_gemm<8, DENSE, EPI_SWIGLU, false, false, false>(a, (M + 15) / 16, stream);
        GemmArgs b = make_args(dv, 1, sh_h, sh_s, H);
        b.M = M;
        launch_gemm<8, DENSE, EPI_BF16, false, false, false>(b, (M + 15) / 16, stream);
        STRIX_HIP_CHECK_LAUNCH(fn, " shared expert M=", M);
    }
    {
        const QV dv = q8 ? qv(dn8) : qv(w.down);
        check_view(fn, dv, E);
        GemmArgs a = make_args(dv, E, h, partial, H);
        a.A = k, a.ws = static_cast<const int32_t *>(route);
        if (q8) launch_gemm<8, GROUPED, EPI_F32, true, false, false>(a, grouped_tiles(M, k, E), stream);
        else launch_gemm<4, GROUPED, EPI_F32, true, false, false>(a, grouped_tiles(M, k, E), stream);
    }
    const MoeSharedAdd sh{sh_s, lg + E, ld, (uint32_t)E, err_router};
    combine_reduce(partial, ids, coef, M, k, E, H, static_cast<uint16_t *>(y), w.has_shared ? &sh : nullptr,
                   static_cast<const uint16_t *>(x), static_cast<uint16_t *>(x_out), stream);
    STRIX_HIP_CHECK_LAUNCH(fn, " M=", M, " E=", E, " k=", k);
}

}  // namespace strix
