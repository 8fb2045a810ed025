// The hyper-connection mix that produces the MoE sublayer's input (strixite kernels/hc.hpp:31-50, the step before the
// path: hc_mix(l.hc_mlp), runtime/qwen4exp.cpp:2801-2832) on gfx950: hc_mix_down (the low-rank projection of the
// four RMS-normalized residual streams, the injection gates and the streams' inverse RMS) and hc_mix_up (the gated
// up projection combined over the streams into u). hc_inject, the other end, lives with the shared-expert add
// (router.hip).
//
// Semantics (strixite kernels/hc.hpp:3-18, :31-50): X [T, 4 d] in the activation dtype, u rounded once to it.
//   hc_mix_down: inv[t, s] = 1 / sqrt(mean_j X[t, s d + j]^2 + eps); a[t, n] = sum_s inv[t, s] (W[n, s-block] .
//     X[t, s-block]) for the rows n of the folded weight W [r (+ 4), 4 d] (Q4 or Q8, row-major); h[t, n] = silu(a /
//     4) for n < r, w_in[t, n - r] = 2 sigmoid(a / 4) for the 4 injection rows.
//   hc_mix_up: u[t, j] = (1/4) sum_s sigmoid(W_up[s d + j] . h[t]) * (X[t, s d + j] * inv[t, s] * (1 + norm_w[s d +
//     j])), W_up [4 d, r] chunk-major (32-code chunk c of row n at q[(c N + n) * 16] (Q4) or [(c N + n) * 32] (Q8),
//     group g's scale / min at [g N + n]; strixite formats/q4.hpp:43-55).
//
// Two kernel designs, chosen by the token count:
//
// * Matrix-core tiles (the up mix from 1 token; the down mix from 256 tokens and d % 128 == 0). Weights enter the
//   bf16 MFMA (v_mfma_f32_16x16x32_bf16) as their exact integer codes and each quantization group's partial product D is
//   rescaled on the FP32 accumulator: w . x = s D + m' sum(x) (Q4 codes enter as 128 + n with m' = m - 128 s, Q8
//   codes as c - 128 with m' = m + 128 s). The min terms of a whole K stage are one FP32 MFMA
//   (v_mfma_f32_16x16x4f32: sums of x per group against m' per group). BF16 activations are exact in bf16; an FP32
//   operand (F32 streams, and h, which is always FP32) enters as three bf16 pieces hi + mid + lo that sum to it
//   exactly (24 significant bits) and takes three MFMAs. So every product is exact and only the FP32 accumulation
//   order differs from the per-chunk FP32 form.
//   - down (mix_down_tile_kernel): a block takes 32 tokens x 192 weight rows (4 waves x 3 row tiles of 16, each wave
//     both 16-token tiles). K runs in stages of 128 (a stage never crosses a stream as d % 128 == 0). All 256
//     threads stage the next stage into LDS while the waves compute the current one: the weight rows' codes (16-byte
//     loads, stored so that one 16-byte LDS read gives a lane its codes for the stage's 4 MFMAs), the activations
//     (converted once to bf16 [hi, mid, lo] in the paired k order the Q4 decoder produces), each token's sums per group
//     and its running sum of squares; at a stream's last stage the staging threads turn that into inv[t, s]. The
//     waves fold each stream's total into a = sum_s inv_s P_s as the stream ends. Blocks are numbered
//     XCD-contiguously, so the row blocks of one token tile share its activations in one XCD's L2.
//   - up (mix_up_tile_kernel): a block takes 16 or 32 tokens and 4 or 8 column tiles of 16 output positions j; a
//     wave owns one column tile: the 4 weight tiles of rows s d + j0 .. + 15 (s = 0..3), so the stream combine of
//     the epilogue happens in registers. h is converted to bf16 [hi, mid, lo] into LDS once per block (with its group
//     sums); the chunk-major codes of a chunk's 16 rows are 256 (Q4) or 512 (Q8) contiguous bytes, read by the
//     wave's lanes directly, four chunks ahead.
// * Vector rows (down mix below 256 tokens, or d % 128 != 0): a block of 4 waves computes the group's inverse RMS into
//   LDS, then each wave takes one weight row (T = 1: a row's chunks split over the 4 waves): lane l dots the row's
//   32-code chunks l, l + 64, ... with the chunk of every token of the group (the codes converted to floats once for
//   the group) and adds each dot scaled by its stream's inverse RMS into one accumulator a token; a butterfly ends it.
#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

namespace strix::kernels {

namespace {

using namespace strix::dev;
constexpr int kWave = 64, kStreams = 4, kChunk = 32;
constexpr int64_t kMaxR = 1024, kMaxTokens = 65535, kMaxD = 1 << 20;
// the down mix's matrix-core tiles from this many tokens: a 32-token tile block streams the whole weight, so with fewer
// tiles than CUs the vector-row kernel, which spreads the rows over the CUs, is faster (measured at d 2560, r 320: tiles
// ~100 us flat up to a few hundred tokens; rows 8 us at 1 token, ~60 at 64)
constexpr int64_t kDownTileMinTokens = 256;

__device__ __forceinline__ float ld_act(const float *p, int64_t i) { return p[i]; }
__device__ __forceinline__ float ld_act(const uint16_t *p, int64_t i) { return bf16_to_f32(p[i]); }
__device__ __forceinline__ void st_act(float *p, int64_t i, float v) { p[i] = v; }
__device__ __forceinline__ void st_act(uint16_t *p, int64_t i, float v) { p[i] = f32_to_bf16(v); }

// 8 consecutive activations at element offset i (16-byte aligned for BF16, 32 for F32)
__device__ __forceinline__ void ld8(const uint16_t *p, int64_t i, float (&v)[8]) {
    const uint4 u = *reinterpret_cast<const uint4 *>(p + i);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) v[2 * k] = __uint_as_float(w[k] << 16), v[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
}
__device__ __forceinline__ void ld8(const float *p, int64_t i, float (&v)[8]) {
    const float4 a = *reinterpret_cast<const float4 *>(p + i), b = *reinterpret_cast<const float4 *>(p + i + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// 8 Q4 codes (a dword, code i at bits 4 i) -> bf16 128 + code in the paired k order k0 k2 k4 k6 k1 k3 k5 k7
__device__ __forceinline__ Frag q4_paired(uint32_t w) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu, c = 0x43434343u;
    return Frag{{__builtin_amdgcn_perm(c, lo, 0x04010400u), __builtin_amdgcn_perm(c, lo, 0x04030402u),
                 __builtin_amdgcn_perm(c, hi, 0x04010400u), __builtin_amdgcn_perm(c, hi, 0x04030402u)}};
}
// 8 Q8 codes (two dwords, natural order) -> bf16 of the signed codes c - 128 (exact) in the paired k order; the
// offset is folded into the min: m' = m + 128 s. Signed codes keep a group's partial product near the size of the
// result instead of 128 sum(x) (no cancellation against the min term).
__device__ __forceinline__ Frag q8_paired(uint32_t a, uint32_t b) {
    a ^= 0x80808080u, b ^= 0x80808080u;
    auto cv = [](uint32_t w, int byte) { return (float)(int8_t)(uint8_t)(w >> (8 * byte)); };
    return Frag{{hi16_pair(cv(a, 0), cv(a, 2)), hi16_pair(cv(b, 0), cv(b, 2)), hi16_pair(cv(a, 1), cv(a, 3)),
                 hi16_pair(cv(b, 1), cv(b, 3))}};
}
// m' for the decoded codes: Q4 enters as 128 + n, Q8 as c - 128
template <int BITS> __device__ __forceinline__ float min_prime(float s, float m) {
    return BITS == 4 ? fmaf(-128.0f, s, m) : fmaf(128.0f, s, m);
}
// 8 floats in natural k order -> three bf16 pieces (hi: the top 16 bits, mid: the top 16 bits of the rest, lo: the
// rest rounded, exact as it holds at most 8 significant bits), each in the paired order: hi + mid + lo == x exactly
struct Split {
    Frag hi, mid, lo;
    float sum;  // FP32 sum of the 8 values
    float sq;   // sum of their squares
};
__device__ __forceinline__ Split split8(const float (&v)[8]) {
    constexpr int ord[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    uint16_t a[8], b[8], c[8];
    Split r{};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float x = v[ord[i]];
        const float xh = __uint_as_float(__float_as_uint(x) & 0xFFFF0000u), r1 = x - xh;
        const float xm = __uint_as_float(__float_as_uint(r1) & 0xFFFF0000u);
        a[i] = (uint16_t)(__float_as_uint(x) >> 16);
        b[i] = (uint16_t)(__float_as_uint(r1) >> 16);
        c[i] = f32_to_bf16(r1 - xm);
        r.sum += x;
        r.sq = fmaf(x, x, r.sq);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        r.hi.d[i] = (uint32_t)a[2 * i] | ((uint32_t)a[2 * i + 1] << 16);
        r.mid.d[i] = (uint32_t)b[2 * i] | ((uint32_t)b[2 * i + 1] << 16);
        r.lo.d[i] = (uint32_t)c[2 * i] | ((uint32_t)c[2 * i + 1] << 16);
    }
    return r;
}
// 8 bf16 in natural k order (a uint4) -> the paired order, with their FP32 sum and sum of squares
__device__ __forceinline__ Split pair8(const uint4 &v) {
    Split r{};
    r.hi = Frag{{__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x05040100u),
                 __builtin_amdgcn_perm(v.y, v.x, 0x07060302u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u)}};
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = __uint_as_float(w[i] << 16), b = __uint_as_float(w[i] & 0xFFFF0000u);
        r.sum += a + b;
        r.sq = fmaf(b, b, fmaf(a, a, r.sq));
    }
    return r;
}

__device__ __forceinline__ float4v mfma_f32x4(float a, float b, float4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ uint4 lds16(const uint32_t *p) { return *reinterpret_cast<const uint4 *>(p); }

// XCD-contiguous block numbering: the hardware deals consecutive block ids round-robin to the 8 XCDs; this maps
// them so XCD x runs the logical blocks [x nb / 8, (x + 1) nb / 8) (when nb % 8 == 0), in order.
__device__ __forceinline__ uint32_t xcd_block(uint32_t b, uint32_t nb) {
    return nb % 8 == 0 ? (b % 8) * (nb / 8) + b / 8 : b;
}

// ================================================================================================ down: MFMA tiles
namespace dn {
constexpr int kWaves = 4, kThreads = kWaves * kWave;
constexpr int kTilesPW = 3;                            // 16-row weight tiles a wave
constexpr int kRows = kWaves * kTilesPW * 16;          // weight rows a block
constexpr int kTok = 32;                               // tokens a block: two 16-token MFMA tiles
constexpr int kK = 128;                                // k a stage
constexpr int kAdw = kK / 2 + 4;                       // dwords of a staged activation row (bf16, padded)
template <int BITS> constexpr int wdw() { return BITS == 4 ? 20 : 36; }  // dwords of a staged weight row (padded)
// stage layout in dwords: W [kRows][wdw] | A hi [kTok][kAdw] | A lo (F32) | xs [4][kTok] | sc [kRows][4] |
// mp [kRows][4]
template <int BITS, bool F32> struct Stage {
    static constexpr int W = 0, AH = W + kRows * wdw<BITS>(), AM = AH + kTok * kAdw;
    static constexpr int AL = AM + (F32 ? kTok * kAdw : 0);
    static constexpr int XS = AL + (F32 ? kTok * kAdw : 0), SC = XS + 4 * kTok, MP = SC + kRows * 4;
    static constexpr int SIZE = MP + kRows * 4;
};
}  // namespace dn

template <typename T, int BITS, int G>
__global__ void __launch_bounds__(dn::kThreads)
    mix_down_tile_kernel(const T *x, const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t R,
                         int64_t d, int64_t r, float eps, int64_t Tn, float *h, float *w_in, float *inv_out) {
    using namespace dn;
    constexpr bool F32 = std::is_same<T, float>::value;
    using S = Stage<BITS, F32>;
    constexpr int GPS = kK / G;  // groups a stage
    constexpr int WDW = wdw<BITS>();
    extern __shared__ uint32_t lds[];  // two stages
    __shared__ float invs[2][kTok];    // by stream parity

    const int64_t K = kStreams * d;
    const uint32_t stages = (uint32_t)(K / kK), sps = (uint32_t)(d / kK);  // stages, stages a stream (32-bit: cheap
                                                                           // division in the loop)
    const uint32_t nrb = (uint32_t)((R + kRows - 1) / kRows);
    const uint32_t L = xcd_block(blockIdx.x, gridDim.x);
    const int64_t t0 = (int64_t)(L / nrb) * kTok, rb = (int64_t)(L % nrb) * kRows;
    const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave, n = lane % 16, qd = lane / 16;

    // ---- staging (all threads): registers for the next stage
    constexpr int WP = BITS == 4 ? 3 : 6;  // 16-byte weight pieces a thread a stage
    struct Regs {
        uint4 w[WP];
        uint4 xa[F32 ? 4 : 2];
        uint16_t sc[(kRows * GPS + dn::kThreads - 1) / dn::kThreads], mn[(kRows * GPS + dn::kThreads - 1) / dn::kThreads];
    } rgs[2];  // two stages in flight: the one being written to LDS and the next one's loads
    const int tt = tid / 8, seg = tid % 8;  // the thread's token and 16-k segment of the activation stage
    const int64_t xrow = (t0 + tt < Tn ? t0 + tt : Tn - 1) * K;
    auto load_stage = [&](uint32_t st, Regs &rg) {
        const int64_t kb = (int64_t)st * kK;
#pragma unroll
        for (int i = 0; i < WP; ++i) {
            const int p = tid + dn::kThreads * i;
            const int row = BITS == 4 ? p / 4 : p / 8, piece = BITS == 4 ? p % 4 : p % 8;
            const int64_t grow = rb + row < R ? rb + row : R - 1;
            rg.w[i] = *reinterpret_cast<const uint4 *>(q + grow * (K * BITS / 8) + kb * BITS / 8 + 16 * piece);
        }
        if constexpr (F32) {
#pragma unroll
            for (int i = 0; i < 4; ++i) rg.xa[i] = *reinterpret_cast<const uint4 *>(x + xrow + kb + 16 * seg + 4 * i);
        } else {
#pragma unroll
            for (int i = 0; i < 2; ++i) rg.xa[i] = *reinterpret_cast<const uint4 *>(x + xrow + kb + 16 * seg + 8 * i);
        }
#pragma unroll
        // scales and mins: loaded by every thread (a clamped index past the table), so the loads are unconditional
        // and the compiler's wait for them counts exactly; kept as raw halves until written
        for (int i = 0; i < (int)(sizeof(rg.sc) / 2); ++i) {
            const int p = min(tid + dn::kThreads * i, kRows * GPS - 1);
            const int row = p / GPS, g = p % GPS;
            const int64_t grow = rb + row < R ? rb + row : R - 1;
            const int64_t gi = grow * (K / G) + kb / G + g;
            rg.sc[i] = scale[gi], rg.mn[i] = minv[gi];
        }
    };
    float sq = 0.f;  // the thread's running sum of squares of its token in the current stream
    auto write_stage = [&](uint32_t st, uint32_t *sb, const Regs &rg) {
#pragma unroll
        for (int i = 0; i < WP; ++i) {
            const int p = tid + dn::kThreads * i;
            const uint32_t dw[4] = {rg.w[i].x, rg.w[i].y, rg.w[i].z, rg.w[i].w};
            if constexpr (BITS == 4) {  // piece j = chunk j: its dword qq is quarter qq's 8 codes
                const int row = p / 4, j = p % 4;
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) sb[S::W + row * WDW + qq * 4 + j] = dw[qq];
            } else {  // piece (j, half): quarters 2 half, 2 half + 1 of chunk j, two dwords each
                const int row = p / 8, j = (p % 8) / 2, half = p % 2;
#pragma unroll
                for (int e = 0; e < 2; ++e)
                    *reinterpret_cast<uint2 *>(&sb[S::W + row * WDW + ((2 * half + e) * 4 + j) * 2]) =
                        uint2{dw[2 * e], dw[2 * e + 1]};
            }
        }
        // activations: 16 k of token tt as two paired-order 8-groups (hi, and lo for F32)
        float part_sum = 0.f;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            Split v;
            if constexpr (F32) {
                float f[8];
                const uint4 a = rg.xa[2 * e], b = rg.xa[2 * e + 1];
                f[0] = __uint_as_float(a.x), f[1] = __uint_as_float(a.y), f[2] = __uint_as_float(a.z);
                f[3] = __uint_as_float(a.w), f[4] = __uint_as_float(b.x), f[5] = __uint_as_float(b.y);
                f[6] = __uint_as_float(b.z), f[7] = __uint_as_float(b.w);
                v = split8(f);
                *reinterpret_cast<uint4 *>(&sb[S::AM + tt * kAdw + 8 * seg + 4 * e]) =
                    uint4{v.mid.d[0], v.mid.d[1], v.mid.d[2], v.mid.d[3]};
                *reinterpret_cast<uint4 *>(&sb[S::AL + tt * kAdw + 8 * seg + 4 * e]) =
                    uint4{v.lo.d[0], v.lo.d[1], v.lo.d[2], v.lo.d[3]};
            } else {
                v = pair8(rg.xa[e]);
            }
            *reinterpret_cast<uint4 *>(&sb[S::AH + tt * kAdw + 8 * seg + 4 * e]) =
                uint4{v.hi.d[0], v.hi.d[1], v.hi.d[2], v.hi.d[3]};
            part_sum += v.sum;
            sq += v.sq;
        }
        // group sums: the G / 16 segments of a group are neighbouring lanes
#pragma unroll
        for (int o = 1; o < G / 16; o <<= 1) part_sum += __shfl_xor(part_sum, o, kWave);
        if (seg % (G / 16) == 0) sb[S::XS + (seg * 16 / G) * kTok + tt] = __float_as_uint(part_sum);
        // scales and mins as floats; m' = m - 128 s for Q4's 128 + n codes
#pragma unroll
        for (int i = 0; i < (int)(sizeof(rg.sc) / 2); ++i) {  // clamped as loaded: a repeat writes the same value
            const int p = min(tid + dn::kThreads * i, kRows * GPS - 1);
            const int row = p / GPS, g = p % GPS;
            const float s = bf16_to_f32(rg.sc[i]), m = bf16_to_f32(rg.mn[i]);
            sb[S::SC + row * 4 + g] = __float_as_uint(s);
            sb[S::MP + row * 4 + g] = __float_as_uint(min_prime<BITS>(s, m));
        }
        // the stream's last stage: its inverse RMS per token
        if ((st + 1) % sps == 0) {
#pragma unroll
            for (int o = 1; o < 8; o <<= 1) sq += __shfl_xor(sq, o, kWave);
            const uint32_t s = st / sps;
            const float iv = 1.0f / sqrtf(sq / (float)d + eps);
            if (seg == 0) {
                invs[s & 1][tt] = iv;
                if (L % nrb == 0 && t0 + tt < Tn) inv_out[(t0 + tt) * kStreams + s] = iv;
            }
            sq = 0.f;
        }
    };
    // zero the unused group slots (GPS < 4) of both stages once: the min MFMA reads all four
    for (int i = tid; i < 2 * kRows * 4; i += dn::kThreads) {
        const int stg = i / (kRows * 4), e = i % (kRows * 4);
        if (e % 4 >= GPS) lds[stg * S::SIZE + S::SC + e] = 0u, lds[stg * S::SIZE + S::MP + e] = 0u;
    }
    for (int i = tid; i < 2 * 4 * kTok; i += dn::kThreads) {
        const int stg = i / (4 * kTok), e = i % (4 * kTok);
        if (e / kTok >= GPS) lds[stg * S::SIZE + S::XS + e] = 0u;
    }

    // ---- compute (each wave): 3 row tiles x 2 token tiles
    float4v D[kTilesPW][2], P[kTilesPW][2], A[kTilesPW][2];
#pragma unroll
    for (int nt = 0; nt < kTilesPW; ++nt)
#pragma unroll
        for (int m = 0; m < 2; ++m) D[nt][m] = P[nt][m] = A[nt][m] = float4v{0, 0, 0, 0};
    const int wrow0 = (wave * kTilesPW) * 16 + n;  // the lane's staged weight row in tile 0
    auto compute = [&](uint32_t st, const uint32_t *sb) {
        uint4 bw[kTilesPW][BITS == 4 ? 1 : 2];
#pragma unroll
        for (int nt = 0; nt < kTilesPW; ++nt) {
            const uint32_t *wr = sb + S::W + (wrow0 + 16 * nt) * WDW;
            if constexpr (BITS == 4) bw[nt][0] = lds16(wr + 4 * qd);
            else bw[nt][0] = lds16(wr + 8 * qd), bw[nt][1] = lds16(wr + 8 * qd + 4);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            Frag ah[2], am[2], al[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                const uint4 v = lds16(sb + S::AH + (16 * m + n) * kAdw + 16 * j + 4 * qd);
                ah[m] = Frag{{v.x, v.y, v.z, v.w}};
                if constexpr (F32) {
                    const uint4 u = lds16(sb + S::AM + (16 * m + n) * kAdw + 16 * j + 4 * qd);
                    am[m] = Frag{{u.x, u.y, u.z, u.w}};
                    const uint4 w = lds16(sb + S::AL + (16 * m + n) * kAdw + 16 * j + 4 * qd);
                    al[m] = Frag{{w.x, w.y, w.z, w.w}};
                }
            }
#pragma unroll
            for (int nt = 0; nt < kTilesPW; ++nt) {
                Frag b;
                if constexpr (BITS == 4) {
                    const uint32_t c[4] = {bw[nt][0].x, bw[nt][0].y, bw[nt][0].z, bw[nt][0].w};
                    b = q4_paired(c[j]);
                } else {
                    const uint32_t c[8] = {bw[nt][0].x, bw[nt][0].y, bw[nt][0].z, bw[nt][0].w,
                                           bw[nt][1].x, bw[nt][1].y, bw[nt][1].z, bw[nt][1].w};
                    b = q8_paired(c[2 * j], c[2 * j + 1]);
                }
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    D[nt][m] = mfma_bf16(ah[m], b, D[nt][m]);
                    if constexpr (F32) D[nt][m] = mfma_bf16(al[m], b, mfma_bf16(am[m], b, D[nt][m]));
                }
            }
            if ((32 * (j + 1)) % G == 0) {  // a group closes: P += s D
                const int g = 32 * j / G;
#pragma unroll
                for (int nt = 0; nt < kTilesPW; ++nt) {
                    const float s = __uint_as_float(sb[S::SC + (wrow0 + 16 * nt) * 4 + g]);
#pragma unroll
                    for (int m = 0; m < 2; ++m) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) P[nt][m][i] = fmaf(s, D[nt][m][i], P[nt][m][i]);
                        D[nt][m] = float4v{0, 0, 0, 0};
                    }
                }
            }
        }
        // the stage's min terms: sum over its groups of m'[n, g] xs[t, g], one FP32 MFMA per tile pair
#pragma unroll
        for (int nt = 0; nt < kTilesPW; ++nt) {
            const float mp = __uint_as_float(sb[S::MP + (wrow0 + 16 * nt) * 4 + qd]);
#pragma unroll
            for (int m = 0; m < 2; ++m)
                P[nt][m] = mfma_f32x4(__uint_as_float(sb[S::XS + qd * kTok + 16 * m + n]), mp, P[nt][m]);
        }
        if ((st + 1) % sps == 0) {  // the stream ends: A += inv_s P
            const int par = (int)((st / sps) & 1);
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                const float4 iv = *reinterpret_cast<const float4 *>(&invs[par][16 * m + 4 * qd]);
                const float ivv[4] = {iv.x, iv.y, iv.z, iv.w};
#pragma unroll
                for (int nt = 0; nt < kTilesPW; ++nt) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) A[nt][m][i] = fmaf(ivv[i], P[nt][m][i], A[nt][m][i]);
                    P[nt][m] = float4v{0, 0, 0, 0};
                }
            }
        }
    };

    // stage st computes from LDS buffer st % 2 while stage st + 1 goes from registers to the other buffer and stage
    // st + 2's loads are in flight (register set st % 2, free since stage st reached LDS)
    auto step = [&](uint32_t st, Regs &mine, Regs &other) {
        load_stage(st + 2 < stages ? st + 2 : stages - 1, mine);  // unconditional, so the waits below count exactly
        compute(st, lds + (st & 1) * S::SIZE);
        if (st + 1 < stages) write_stage(st + 1, lds + ((st + 1) & 1) * S::SIZE, other);
        __syncthreads();
    };
    load_stage(0, rgs[0]);
    load_stage(stages > 1 ? 1 : 0, rgs[1]);
    write_stage(0, lds, rgs[0]);
    __syncthreads();
    for (uint32_t st = 0; st < stages; st += 2) {
        step(st, rgs[0], rgs[1]);
        if (st + 1 < stages) step(st + 1, rgs[1], rgs[0]);
    }

    // ---- epilogue: z = a / 4 -> h (rows < r) or the injection gates (rows r .. r + 3)
#pragma unroll
    for (int nt = 0; nt < kTilesPW; ++nt) {
        const int64_t row = rb + wrow0 + 16 * nt;
        if (row >= R) continue;
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t t = t0 + 16 * m + 4 * qd + i;
                if (t >= Tn) continue;
                const float z = A[nt][m][i] * 0.25f;
                if (row < r) h[t * r + row] = z / (1.0f + expf(-z));
                else w_in[t * kStreams + (row - r)] = 2.0f / (1.0f + expf(-z));
            }
    }
}

template <int BITS, bool F32> constexpr size_t down_tile_lds() { return (size_t)2 * dn::Stage<BITS, F32>::SIZE * 4; }

// ================================================================================================ down: vector rows
// KS waves share a row (its chunks split over them, their totals meeting in LDS) or, KS = 1, a wave takes one row; MT
// tokens a block. The streams' inverse RMS is known before the dot products (the block's first phase), so each
// chunk's dot goes straight into one accumulator a token, scaled by its stream's inverse RMS:
// a = sum over chunks of inv[stream(chunk)] (s dot + m sum(x)).
template <typename T, int BITS, int MT, int KS>
__global__ void __launch_bounds__(256)
    mix_down_rows_kernel(const T *x, const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t R,
                         int64_t d, int64_t G, int64_t r, float eps, int64_t Tn, float *h, float *w_in, float *inv) {
    constexpr int kWaves = 4;
    __shared__ float invs[MT][kStreams];
    __shared__ float red[KS > 1 ? kWaves : 1][MT];  // KS > 1: wave w's totals (its row w / KS, part w % KS)
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int64_t K = kStreams * d, t0 = (int64_t)blockIdx.y * MT;
    const int nt = (int)(Tn - t0 < MT ? Tn - t0 : MT);
    // wave s: the inverse RMS of stream s of each token of the group (the tokens' loads of a step issued together)
    {
        float sq[MT];
#pragma unroll
        for (int tt = 0; tt < MT; ++tt) sq[tt] = 0.f;
        for (int64_t i = 8 * lane; i < d; i += 8 * kWave) {
            float v[MT][8];
#pragma unroll
            for (int tt = 0; tt < MT; ++tt)
                if (tt < nt) ld8(x + (t0 + tt) * K + (int64_t)wave * d, i, v[tt]);
#pragma unroll
            for (int tt = 0; tt < MT; ++tt)
                if (tt < nt)
#pragma unroll
                    for (int k = 0; k < 8; ++k) sq[tt] = fmaf(v[tt][k], v[tt][k], sq[tt]);
        }
#pragma unroll
        for (int tt = 0; tt < MT; ++tt) {
            const float tot = wave_sum(sq[tt]);
            if (lane == 0 && tt < nt) invs[tt][wave] = 1.0f / sqrtf(tot / (float)d + eps);
        }
    }
    __syncthreads();
    if (blockIdx.x == 0 && lane == 0)
        for (int tt = 0; tt < nt; ++tt) inv[(t0 + tt) * kStreams + wave] = invs[tt][wave];
    const int64_t row = (int64_t)blockIdx.x * (kWaves / KS) + wave / KS;
    const int part = wave % KS;
    if (KS == 1 && row >= R) return;  // after the block's only barrier (KS > 1: the grid holds whole rows)
    const int64_t grow = row < R ? row : R - 1;
    const uint8_t *qrow = q + grow * (K * BITS / 8);
    const int64_t nc = K / kChunk, cps = d / kChunk;  // chunks of the row, chunks a stream
    float iv[MT][kStreams];
#pragma unroll
    for (int tt = 0; tt < MT; ++tt)
#pragma unroll
        for (int st = 0; st < kStreams; ++st) iv[tt][st] = tt < nt ? invs[tt][st] : 0.f;
    float acc[MT];
#pragma unroll
    for (int tt = 0; tt < MT; ++tt) acc[tt] = 0.f;
#pragma unroll 2
    for (int64_t c = (int64_t)part * kWave + lane; c < nc; c += (int64_t)kWave * KS) {
        uint32_t w[BITS];
#pragma unroll
        for (int i = 0; i < BITS / 4; ++i) {
            const uint4 u = reinterpret_cast<const uint4 *>(qrow + c * (kChunk * BITS / 8))[i];
            w[4 * i] = u.x, w[4 * i + 1] = u.y, w[4 * i + 2] = u.z, w[4 * i + 3] = u.w;
        }
        const int64_t gi = grow * (K / G) + c * kChunk / G;
        const float sc = bf16_to_f32(scale[gi]), mn = bf16_to_f32(minv[gi]);
        const int sg = (int)(c / cps);  // the chunk's stream
        float cf[kChunk];
#pragma unroll
        for (int k = 0; k < kChunk; ++k)
            cf[k] = (float)((w[k * BITS / 32] >> ((k * BITS) % 32)) & ((1u << BITS) - 1u));
#pragma unroll
        for (int tt = 0; tt < MT; ++tt) {
            if (tt >= nt) break;
            const T *xc = x + (t0 + tt) * K + c * kChunk;
            float dot = 0.f, xsum = 0.f;
#pragma unroll
            for (int p8 = 0; p8 < kChunk / 8; ++p8) {
                float v[8];
                ld8(xc, 8 * p8, v);
#pragma unroll
                for (int k = 0; k < 8; ++k) dot = fmaf(v[k], cf[8 * p8 + k], dot), xsum += v[k];
            }
            const float s_inv = sg == 0 ? iv[tt][0] : sg == 1 ? iv[tt][1] : sg == 2 ? iv[tt][2] : iv[tt][3];
            acc[tt] = fmaf(s_inv, fmaf(sc, dot, mn * xsum), acc[tt]);
        }
    }
    float tot[MT];
#pragma unroll
    for (int tt = 0; tt < MT; ++tt) tot[tt] = wave_sum(acc[tt]);
    if constexpr (KS > 1) {
        if (lane == 0)
#pragma unroll
            for (int tt = 0; tt < MT; ++tt) red[wave][tt] = tot[tt];
        __syncthreads();
        if (part != 0) return;
#pragma unroll
        for (int tt = 0; tt < MT; ++tt) {
            float v = 0.f;
            for (int k = 0; k < KS; ++k) v += red[wave + k][tt];  // part 0's wave: its row's KS waves from here
            tot[tt] = v;
        }
    }
    if (lane != 0 || row >= R) return;
    for (int tt = 0; tt < nt; ++tt) {
        const int64_t t = t0 + tt;
        const float z = tot[tt] * 0.25f;
        if (row < r) h[t * r + row] = z / (1.0f + expf(-z));
        else w_in[t * kStreams + (row - r)] = 2.0f / (1.0f + expf(-z));
    }
}

// ================================================================================================ up: MFMA tiles
// WAVES column tiles of 16 positions j a block (a wave each), MT 16-token tiles; LDS: h as bf16 hi / mid / lo [16 MT][r + 8]
// in the paired k order, then its group sums [r / G][16 MT] (FP32)
template <typename T, int BITS, int MT, int WAVES>
__global__ void __launch_bounds__(WAVES * kWave)
    mix_up_tile_kernel(const float *h, const uint8_t *q, const uint16_t *scale, const uint16_t *minv, const T *x,
                       const float *norm_w, const float *inv, int64_t d, int64_t r, int64_t G, int64_t Tn, T *u) {
    constexpr int NTHR = WAVES * kWave, TOK = 16 * MT, CB = kChunk * BITS / 8;
    extern __shared__ uint32_t lds[];
    const int rdw = (int)(r / 2 + 4);  // dwords a staged h row
    uint32_t *hh = lds, *hm = lds + TOK * rdw, *hl = lds + 2 * TOK * rdw;
    float *hsum = reinterpret_cast<float *>(lds + 3 * TOK * rdw);
    const int64_t N = kStreams * d, ngr = r / G;
    const uint32_t njb = (uint32_t)((d / 16 + WAVES - 1) / WAVES);
    const uint32_t L = xcd_block(blockIdx.x, gridDim.x);
    const int64_t t0 = (int64_t)(L / njb) * TOK;
    const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave, n = lane % 16, qd = lane / 16;

    // h -> LDS as hi / mid / lo, 8 consecutive k a thread; the G / 8 threads of a group are neighbouring lanes
    // (a token's units are consecutive and G / 8 divides both r / 8 and the block), and their partial sums meet by
    // butterfly into the group sums, padded with zeros to a multiple of 4 groups
    const int ngr4 = (int)((ngr + 3) / 4 * 4);
    for (int p = tid; p < (ngr4 - (int)ngr) * TOK; p += NTHR) hsum[(ngr + p / TOK) * TOK + p % TOK] = 0.f;
    const int units = TOK * (int)(r / 8), upg = (int)(G / 8);
    for (int ub = 0; ub < units; ub += NTHR) {
        const int uix = ub + tid;
        float part = 0.f;
        int t = 0, k8 = 0;
        if (uix < units) {
            t = uix / (int)(r / 8), k8 = uix % (int)(r / 8);
            // rows past the tokens are zeros (their outputs are not stored), so a short batch loads only its rows
            float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
            if (t0 + t < Tn) {
                a = *reinterpret_cast<const float4 *>(h + (t0 + t) * r + 8 * k8);
                b = *reinterpret_cast<const float4 *>(h + (t0 + t) * r + 8 * k8 + 4);
            }
            const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            const Split v = split8(f);
            *reinterpret_cast<uint4 *>(hh + t * rdw + 4 * k8) = uint4{v.hi.d[0], v.hi.d[1], v.hi.d[2], v.hi.d[3]};
            *reinterpret_cast<uint4 *>(hm + t * rdw + 4 * k8) = uint4{v.mid.d[0], v.mid.d[1], v.mid.d[2], v.mid.d[3]};
            *reinterpret_cast<uint4 *>(hl + t * rdw + 4 * k8) = uint4{v.lo.d[0], v.lo.d[1], v.lo.d[2], v.lo.d[3]};
            part = v.sum;
        }
        for (int o = 1; o < upg; o <<= 1) part += __shfl_xor(part, o, kWave);
        if (uix < units && k8 % upg == 0) hsum[(k8 / upg) * TOK + t] = part;
    }
    __syncthreads();

    const int64_t j0 = ((int64_t)(L % njb) * WAVES + wave) * 16;
    if (j0 >= d) return;  // after the block's barriers
    const int64_t nc = r / kChunk;
    // the wave's 4 weight tiles: rows s d + j0 .. + 15; lane row s d + j0 + n
    const uint8_t *qb = q + (j0 + n) * CB + (BITS == 4 ? 4 : 8) * qd;
    float4v acc[kStreams][MT], D[kStreams][MT];
#pragma unroll
    for (int s = 0; s < kStreams; ++s)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[s][m] = D[s][m] = float4v{0, 0, 0, 0};
    using CodeT = typename std::conditional<BITS == 4, uint32_t, uint2>::type;
    struct Ahead {
        CodeT q[kStreams];
        uint16_t sc[kStreams];  // the chunk's group's scales
    };
    // unconditional loads (the last chunk re-reads itself), so the compiler's waits count them exactly
    auto ld_chunk = [&](int64_t c, Ahead &a) {
        c = c < nc ? c : nc - 1;
        const int64_t g = kChunk * c / G;
#pragma unroll
        for (int s = 0; s < kStreams; ++s) {
            a.q[s] = *reinterpret_cast<const CodeT *>(qb + (c * N + s * d) * CB);
            a.sc[s] = scale[g * N + s * d + j0 + n];
        }
    };
    // the operands of the min terms and of the epilogue depend on nothing the loop computes: for a 16-token tile (a
    // short, latency-bound kernel) they are loaded now, so their round trips overlap the loop instead of following it
    // (all loads unconditional, indices clamped); a 32-token tile has no registers to spare and loads them after it
    constexpr bool kHoist = MT == 1;
    constexpr int kMinPre = kHoist ? 2 : 1;  // four-group steps of the min terms held here; more load after the loop
    uint16_t pre_s[kMinPre][kStreams], pre_m[kMinPre][kStreams];
#pragma unroll
    for (int gs = 0; gs < kMinPre; ++gs) {
        if (!kHoist) break;
        const int g = 4 * gs + qd < ngr ? 4 * gs + qd : 0;
#pragma unroll
        for (int s = 0; s < kStreams; ++s) {
            const int64_t gi = g * N + s * d + j0 + n;
            pre_s[gs][s] = scale[gi], pre_m[gs][s] = minv[gi];
        }
    }
    const int64_t j = j0 + n;  // < d: d is a multiple of 16
    float nwv[kStreams], xe[MT][4][kStreams], ie[MT][4][kStreams];
    auto load_epilogue = [&]() {
#pragma unroll
        for (int s = 0; s < kStreams; ++s) nwv[s] = 1.0f + norm_w[s * d + j];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t t = t0 + 16 * m + 4 * qd + i, tc = t < Tn ? t : Tn - 1;
#pragma unroll
            for (int s = 0; s < kStreams; ++s) xe[m][i][s] = ld_act(x, tc * N + s * d + j), ie[m][i][s] = inv[tc * kStreams + s];
        }
    };
    if constexpr (kHoist) load_epilogue();

    // a ring of kAhead chunks in flight: chunk c computes from slot c % kAhead, then that slot loads chunk c + kAhead
    constexpr int kAhead = 4;  // (8 for the 16-token tiles measured slower: 15.1 against 13.2 us at 1 token)
    Ahead ring[kAhead];
#pragma unroll
    for (int p = 0; p < kAhead; ++p) ld_chunk(p, ring[p]);
    auto chunk = [&](int64_t c, Ahead &a) {
        if (c < nc) {
            Frag ah[MT], am[MT], al[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const int at = (16 * m + n) * rdw + 16 * (int)c + 4 * qd;
                const uint4 v = lds16(hh + at), w = lds16(hm + at), z = lds16(hl + at);
                ah[m] = Frag{{v.x, v.y, v.z, v.w}}, am[m] = Frag{{w.x, w.y, w.z, w.w}}, al[m] = Frag{{z.x, z.y, z.z, z.w}};
            }
#pragma unroll
            for (int s = 0; s < kStreams; ++s) {
                Frag b;
                if constexpr (BITS == 4) b = q4_paired(a.q[s]);
                else b = q8_paired(a.q[s].x, a.q[s].y);
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    D[s][m] = mfma_bf16(al[m], b, mfma_bf16(am[m], b, mfma_bf16(ah[m], b, D[s][m])));
            }
            if ((kChunk * (c + 1)) % G == 0) {  // a group closes: acc += s D
#pragma unroll
                for (int s = 0; s < kStreams; ++s) {
                    const float sc = bf16_to_f32(a.sc[s]);
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[s][m][i] = fmaf(sc, D[s][m][i], acc[s][m][i]);
                        D[s][m] = float4v{0, 0, 0, 0};
                    }
                }
            }
        }
        ld_chunk(c + kAhead, a);  // unconditional (clamped), so the waits count it exactly
    };
    for (int64_t c = 0; c < nc; c += kAhead) {
#pragma unroll
        for (int p = 0; p < kAhead; ++p) chunk(c + p, ring[p]);
    }
    // the min terms: sum_g m'[row, g] hsum[t, g], four groups an FP32 MFMA
    for (int g4 = 0; g4 < ngr4; g4 += 4) {
        const int g = g4 + qd;
#pragma unroll
        for (int s = 0; s < kStreams; ++s) {
            float mp = 0.f;
            if (g < ngr) {
                float sc, mn;
                if (kHoist && g4 / 4 < kMinPre) {
                    const int gs = g4 / 4;
                    sc = bf16_to_f32(gs == 0 ? pre_s[0][s] : pre_s[kMinPre - 1][s]);
                    mn = bf16_to_f32(gs == 0 ? pre_m[0][s] : pre_m[kMinPre - 1][s]);
                } else {
                    const int64_t gi = g * N + s * d + j0 + n;
                    sc = bf16_to_f32(scale[gi]), mn = bf16_to_f32(minv[gi]);
                }
                mp = min_prime<BITS>(sc, mn);
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) acc[s][m] = mfma_f32x4(hsum[g * TOK + 16 * m + n], mp, acc[s][m]);
        }
    }
    // epilogue: gates and the stream combine, in registers
    if constexpr (!kHoist) load_epilogue();
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t t = t0 + 16 * m + 4 * qd + i;
            if (t >= Tn) continue;
            float sum = 0.f;
#pragma unroll
            for (int s = 0; s < kStreams; ++s) {
                const float gate = 1.0f / (1.0f + expf(-acc[s][m][i]));
                sum += gate * (xe[m][i][s] * ie[m][i][s] * nwv[s]);
            }
            st_act(u, t * d + j, sum * 0.25f);
        }
}

inline size_t up_tile_lds(int MT, int64_t r, int64_t G) {
    const int64_t ngr4 = (r / G + 3) / 4 * 4;
    return (size_t)(3 * 16 * MT * (r / 2 + 4) + ngr4 * 16 * MT) * 4;
}

// ================================================================================================ launchers
// Raises a tile kernel's dynamic LDS allowance to `bytes` when it is below (kept per kernel, so a launch that needs
// no more than before makes no runtime call).
void allow_lds(const void *kernel, size_t bytes) {
    static std::mutex mu;
    static std::vector<std::pair<const void *, size_t>> granted;
    std::lock_guard<std::mutex> lock(mu);
    auto it = std::find_if(granted.begin(), granted.end(), [&](const auto &e) { return e.first == kernel; });
    if (it != granted.end() && it->second >= bytes) return;
    STRIX_HIP_CHECK(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes),
                    "hc mix: allowing ", bytes, " bytes of LDS");
    if (it != granted.end()) it->second = bytes;
    else granted.emplace_back(kernel, bytes);
}

struct Weights {  // either format's arrays
    const uint8_t *q;
    const uint16_t *scale, *minv;
    int64_t N, K, G;
};

// Shape rules both mixes share (strixite kernels/hc.hpp:20-50); `what` names the mix in messages.
void require_common(const char *what, const Weights &w, const void *x, int64_t T, int64_t H, int64_t d, Act act) {
    STRIX_CHECK(H == kStreams, what, ": ", H, " residual streams given; this build mixes exactly ", kStreams);
    STRIX_CHECK(T >= 1 && T <= kMaxTokens, what, ": ", T, " tokens; 1 to ", kMaxTokens, " are taken");
    STRIX_CHECK(d >= kChunk && d <= kMaxD && d % kChunk == 0, what, ": stream width d = ", d,
                " must be a multiple of ", kChunk, " between ", kChunk, " and ", kMaxD);
    STRIX_CHECK(act == Act::F32 || act == Act::BF16, what, ": activation type ", (int)act, " is neither F32 nor BF16");
    STRIX_CHECK(w.q && w.scale && w.minv, what, ": the weight view has a null array");
    STRIX_CHECK(w.G == 32 || w.G == 64 || w.G == 128, what, ": weight group size ", w.G, " (32, 64 or 128 expected)");
    STRIX_CHECK(w.K >= w.G && w.K % w.G == 0, what, ": weight K = ", w.K, " is not a whole number of ", w.G,
                "-code groups");
    STRIX_CHECK(reinterpret_cast<uintptr_t>(w.q) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0, what,
                ": the codes and the streams must start on 16-byte boundaries");
}

template <int BITS>
void run_mix_down(const void *x, const Weights &w, int64_t T, int64_t H, int64_t d, int64_t r, bool inject, float eps,
                  float *h, float *w_in, float *inv, Act act, hipStream_t stream) {
    const char *what = "hc_mix_down";
    require_common(what, w, x, T, H, d, act);
    STRIX_CHECK(h && inv, what, ": h and inv are required outputs");
    STRIX_CHECK(inject ? w_in != nullptr : w_in == nullptr, what, ": the injection gates w_in go with inject = true, "
                "and only with it");
    STRIX_CHECK(r >= 1 && r <= kMaxR, what, ": rank r = ", r, " outside 1..", kMaxR);
    STRIX_CHECK(w.K == H * d, what, ": the weight spans K = ", w.K, " inputs, the streams H d = ", H * d);
    const int64_t R = r + (inject ? H : 0);
    STRIX_CHECK(w.N == R, what, ": the weight holds ", w.N, " rows; r", inject ? " + H" : "", " = ", R,
                " rows are needed");
    STRIX_CHECK(std::isfinite(eps) && eps > 0.f, what, ": eps = ", eps, " (a finite positive value is needed)");
    const bool f32 = act == Act::F32;
    if (T >= kDownTileMinTokens && d % dn::kK == 0) {  // matrix-core tiles
        const int64_t nrb = (R + dn::kRows - 1) / dn::kRows, ntt = (T + dn::kTok - 1) / dn::kTok;
        const size_t lds = f32 ? down_tile_lds<BITS, true>() : down_tile_lds<BITS, false>();
        auto go = [&](auto tag, auto gtag) {
            using TT = decltype(tag);
            constexpr int GG = decltype(gtag)::value;
            auto k = mix_down_tile_kernel<TT, BITS, GG>;
            allow_lds((const void *)k, lds);
            k<<<(unsigned)(nrb * ntt), dn::kThreads, lds, stream>>>(static_cast<const TT *>(x), w.q, w.scale, w.minv,
                                                                    R, d, r, eps, T, h, w_in, inv);
        };
        auto by_g = [&](auto tag) {
            if (w.G == 32) go(tag, std::integral_constant<int, 32>{});
            else if (w.G == 64) go(tag, std::integral_constant<int, 64>{});
            else go(tag, std::integral_constant<int, 128>{});
        };
        if (f32) by_g(float{});
        else by_g(uint16_t{});
    } else {  // vector rows: up to 16 tokens the 4 waves split each row; more tokens share a row's code loads
        const int mt = T == 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : 8;
        // up to 16 tokens, 4 waves split each row's K (measured at d 2560, r 320: 16 tokens 29.4 -> 24.3 us, 5 tokens
        // 21.3 -> 16.2); above, a wave a row
        const int ks = T <= 16 ? 4 : 1;
        const int rows_pb = 4 / ks;
        const dim3 grid((unsigned)((R + rows_pb - 1) / rows_pb), (unsigned)((T + mt - 1) / mt));
        auto go = [&](auto tag, auto mtag) {
            using TT = decltype(tag);
            constexpr int MT = decltype(mtag)::value;
            if (T == 1)
                mix_down_rows_kernel<TT, BITS, 1, 4><<<grid, 256, 0, stream>>>(
                    static_cast<const TT *>(x), w.q, w.scale, w.minv, R, d, w.G, r, eps, T, h, w_in, inv);
            else if (ks == 4)
                mix_down_rows_kernel<TT, BITS, MT, 4><<<grid, 256, 0, stream>>>(
                    static_cast<const TT *>(x), w.q, w.scale, w.minv, R, d, w.G, r, eps, T, h, w_in, inv);
            else
                mix_down_rows_kernel<TT, BITS, MT, 1><<<grid, 256, 0, stream>>>(
                    static_cast<const TT *>(x), w.q, w.scale, w.minv, R, d, w.G, r, eps, T, h, w_in, inv);
        };
        auto by_mt = [&](auto tag) {
            switch (mt) {
                case 1: go(tag, std::integral_constant<int, 1>{}); break;
                case 2: go(tag, std::integral_constant<int, 2>{}); break;
                case 4: go(tag, std::integral_constant<int, 4>{}); break;
                default: go(tag, std::integral_constant<int, 8>{}); break;
            }
        };
        if (f32) by_mt(float{});
        else by_mt(uint16_t{});
    }
    STRIX_HIP_CHECK_LAUNCH(what, " Q", BITS, " ", act_str(act), " T=", T, " R=", R, " K=", w.K, " G=", w.G);
}

template <int BITS>
void run_mix_up(const float *h, const Weights &w, const void *x, const float *norm_w, const float *inv, int64_t T,
                int64_t H, int64_t d, void *u, Act act, hipStream_t stream) {
    const char *what = "hc_mix_up";
    require_common(what, w, x, T, H, d, act);
    STRIX_CHECK(h && norm_w && inv && u, what, ": h, norm_w, inv and u must all be given");
    STRIX_CHECK(w.N == H * d, what, ": W_up holds ", w.N, " rows; H d = ", H * d, " are needed");
    STRIX_CHECK(w.K % kChunk == 0 && w.K <= kMaxR, what, ": W_up's K (the rank r) = ", w.K, " must be a multiple of ",
                kChunk, " up to ", kMaxR);
    STRIX_CHECK(reinterpret_cast<uintptr_t>(h) % 16 == 0, what, ": h must start on a 16-byte boundary");
    const int64_t es = act == Act::F32 ? 4 : 2;
    STRIX_CHECK(disjoint(u, T * d * es, x, T * H * d * es), what, ": u and the streams x overlap");
    // 16-token tiles of 4 waves a block up to 16 tokens, 32-token tiles of 8 waves above (the h tile shared by more
    // columns); 32-token tiles of h fit the LDS up to r = 768
    const bool small = T <= 16 || w.K > 768;
    const int MT = small ? 1 : 2, WAVES = small ? 4 : 8;
    const size_t lds = up_tile_lds(MT, w.K, w.G);
    const int64_t njb = (d / 16 + WAVES - 1) / WAVES, ntt = (T + 16 * MT - 1) / (16 * MT);
    auto go = [&](auto tag, auto mtag) {
        using TT = decltype(tag);
        constexpr int M = decltype(mtag)::value, WV = M == 1 ? 4 : 8;
        auto k = mix_up_tile_kernel<TT, BITS, M, WV>;
        allow_lds((const void *)k, lds);
        k<<<(unsigned)(njb * ntt), WV * kWave, lds, stream>>>(h, w.q, w.scale, w.minv, static_cast<const TT *>(x),
                                                              norm_w, inv, d, w.K, w.G, T, static_cast<TT *>(u));
    };
    auto by_mt = [&](auto tag) {
        if (small) go(tag, std::integral_constant<int, 1>{});
        else go(tag, std::integral_constant<int, 2>{});
    };
    if (act == Act::F32) by_mt(float{});
    else by_mt(uint16_t{});
    STRIX_HIP_CHECK_LAUNCH(what, " Q", BITS, " ", act_str(act), " T=", T, " d=", d, " r=", w.K, " G=", w.G);
}

}  // namespace

void hc_mix_down(const void *x, const Q4DeviceView &w, int64_t T, int64_t H, int64_t d, int64_t r, bool inject,
                 float eps, float *h, float *w_in, float *inv, Act act, hipStream_t stream) {
    run_mix_down<4>(x, {w.q, w.scale, w.minv, w.N, w.K, w.G}, T, H, d, r, inject, eps, h, w_in, inv, act, stream);
}
void hc_mix_down(const void *x, const Q8DeviceView &w, int64_t T, int64_t H, int64_t d, int64_t r, bool inject,
                 float eps, float *h, float *w_in, float *inv, Act act, hipStream_t stream) {
    run_mix_down<8>(x, {w.q, w.scale, w.minv, w.N, w.K, w.G}, T, H, d, r, inject, eps, h, w_in, inv, act, stream);
}
void hc_mix_up(const float *h, const Q4ChunkMajorView &w, const void *x, const float *norm_w, const float *inv,
               int64_t T, int64_t H, int64_t d, void *u, Act act, hipStream_t stream) {
    run_mix_up<4>(h, {w.q, w.scale, w.minv, w.N, w.K, w.G}, x, norm_w, inv, T, H, d, u, act, stream);
}
void hc_mix_up(const float *h, const Q8ChunkMajorView &w, const void *x, const float *norm_w, const float *inv,
               int64_t T, int64_t H, int64_t d, void *u, Act act, hipStream_t stream) {
    run_mix_up<8>(h, {w.q, w.scale, w.minv, w.N, w.K, w.G}, x, norm_w, inv, T, H, d, u, act, stream);
}

}  // namespace strix::kernels
