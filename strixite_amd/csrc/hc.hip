// The hyper-connection mix that produces the MoE sublayer's input (strixite kernels/hc.hpp:31-50, the step before the
// path: hc_mix(l.hc_mlp), runtime/qwen4exp.cpp:2801-2832) on gfx950: hc_mix_down (the low-rank projection of the
// four RMS-normalized residual streams, the injection gates and the streams' inverse RMS) and hc_mix_up (the gated
// up projection combined over the streams into u). hc_inject, the other end, lives with the shared-expert add
// (router.hip).
//
// Semantics (strixite kernels/hc.hpp:3-18, :31-50): X [T, 4 d] in the activation dtype, everything inside FP32, u
// rounded once to the activation dtype.
//   hc_mix_down: inv[t, s] = 1 / sqrt(mean_j X[t, s d + j]^2 + eps); a[t, n] = sum_s inv[t, s] (W[n, s-block] .
//     X[t, s-block]) for the rows n of the folded weight W [r (+ 4), 4 d] (Q4 or Q8, row-major); h[t, n] = silu(a /
//     4) for n < r, w_in[t, n - r] = 2 sigmoid(a / 4) for the 4 injection rows. Per 32-code chunk the dot is
//     s * sum(x * code) + m * sum(x), FP32.
//   hc_mix_up: u[t, j] = (1/4) sum_s sigmoid(W_up[s d + j] . h[t]) * (X[t, s d + j] * inv[t, s] * (1 + norm_w[s d +
//     j])), W_up [4 d, r] chunk-major (32-code chunk c of row n at q[(c N + n) * 16] (Q4) or [(c N + n) * 32] (Q8),
//     group g's scale / min at [g N + n]; strixite formats/q4.hpp:43-55).
//
// hc_mix_down: a block of 4 waves serves 4 weight rows for a group of MT tokens. Its waves first compute the
// streams' inverse RMS of those tokens (wave s: stream s, 8 elements a lane a step, a butterfly) into LDS; then each
// wave takes one row: lane l walks the row's 32-code chunks l, l + 64, ... (the 64 lanes' code loads are one
// contiguous run of the row; a chunk lies inside one stream as d % 32 == 0), dots each with the chunk of every token
// of the group (x rows from L2, one contiguous 4 KB run across the lanes) into per-stream sums, then a butterfly.
// hc_mix_up: a block covers 64 output columns j; its thread (s, jl) owns row s d + j of W_up for the group's tokens,
// so the 64 threads of a stream read 64 consecutive rows, which the chunk-major layout puts next to each other (one
// contiguous run per 16-byte load instruction); a thread issues 8 chunks' loads before it uses them; the tokens' h live
// in LDS with each chunk's sum of h, and the 4 streams' gated terms meet in LDS, summed in stream order.
#include "common.hpp"

#include <cmath>

namespace strix::kernels {

namespace {

using namespace strix::dev;
constexpr int kWave = 64, kThreads = 256, kStreams = 4, kChunk = 32;
constexpr int64_t kMaxR = 1024, kMaxTokens = 65535, kMaxD = 1 << 20;

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

// a 32-code chunk: BITS / 4 16-byte loads; code i
template <int BITS> __device__ __forceinline__ void ld_chunk(const uint8_t *p, uint32_t (&w)[BITS]) {
#pragma unroll
    for (int i = 0; i < BITS / 4; ++i) {
        const uint4 u = reinterpret_cast<const uint4 *>(p)[i];
        w[4 * i] = u.x, w[4 * i + 1] = u.y, w[4 * i + 2] = u.z, w[4 * i + 3] = u.w;
    }
}
template <int BITS> __device__ __forceinline__ float code_at(const uint32_t (&w)[BITS], int i) {
    constexpr int per = 32 / BITS;
    return (float)((w[i / per] >> (BITS * (i % per))) & ((1u << BITS) - 1u));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// KS waves share a row (split over its chunks, sums meeting in LDS), or a wave takes RW consecutive rows and loads
// each activation chunk once for them; 4 RW / KS rows a block
template <typename T, int BITS, int MT, int KS, int RW>
__global__ void __launch_bounds__(kThreads)
    hc_down_kernel(const T *x, const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t R, int64_t K,
                   int64_t d, int64_t G, int64_t r, float eps, int64_t Tn, float *h, float *w_in, float *inv) {
    __shared__ float invs[MT][kStreams];
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int64_t t0 = (int64_t)blockIdx.y * MT;
    const int nt = (int)(Tn - t0 < MT ? Tn - t0 : MT);
    // the inverse RMS of stream `wave` of each token
    for (int tt = 0; tt < nt; ++tt) {
        const T *xs = x + (t0 + tt) * K + (int64_t)wave * d;
        float sq = 0.f;
#pragma unroll 8
        for (int64_t i = 8 * lane; i < d; i += 8 * kWave) {
            float v[8];
            ld8(xs, i, v);
#pragma unroll
            for (int k = 0; k < 8; ++k) sq = fmaf(v[k], v[k], sq);
        }
        sq = wave_sum(sq);
        if (lane == 0) invs[tt][wave] = 1.0f / sqrtf(sq / (float)d + eps);
    }
    __syncthreads();
    if (blockIdx.x == 0 && lane == 0)
        for (int tt = 0; tt < nt; ++tt) inv[(t0 + tt) * kStreams + wave] = invs[tt][wave];
    constexpr int RPB = kThreads / kWave / KS;  // rows a block
    const int64_t n0 = ((int64_t)blockIdx.x * RPB + wave / KS) * RW;  // the wave's first row
    const int kw = wave % KS;
    if (KS == 1 && n0 >= R) return;  // after the only barrier (KS > 1: the grid holds whole rows)
    float acc[RW][MT][kStreams];
#pragma unroll
    for (int rr = 0; rr < RW; ++rr)
#pragma unroll
        for (int tt = 0; tt < MT; ++tt)
#pragma unroll
            for (int s = 0; s < kStreams; ++s) acc[rr][tt][s] = 0.f;
    const int64_t nc = K / kChunk;
#pragma unroll 2
    for (int64_t c = (int64_t)kw * kWave + lane; c < nc; c += (int64_t)kWave * KS) {
        uint32_t w[RW][BITS];
        float sc[RW], mn[RW];
#pragma unroll
        for (int rr = 0; rr < RW; ++rr) {  // rows past R read the last one (not stored)
            const int64_t n = n0 + rr < R ? n0 + rr : R - 1;
            ld_chunk<BITS>(q + (n * nc + c) * (kChunk * BITS / 8), w[rr]);
            const int64_t gi = n * (K / G) + c * kChunk / G;
            sc[rr] = bf16_to_f32(scale[gi]), mn[rr] = bf16_to_f32(minv[gi]);
        }
        const int sg = (int)(c * kChunk / d);
        float cf[RW][kChunk];  // the codes as floats, once for the token group
#pragma unroll
        for (int rr = 0; rr < RW; ++rr)
#pragma unroll
            for (int k = 0; k < kChunk; ++k) cf[rr][k] = code_at<BITS>(w[rr], k);
#pragma unroll
        for (int tt = 0; tt < MT; ++tt) {
            if (tt >= nt) break;
            const T *xc = x + (t0 + tt) * K + c * kChunk;  // one load of the chunk for the wave's RW rows
            float xv[kChunk], xsum = 0.f;
#pragma unroll
            for (int p = 0; p < kChunk / 8; ++p) {
                float v[8];
                ld8(xc, 8 * p, v);
#pragma unroll
                for (int k = 0; k < 8; ++k) xv[8 * p + k] = v[k], xsum += v[k];
            }
#pragma unroll
            for (int rr = 0; rr < RW; ++rr) {
                float dot = 0.f;
#pragma unroll
                for (int k = 0; k < kChunk; ++k) dot = fmaf(xv[k], cf[rr][k], dot);
                const float pv = fmaf(sc[rr], dot, mn[rr] * xsum);
#pragma unroll
                for (int s = 0; s < kStreams; ++s)  // constant indices keep acc in registers
                    if (s == sg) acc[rr][tt][s] += pv;
            }
        }
    }
    if constexpr (KS > 1) {  // (RW 1) the waves' per-stream sums meet in LDS; wave 0 adds them in wave order
        __shared__ float red[KS][MT][kStreams];
#pragma unroll
        for (int tt = 0; tt < MT; ++tt)
#pragma unroll
            for (int s = 0; s < kStreams; ++s) {
                const float v = wave_sum(acc[0][tt][s]);
                if (lane == 0) red[kw][tt][s] = v;
            }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int tt = 0; tt < MT; ++tt)
#pragma unroll
            for (int s = 0; s < kStreams; ++s) {
                float v = 0.f;
                for (int k = 0; k < KS; ++k) v += red[k][tt][s];
                acc[0][tt][s] = v;
            }
    }
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) {
        const int64_t n = n0 + rr;
        if (n >= R) break;
#pragma unroll
        for (int tt = 0; tt < MT; ++tt) {
            if (tt >= nt) break;
            float a = 0.f;
#pragma unroll
            for (int s = 0; s < kStreams; ++s)
                a = fmaf(invs[tt][s], KS > 1 ? acc[rr][tt][s] : wave_sum(acc[rr][tt][s]), a);
            if (lane == 0) {
                const int64_t t = t0 + tt;
                const float z = a / (float)kStreams;
                if (n < r) h[t * r + n] = z / (1.0f + expf(-z));
                else w_in[t * kStreams + (n - r)] = 2.0f / (1.0f + expf(-z));
            }
        }
    }
}

constexpr int kUpCols = kThreads / kStreams;  // output columns a block (its threads: 4 streams x 64 columns)
constexpr int kUpBatch = 8;                   // chunk loads a thread issues before it uses them

template <typename T, int BITS, int MT>
__global__ void __launch_bounds__(kThreads)
    hc_up_kernel(const float *h, const uint8_t *q, const uint16_t *scale, const uint16_t *minv, const T *x,
                 const float *norm_w, const float *inv, int64_t d, int64_t r, int64_t G, int64_t Tn, T *u) {
    __shared__ float hs[MT][kMaxR];
    __shared__ float hsum[MT][kMaxR / kChunk];
    __shared__ float part[MT][kStreams][kUpCols];
    const int64_t t0 = (int64_t)blockIdx.y * MT;
    const int nt = (int)(Tn - t0 < MT ? Tn - t0 : MT);
    for (int i = threadIdx.x; i < nt * r; i += kThreads) hs[i / r][i % r] = h[(t0 + i / r) * r + i % r];
    __syncthreads();
    const int nc = (int)(r / kChunk);
    for (int i = threadIdx.x; i < nt * nc; i += kThreads) {
        float s = 0.f;
        for (int k = 0; k < kChunk; ++k) s += hs[i / nc][(i % nc) * kChunk + k];
        hsum[i / nc][i % nc] = s;
    }
    __syncthreads();
    // thread (s, jl): row s d + j of W_up; the 64 threads of a stream read 64 consecutive rows (contiguous in the
    // chunk-major layout)
    const int s = threadIdx.x / kUpCols, jl = threadIdx.x % kUpCols;
    const int64_t j = (int64_t)blockIdx.x * kUpCols + jl, N = kStreams * d;
    const bool live = j < d;
    const int64_t row = s * d + (live ? j : d - 1);
    float acc[MT];
#pragma unroll
    for (int tt = 0; tt < MT; ++tt) acc[tt] = 0.f;
    for (int c0 = 0; c0 < nc; c0 += kUpBatch) {
        uint32_t w[kUpBatch][BITS];
        float sc[kUpBatch], mn[kUpBatch];
#pragma unroll
        for (int b = 0; b < kUpBatch; ++b)  // the batch's loads first (one round trip), then its math
            if (c0 + b < nc) {
                const int c = c0 + b;
                ld_chunk<BITS>(q + ((int64_t)c * N + row) * (kChunk * BITS / 8), w[b]);
                const int64_t gi = (int64_t)c * kChunk / G * N + row;
                sc[b] = bf16_to_f32(scale[gi]), mn[b] = bf16_to_f32(minv[gi]);
            }
#pragma unroll
        for (int b = 0; b < kUpBatch; ++b) {
            const int c = c0 + b;
            if (c >= nc) break;
#pragma unroll
            for (int tt = 0; tt < MT; ++tt) {
                if (tt >= nt) break;
                float dot = 0.f;
#pragma unroll
                for (int k = 0; k < kChunk; ++k) dot = fmaf(hs[tt][c * kChunk + k], code_at<BITS>(w[b], k), dot);
                acc[tt] = fmaf(sc[b], dot, fmaf(mn[b], hsum[tt][c], acc[tt]));
            }
        }
    }
    const float nw = 1.0f + norm_w[row];
#pragma unroll
    for (int tt = 0; tt < MT; ++tt) {
        if (tt >= nt) break;
        const int64_t t = t0 + tt;
        const float g = 1.0f / (1.0f + expf(-acc[tt]));
        part[tt][s][jl] = g * (ld_act(x, t * N + row) * inv[t * kStreams + s] * nw);
    }
    __syncthreads();
    if (s == 0 && live)  // the streams in order, as a running sum from 0
        for (int tt = 0; tt < nt; ++tt) {
            float sum = 0.f;
#pragma unroll
            for (int k = 0; k < kStreams; ++k) sum += part[tt][k][jl];
            st_act(u, (t0 + tt) * d + j, sum / (float)kStreams);
        }
}

struct QArr {
    const uint8_t *q;
    const uint16_t *scale, *minv;
    int64_t N, K, G;
};

void check_q(const char *fn, const QArr &w) {
    STRIX_CHECK(w.q != nullptr && w.scale != nullptr && w.minv != nullptr, fn, ": null weight pointer");
    STRIX_CHECK(w.G == 32 || w.G == 64 || w.G == 128, fn, ": group size ", w.G, " unsupported (32, 64 or 128)");
    STRIX_CHECK(w.K >= w.G && w.K % w.G == 0, fn, ": K = ", w.K, " must be a positive multiple of group size ", w.G);
    STRIX_CHECK(reinterpret_cast<uintptr_t>(w.q) % 16 == 0, fn, ": code array must be 16-byte aligned");
}

void check_shape(const char *fn, int64_t T, int64_t H, int64_t d, Act act) {
    STRIX_CHECK(H == kStreams, fn, ": H = ", H, " streams, only ", kStreams, " is supported");
    STRIX_CHECK(T >= 1 && T <= kMaxTokens, fn, ": T = ", T, " tokens, expected 1..", kMaxTokens);
    STRIX_CHECK(d >= kChunk && d <= kMaxD && d % kChunk == 0, fn, ": d = ", d, ", expected a multiple of ", kChunk,
                " in ", kChunk, "..", kMaxD);
    STRIX_CHECK(act == Act::F32 || act == Act::BF16, fn, ": unsupported activation dtype ", (int)act);
}

int tokens_per_block(int64_t T) { return T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : 8; }

template <int BITS>
void mix_down(const void *x, const QArr &w, int64_t T, int64_t H, int64_t d, int64_t r, bool inject, float eps,
              float *h, float *w_in, float *inv, Act act, hipStream_t stream) {
    const char *fn = "hc_mix_down";
    check_shape(fn, T, H, d, act);
    check_q(fn, w);
    STRIX_CHECK(x != nullptr && h != nullptr && inv != nullptr, fn, ": null pointer (x, h or inv)");
    STRIX_CHECK(inject == (w_in != nullptr), fn, ": w_in must be given exactly when inject");
    STRIX_CHECK(r >= 1 && r <= kMaxR, fn, ": r = ", r, ", expected 1..", kMaxR);
    STRIX_CHECK(w.K == H * d, fn, ": weight K = ", w.K, " != H*d = ", H * d);
    const int64_t R = r + (inject ? H : 0);
    STRIX_CHECK(w.N == R, fn, ": weight has ", w.N, " rows, expected ", R);
    STRIX_CHECK(reinterpret_cast<uintptr_t>(x) % 16 == 0, fn, ": x must be 16-byte aligned");
    STRIX_CHECK(std::isfinite(eps) && eps > 0.f, fn, ": eps must be finite and > 0, got ", eps);
    const int MT = tokens_per_block(T);
    // one token: a row's chunks split over the block's 4 waves (a round trip or two a lane, 4x the blocks); more
    // tokens: 4 rows a block, each wave's code loads shared by its token group (splitting measured no faster at 5)
    const bool split = T == 1;
    constexpr int kRW = 1;  // rows a wave when tokens share the waves' code loads (2: slower, measured)
    const int64_t rpb = split ? 1 : kThreads / kWave * kRW;
    const dim3 grid((unsigned)((R + rpb - 1) / rpb), (unsigned)((T + MT - 1) / MT));
    auto go = [&](auto tc, auto mtc) {
        using TT = decltype(tc);
        constexpr int MTV = decltype(mtc)::value;
        if constexpr (MTV == 1) {
            if (split) {
                hc_down_kernel<TT, BITS, 1, 4, 1><<<grid, kThreads, 0, stream>>>(
                    static_cast<const TT *>(x), w.q, w.scale, w.minv, R, w.K, d, w.G, r, eps, T, h, w_in, inv);
                return;
            }
        }
        hc_down_kernel<TT, BITS, MTV, 1, kRW><<<grid, kThreads, 0, stream>>>(
            static_cast<const TT *>(x), w.q, w.scale, w.minv, R, w.K, d, w.G, r, eps, T, h, w_in, inv);
    };
    auto by_mt = [&](auto tc) {
        switch (MT) {
            case 1: go(tc, std::integral_constant<int, 1>{}); break;
            case 2: go(tc, std::integral_constant<int, 2>{}); break;
            case 4: go(tc, std::integral_constant<int, 4>{}); break;
            default: go(tc, std::integral_constant<int, 8>{}); break;
        }
    };
    if (act == Act::F32) by_mt(float{});
    else by_mt(uint16_t{});
    STRIX_HIP_CHECK_LAUNCH(fn, " Q", BITS, " ", act_str(act), " T=", T, " R=", R, " K=", w.K, " G=", w.G);
}

template <int BITS>
void mix_up(const float *h, const QArr &w, const void *x, const float *norm_w, const float *inv, int64_t T,
            int64_t H, int64_t d, void *u, Act act, hipStream_t stream) {
    const char *fn = "hc_mix_up";
    check_shape(fn, T, H, d, act);
    check_q(fn, w);
    STRIX_CHECK(h != nullptr && x != nullptr && norm_w != nullptr && inv != nullptr && u != nullptr, fn,
                ": null pointer (h, x, norm_w, inv or u)");
    STRIX_CHECK(w.N == H * d, fn, ": W_up has ", w.N, " rows, expected H*d = ", H * d);
    STRIX_CHECK(w.K >= kChunk && w.K <= kMaxR && w.K % kChunk == 0, fn, ": W_up K (the rank r) = ", w.K,
                ", expected a multiple of ", kChunk, " up to ", kMaxR);
    const int64_t es = act == Act::F32 ? 4 : 2;
    STRIX_CHECK(disjoint(u, T * d * es, x, T * H * d * es), fn, ": u overlaps the streams x");
    const int MT = tokens_per_block(T);
    const dim3 grid((unsigned)((d + kUpCols - 1) / kUpCols), (unsigned)((T + MT - 1) / MT));
    auto go = [&](auto tc, auto mtc) {
        using TT = decltype(tc);
        hc_up_kernel<TT, BITS, decltype(mtc)::value><<<grid, kThreads, 0, stream>>>(
            h, w.q, w.scale, w.minv, static_cast<const TT *>(x), norm_w, inv, d, w.K, w.G, T, static_cast<TT *>(u));
    };
    auto by_mt = [&](auto tc) {
        switch (MT) {
            case 1: go(tc, std::integral_constant<int, 1>{}); break;
            case 2: go(tc, std::integral_constant<int, 2>{}); break;
            case 4: go(tc, std::integral_constant<int, 4>{}); break;
            default: go(tc, std::integral_constant<int, 8>{}); break;
        }
    };
    if (act == Act::F32) by_mt(float{});
    else by_mt(uint16_t{});
    STRIX_HIP_CHECK_LAUNCH(fn, " Q", BITS, " ", act_str(act), " T=", T, " d=", d, " r=", w.K, " G=", w.G);
}

}  // namespace

void hc_mix_down(const void *x, const Q4DeviceView &w, int64_t T, int64_t H, int64_t d, int64_t r, bool inject,
                 float eps, float *h, float *w_in, float *inv, Act act, hipStream_t stream) {
    mix_down<4>(x, {w.q, w.scale, w.minv, w.N, w.K, w.G}, T, H, d, r, inject, eps, h, w_in, inv, act, stream);
}
void hc_mix_down(const void *x, const Q8DeviceView &w, int64_t T, int64_t H, int64_t d, int64_t r, bool inject,
                 float eps, float *h, float *w_in, float *inv, Act act, hipStream_t stream) {
    mix_down<8>(x, {w.q, w.scale, w.minv, w.N, w.K, w.G}, T, H, d, r, inject, eps, h, w_in, inv, act, stream);
}
void hc_mix_up(const float *h, const Q4ChunkMajorView &w, const void *x, const float *norm_w, const float *inv,
               int64_t T, int64_t H, int64_t d, void *u, Act act, hipStream_t stream) {
    mix_up<4>(h, {w.q, w.scale, w.minv, w.N, w.K, w.G}, x, norm_w, inv, T, H, d, u, act, stream);
}
void hc_mix_up(const float *h, const Q8ChunkMajorView &w, const void *x, const float *norm_w, const float *inv,
               int64_t T, int64_t H, int64_t d, void *u, Act act, hipStream_t stream) {
    mix_up<8>(h, {w.q, w.scale, w.minv, w.N, w.K, w.G}, x, norm_w, inv, T, H, d, u, act, stream);
}

}  // namespace strix::kernels
