// Router side of the MoE sublayer on gfx950: the router projection (linear_bf16w, one fixed FP32 summation order),
// the top-k / softmax (moe_router, one wave64 per token, logits in registers), and the shared expert's gated add
// (moe_shared_add, moe_shared_add_inject).
#include "common.hpp"
#include "router_small.hpp"
#include "topk.hpp"

#include <climits>
#include <type_traits>

namespace strix::kernels {

const char *act_str(Act a) { return a == Act::F32 ? "F32" : a == Act::BF16 ? "BF16" : "?"; }

namespace {

using namespace strix::dev;

constexpr int kWave = 64;
constexpr int kThreads = 256;

// ---- router projection ----------------------------------------------------------------------------------------
// One wave per (output row n, group of MR token rows); a block is RB rows x TG token groups (RB * TG = 4 waves), so
// the waves sharing a weight row share it through L1. Lane l owns the 8-element chunks c = l, l + 64, ...: its
// partial is an fmaf chain over them (chunk order, then element order), then a butterfly over the 64 lanes. The order
// depends on nothing but K, so every M, grid and launch gives the same bits (oracle: orc_router_logits).
// A lane's weight chunks are loaded in batches of NB before the token loop. VEC: K % 8 == 0 and 16-byte aligned x / w
// rows - 16-byte loads; else element loads, the same arithmetic.
template <typename TY, int MR, bool VEC>
__global__ void __launch_bounds__(kThreads)
    router_rows_kernel(const uint16_t *x, const uint16_t *w, TY *y, int64_t M, int64_t N, int64_t K, int TG) {
    constexpr int NB = 8;
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int RB = (kThreads / kWave) / TG;
    const int64_t n = (int64_t)blockIdx.x * RB + wave / TG;
    const int64_t m0 = ((int64_t)blockIdx.y * TG + wave % TG) * MR;
    if (n >= N || m0 >= M) return;  // no barrier in this kernel
    const int rows = (int)(M - m0 < MR ? M - m0 : MR);
    float acc[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = 0.f;
    const int64_t chunks = (K + 7) / 8;
    const uint16_t *wr = w + n * K;
    for (int64_t cb = lane; cb < chunks; cb += (int64_t)NB * kWave) {
        uint4 wu[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int64_t c = cb + (int64_t)b * kWave;
            if constexpr (VEC) {
                wu[b] = c < chunks ? *reinterpret_cast<const uint4 *>(wr + c * 8) : make_uint4(0, 0, 0, 0);
            } else {
                uint16_t e[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) e[i] = c * 8 + i < K ? wr[c * 8 + i] : 0;
                wu[b] = make_uint4(e[0] | (uint32_t)e[1] << 16, e[2] | (uint32_t)e[3] << 16, e[4] | (uint32_t)e[5] << 16,
                                   e[6] | (uint32_t)e[7] << 16);
            }
        }
        // every token row's chunks are loaded before any arithmetic (rows past M re-read the last row, unused), so a
        // batch costs one memory round trip, not one per token
        uint4 xu[MR][NB];
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            const uint16_t *xr = x + (m0 + (r < rows ? r : rows - 1)) * K;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int64_t c = cb + (int64_t)b * kWave;
                if constexpr (VEC) {
                    xu[r][b] = c < chunks ? *reinterpret_cast<const uint4 *>(xr + c * 8) : make_uint4(0, 0, 0, 0);
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) e[i] = c * 8 + i < K ? xr[c * 8 + i] : 0;
                    xu[r][b] = make_uint4(e[0] | (uint32_t)e[1] << 16, e[2] | (uint32_t)e[3] << 16,
                                          e[4] | (uint32_t)e[5] << 16, e[6] | (uint32_t)e[7] << 16);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < MR; ++r) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int64_t c = cb + (int64_t)b * kWave;
                if (c >= chunks) break;
                const uint32_t wd[4] = {wu[b].x, wu[b].y, wu[b].z, wu[b].w};
                const uint32_t xd[4] = {xu[r][b].x, xu[r][b].y, xu[r][b].z, xu[r][b].w};
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    if (!VEC && c * 8 + i >= K) break;
                    const float xv = __uint_as_float(i % 2 ? xd[i / 2] & 0xffff0000u : xd[i / 2] << 16);
                    const float wv = __uint_as_float(i % 2 ? wd[i / 2] & 0xffff0000u : wd[i / 2] << 16);
                    acc[r] = fmaf(xv, wv, acc[r]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1) acc[r] = acc[r] + __shfl_xor(acc[r], off, kWave);
    if (lane == 0)
#pragma unroll
        for (int r = 0; r < MR; ++r)
            if (r < rows) {
                if constexpr (std::is_same_v<TY, float>) y[(m0 + r) * N + n] = acc[r];
                else y[(m0 + r) * N + n] = f32_to_bf16(acc[r]);
            }
}

// Register-tiled form for larger M (same arithmetic, same bits): a wave computes 8 tokens x 8 output rows, so each
// loaded chunk feeds 8 fmaf chains; lane l still owns chunks l, l + 64, ... of every pair. The 64 pairs' lane
// partials then meet in a reduce-scatter along the same butterfly (offsets 32 .. 1): at offset o a lane keeps half of
// its pairs - the upper half when bit o of its lane is set - and adds the partner's partials of that half, own +
// partner as in the butterfly. Lane l ends with pair l. A block is 4 waves on the same 8 tokens (32 rows).
constexpr int kTT = 8, kTE = 8;
template <typename TY>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
    router_tile_kernel(const uint16_t *x, const uint16_t *w, TY *y, int64_t M, int64_t N, int64_t K) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int64_t n0 = ((int64_t)blockIdx.x * (kThreads / kWave) + wave) * kTE, m0 = (int64_t)blockIdx.y * kTT;
    if (n0 >= N) return;  // no barrier in this kernel
    float v[kTT * kTE];
#pragma unroll
    for (int p = 0; p < kTT * kTE; ++p) v[p] = 0.f;
    const int64_t chunks = K / 8;
    for (int64_t c = lane; c < chunks; c += kWave) {
        uint4 wu[kTE];
#pragma unroll
        for (int e = 0; e < kTE; ++e)
            wu[e] = n0 + e < N ? *reinterpret_cast<const uint4 *>(w + (n0 + e) * K + c * 8) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int t = 0; t < kTT; ++t) {
            const uint4 xu = m0 + t < M ? *reinterpret_cast<const uint4 *>(x + (m0 + t) * K + c * 8) : make_uint4(0, 0, 0, 0);
            const uint32_t xd[4] = {xu.x, xu.y, xu.z, xu.w};
#pragma unroll
            for (int e = 0; e < kTE; ++e) {
                const uint32_t wd[4] = {wu[e].x, wu[e].y, wu[e].z, wu[e].w};
                float a = v[t * kTE + e];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float xv = __uint_as_float(i % 2 ? xd[i / 2] & 0xffff0000u : xd[i / 2] << 16);
                    const float wv = __uint_as_float(i % 2 ? wd[i / 2] & 0xffff0000u : wd[i / 2] << 16);
                    a = fmaf(xv, wv, a);
                }
                v[t * kTE + e] = a;
            }
        }
    }
    // reduce-scatter along the butterfly: n live pairs halve at each offset
#pragma unroll
    for (int lvl = 0; lvl < 6; ++lvl) {
        const int o = kWave / 2 >> lvl, n = kTT * kTE >> lvl;
        const bool up = lane & o;
#pragma unroll
        for (int i = 0; i < n / 2; ++i) {
            const float send = up ? v[i] : v[n / 2 + i];
            const float keep = up ? v[n / 2 + i] : v[i];
            v[i] = keep + __shfl_xor(send, o, kWave);
        }
    }
    constexpr int PL = kTT * kTE / kWave;  // pairs a lane ends with
#pragma unroll
    for (int h = 0; h < PL; ++h) {
        const int p = PL * lane + h, t = p / kTE, e = p % kTE;
        if (m0 + t < M && n0 + e < N) {
            if constexpr (std::is_same_v<TY, float>) y[(m0 + t) * N + n0 + e] = v[h];
            else y[(m0 + t) * N + n0 + e] = f32_to_bf16(v[h]);
        }
    }
}

// Small batches (M <= 64): a wave computes TT tokens x TE rows (router_small.hpp).
template <typename TY, int TT, int TE, int NCH>
__global__ void __launch_bounds__(kThreads)
    router_small_kernel(const uint16_t *x, const uint16_t *w, TY *y, int64_t M, int64_t N, int64_t K) {
    const int wave = threadIdx.x / kWave;
    const int64_t n0 = ((int64_t)blockIdx.x * (kThreads / kWave) + wave) * TE, m0 = (int64_t)blockIdx.y * TT;
    if (n0 >= N) return;  // no barrier in this kernel
    rsmall::router_small_wave<TY, TT, TE, NCH>(x, w, y, M, N, K, n0, m0);
}

// Act::F32 activations (the reference's FP32-activation form of linear_bf16w): one wave per (token, row) in the same
// canonical order - lane l takes the 8-element chunks l, l + 64, ... with fmaf in element order, then the butterfly
// over offsets 32 .. 1 - so an FP32 x holding BF16 values gives the BF16 path's bits. A compatibility path: every
// wave reads its token's and its row's whole K from L2.
template <typename TY>
__global__ void __launch_bounds__(kThreads)
    router_f32x_kernel(const float *x, const uint16_t *w, TY *y, int64_t M, int64_t N, int64_t K) {
    const int lane = threadIdx.x % kWave;
    const int64_t item = (int64_t)blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
    if (item >= M * N) return;  // whole wave; no barrier in this kernel
    const int64_t m = item / N, n = item % N;
    const float *xr = x + m * K;
    const uint16_t *wr = w + n * K;
    float a = 0.f;
    for (int64_t c = lane; c * 8 < K; c += kWave)
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int64_t i = c * 8 + k;
            if (i < K) a = fmaf(xr[i], bf16_to_f32(wr[i]), a);
        }
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) a += __shfl_xor(a, o, kWave);
    if (lane == 0) {
        if constexpr (std::is_same_v<TY, float>) y[item] = a;
        else y[item] = f32_to_bf16(a);
    }
}

template <typename TY>
void launch_router_rows(const uint16_t *x, const uint16_t *w, TY *y, int64_t M, int64_t N, int64_t K,
                        hipStream_t stream) {
    const bool vec = K % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0;
    auto go = [&](auto mr) {
        constexpr int MR = decltype(mr)::value;
        const int64_t groups = (M + MR - 1) / MR;
        const int TG = groups >= 4 ? 4 : groups >= 2 ? 2 : 1, RB = 4 / TG;
        const int64_t by = (groups + TG - 1) / TG;
        STRIX_CHECK(by <= 65535, "linear_bf16w: M = ", M, " needs ", by, " row blocks, grid.y holds 65535");
        dim3 grid((unsigned)((N + RB - 1) / RB), (unsigned)by), block(kThreads);
        if (vec) router_rows_kernel<TY, MR, true><<<grid, block, 0, stream>>>(x, w, y, M, N, K, TG);
        else router_rows_kernel<TY, MR, false><<<grid, block, 0, stream>>>(x, w, y, M, N, K, TG);
    };
    if (M <= 64 && vec && K % 512 == 0 && (K / 512 == 4 || K / 512 == 6 || K / 512 == 8)) {
        // 4 tokens x 1 row a wave (one row a wave keeps enough waves in flight; measured on MI355X at M 16, N 513,
        // K 3072: 4 x 1 5.1 us, 4 x 2 6.0, 4 x 4 8.9, the per-row form with loads in order 8.3)
        constexpr int TT = 4, TE = 1;
        const int64_t per_block = TE * (kThreads / kWave);
        dim3 grid((unsigned)((N + per_block - 1) / per_block), (unsigned)((M + TT - 1) / TT)), block(kThreads);
        if (K / 512 == 4) router_small_kernel<TY, TT, TE, 4><<<grid, block, 0, stream>>>(x, w, y, M, N, K);
        else if (K / 512 == 6) router_small_kernel<TY, TT, TE, 6><<<grid, block, 0, stream>>>(x, w, y, M, N, K);
        else router_small_kernel<TY, TT, TE, 8><<<grid, block, 0, stream>>>(x, w, y, M, N, K);
    } else if (M >= 256 && vec) {
        const int64_t by = (M + kTT - 1) / kTT;
        STRIX_CHECK(by <= 65535, "linear_bf16w: M = ", M, " needs ", by, " token blocks, grid.y holds 65535");
        const int64_t per_block = kTE * (kThreads / kWave);
        dim3 grid((unsigned)((N + per_block - 1) / per_block), (unsigned)by), block(kThreads);
        router_tile_kernel<TY><<<grid, block, 0, stream>>>(x, w, y, M, N, K);
    } else if (M == 1) go(std::integral_constant<int, 1>{});
    else go(std::integral_constant<int, 4>{});  // a wave holds its 4 tokens' chunks in registers
}

// ---- top-k ----------------------------------------------------------------------------------------------------
// One wave64 per token: a block of 4 waves, or of 1 wave for small batches (the rounds are VALU-bound, so tokens that
// share a CU share its 4 SIMDs; a decode batch spread one token a CU finishes several times sooner). Lane l holds
// experts l, l + 64, ... (NV registers, -inf past E). A round is a 64-lane arg-max over the lanes' bests (larger
// value, then lower index); the winner lane masks its pick and rescans its registers. Lane r keeps the r-th pick, so
// the softmax over the k is one butterfly sum.
template <typename T, int NV>
__global__ void __launch_bounds__(kThreads)
    topk_kernel(const T *logits, int64_t ld, int64_t M, int E, int k, const T *shared, int64_t shared_ld,
                int32_t shared_id, int32_t *ids, float *coef, int A, uint32_t *err) {
    const int lane = threadIdx.x % kWave;
    const int64_t m = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (m >= M) return;  // whole wave; no barrier in this kernel
    int32_t *id_row = ids + m * A;
    float *coef_row = coef + m * A;
    float sl = 0.f;
    int bad = INT_MAX;
    if (shared != nullptr) {
        sl = topk::load_logit(shared, m * shared_ld);
        if (!isfinite(sl)) bad = E;
    }
    __shared__ uint2 cand[kThreads / kWave][topk::kCandScratch];
    int id;
    float cf;
    const int rb = topk::wave_topk<T, NV>(logits + m * ld, E, k, id, cf, cand[threadIdx.x / kWave]);
    bad = rb < bad ? rb : bad;
    if (bad != INT_MAX) {
        if (lane == 0 && atomicCAS(&err[0], 0u, 1u) == 0u) {
            err[1] = (uint32_t)m;
            err[2] = (uint32_t)bad;
        }
        for (int a = lane; a < A; a += kWave) id_row[a] = -1, coef_row[a] = qnan();
        return;
    }
    if (lane < k) {
        id_row[lane] = id;
        coef_row[lane] = cf;
    }
    if (shared != nullptr && lane == 0) {
        id_row[k] = shared_id;
        coef_row[k] = 1.0f / (1.0f + expf(-sl));
    }
}

// ---- shared expert add ----------------------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ float ld_act(const T *p, int64_t i);
template <> __device__ __forceinline__ float ld_act<float>(const float *p, int64_t i) { return p[i]; }
template <> __device__ __forceinline__ float ld_act<uint16_t>(const uint16_t *p, int64_t i) { return bf16_to_f32(p[i]); }
template <typename T> __device__ __forceinline__ void st_act(T *p, int64_t i, float v);
template <> __device__ __forceinline__ void st_act<float>(float *p, int64_t i, float v) { p[i] = v; }
template <> __device__ __forceinline__ void st_act<uint16_t>(uint16_t *p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
template <typename T> __device__ __forceinline__ float as_stored(float v) {
    if constexpr (std::is_same_v<T, float>) return v;
    else return bf16_round(v);
}

// y = stored(y + sigmoid(gl) * s) (strixite kernels/moe_router.hip:129-146); INJECT: then for the H streams
// x[m, st * N + n] = stored(fma(w_in[m, st], y, x)) (moe_router.hip:154-180). Grid-stride over M * N.
template <typename T, bool INJECT>
__global__ void __launch_bounds__(kThreads)
    shared_add_kernel(T *y, const T *s, const float *gate_logit, int64_t gate_ld, int64_t M, int64_t N,
                      uint32_t gate_index, T *x, const float *w_in, int64_t H, uint32_t *err) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < M * N; i += (int64_t)gridDim.x * kThreads) {
        const int64_t m = i / N, n = i % N;
        const float gl = gate_logit[m * gate_ld];
        const bool ok = isfinite(gl);
        if (!ok && n == 0 && atomicCAS(&err[0], 0u, 1u) == 0u) {
            err[1] = (uint32_t)m;
            err[2] = gate_index;
        }
        const float g = ok ? 1.f / (1.f + expf(-gl)) : qnan();
        const float v = as_stored<T>(ld_act(y, i) + g * ld_act(s, i));
        st_act(y, i, v);
        if constexpr (INJECT)
            for (int64_t st = 0; st < H; ++st) {
                const int64_t xi = (m * H + st) * N + n;
                st_act(x, xi, fmaf(w_in[m * H + st], v, ld_act(x, xi)));
            }
    }
}

// strixite kernels/hc.hpp:51-55: x[t, s d + j] = stored(fma(w_in[t, s], y[t, j], x[t, s d + j])), in place
template <typename T>
__global__ void __launch_bounds__(kThreads)
    hc_inject_kernel(T *x, const float *w_in, const T *y, int64_t T_, int64_t H, int64_t d) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < T_ * H * d; i += (int64_t)gridDim.x * kThreads) {
        const int64_t t = i / (H * d), s = (i / d) % H, jj = i % d;
        st_act(x, i, fmaf(w_in[t * H + s], ld_act(y, t * d + jj), ld_act(x, i)));
    }
}

unsigned elementwise_blocks(int64_t n) {
    const int64_t b = (n + kThreads - 1) / kThreads;
    return (unsigned)(b < 65536 ? b : 65536);
}

}  // namespace

void linear_bf16w(const void *x, const uint16_t *w, void *y, int64_t M, int64_t N, int64_t K, Act act,
                  hipStream_t stream) {
    linear_bf16w(x, w, y, M, N, K, act, act, stream);
}

void linear_bf16w(const void *x, const uint16_t *w, void *y, int64_t M, int64_t N, int64_t K, Act act, Act out_act,
                  hipStream_t stream) {
    STRIX_CHECK(x != nullptr && w != nullptr && y != nullptr, "linear_bf16w: null pointer (x=", x, ", w=",
                (const void *)w, ", y=", y, ")");
    STRIX_CHECK(M >= 1 && N >= 1 && K >= 1 && K <= (1 << 24) && N <= 0x7fffffff, "linear_bf16w: M = ", M, ", N = ",
                N, ", K = ", K, " out of range");
    STRIX_CHECK(act == Act::F32 || act == Act::BF16, "linear_bf16w: unsupported activation dtype ", (int)act);
    STRIX_CHECK(out_act == Act::F32 || out_act == Act::BF16, "linear_bf16w: output dtype ", (int)out_act);
    const int64_t oes = out_act == Act::F32 ? 4 : 2, xes = act == Act::F32 ? 4 : 2;
    STRIX_CHECK(disjoint(y, M * N * oes, x, M * K * xes), "linear_bf16w: output y overlaps input x");
    if (act == Act::F32) {
        const int64_t blocks = (M * N + kThreads / kWave - 1) / (kThreads / kWave);
        STRIX_CHECK(blocks < (1ll << 31), "linear_bf16w: M * N = ", M * N, " too large for the FP32-activation path");
        if (out_act == Act::F32)
            router_f32x_kernel<float><<<(unsigned)blocks, kThreads, 0, stream>>>(static_cast<const float *>(x), w,
                                                                                 static_cast<float *>(y), M, N, K);
        else
            router_f32x_kernel<uint16_t><<<(unsigned)blocks, kThreads, 0, stream>>>(
                static_cast<const float *>(x), w, static_cast<uint16_t *>(y), M, N, K);
    } else if (out_act == Act::F32)
        launch_router_rows(static_cast<const uint16_t *>(x), w, static_cast<float *>(y), M, N, K, stream);
    else
        launch_router_rows(static_cast<const uint16_t *>(x), w, static_cast<uint16_t *>(y), M, N, K, stream);
    STRIX_HIP_CHECK_LAUNCH("linear_bf16w M=", M, " N=", N, " K=", K);
}

void moe_router(const void *logits, int64_t ld, int64_t M, int64_t E, int64_t k, const void *shared_logit,
                int64_t shared_ld, int32_t shared_id, int32_t *ids, float *coef, Act act, uint32_t *err,
                hipStream_t stream) {
    STRIX_CHECK(logits != nullptr && ids != nullptr && coef != nullptr && err != nullptr,
                "moe_router: null pointer (logits=", logits, ", ids=", (const void *)ids, ", coef=",
                (const void *)coef, ", err=", (const void *)err, ")");
    STRIX_CHECK(M >= 1 && M <= 0x7fffffff, "moe_router: M = ", M, " tokens, expected 1..2^31-1");
    STRIX_CHECK(E >= 1 && E <= 1024, "moe_router: E = ", E, " experts, expected 1..1024");
    STRIX_CHECK(k >= 1 && k <= E && k <= 32, "moe_router: k = ", k, ", expected 1..min(E = ", E, ", 32)");
    STRIX_CHECK(ld >= E, "moe_router: logits row stride ld = ", ld, " < E = ", E);
    if (shared_logit != nullptr) {
        STRIX_CHECK(shared_ld >= 1, "moe_router: shared_ld = ", shared_ld, ", expected >= 1");
        STRIX_CHECK(shared_id >= 0, "moe_router: shared_id = ", shared_id, ", expected >= 0");
    }
    STRIX_CHECK((const void *)ids != (const void *)coef, "moe_router: ids and coef are the same buffer");
    STRIX_CHECK(act == Act::F32 || act == Act::BF16, "moe_router: unsupported logit dtype ", (int)act);
    const int A = (int)k + (shared_logit != nullptr ? 1 : 0);
    const unsigned per_block = M <= 1024 ? 1 : kThreads / kWave;  // tokens a block
    dim3 grid((unsigned)((M + per_block - 1) / per_block)), block(per_block * kWave);
    const int nv = E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : 16;
    auto go = [&](auto tag, auto nvc) {
        using T = decltype(tag);
        topk_kernel<T, decltype(nvc)::value><<<grid, block, 0, stream>>>(
            static_cast<const T *>(logits), ld, M, (int)E, (int)k, static_cast<const T *>(shared_logit), shared_ld,
            shared_id, ids, coef, A, err);
    };
    auto by_nv = [&](auto tag) {
        switch (nv) {
            case 1: go(tag, std::integral_constant<int, 1>{}); break;
            case 2: go(tag, std::integral_constant<int, 2>{}); break;
            case 4: go(tag, std::integral_constant<int, 4>{}); break;
            case 8: go(tag, std::integral_constant<int, 8>{}); break;
            default: go(tag, std::integral_constant<int, 16>{}); break;
        }
    };
    if (act == Act::F32) by_nv(float{});
    else by_nv(uint16_t{});
    STRIX_HIP_CHECK_LAUNCH("moe_router ", act_str(act), " M=", M, " E=", E, " k=", k, shared_logit ? " +shared" : "");
}

void check_router_error(const uint32_t *err, const char *what) {
    STRIX_CHECK(err != nullptr, "check_router_error(", what, "): null err");
    uint32_t e[3];
    STRIX_HIP_CHECK(hipMemcpy(e, err, sizeof(e), hipMemcpyDeviceToHost), "reading the router error word for ", what);
    report_router_error(e, what);
}

void report_router_error(const uint32_t e[3], const char *what) {
    STRIX_CHECK(e[0] == 0, what, ": non-finite router logit at token ", e[1], ", expert ", e[2],
                " (E = the shared-expert gate); that token's ids are -1 and its coefficients NaN");
}

namespace {
template <bool INJECT>
void shared_add_common(const char *fn, void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M,
                       int64_t N, uint32_t gate_index, void *x, const float *w_in, int64_t H, Act act, uint32_t *err,
                       hipStream_t stream) {
    STRIX_CHECK(y != nullptr && s != nullptr && gate_logit != nullptr && err != nullptr, fn, ": null pointer");
    STRIX_CHECK(!INJECT || (x != nullptr && w_in != nullptr), fn, ": null x or w_in");
    STRIX_CHECK(M >= 1 && N >= 1 && N <= (1ll << 24), fn, ": M = ", M, ", N = ", N, " out of range");
    STRIX_CHECK(gate_ld >= 1, fn, ": gate_ld = ", gate_ld, ", expected >= 1");
    STRIX_CHECK(!INJECT || H == 4, fn, ": H = ", H, " streams, expected 4 (strixite's hc_count)");
    STRIX_CHECK(act == Act::F32 || act == Act::BF16, fn, ": unsupported activation dtype ", (int)act);
    const int64_t es = act == Act::F32 ? 4 : 2;
    STRIX_CHECK(disjoint(y, M * N * es, s, M * N * es), fn, ": s overlaps y");
    if (INJECT)
        STRIX_CHECK(disjoint(x, M * H * N * es, y, M * N * es) && disjoint(x, M * H * N * es, s, M * N * es), fn,
                    ": x overlaps y or s");
    const unsigned blocks = elementwise_blocks(M * N);
    if (act == Act::F32)
        shared_add_kernel<float, INJECT><<<blocks, kThreads, 0, stream>>>(
            static_cast<float *>(y), static_cast<const float *>(s), gate_logit, gate_ld, M, N, gate_index,
            static_cast<float *>(x), w_in, H, err);
    else
        shared_add_kernel<uint16_t, INJECT><<<blocks, kThreads, 0, stream>>>(
            static_cast<uint16_t *>(y), static_cast<const uint16_t *>(s), gate_logit, gate_ld, M, N, gate_index,
            static_cast<uint16_t *>(x), w_in, H, err);
    STRIX_HIP_CHECK_LAUNCH(fn, " ", act_str(act), " M=", M, " N=", N);
}
}  // namespace

void moe_shared_add(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M, int64_t N,
                    uint32_t gate_index, Act act, uint32_t *err, hipStream_t stream) {
    shared_add_common<false>("moe_shared_add", y, s, gate_logit, gate_ld, M, N, gate_index, nullptr, nullptr, 0, act,
                             err, stream);
}

void hc_inject(void *x, const float *w_in, const void *y, int64_t T, int64_t H, int64_t d, Act act,
               hipStream_t stream) {
    const char *fn = "hc_inject";
    STRIX_CHECK(x != nullptr && w_in != nullptr && y != nullptr, fn, ": null pointer");
    STRIX_CHECK(T >= 1 && H >= 1 && d >= 1 && T * H * d <= (1ll << 40), fn, ": T = ", T, ", H = ", H, ", d = ", d);
    STRIX_CHECK(act == Act::F32 || act == Act::BF16, fn, ": unsupported activation dtype ", (int)act);
    const int64_t es = act == Act::F32 ? 4 : 2;
    STRIX_CHECK(disjoint(x, T * H * d * es, y, T * d * es), fn, ": y overlaps x");
    const unsigned blocks = elementwise_blocks(T * H * d);
    if (act == Act::F32)
        hc_inject_kernel<float><<<blocks, kThreads, 0, stream>>>(static_cast<float *>(x), w_in,
                                                                static_cast<const float *>(y), T, H, d);
    else
        hc_inject_kernel<uint16_t><<<blocks, kThreads, 0, stream>>>(static_cast<uint16_t *>(x), w_in,
                                                                   static_cast<const uint16_t *>(y), T, H, d);
    STRIX_HIP_CHECK_LAUNCH(fn, " ", act_str(act), " T=", T, " H=", H, " d=", d);
}

void moe_shared_add_inject(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M, int64_t N,
                           uint32_t gate_index, void *x, const float *w_in, int64_t H, Act act, uint32_t *err,
                           hipStream_t stream) {
    shared_add_common<true>("moe_shared_add_inject", y, s, gate_logit, gate_ld, M, N, gate_index, x, w_in, H, act,
                            err, stream);
}

}  // namespace strix::kernels
