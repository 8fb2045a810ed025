// Prefill-size routing on gfx950's matrix cores with the routing of the canonical FP32 order, bit for bit.
//
// The router projection (strixite kernels/linear.hip:83-147 semantics, FP32) is the one place on the path whose result
// decides a discrete choice (the top-k), so it must be reproduced exactly - in this library's canonical summation
// order (lane l of a wave64 takes the 8-element chunks l, l + 64, ... with fmaf, then a butterfly over the 64 lanes;
// oracle: orc_router_logits). That order does not map onto MFMA, and at 4096 tokens x 513 rows x 3072 the VALU form
// costs ~0.3 ms. So the projection runs in two passes:
//   1. approx: logits a = x . w^T with bf16 MFMA (FP32 accumulation, any internal order), and the 2-norms |w_e|
//      (|x_m| comes from pass 2, which loads the token's row). For ANY order of summing the K exact bf16 x bf16 products in FP32 - rounded to nearest or toward zero,
//      FP32 denormals kept or flushed - the result differs from the exact sum by at most (2K u) S + K 2^-125 with
//      u = 2^-24 and S = sum_k |x_k w_k| <= |x| |w| (Cauchy-Schwarz). Both the canonical and the MFMA sums obey it, so
//      |a - c| <= delta = (4K + 64) u |x| |w| + K 2^-124 (norms rounded up).
//   2. select (a wave per token): with the (optional FP32) bias, a value v = fl(c + b) lies within delta' = delta +
//      2^-22 (|a| + |b|) of fl(a + b). tau = the k-th largest of (fl(a + b) - delta'); an expert with fl(a + b) +
//      delta' < tau has at least k experts whose exact value is larger, so it is never chosen, ties included. The
//      others (the candidates, typically k + 1 or 2) and the shared-expert gate row are recomputed in the canonical
//      order; the top-k over the candidates' exact values (value desc, index asc) and the softmax over the picks are
//      then exactly those of the full exact row. Any non-finite a, b, or norm sends the token to the exact path for
//      all of its experts (the non-finite handling of strixite kernels/moe_router.hip:40-67).
// The logits workspace row of a token ends with exact values at the candidates and the shared gate (the entries the
// layer reads later) and approximate values elsewhere.
#include "common.hpp"
#include "topk.hpp"

#include <climits>

namespace strix::kernels {
namespace {

using namespace strix::dev;
constexpr int kWave = 64, kThreads = 256;


// ---- pass 1: approximate logits + router row norms ------------------------------------------------------------------
// Only the E routed rows (the shared gate row is computed exactly by pass 2). kNormRows extra rows of blocks (grid y)
// only sum the squares of the router rows, so the GEMM blocks carry no norm work. Block tile 128 tokens x 128 rows, K in
// steps of 64 through LDS (rows padded to 144 bytes: the 16 lanes of a fragment read hit 16 distinct 16-byte bank
// groups); wave w computes tokens 64 (w / 2) .. + 63 x rows 64 (w % 2) .. + 63 as 4 x 4 v_mfma_f32_16x16x32_bf16
// tiles whose A and B fragments are both 16-byte row segments (x rows for tokens, w rows for experts). The next K
// step's tiles are loaded into registers while the current one is multiplied. K is split into kParts parts (grid z),
// each summed by its own blocks into its own output (the pass is bound by latency and by L2 re-reads of the tiles,
// which the large tiles keep to 4 reads of x and 32 of w at E 512, M 4096).
// (parts: 1, 2, 4 measured 139, 122, 124 us for both passes at 4096 x 512 x 3072 on MI355X - more parts shorten this
// pass but their partial logits push the router rows out of L2 before pass 2 re-reads them)
constexpr int kBM = 128, kBN = 128, kBK = 64, kLd = kBK + 8, kParts = 2, kNormRows = kBN / 16;

__device__ __forceinline__ float sumsq8(const uint4 &v) {
    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = __uint_as_float(d[i] << 16), b = __uint_as_float(d[i] & 0xffff0000u);
        s = fmaf(a, a, s);
        s = fmaf(b, b, s);
    }
    return s;
}

__global__ void __launch_bounds__(kThreads)
    router_approx_kernel(const uint16_t *x, const uint16_t *w, float *a_out, int64_t ld, int64_t M, int64_t N,
                         int64_t K, float *nw) {
    __shared__ __attribute__((aligned(16))) uint16_t As[kBM * kLd], Bs[kBN * kLd];
    // K part blockIdx.z of gridDim.z: its sums go to part z of the outputs ([parts][M][ld], [parts][M], [parts][N])
    const int64_t kp = K / gridDim.z, kbeg = kp * blockIdx.z, kend = kbeg + kp;
    a_out += (int64_t)blockIdx.z * M * ld, nw += (int64_t)blockIdx.z * N;
    const int t = threadIdx.x, lane = t % kWave, wave = t / kWave, g = lane / 16, j = lane % 16;
    const int wm = 64 * (wave / 2), wn = 64 * (wave % 2);
    const int64_t n0 = (int64_t)blockIdx.x * kBN, m0 = (int64_t)blockIdx.y * kBM;
    // staging: chunk u covers row (t >> 3) + 32 u, 16 bytes at column 8 (t & 7), of A and of B
    const int sr = t >> 3, sc = (t & 7) * 8;
    const int64_t gemm_rows = (int64_t)gridDim.y - kNormRows;
    if ((int64_t)blockIdx.y >= gemm_rows) {
        // the last kNormRows rows of blocks: the squared norms of the router rows over this K part, 16 rows a block
        // (16 threads a row, each summing every 16th 16-byte piece; the tokens' norms come from the select pass,
        // which loads each token's whole row anyway)
        const int64_t c = n0 + 16 * (blockIdx.y - gemm_rows) + t / 16;
        float q = 0.f;
        if (c < N) {
            const uint4 *wr = reinterpret_cast<const uint4 *>(w + c * K + kbeg);
            const int n16 = (int)(kp / 8);
#pragma unroll 12
            for (int i = t % 16; i < n16; i += 16) q += sumsq8(wr[i]);
        }
        q += __shfl_xor(q, 1, kWave);
        q += __shfl_xor(q, 2, kWave);
        q += __shfl_xor(q, 4, kWave);
        q += __shfl_xor(q, 8, kWave);
        if (t % 16 == 0 && c < N) nw[c] = q;
        return;
    }
    uint4 ra[4], rb[4];
    auto load = [&](int64_t k0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t r = m0 + sr + 32 * u, c = n0 + sr + 32 * u;
            ra[u] = r < M ? *reinterpret_cast<const uint4 *>(x + r * K + k0 + sc) : make_uint4(0, 0, 0, 0);
            rb[u] = c < N ? *reinterpret_cast<const uint4 *>(w + c * K + k0 + sc) : make_uint4(0, 0, 0, 0);
        }
    };
    float4v acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = float4v{0, 0, 0, 0};
    load(kbeg);
    for (int64_t k0 = kbeg; k0 < kend; k0 += kBK) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            *reinterpret_cast<uint4 *>(&As[(sr + 32 * u) * kLd + sc]) = ra[u];
            *reinterpret_cast<uint4 *>(&Bs[(sr + 32 * u) * kLd + sc]) = rb[u];
        }
        __syncthreads();
        if (k0 + kBK < kend) load(k0 + kBK);
#pragma unroll
        for (int s = 0; s < kBK / 32; ++s) {
            Frag af[4], bf[4];
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const uint4 v = *reinterpret_cast<const uint4 *>(&As[(wm + 16 * a + j) * kLd + 32 * s + 8 * g]);
                af[a] = Frag{{v.x, v.y, v.z, v.w}};
            }
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint4 v = *reinterpret_cast<const uint4 *>(&Bs[(wn + 16 * b + j) * kLd + 32 * s + 8 * g]);
                bf[b] = Frag{{v.x, v.y, v.z, v.w}};
            }
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b) acc[a][b] = mfma_bf16(af[a], bf[b], acc[a][b]);
        }
        __syncthreads();
    }
    // D: lane (j, g) holds tokens 4 g + r of column j
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + wm + 16 * a + 4 * g + r, n = n0 + wn + 16 * b + j;
                if (m < M && n < N) a_out[m * ld + n] = acc[a][b][r];
            }
}

// ---- pass 2: select -------------------------------------------------------------------------------------------------
// The canonical lane partial of token row xr (this lane's NCH chunks) with weight row chunks c: the fmaf chain over
// chunks l, l + 64, ... in element order; the wave's butterfly then gives the canonical sum.
template <int NCH>
__device__ __forceinline__ float lane_chain(const uint4 (&xr)[NCH], const uint4 (&c)[NCH]) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const uint32_t xd[4] = {xr[i].x, xr[i].y, xr[i].z, xr[i].w}, wd[4] = {c[i].x, c[i].y, c[i].z, c[i].w};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float xv = __uint_as_float(k % 2 ? xd[k / 2] & 0xffff0000u : xd[k / 2] << 16);
            const float wv = __uint_as_float(k % 2 ? wd[k / 2] & 0xffff0000u : wd[k / 2] << 16);
            acc = fmaf(xv, wv, acc);
        }
    }
    return acc;
}

// One wave per token. parts: the approx pass's K parts [kParts][M][ld] (part 0 is the layer's logits buffer: the
// exact values are written there); nw2: the parts' squared norms of the router rows.
template <int NV, int NCH>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
    router_select_kernel(const uint16_t *x, const uint16_t *w, const float *bias, float *logits, int64_t ld,
                         int64_t M, int E, int k, bool shared, bool shared_slot, const float *nw2,
                         int32_t *ids, float *coef, uint32_t *err, uint4 *x16) {
    __shared__ int cand_lds[kThreads / kWave][1040];  // a wave's candidate list (at most E + 1 <= 1025)
    __shared__ uint2 pick_lds[kThreads / kWave][topk::kCandScratch];  // the picks' scratch (topk::wave_picks)
    const int lane = threadIdx.x % kWave;
    const int64_t m = (int64_t)blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
    if (m >= M) return;  // whole wave; no barrier in this kernel
    constexpr int64_t K = (int64_t)NCH * 512;
    const int64_t N = E;  // rows of the approximate pass (the routed ones)
    const uint16_t *xm = x + m * K;
    float *row = logits + m * ld;
    uint4 xr[NCH];
#pragma unroll
    for (int i = 0; i < NCH; ++i) xr[i] = *reinterpret_cast<const uint4 *>(xm + (lane + i * kWave) * 8);
    if (x16 != nullptr) {  // the row as F16 toward zero, each 8-element block in the paired order k0 k4 k1 k5 ..
        auto lo = [](uint32_t d) { return __uint_as_float(d << 16); };
        auto hi = [](uint32_t d) { return __uint_as_float(d & 0xFFFF0000u); };
        auto pk = [](float a, float b) { return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b)); };
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const uint4 v = xr[i];
            x16[m * (K / 8) + lane + i * kWave] =
                make_uint4(pk(lo(v.x), lo(v.z)), pk(hi(v.x), hi(v.z)), pk(lo(v.y), lo(v.w)), pk(hi(v.y), hi(v.w)));
        }
    }
    // the token's squared norm from the row just loaded (any FP32 order is within the bound's allowance)
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; ++i) q += sumsq8(xr[i]);
#pragma unroll
    for (int s = 1; s < kWave; s *= 2) q += __shfl_xor(q, s, kWave);
    constexpr float up = 1.0f + 1.0f / 256;  // the FP32 sums of squares are within 2^-10 of the exact ones
    const float nxm = sqrtf(q) * up;
    float va[NV], dl[NV];
    bool fin = isfinite(nxm);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e = lane + j * kWave;
        float a = 0.f, n2 = 0.f;
        if (e < E)
#pragma unroll
            for (int p = 0; p < kParts; ++p) a += row[p * M * ld + e], n2 += nw2[p * N + e];
        const float b = e < E && bias ? bias[e] : 0.f, n = sqrtf(n2) * up;
        va[j] = bias ? a + b : a;
        fin = fin && isfinite(va[j]) && isfinite(n);
        // delta' = (4K + 64) u |x| |w| + K 2^-124 + 2^-22 (|a| + |b|), rounded up by the 1 + 2^-10 factor
        dl[j] = ((4.0f * (float)K + 64.0f) * 0x1p-24f * nxm * n + (float)K * 0x1p-124f +
                 0x1p-22f * (fabsf(a) + fabsf(b))) * (1.0f + 0x1p-10f);
    }
    const bool exact_all = __ballot(!fin) != 0;  // uniform
    uint32_t key[NV];
    bool cand[NV];
    if (!exact_all) {
        // tau: the k-th largest lower bound (the key of pick k - 1, held by lane k - 1)
#pragma unroll
        for (int j = 0; j < NV; ++j) key[j] = lane + j * kWave < E ? topk::order_key(va[j] - dl[j]) : 0u;
        int id_unused;
        uint32_t kth, top_unused;
        topk::wave_picks<NV>(key, k, pick_lds[threadIdx.x / kWave], id_unused, kth, top_unused);
        const uint32_t tau = __builtin_amdgcn_readlane(kth, k - 1);
#pragma unroll
        for (int j = 0; j < NV; ++j) cand[j] = lane + j * kWave < E && topk::order_key(va[j] + dl[j]) >= tau;
    } else {
#pragma unroll
        for (int j = 0; j < NV; ++j) cand[j] = lane + j * kWave < E;
    }
    // the candidates in ascending expert order (then the shared gate row E) as a list in this wave's LDS
    int *cl = cand_lds[threadIdx.x / kWave];
    int nc = 0;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint64_t mk = __ballot(cand[j]);
        if (cand[j]) cl[nc + __popcll(mk & ((1ull << lane) - 1ull))] = lane + j * kWave;
        nc += __popcll(mk);
    }
    if (shared && lane == 0) cl[nc] = E;
    nc += shared ? 1 : 0;

    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's list writes are done (its lanes read them next)
    float ex[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) ex[j] = 0.f;
    // the candidates in batches of kBatch: a batch's rows are loaded together (one L2 round trip for the batch, the
    // loads unconditional: a slot past the list repeats the batch's first candidate and is not stored), then their
    // chains and butterflies run interleaved (independent, so they overlap); each chain is the canonical order
    constexpr int kBatch = 6;
    float sd = 0.f;  // the shared gate logit (wave-uniform)
    for (int b0 = 0; b0 < nc; b0 += kBatch) {
        uint4 rows[kBatch][NCH];
        int ecs[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            ecs[i] = __builtin_amdgcn_readfirstlane(cl[b0 + i < nc ? b0 + i : b0]);
#pragma unroll
            for (int c = 0; c < NCH; ++c)
                rows[i][c] = *reinterpret_cast<const uint4 *>(w + (int64_t)ecs[i] * K + (lane + c * kWave) * 8);
        }
        float d[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) d[i] = lane_chain<NCH>(xr, rows[i]);
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1)
#pragma unroll
            for (int i = 0; i < kBatch; ++i) d[i] = d[i] + __shfl_xor(d[i], off, kWave);
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            if (b0 + i >= nc) break;
            const int ec = ecs[i];
            if (ec == E) {
                sd = d[i];
                if (lane == 0) row[E] = d[i];  // the shared gate logit, unbiased
            } else {
                const float vb = bias ? d[i] + bias[ec] : d[i];  // one FP32 add, as the unfused path
                if (lane == ec % kWave) {
                    const int js = ec / kWave;
#pragma unroll
                    for (int j = 0; j < NV; ++j)
                        if (j == js) ex[j] = vb;
                    row[ec] = vb;
                }
            }
        }
    }
    int bad = INT_MAX;
    if (exact_all) {
#pragma unroll
        for (int j = 0; j < NV; ++j)
            if (lane + j * kWave < E && !isfinite(ex[j]) && lane + j * kWave < bad) bad = lane + j * kWave;
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1) bad = min(bad, __shfl_xor(bad, off, kWave));
    }
    // shared_slot: the shared expert routed as slot k, id E, coefficient sigmoid(its gate logit) (strixite
    // kernels/moe_router.hip:108-111); a non-finite gate logit is bad index E
    const int A = k + (shared_slot ? 1 : 0);
    if (shared_slot && !isfinite(sd)) bad = min(bad, E);
    int32_t *id_row = ids + m * A;
    float *coef_row = coef + m * A;
    if (bad != INT_MAX) {  // strixite kernels/moe_router.hip:40-67: the token's ids -1, coefficients NaN, err
        if (lane == 0 && atomicCAS(&err[0], 0u, 1u) == 0u) {
            err[1] = (uint32_t)m;
            err[2] = (uint32_t)bad;
        }
        if (lane < A) id_row[lane] = -1, coef_row[lane] = qnan();
        return;
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) key[j] = cand[j] ? topk::order_key(ex[j]) : 0u;
    int id;
    uint32_t my_k, top;
    topk::wave_picks<NV>(key, k, pick_lds[threadIdx.x / kWave], id, my_k, top);
    const float e0 = lane < k ? expf(topk::key_value(my_k) - topk::key_value(top)) : 0.f;
    const float sum = topk::wave_butterfly_sum(e0);  // the standalone top-k's order: the same coefficient bits
    if (lane < k) id_row[lane] = id, coef_row[lane] = e0 / sum;
    if (shared_slot && lane == 0) id_row[k] = E, coef_row[k] = 1.0f / (1.0f + expf(-sd));
}

}  // namespace

bool moe_router_prefill(const void *x, const uint16_t *w, const float *bias, int64_t M, int64_t H, int64_t E,
                        int64_t k, bool shared, float *logits, float *norms, int32_t *ids, float *coef, uint32_t *err,
                        hipStream_t stream, bool shared_slot, void *x16) {
    const int64_t nch = H / 512, ld = E + (shared ? 1 : 0);
    if (H % 512 != 0 || nch < 1 || nch > 8 || E > 1024 || k > 32 || k > E || (H / kParts) % kBK != 0 ||
        reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(w) % 16 != 0)
        return false;
    float *nw = norms + (int64_t)kParts * M;  // (the first kParts * M floats: unused)
    // kNormRows more rows of blocks for the router rows' norms
    dim3 g1((unsigned)((E + kBN - 1) / kBN), (unsigned)((M + kBM - 1) / kBM + kNormRows), (unsigned)kParts);
    STRIX_CHECK(g1.y <= 65535, "moe_router_prefill: M = ", M, " too large");
    router_approx_kernel<<<g1, kThreads, 0, stream>>>(static_cast<const uint16_t *>(x), w, logits, ld, M, E, H, nw);
    const unsigned g2 = (unsigned)((M + 3) / 4);
    const int nv = E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : 16;
    auto go = [&](auto nvc, auto nchc) {
        router_select_kernel<decltype(nvc)::value, decltype(nchc)::value><<<g2, kThreads, 0, stream>>>(
            static_cast<const uint16_t *>(x), w, bias, logits, ld, M, (int)E, (int)k, shared, shared && shared_slot, nw,
            ids, coef, err, static_cast<uint4 *>(x16));
    };
    auto by_nch = [&](auto nvc) {
        switch (nch) {
            case 4: go(nvc, std::integral_constant<int, 4>{}); break;
            case 6: go(nvc, std::integral_constant<int, 6>{}); break;
            case 8: go(nvc, std::integral_constant<int, 8>{}); break;
            default: go(nvc, std::integral_constant<int, 2>{}); break;
        }
    };
    if (nch != 2 && nch != 4 && nch != 6 && nch != 8) return false;
    switch (nv) {
        case 1: by_nch(std::integral_constant<int, 1>{}); break;
        case 2: by_nch(std::integral_constant<int, 2>{}); break;
        case 4: by_nch(std::integral_constant<int, 4>{}); break;
        case 8: by_nch(std::integral_constant<int, 8>{}); break;
        default: by_nch(std::integral_constant<int, 16>{}); break;
    }
    STRIX_HIP_CHECK_LAUNCH("moe_router_prefill M=", M, " E=", E, " k=", k, " H=", H);
    return true;
}

}  // namespace strix::kernels
