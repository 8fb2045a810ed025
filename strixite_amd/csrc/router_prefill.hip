// Prefill-size routing on gfx950's matrix cores with the routing of the canonical FP32 order, bit for bit.
//
// The router projection (strixite kernels/linear.hip:83-147 semantics, FP32) is the one place on the path whose result
// decides a discrete choice (the top-k), so it must be reproduced exactly - in this library's canonical summation
// order (lane l of a wave64 takes the 8-element chunks l, l + 64, ... with fmaf, then a butterfly over the 64 lanes;
// oracle: orc_router_logits). That order does not map onto MFMA, and at 4096 tokens x 513 rows x 3072 the VALU form
// costs ~0.3 ms. So the projection runs in two passes:
//   1. approx: logits a = x . w^T as a plain bf16 GEMM on the matrix cores (hipBLASLt, FP32 accumulation, any
//      internal order), and the 2-norms |w_e| (|x_m| comes from pass 2, which loads the token's row). For ANY order of
//      summing the K exact bf16 x bf16 products in FP32 - rounded to nearest or toward zero,
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
// layer reads later); the approximate values sit in the buffer's second quarter.
#include "common.hpp"
#include "topk.hpp"

#include <hipblaslt/hipblaslt.h>

#include <climits>
#include <cstdlib>
#include <mutex>
#include <tuple>
#include <vector>

namespace strix::kernels {
namespace {

using namespace strix::dev;
constexpr int kWave = 64, kThreads = 256;


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

// The approximate logits as pass 1 left them: token m's at a[m ld + e].
struct ApproxIn {
    const float *a;
    int64_t ld;
};

// One wave per token. The exact values are written into the layer's logits row (ld); nw2: the squared norms of the
// router rows.
template <int NV, int NCH>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
    router_select_kernel(const uint16_t *x, const uint16_t *w, const float *bias, float *logits, int64_t ld,
                         int64_t M, int E, int k, bool shared, bool shared_slot, const float *nw2,
                         int32_t *ids, float *coef, uint32_t *err, uint4 *x16, ApproxIn ap) {
    __shared__ int cand_lds[kThreads / kWave][1040];  // a wave's candidate list (at most E + 1 <= 1025)
    __shared__ uint2 pick_lds[kThreads / kWave][topk::kCandScratch];  // the picks' scratch (topk::wave_picks)
    const int lane = threadIdx.x % kWave;
    const int64_t m = (int64_t)blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
    if (m >= M) return;  // whole wave; no barrier in this kernel
    constexpr int64_t K = (int64_t)NCH * 512;
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
    float va[NV], dl[NV], av[NV], n2v[NV], bv[NV];
    bool fin = isfinite(nxm);
    // every lane's approximate values, norms and biases loaded together (clamped indices: one round trip)
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e = lane + j * kWave, ec = e < E ? e : E - 1;
        av[j] = ap.a[m * ap.ld + ec], n2v[j] = nw2[ec], bv[j] = bias ? bias[ec] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e = lane + j * kWave;
        const float a = e < E ? av[j] : 0.f, n2 = e < E ? n2v[j] : 0.f;
        const float b = e < E ? bv[j] : 0.f, n = sqrtf(n2) * up;
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

// ---- pass 1 through hipBLASLt ---------------------------------------------------------------------------------------
// The approximate logits are a plain bf16 GEMM (any FP32 summation order is within the bound above), so at prefill
// sizes they come from the library GEMM: C [M, N] (ld N) = x [M, K] w [N, K]^T, FP32 accumulation. Column-major in
// hipBLASLt's terms: C^T (N x M) = op_T(w as K x N) * (x as K x M). The handle lives per device and the chosen
// algorithm per shape (no workspace); a shape the library declines returns false (the caller then routes through the
// canonical-order projection and top-k).
struct BltShape {
    int device;
    int64_t M, N, K;
    hipblasLtMatrixLayout_t la, lb, lc;
    hipblasLtMatmulAlgo_t algo;
};
struct BltState {
    std::mutex mu;
    std::vector<std::pair<int, hipblasLtHandle_t>> handles;
    std::vector<std::pair<int, hipblasLtMatmulDesc_t>> descs;
    std::vector<BltShape> shapes;
    std::vector<std::tuple<int, int64_t, int64_t, int64_t>> declined;
};
BltState &blt_state() {
    static BltState *s = new BltState;  // lives until the process ends (the library's handles with it)
    return *s;
}

bool approx_blaslt(const uint16_t *x, const uint16_t *w, float *c, int64_t M, int64_t N, int64_t K,
                   hipStream_t stream) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    BltState &st = blt_state();
    hipblasLtHandle_t h = nullptr;
    hipblasLtMatmulDesc_t op = nullptr;
    BltShape use{};
    {
        std::lock_guard<std::mutex> lock(st.mu);
        for (const auto &d : st.declined)
            if (d == std::make_tuple(dev, M, N, K)) return false;
        for (auto &e : st.handles)
            if (e.first == dev) h = e.second;
        for (auto &e : st.descs)
            if (e.first == dev) op = e.second;
        if (h == nullptr) {
            if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) return false;
            st.handles.emplace_back(dev, h);
        }
        if (op == nullptr) {
            if (hipblasLtMatmulDescCreate(&op, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) return false;
            const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
            hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta);
            hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb);
            st.descs.emplace_back(dev, op);
        }
        bool found = false;
        for (const BltShape &e : st.shapes)
            if (e.device == dev && e.M == M && e.N == N && e.K == K) use = e, found = true;
        if (!found) {
            BltShape ns{dev, M, N, K, nullptr, nullptr, nullptr, {}};
            bool ok = hipblasLtMatrixLayoutCreate(&ns.la, HIP_R_16BF, K, N, K) == HIPBLAS_STATUS_SUCCESS &&
                      hipblasLtMatrixLayoutCreate(&ns.lb, HIP_R_16BF, K, M, K) == HIPBLAS_STATUS_SUCCESS &&
                      hipblasLtMatrixLayoutCreate(&ns.lc, HIP_R_32F, N, M, N) == HIPBLAS_STATUS_SUCCESS;
            hipblasLtMatmulPreference_t pref = nullptr;
            ok = ok && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
            uint64_t wsb = 0;
            ok = ok && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb,
                                                             sizeof wsb) == HIPBLAS_STATUS_SUCCESS;
            hipblasLtMatmulHeuristicResult_t res{};
            int n = 0;
            ok = ok && hipblasLtMatmulAlgoGetHeuristic(h, op, ns.la, ns.lb, ns.lc, ns.lc, pref, 1, &res, &n) ==
                           HIPBLAS_STATUS_SUCCESS && n >= 1;
            if (pref) hipblasLtMatmulPreferenceDestroy(pref);
            if (!ok) {
                st.declined.emplace_back(dev, M, N, K);
                return false;
            }
            ns.algo = res.algo;
            st.shapes.push_back(ns);
            use = ns;
        }
    }
    const float alpha = 1.0f, beta = 0.0f;
    return hipblasLtMatmul(h, op, &alpha, w, use.la, x, use.lb, &beta, c, use.lc, c, use.lc, &use.algo, nullptr, 0,
                           stream) == HIPBLAS_STATUS_SUCCESS;
}

// The router rows' squared norms (any FP32 order; rounded up by the bound's allowance): 16 rows a block, 16 threads
// a row
__global__ void __launch_bounds__(kThreads) router_norms_kernel(const uint16_t *w, int64_t N, int64_t K, float *nw) {
    const int t = threadIdx.x;
    const int64_t c = (int64_t)blockIdx.x * 16 + t / 16;
    float q = 0.f;
    if (c < N) {
        const uint4 *wr = reinterpret_cast<const uint4 *>(w + c * K);
#pragma unroll 12
        for (int64_t i = t % 16; i < K / 8; i += 16) q += sumsq8(wr[i]);
    }
    q += __shfl_xor(q, 1, kWave);
    q += __shfl_xor(q, 2, kWave);
    q += __shfl_xor(q, 4, kWave);
    q += __shfl_xor(q, 8, kWave);
    if (t % 16 == 0 && c < N) nw[c] = q;
}

}  // namespace

namespace {
bool prefill_shape_fits(const void *x, const uint16_t *w, int64_t H, int64_t E, int64_t k) {
    const int64_t nch = H / 512;
    return H % 512 == 0 && (nch == 2 || nch == 4 || nch == 6 || nch == 8) && E <= 1024 && k <= 32 && k <= E &&
           reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0;
}
}  // namespace

bool moe_router_prefill_approx(const void *x, const uint16_t *w, int64_t M, int64_t H, int64_t E, int64_t k,
                               bool shared, float *logits, float *norms, hipStream_t stream) {
    if (!prefill_shape_fits(x, w, H, E, k)) return false;
    const int64_t ld = E + (shared ? 1 : 0);
    // pass 1: the library GEMM into the logits buffer's second part ([M][E], ld E; parts 1..3 of the [4][M][ld]
    // buffer are scratch) and the row norms. A shape the library declines: false, and the caller routes through the
    // canonical-order projection and top-k instead
    if (!approx_blaslt(static_cast<const uint16_t *>(x), w, logits + M * ld, M, E, H, stream)) return false;
    router_norms_kernel<<<(unsigned)((E + 15) / 16), kThreads, 0, stream>>>(w, E, H, norms + M);
    STRIX_HIP_CHECK_LAUNCH("moe_router_prefill (row norms) E=", E, " H=", H);
    return true;
}

void moe_router_prefill_select(const void *x, const uint16_t *w, const float *bias, int64_t M, int64_t H, int64_t E,
                               int64_t k, bool shared, float *logits, float *norms, int32_t *ids, float *coef,
                               uint32_t *err, hipStream_t stream, bool shared_slot, void *x16) {
    const int64_t nch = H / 512, ld = E + (shared ? 1 : 0);
    const ApproxIn ap{logits + M * ld, E};
    const float *nw = norms + M;  // (the first M floats: unused)
    const unsigned g2 = (unsigned)((M + 3) / 4);
    const int nv = E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : 16;
    auto go = [&](auto nvc, auto nchc) {
        router_select_kernel<decltype(nvc)::value, decltype(nchc)::value><<<g2, kThreads, 0, stream>>>(
            static_cast<const uint16_t *>(x), w, bias, logits, ld, M, (int)E, (int)k, shared, shared && shared_slot, nw,
            ids, coef, err, static_cast<uint4 *>(x16), ap);
    };
    auto by_nch = [&](auto nvc) {
        switch (nch) {
            case 4: go(nvc, std::integral_constant<int, 4>{}); break;
            case 6: go(nvc, std::integral_constant<int, 6>{}); break;
            case 8: go(nvc, std::integral_constant<int, 8>{}); break;
            default: go(nvc, std::integral_constant<int, 2>{}); break;
        }
    };
    switch (nv) {
        case 1: by_nch(std::integral_constant<int, 1>{}); break;
        case 2: by_nch(std::integral_constant<int, 2>{}); break;
        case 4: by_nch(std::integral_constant<int, 4>{}); break;
        case 8: by_nch(std::integral_constant<int, 8>{}); break;
        default: by_nch(std::integral_constant<int, 16>{}); break;
    }
    STRIX_HIP_CHECK_LAUNCH("moe_router_prefill M=", M, " E=", E, " k=", k, " H=", H);
}

bool moe_router_prefill(const void *x, const uint16_t *w, const float *bias, int64_t M, int64_t H, int64_t E,
                        int64_t k, bool shared, float *logits, float *norms, int32_t *ids, float *coef, uint32_t *err,
                        hipStream_t stream, bool shared_slot, void *x16) {
    if (!moe_router_prefill_approx(x, w, M, H, E, k, shared, logits, norms, stream)) return false;
    moe_router_prefill_select(x, w, bias, M, H, E, k, shared, logits, norms, ids, coef, err, stream, shared_slot, x16);
    return true;
}

}  // namespace strix::kernels
