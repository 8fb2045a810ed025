// The router projection's small-batch wave (router.hip's router_small_kernel, and the layer's fused decode routing
// launch in experts.hip): one wave computes TT tokens x TE rows of logits in the canonical FP32 order.
#pragma once

#include "common.hpp"

#include <type_traits>

namespace strix::kernels::rsmall {

constexpr int kWave = 64;

// Small batches (M <= 64): a wave computes TT tokens x TE rows (rows n0 .., tokens m0 ..) with all of its loads
// issued at once (NCH chunks a lane: K = 8 * 64 * NCH), so a wave costs one memory round trip. The TT * TE lane
// partials meet in a reduce-scatter along the butterfly: bit-identical to the canonical order (lane l takes the
// 8-element chunks l, l + 64, ... with fmaf, then a butterfly over the 64 lanes).
// COH: FP32 logits stored device-coherent (agent-scope relaxed atomic stores: through to memory, for a reader on
// another XCD in the same launch).
template <typename TY, int TT, int TE, int NCH, bool COH = false>
__device__ __forceinline__ void router_small_wave(const uint16_t *x, const uint16_t *w, TY *y, int64_t M, int64_t N,
                                                  int64_t K, int64_t n0, int64_t m0, const float *bias = nullptr,
                                                  int64_t nbias = 0) {
    using namespace strix::dev;
    constexpr int P = TT * TE;
    static_assert(P <= kWave && (P & (P - 1)) == 0, "pairs: a power of two, at most a wave");
    const int lane = threadIdx.x % kWave;
    uint4 wu[NCH][TE], xu[NCH][TT];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int64_t c = lane + (int64_t)i * kWave;
#pragma unroll
        for (int e = 0; e < TE; ++e)
            wu[i][e] = *reinterpret_cast<const uint4 *>(w + (n0 + e < N ? n0 + e : N - 1) * K + c * 8);
#pragma unroll
        for (int t = 0; t < TT; ++t)
            xu[i][t] = *reinterpret_cast<const uint4 *>(x + (m0 + t < M ? m0 + t : M - 1) * K + c * 8);
    }
    float v[P];
#pragma unroll
    for (int p = 0; p < P; ++p) v[p] = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; ++i)
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            const uint32_t xd[4] = {xu[i][t].x, xu[i][t].y, xu[i][t].z, xu[i][t].w};
#pragma unroll
            for (int e = 0; e < TE; ++e) {
                const uint32_t wd[4] = {wu[i][e].x, wu[i][e].y, wu[i][e].z, wu[i][e].w};
                float a = v[t * TE + e];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float xv = __uint_as_float(k % 2 ? xd[k / 2] & 0xffff0000u : xd[k / 2] << 16);
                    const float wv = __uint_as_float(k % 2 ? wd[k / 2] & 0xffff0000u : wd[k / 2] << 16);
                    a = fmaf(xv, wv, a);
                }
                v[t * TE + e] = a;
            }
        }
    // reduce-scatter along the butterfly while pairs remain, then a plain butterfly; lane l ends with pair
    // (l / (64 / P)) (every lane of its group holds the same sum)
#pragma unroll
    for (int lvl = 0; lvl < 6; ++lvl) {
        const int o = kWave / 2 >> lvl, n = P >> lvl;
        if (n > 1) {
            const bool up = lane & o;
#pragma unroll
            for (int i = 0; i < n / 2; ++i) {
                const float send = up ? v[i] : v[n / 2 + i];
                const float keep = up ? v[n / 2 + i] : v[i];
                v[i] = keep + __shfl_xor(send, o, kWave);
            }
        } else {
            v[0] = v[0] + __shfl_xor(v[0], o, kWave);
        }
    }
    constexpr int G = kWave / P;  // lanes holding one pair
    if (lane % G == 0) {
        const int p = lane / G, t = p / TE, e = p % TE;
        if (m0 + t < M && n0 + e < N) {
            // bias: the router's bias added to the first nbias rows, one rounding (as a separate pass adds it)
            if constexpr (std::is_same_v<TY, float>) {
                const float r = bias != nullptr && n0 + e < nbias ? v[0] + bias[n0 + e] : v[0];
                if constexpr (COH) __hip_atomic_store(y + (m0 + t) * N + n0 + e, r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else y[(m0 + t) * N + n0 + e] = r;
            }
            else y[(m0 + t) * N + n0 + e] = f32_to_bf16(v[0]);
        }
    }
}

}  // namespace strix::kernels::rsmall
