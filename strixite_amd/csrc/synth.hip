// Seeded synthetic tensors generated on the GPU (the bench's weights: ~10 GB for an 8-layer stack would take minutes
// on the host). Counter-based SplitMix64 (Steele, Lea, Flood 2014): element i of a tensor is a pure function of
// (key, i), so any launch shape gives the same bytes, and a host generator that follows the same definition matches
// bit for bit. Normals: the Irwin-Hall sum of four 16-bit uniforms, standardized by one float multiply - no
// transcendental function, hence no library-dependent rounding.
#include "common.hpp"

namespace strix::synth {

namespace {

__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t hash_at(uint64_t key, uint64_t i) { return splitmix64(key ^ (i * 0xD1B54A32D192ED03ull)); }

constexpr float kInvSd = 2.6428722e-05f;  // 1 / sqrt((65536^2 - 1) / 3)
constexpr int32_t kMean = 131070;         // 4 * 65535 / 2

__device__ __forceinline__ float normal_at(uint64_t key, uint64_t i, float sigma) {
    const uint64_t h = hash_at(key, i);
    const int32_t n = (int32_t)(h & 0xFFFF) + (int32_t)((h >> 16) & 0xFFFF) + (int32_t)((h >> 32) & 0xFFFF) + (int32_t)(h >> 48);
    const float sf = sigma * kInvSd;
    return __fmul_rn((float)(n - kMean), sf);
}

constexpr int kThreads = 256;

__global__ void bf16_normal_kernel(uint64_t key, float sigma, uint16_t *out, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
        out[i] = dev::f32_to_bf16(normal_at(key, (uint64_t)i, sigma));
}

__global__ void q4_codes_kernel(uint64_t key, uint8_t *q, int64_t nbytes) {
    // 8 bytes per hash: byte i = bits 8 (i % 8) .. of hash(i / 8)
    for (int64_t w = (int64_t)blockIdx.x * kThreads + threadIdx.x; w * 8 < nbytes; w += (int64_t)gridDim.x * kThreads) {
        const uint64_t h = hash_at(key, (uint64_t)w);
        if (w * 8 + 8 <= nbytes && ((uintptr_t)q % 8) == 0) {
            reinterpret_cast<uint64_t *>(q)[w] = h;
        } else {
            for (int b = 0; b < 8 && w * 8 + b < nbytes; ++b) q[w * 8 + b] = (uint8_t)(h >> (8 * b));
        }
    }
}

__global__ void q8_codes_kernel(uint64_t key, uint8_t *q, int64_t n) {
    // 4 codes per hash: code i = (16-bit field i % 4 of hash(i / 4)) % 255 + 1
    for (int64_t w = (int64_t)blockIdx.x * kThreads + threadIdx.x; w * 4 < n; w += (int64_t)gridDim.x * kThreads) {
        const uint64_t h = hash_at(key, (uint64_t)w);
        for (int b = 0; b < 4 && w * 4 + b < n; ++b) q[w * 4 + b] = (uint8_t)((uint32_t)((h >> (16 * b)) & 0xFFFF) % 255u + 1u);
    }
}

__global__ void scales_kernel(uint64_t key, float min_mul, uint16_t *scale, uint16_t *minv, int64_t n) {
    for (int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x; g < n; g += (int64_t)gridDim.x * kThreads) {
        const uint16_t sb = dev::f32_to_bf16(fabsf(normal_at(key, (uint64_t)g, 0.02f)));
        scale[g] = sb;
        minv[g] = dev::f32_to_bf16(__fmul_rn(min_mul, dev::bf16_to_f32(sb)));
    }
}

__global__ void uniform_pm1_kernel(uint64_t key, float *out, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
        const uint32_t v = (uint32_t)(hash_at(key, (uint64_t)i) >> 40);
        out[i] = __fsub_rn(__fmul_rn((float)v, 1.1920928955078125e-07f), 1.0f);
    }
}

unsigned blocks_for(int64_t n) {
    const int64_t b = (n + kThreads - 1) / kThreads;
    return (unsigned)(b < 8192 ? (b > 0 ? b : 1) : 8192);
}

}  // namespace

uint64_t tensor_key(uint64_t seed, uint32_t tensor, uint32_t layer) {
    return splitmix64(splitmix64(seed) ^ ((uint64_t)tensor << 32) ^ (uint64_t)layer);
}

void bf16_normal(uint64_t key, float sigma, uint16_t *out, int64_t n, hipStream_t stream) {
    STRIX_CHECK(out != nullptr && n >= 0, "synth bf16_normal: null output or negative count");
    bf16_normal_kernel<<<blocks_for(n), kThreads, 0, stream>>>(key, sigma, out, n);
    STRIX_HIP_CHECK_LAUNCH("synth bf16_normal n=", n);
}

void q_weight(int bits, uint64_t key_codes, uint64_t key_scales, int64_t rows, int64_t K, int64_t G, uint8_t *q,
              uint16_t *scale, uint16_t *minv, hipStream_t stream) {
    STRIX_CHECK(bits == 4 || bits == 8, "synth q_weight: bits = ", bits);
    STRIX_CHECK(q && scale && minv && rows >= 1 && K >= G && (G == 32 || G == 64 || G == 128) && K % G == 0,
                "synth q_weight: bad view (rows = ", rows, ", K = ", K, ", G = ", G, ")");
    if (bits == 4) q4_codes_kernel<<<blocks_for(rows * K / 16), kThreads, 0, stream>>>(key_codes, q, rows * K / 2);
    else q8_codes_kernel<<<blocks_for(rows * K / 4), kThreads, 0, stream>>>(key_codes, q, rows * K);
    const int64_t ng = rows * (K / G);
    scales_kernel<<<blocks_for(ng), kThreads, 0, stream>>>(key_scales, bits == 4 ? -8.0f : -128.0f, scale, minv, ng);
    STRIX_HIP_CHECK_LAUNCH("synth q_weight rows=", rows, " K=", K);
}

void uniform_pm1(uint64_t key, float *out, int64_t n, hipStream_t stream) {
    STRIX_CHECK(out != nullptr && n >= 0, "synth uniform_pm1: null output");
    uniform_pm1_kernel<<<blocks_for(n), kThreads, 0, stream>>>(key, out, n);
    STRIX_HIP_CHECK_LAUNCH("synth uniform_pm1 n=", n);
}

}  // namespace strix::synth
