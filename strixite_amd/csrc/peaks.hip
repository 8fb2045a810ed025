// Calibration kernels for the bench (no counterpart in the reference): what this device's matrix cores and HBM deliver
// on plain, dependency-free work, so the bench can quote the measured peaks next to the published ones.
#include "common.hpp"
#include "strixite_moe.h"

#include <algorithm>

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// 4 independent chains of v_mfma_f32_32x32x16_f16 a wave (2 * 32 * 32 * 16 flops each), no memory traffic
__global__ void __launch_bounds__(256) mfma_peak_kernel(int iters, float *out) {
    const float s = (float)(threadIdx.x % 7) * 0.001f;
    const f16x8 a = {(_Float16)s, (_Float16)1, (_Float16)0, (_Float16)s, (_Float16)1, (_Float16)0, (_Float16)s, (_Float16)1};
    const f16x8 b = a * (_Float16)0.5f;
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int i = 0; i < iters; ++i) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, a, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, a, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, b, c3, 0, 0, 0);
    }
    const float v = c0[0] + c1[1] + c2[2] + c3[3];
    if (v == 1234.5f) out[0] = v;  // keeps the chains alive; never true for these inputs
}

// a plain streaming read: 16 bytes a lane, grid-stride
__global__ void __launch_bounds__(256) read_peak_kernel(const uint4 *p, int64_t n, float *out) {
    uint32_t acc = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        acc ^= p[i].x ^ p[i].w;
    if (acc == 0x9E3779B9u) out[0] = 1.0f;  // keeps the loads alive
}

// the library's FP32 -> BF16 rounding, element by element
__global__ void __launch_bounds__(256) bf16_round_kernel(const float *x, uint16_t *y, int64_t n) {
    using namespace strix::dev;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = f32_to_bf16(x[i]);
}

}  // namespace

extern "C" {

int strix_calib_bf16_round(const float *x, uint16_t *y, int64_t n, void *stream) {
    if (x == nullptr || y == nullptr || n < 0) return 1;
    if (n == 0) return 0;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 8192);
    bf16_round_kernel<<<(unsigned)blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(x, y, n);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

int64_t strix_calib_mfma_peak(int64_t blocks, int iters, float *out, void *stream) {
    if (blocks < 1 || iters < 1 || out == nullptr) return -1;
    mfma_peak_kernel<<<(unsigned)blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(iters, out);
    if (hipGetLastError() != hipSuccess) return -1;
    return blocks * 4 * (int64_t)iters * 4 * 2 * 32 * 32 * 16;  // flops
}

int strix_calib_read_peak(const void *p, int64_t bytes, int64_t blocks, float *out, void *stream) {
    if (p == nullptr || out == nullptr || bytes < 16 || blocks < 1 || reinterpret_cast<uintptr_t>(p) % 16) return 1;
    read_peak_kernel<<<(unsigned)blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(static_cast<const uint4 *>(p),
                                                                                   bytes / 16, out);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
