// The boundary types of the MoE launch interface, for a build WITHOUT strixite's own headers (this library itself,
// its C-ABI, tests). Inside the strixite tree these types come from strixite's headers instead and this file is not
// included (strixite_moe_extras.hpp with STRIXITE_MOE_DROPIN defined). Each type has the fields and meaning of the
// strixite declaration cited beside it, so code compiled against either sees the same layout.
#pragma once

#define STRIXITE_MOE_TYPES_HPP 1

#include <cstddef>
#include <cstdint>
#include <stdexcept>

namespace strix {

// strixite common/check.hpp:21-30: a failed host-side precondition; a HIP runtime failure after which the device
// context is not trusted.
class Error : public std::runtime_error {
public:
    using std::runtime_error::runtime_error;
};
class GpuFatalError : public Error {
public:
    using Error::Error;
};

// strixite runtime/q4_device.hpp:13-18, runtime/q8_device.hpp:12-17: non-owning device views of the formats/q4.hpp
// and formats/q8.hpp layouts (q [N, K/2] or [N, K] bytes, scale / min [N, K/G] BF16 bits, w = q * scale + min).
struct Q4DeviceView {
    const uint8_t *q = nullptr;
    const uint16_t *scale = nullptr;
    const uint16_t *minv = nullptr;
    int64_t N = 0, K = 0, G = 0;
};
struct Q8DeviceView {
    const uint8_t *q = nullptr;
    const uint16_t *scale = nullptr;
    const uint16_t *minv = nullptr;
    int64_t N = 0, K = 0, G = 0;
};
// strixite runtime/q5_device.hpp:13-18: formats/q5.hpp rows (K % 128 == 0): per row a low plane [K/2] of 4-bit
// codes (low nibble = even k) and a high plane [K/8] of bit 4 (code k at bit k % 8 of byte k / 8), scale / min
// [N, K/G] BF16 bits, w = q * scale + min.
struct Q5DeviceView {
    const uint8_t *q = nullptr;
    const uint16_t *scale = nullptr;
    const uint16_t *minv = nullptr;
    int64_t N = 0, K = 0, G = 0;
};
// strixite runtime/q4_device.hpp:37-43, runtime/q8_device.hpp:36-42: the same codes, scales and mins laid out
// chunk-major (formats/q4.hpp:43-55): 32-code chunk c of row n at q[(c N + n) * 16] (Q4) or [(c N + n) * 32] (Q8),
// group g's scale / min at [g N + n].
struct Q4ChunkMajorView {
    const uint8_t *q = nullptr;
    const uint16_t *scale = nullptr;
    const uint16_t *minv = nullptr;
    int64_t N = 0, K = 0, G = 0;
};
struct Q8ChunkMajorView {
    const uint8_t *q = nullptr;
    const uint16_t *scale = nullptr;
    const uint16_t *minv = nullptr;
    int64_t N = 0, K = 0, G = 0;
};

namespace kernels {

// strixite kernels/norm.hpp:20
enum class Act { F32, BF16 };

// strixite kernels/moe_grouped.hpp:38. The F16 kinds (WmmaF16, Narrow, Wide, Wide256: one math, tiles picked by
// shape) run Q4 experts' prefill-size grouped GEMMs in the reference's F16 math (x rounded to F16 toward zero, each
// weight one F16 rounding of code * s + m, FP32 accumulation); F32 and WmmaBf16 keep the weights exact (scaled
// codes, FP32 accumulation). Q8 experts and decode-size calls use the exact weights under every kind.
enum class MoeMath { F32, WmmaBf16, WmmaF16, WmmaF16Narrow, WmmaF16Wide, WmmaF16Wide256 };

constexpr int64_t kMoeMaxExperts = 1023;  // strixite kernels/moe_grouped.hpp:43: E + 1 buckets
constexpr int64_t kMoeMaxSlots = 1 << 20;  // strixite kernels/moe_grouped.hpp:44

// strixite kernels/moe_grouped.hpp:75-81
struct MoeSharedAdd {
    const void *s = nullptr;
    const float *gate_logit = nullptr;
    int64_t gate_ld = 0;
    uint32_t gate_index = 0;
    uint32_t *err = nullptr;
};

}  // namespace kernels
}  // namespace strix
