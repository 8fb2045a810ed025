// C-ABI shim over the reference's own quantizers, built from the reference's sources where they lie
// (strixite formats/q4.cpp, formats/q8.cpp, formats/q5.cpp; nothing is copied) into oracle/_ref/. Test infrastructure only: it
// writes the golden vectors under tests/golden/ that pin this oracle's orc_quantize_* / orc_dequantize.
#include "formats/q4.hpp"
#include "formats/q8.hpp"
#include "formats/q5.hpp"

#include <cstring>
#include <exception>

extern "C" {

// strixite formats/q4.hpp:29 quantize_q4, :39 dequantize_q4. Returns 0, or -1 when the reference throws.
int ref_quantize_q4(const float *w, int64_t N, int64_t K, int64_t G, uint8_t *q, uint16_t *scale, uint16_t *minv) {
    try {
        const strix::Q4Weight r = strix::quantize_q4(w, N, K, G);
        std::memcpy(q, r.q.data(), r.q.size());
        std::memcpy(scale, r.scale.data(), r.scale.size() * 2);
        std::memcpy(minv, r.minv.data(), r.minv.size() * 2);
        return 0;
    } catch (const std::exception &) {
        return -1;
    }
}

int ref_dequantize_q4(const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t N, int64_t K, int64_t G,
                      float *w) {
    try {
        strix::Q4Weight r;
        r.N = N, r.K = K, r.G = G;
        r.q.assign(q, q + N * K / 2);
        r.scale.assign(scale, scale + N * (K / G));
        r.minv.assign(minv, minv + N * (K / G));
        const std::vector<float> d = strix::dequantize_q4(r);
        std::memcpy(w, d.data(), d.size() * 4);
        return 0;
    } catch (const std::exception &) {
        return -1;
    }
}

// strixite formats/q8.hpp:28 quantize_q8, :34 dequantize_q8.
int ref_quantize_q8(const float *w, int64_t N, int64_t K, int64_t G, uint8_t *q, uint16_t *scale, uint16_t *minv) {
    try {
        const strix::Q8Weight r = strix::quantize_q8(w, N, K, G);
        std::memcpy(q, r.q.data(), r.q.size());
        std::memcpy(scale, r.scale.data(), r.scale.size() * 2);
        std::memcpy(minv, r.minv.data(), r.minv.size() * 2);
        return 0;
    } catch (const std::exception &) {
        return -1;
    }
}

int ref_dequantize_q8(const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t N, int64_t K, int64_t G,
                      float *w) {
    try {
        strix::Q8Weight r;
        r.N = N, r.K = K, r.G = G;
        r.q.assign(q, q + N * K);
        r.scale.assign(scale, scale + N * (K / G));
        r.minv.assign(minv, minv + N * (K / G));
        const std::vector<float> d = strix::dequantize_q8(r);
        std::memcpy(w, d.data(), d.size() * 4);
        return 0;
    } catch (const std::exception &) {
        return -1;
    }
}


// strixite formats/q5.hpp:36 quantize_q5, :42 dequantize_q5. Returns 0, or -1 when the reference throws.
int ref_quantize_q5(const float *w, int64_t N, int64_t K, int64_t G, uint8_t *q, uint16_t *scale, uint16_t *minv) {
    try {
        const strix::Q5Weight r = strix::quantize_q5(w, N, K, G);
        std::memcpy(q, r.q.data(), r.q.size());
        std::memcpy(scale, r.scale.data(), r.scale.size() * 2);
        std::memcpy(minv, r.minv.data(), r.minv.size() * 2);
        return 0;
    } catch (const std::exception &) {
        return -1;
    }
}

int ref_dequantize_q5(const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t N, int64_t K, int64_t G,
                      float *w) {
    try {
        strix::Q5Weight r;
        r.N = N, r.K = K, r.G = G;
        r.q.assign(q, q + N * (K / 2 + K / 8));
        r.scale.assign(scale, scale + N * (K / G));
        r.minv.assign(minv, minv + N * (K / G));
        const std::vector<float> d = strix::dequantize_q5(r);
        std::memcpy(w, d.data(), d.size() * 4);
        return 0;
    } catch (const std::exception &) {
        return -1;
    }
}

}  // extern "C"
