// oracle: f16 conversion and Q8_0 blocks — TEST INFRASTRUCTURE ONLY (see oracle.h).
//
// Q8_0 is ggml's block_q8_0 (32 int8 quants + one f16 scale, 34 bytes), the GGUF type the
// reference's quantizer writes (tools/sa3-quantize.cpp:43-56) and its inference path reads
// (src/lora.h:51-74, 239-268). ggml is not vendored (docs/GGML_FORK.md:84-88), so the encoder
// restates ggml's published quantize_row_q8_0_ref: d = amax/127, id = 1/d (0 if d == 0),
// q = roundf(x*id), d stored as f16 with round-to-nearest-even; the decoder is f32(d)*q.
#include "oracle.h"

#include <cmath>
#include <cstring>

extern "C" {

// IEEE binary32 -> binary16, round to nearest even (software; pinned against numpy.float16)
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u);
    if (ax >= 0x477ff000u) return sign | 0x7c00u;          // >= 65520 rounds to infinity
    if (ax < 0x38800000u) {                                // below 2^-14: f16 subnormal range
        const int e = (int)(ax >> 23);
        if (e < 102) return sign;                          // < 2^-25 rounds to zero
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const int shift = 126 - e;                         // 14..24
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (ax >> 13) - (112u << 10);                // rebias 127 -> 15
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            float v = (float)m * 0x1p-24f;                 // exact
            std::memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float out;
    std::memcpy(&out, &bits, 4);
    return out;
}

void orc_f32_to_f16_row(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_f16(x[i]);
}

void orc_f16_to_f32_row(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f16_to_f32(x[i]);
}

void orc_q8_0_quantize(const float* x, void* blocks, int64_t n) {
    unsigned char* out = static_cast<unsigned char*>(blocks);
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* src = x + b * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = std::fmax(amax, std::fabs(src[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = orc_f32_to_f16(d);
        unsigned char* blk = out + b * 34;
        blk[0] = (unsigned char)(dh & 0xff);
        blk[1] = (unsigned char)(dh >> 8);
        for (int j = 0; j < 32; ++j) {
            const float x0 = src[j] * id;
            blk[2 + j] = (unsigned char)(int8_t)std::round(x0);   // roundf: half away from zero
        }
    }
}

void orc_q8_0_dequant(const void* blocks, float* y, int64_t n) {
    const unsigned char* in = static_cast<const unsigned char*>(blocks);
    for (int64_t b = 0; b < n / 32; ++b) {
        const unsigned char* blk = in + b * 34;
        const float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int j = 0; j < 32; ++j) y[b * 32 + j] = d * (float)(int8_t)blk[2 + j];
    }
}

}  // extern "C"
