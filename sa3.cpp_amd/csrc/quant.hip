// a5: Q8_0 weight blocks — decode to f32 and the reference block encoder.
//
// Block format (ggml block_q8_0, the GGUF Q8_0 tensor layout the reference loads): 32 weights per
// 34-byte block, {uint16 f16 scale d; int8 qs[32]}, packed with 2-byte alignment. A value decodes
// as f32(d) * qs[i]; the product has at most 11 + 7 significant bits, so it is exact in f32 and
// the decode is bit-identical to ggml's dequantize_row_q8_0 (tools/sa3-quant-check.cpp:43).
//
// Compiled with -ffp-contract=off: the encoder's x*id must round before roundf, as ggml's does.
#include "sa3k_internal.h"

namespace {

constexpr int kQK = 32;
constexpr int kBlockBytes = 34;
constexpr int kThreads = 256;

__device__ inline float f16_bits_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

__device__ inline uint16_t f32_to_f16_bits(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);   // round-to-nearest-even
}

// One thread per block: 17 aligned 16-bit loads, 8 float4 stores.
__global__ __launch_bounds__(kThreads) void q8_0_dequant_kernel(const uint16_t* __restrict__ blocks,
                                                                 float4* __restrict__ out, int64_t nb) {
    const int64_t b = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (b >= nb) return;
    const uint16_t* src = blocks + b * (kBlockBytes / 2);
    const float d = f16_bits_to_f32(src[0]);
    float4* dst = out + b * (kQK / 4);
#pragma unroll
    for (int j = 0; j < kQK / 4; ++j) {
        const uint16_t lo = src[1 + 2 * j], hi = src[2 + 2 * j];
        const int8_t q0 = (int8_t)(lo & 0xff), q1 = (int8_t)(lo >> 8);
        const int8_t q2 = (int8_t)(hi & 0xff), q3 = (int8_t)(hi >> 8);
        dst[j] = make_float4(d * (float)q0, d * (float)q1, d * (float)q2, d * (float)q3);
    }
}

// ggml's quantize_row_q8_0_ref, restated: amax over the block, d = amax / 127, id = 1/d (0 when
// d == 0), q = roundf(x * id) (round half away from zero), d stored as f16 (RNE).
__global__ __launch_bounds__(kThreads) void q8_0_quantize_kernel(const float* __restrict__ x,
                                                                  uint16_t* __restrict__ blocks, int64_t nb) {
    const int64_t b = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (b >= nb) return;
    const float* src = x + b * kQK;
    float v[kQK];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < kQK; ++j) {
        v[j] = src[j];
        amax = fmaxf(amax, fabsf(v[j]));
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t* dst = blocks + b * (kBlockBytes / 2);
    dst[0] = f32_to_f16_bits(d);
#pragma unroll
    for (int j = 0; j < kQK / 2; ++j) {
        const float x0 = v[2 * j] * id, x1 = v[2 * j + 1] * id;
        const int8_t q0 = (int8_t)roundf(x0), q1 = (int8_t)roundf(x1);
        dst[1 + j] = (uint16_t)((uint8_t)q0 | ((uint16_t)(uint8_t)q1 << 8));
    }
}

}  // namespace

extern "C" {

SA3K_API int sa3k_q8_0_dequant(sa3k_ctx* ctx, const void* blocks, float* out, int64_t n_elems) {
    return sa3k_guard(ctx, "sa3k_q8_0_dequant", [&] {
        SA3K_REQUIRE(n_elems >= 0 && n_elems % kQK == 0, "element count must be a multiple of 32");
        if (!n_elems) return;
        SA3K_REQUIRE(blocks && out, "null pointer");
        SA3K_REQUIRE((reinterpret_cast<uintptr_t>(blocks) & 1u) == 0, "blocks must be 2-byte aligned");
        SA3K_REQUIRE((reinterpret_cast<uintptr_t>(out) & 15u) == 0, "out must be 16-byte aligned");
        const int64_t nb = n_elems / kQK;
        KernelScope ks(ctx, "q8_0_dequant");
        q8_0_dequant_kernel<<<(unsigned)ceil_div(nb, kThreads), kThreads, 0, ctx->stream>>>(
            static_cast<const uint16_t*>(blocks), reinterpret_cast<float4*>(out), nb);
        SA3K_LAUNCHED();
    });
}

SA3K_API int sa3k_q8_0_quantize(sa3k_ctx* ctx, const float* x, void* blocks, int64_t n_elems) {
    return sa3k_guard(ctx, "sa3k_q8_0_quantize", [&] {
        SA3K_REQUIRE(n_elems >= 0 && n_elems % kQK == 0, "element count must be a multiple of 32");
        if (!n_elems) return;
        SA3K_REQUIRE(blocks && x, "null pointer");
        SA3K_REQUIRE((reinterpret_cast<uintptr_t>(blocks) & 1u) == 0, "blocks must be 2-byte aligned");
        const int64_t nb = n_elems / kQK;
        KernelScope ks(ctx, "q8_0_quantize");
        q8_0_quantize_kernel<<<(unsigned)ceil_div(nb, kThreads), kThreads, 0, ctx->stream>>>(
            x, static_cast<uint16_t*>(blocks), nb);
        SA3K_LAUNCHED();
    });
}

}  // extern "C"
