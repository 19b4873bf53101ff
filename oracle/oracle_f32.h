// oracle (internal, not part of the C interface): the oracle's f32 mode — TEST INFRASTRUCTURE ONLY.
//
// orc_set_f32(1) (oracle.h) makes the linears (dit_lin.cpp) and the attention (attn.cpp) compute in
// float instead of double, with the products in sgemm.cpp; bench.py times the DiT block this way
// as its CPU baseline. The double mode stays the pinned oracle.
#pragma once

#include <cstdint>

extern int g_orc_f32;            // 1: float compute in dit_lin.cpp and attn.cpp
bool orc_f32_kernels_ok();       // the CPU runs sgemm.cpp's AVX2 + FMA code

// sgemm.cpp (call only when orc_f32_kernels_ok())
void orc_sgemm_nt(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K);
float orc_sdot(const float* a, const float* b, int n);
void orc_saxpy(float a, const float* x, float* y, int n);
