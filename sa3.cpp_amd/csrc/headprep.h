// Element math that a separate kernel and a GEMM epilogue both compute (each through the functions
// here, so the two paths give the same bits): the per-head preparation of the DiT's attention
// inputs (src/dit.h:207-217, src/nn.h:40-59: RMS norm over a head's 64 dims with a per-dim gain,
// then NeoX RoPE over its first rope_dims dims; 16 lanes work on one (row, head), lane j holding
// dims 4j..4j+3), the attention backward's row dots and the FFN SwiGLU backward.
#pragma once

#include "sa3k_internal.h"

namespace sa3k {

constexpr int kHeadDim = 64;

// v + its value in another lane of the same 16-lane row, by a DPP lane permutation
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Sum over the 16 lanes of an aligned 16-lane group (every lane of the group active): partners by
// lane ^ 1, lane ^ 2 (quad permutations), then the mirrored lane of the 8- and the 16-lane half.
// Every lane adds the same two partial sums at each step, so all 16 get the same bits.
__device__ inline float group16_sum(float v) {
    v = dpp_add<0xB1>(v);    // quad_perm [1, 0, 3, 2]
    v = dpp_add<0x4E>(v);    // quad_perm [2, 3, 0, 1]
    v = dpp_add<0x141>(v);   // row_half_mirror
    v = dpp_add<0x140>(v);   // row_mirror
    return v;
}

// The RoPE table entries (cos, sin) of this lane's four dims d0..d0+3 from the token's table row
// [rope_dims] (cos of the half pairs, then sin; global memory or LDS). Lanes past rope_dims get
// zeros and do not use them. rope_dims % 8 == 0, so a rotation pair (i, i + half) is the same
// component of lanes j and j + half/4.
__device__ inline void rope_tab4(int d0, int rope, const float* row_tab, float4& cs, float4& sn) {
    const int half = rope >> 1;
    cs = sn = make_float4(0.f, 0.f, 0.f, 0.f);
    if (d0 >= rope) return;
    const int i = d0 < half ? d0 : d0 - half;
    cs = *reinterpret_cast<const float4*>(row_tab + i);
    sn = *reinterpret_cast<const float4*>(row_tab + half + i);
}

// Rotates y in place with the table entries of rope_tab4; lanes past rope_dims keep y. sign -1:
// the inverse rotation. Every lane of the wave takes part (the partner values come by shuffle).
__device__ inline void rope4_cs(float4& y, int d0, int rope, const float4& cs, const float4& sn, float sign) {
    // explicit fused multiply-adds, no contraction left to the compiler: the prep kernels and the
    // projection epilogues compile this in different code and must round alike
#pragma clang fp contract(off)
    const int half = rope >> 1;
    const bool rot = d0 < rope, first = d0 < half;
    const int lane = threadIdx.x & 63;
    const int src = rot ? (first ? lane + (half >> 2) : lane - (half >> 2)) : lane;
    const float4 p = make_float4(__shfl(y.x, src, 64), __shfl(y.y, src, 64), __shfl(y.z, src, 64), __shfl(y.w, src, 64));
    if (!rot) return;
    const float ys[4] = {y.x, y.y, y.z, y.w}, ps[4] = {p.x, p.y, p.z, p.w};
    const float cc[4] = {cs.x, cs.y, cs.z, cs.w}, ss[4] = {sign * sn.x, sign * sn.y, sign * sn.z, sign * sn.w};
    float o[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
        o[u] = first ? __builtin_fmaf(ys[u], cc[u], -(ps[u] * ss[u])) : __builtin_fmaf(ps[u], ss[u], ys[u] * cc[u]);
    y = make_float4(o[0], o[1], o[2], o[3]);
}

// The attention backward's row dot over a head, this lane's share: y . o for four f32 values y and
// four bf16 values o, in a fixed order (one product, then three fused multiply-adds). The separate
// dot kernel and the dX product's epilogue both sum a head's 16 shares with group16_sum, so the two
// paths give the same bits.
__device__ inline float dot4_bf16(const float4& y, uint2 o) {
#pragma clang fp contract(off)
    typedef __bf16 b4 __attribute__((__vector_size__(4 * sizeof(__bf16))));
    const b4 b = __builtin_bit_cast(b4, o);
    float s = y.x * (float)b[0];
    s = __builtin_fmaf(y.y, (float)b[1], s);
    s = __builtin_fmaf(y.z, (float)b[2], s);
    return __builtin_fmaf(y.w, (float)b[3], s);
}

// The FFN SwiGLU backward of four columns (src/dit.h:259-264): g = val * glu * s(glu) with the
// sigmoid s(z) = 1 / (1 + e^-z) on the library exp, so d val = d * glu * s and d glu = d * val *
// (s + glu * s * (1 - s)); no contraction. The block's swiglu_bwd kernel and the FFN
// down-projection's dX epilogue both compute through this function and store_du4.
__device__ inline void swiglu_bwd4(const float4& val, const float4& glu, const float4& d, float4& dv, float4& dgl) {
#pragma clang fp contract(off)
    const float vs[4] = {val.x, val.y, val.z, val.w}, gs[4] = {glu.x, glu.y, glu.z, glu.w};
    const float ds[4] = {d.x, d.y, d.z, d.w};
    float a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const float sg = 1.0f / (1.0f + expf(-gs[u]));
        a[u] = ds[u] * gs[u] * sg;
        b[u] = ds[u] * vs[u] * (sg + gs[u] * sg * (1.0f - sg));
    }
    dv = make_float4(a[0], a[1], a[2], a[3]);
    dgl = make_float4(b[0], b[1], b[2], b[3]);
}
// bf16(v (.) scale[c .. c + 3]) (scale null: v) at p: an adapted linear's dU as its producer writes it
__device__ inline void store_du4(__bf16* p, float4 v, const float* scale, int64_t c) {
    if (scale) {
        const float4 s = *reinterpret_cast<const float4*>(scale + c);
        v = make_float4(v.x * s.x, v.y * s.y, v.z * s.z, v.w * s.w);
    }
    const __bf16 b[4] = {(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
    *reinterpret_cast<uint2*>(p) = __builtin_bit_cast(uint2, b);
}
// four bf16 values as floats
__device__ inline float4 bf16x4_to_f4(uint2 u) {
    typedef __bf16 b4 __attribute__((__vector_size__(4 * sizeof(__bf16))));
    const b4 b = __builtin_bit_cast(b4, u);
    return make_float4((float)b[0], (float)b[1], (float)b[2], (float)b[3]);
}

// y: this lane's four values of the head as the projection produced them. Normalises them in
// place with the gain gm (y * r * g, r = 1 / sqrt(mean(y^2) + eps) over the head, on the hardware
// reciprocal square root), rotates them when rope is set, and returns r.
__device__ inline float head_norm_rope4(float4& y, const float4& gm, bool rope, int d0, int rope_dims, float eps,
                                        const float4& cs, const float4& sn) {
#pragma clang fp contract(off)   // as in rope4_cs: every fused multiply-add written out
    const float ss = __builtin_fmaf(y.w, y.w, __builtin_fmaf(y.z, y.z, __builtin_fmaf(y.y, y.y, y.x * y.x)));
    const float r = __builtin_amdgcn_rsqf(group16_sum(ss) / kHeadDim + eps);
    y = make_float4(y.x * r * gm.x, y.y * r * gm.y, y.z * r * gm.z, y.w * r * gm.w);
    if (rope) rope4_cs(y, d0, rope_dims, cs, sn, 1.0f);
    return r;
}

}  // namespace sa3k
