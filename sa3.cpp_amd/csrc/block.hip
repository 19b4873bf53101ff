// One DiT block forward and backward on the GPU (dit_block, src/dit.h:164-266, autodiff_safe).
//
// The block is the seven adapted linears (lora.hip), the two differential attentions (attn.hip)
// and the element-wise / row-wise ops between them, which are the kernels of this file:
//   norm_fwd/bwd     rms_norm * gamma (+ adaLN modulation h*(1+sc)+sh)       (src/nn.h:40-42, dit.h:177-185)
//   prep_fwd/bwd     per-head rms q/k-norm + partial NEOX RoPE, head-major re-layout
//                                                                            (src/dit.h:194-217, nn.h:53-59)
//   gate_res         x + y * sigmoid(1 - g)                                  (src/dit.h:186-193, 223, 265)
//   swiglu           val * silu(glu)                                         (src/dit.h:259-263)
//   colred           per-sample column sums of the modulation/gate gradients (d gcond)
// Batch-major tokens: x is [B][S][dim], S = memory tokens + latent frames, RoPE position = index
// in S (src/train_loop.h:229-230). The backward of a block consumes the activations its own most
// recent forward left in the workspace: the stack runner either keeps one workspace per block, or
// recomputes block l into a shared one right before its backward (the gradient-checkpointed
// schedule of src/train_ckpt.h:386-431).
#include "block.h"
#include "headprep.h"
#include "lora.h"

#include <cmath>
#include <vector>

using namespace sa3k;

// attn.hip
namespace sa3k {
void attn_forward(sa3k_ctx*, const bf16*, const bf16*, const bf16*, const bf16*, const bf16*, int, int, int, int, int,
                  float, bf16*, bf16*, bf16*, float*, float*);
void attn_backward(sa3k_ctx*, const bf16*, const bf16*, const bf16*, const bf16*, const bf16*, const bf16*,
                   const bf16*, const float*, const float*, const float*, int, int, int, int, int, float, bf16*,
                   float*, float*, float*, float*, float*, float*, float*, bool);
}

namespace {

constexpr int kThreads = 256;
constexpr int HD = 64;
constexpr int NT = 7;   // adapted linears per block

// call a C-ABI entry from inside another entry point: rethrow its failure
void chk(sa3k_ctx* ctx, int rc) {
    if (rc != SA3K_OK) sa3k_throw(rc, ctx->last_error);
}

template <class T>
T* dalloc(size_t n) {
    void* p = nullptr;
    SA3K_HIP(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)));
    return static_cast<T*>(p);
}

__device__ inline float sigmoidf_(float z) { return 1.0f / (1.0f + expf(-z)); }

// ---------------------------------------------------------------- modulation vector
// modv[b][k][c] = ssg[k*dim + c] + gcond[b][k*dim + c]   (src/dit.h:174)
__global__ void modv_kernel(const float* __restrict__ ssg, const float* __restrict__ gcond, int64_t n, int per,
                            float* __restrict__ modv) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) modv[i] = ssg[i % per] + gcond[i];
}

// ---------------------------------------------------------------- row kernels
// One wave per token row; lane l keeps the columns 4 (l + 64 k), k < V, of the row in registers as
// float4 (dim % 4 == 0, dim <= 256 V), so every row is read from memory once.
typedef __bf16 bf16x4 __attribute__((__vector_size__(4 * sizeof(__bf16))));

__device__ inline float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ inline float4 ld4b(const bf16* p) {
    const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
    return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
}
__device__ inline float4 ldx4(const float* p) { return ld4(p); }
__device__ inline float4 ldx4(const bf16* p) { return ld4b(p); }
// An adapted linear's dU = bf16(scale (.) dY) for four consecutive output columns c..c+3 (scale
// null: 1), written by the kernel that produces dY instead of dY itself (lin_du / lin_backward_du)
__device__ inline void st_du4(bf16* p, float4 v, const float* scale, int64_t c) {
    if (scale) {
        const float4 s = ld4(scale + c);
        v = make_float4(v.x * s.x, v.y * s.y, v.z * s.z, v.w * s.w);
    }
    const bf16 b[4] = {(bf16)v.x, (bf16)v.y, (bf16)v.z, (bf16)v.w};
    *reinterpret_cast<uint2*>(p) = __builtin_bit_cast(uint2, b);
}
__device__ inline void st4(float* p, const float4& v) { *reinterpret_cast<float4*>(p) = v; }
__device__ inline void st4(bf16* p, const float4& v) {
    const bf16x4 b = {(bf16)v.x, (bf16)v.y, (bf16)v.z, (bf16)v.w};
    *reinterpret_cast<bf16x4*>(p) = b;
}
__device__ inline float dot4(const float4& a, const float4& b) { return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w; }
__device__ inline float wave_sum(float v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
// apply f to the four components
template <class F>
__device__ inline float4 map4(const float4& a, const float4& b, F f) {
    return make_float4(f(a.x, b.x), f(a.y, b.y), f(a.z, b.z), f(a.w, b.w));
}

// Residual + rms norm (+ modulation), one wave per row:
//   xr = x + y * sigmoid(1 - g_b)  (g_part >= 0)  |  x + y  (g_part < 0)  |  x  (y null);  xo = xr
//   h  = xr * rstd * gamma [* (1 + sc) + sh]  (sc_part >= 0: modulation parts sc_part, sc_part + 1)
template <int V>
__global__ __launch_bounds__(kThreads) void resnorm_fwd_kernel(const float* __restrict__ x, const float* __restrict__ y,
                                                               int g_part, float* __restrict__ xo,
                                                               const float* __restrict__ gamma,
                                                               const float* __restrict__ modv, int sc_part, int S,
                                                               int dim, int rows, float eps, bf16* __restrict__ h,
                                                               float* __restrict__ rstd) {
    const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int64_t base = (int64_t)row * dim;
    const float* mv = modv ? modv + (int64_t)(row / S) * 6 * dim : nullptr;
    float4 v[V];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
        const int c = 4 * (lane + 64 * k);
        v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c < dim) v[k] = ld4(x + base + c);
    }
    if (y) {
#pragma unroll
        for (int k = 0; k < V; ++k) {
            const int c = 4 * (lane + 64 * k);
            if (c >= dim) continue;
            const float4 yv = ld4(y + base + c);
            if (g_part >= 0) {
                const float4 g = ld4(mv + g_part * dim + c);
                v[k] = make_float4(v[k].x + yv.x * sigmoidf_(1.0f - g.x), v[k].y + yv.y * sigmoidf_(1.0f - g.y),
                                   v[k].z + yv.z * sigmoidf_(1.0f - g.z), v[k].w + yv.w * sigmoidf_(1.0f - g.w));
            } else {
                v[k] = map4(v[k], yv, [](float a, float b) { return a + b; });
            }
            st4(xo + base + c, v[k]);
        }
    }
    // the norm weights and modulation rows are loaded before the row sum, not after it
    float4 gw[V], sc[V], sh[V];
#pragma unroll
    for (int k = 0; k < V; ++k) {
        const int c = 4 * (lane + 64 * k);
        gw[k] = sc[k] = sh[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c >= dim) continue;
        gw[k] = ld4(gamma + c);
        if (sc_part >= 0) {
            sc[k] = ld4(mv + sc_part * dim + c);
            sh[k] = ld4(mv + (sc_part + 1) * dim + c);
        }
    }
#pragma unroll
    for (int k = 0; k < V; ++k) ss += dot4(v[k], v[k]);
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / dim + eps);
    if (lane == 0) rstd[row] = r;
#pragma unroll
    for (int k = 0; k < V; ++k) {
        const int c = 4 * (lane + 64 * k);
        if (c >= dim) continue;
        float4 o = map4(v[k], gw[k], [r](float a, float g) { return a * r * g; });
        if (sc_part >= 0) {
            o = map4(o, sc[k], [](float a, float s) { return a * (1.0f + s); });
            o = map4(o, sh[k], [](float a, float s) { return a + s; });
        }
        st4(h + base + c, o);
    }
}

// rms norm backward, one wave per row:
//   dn = dh * (1 + sc) (sc_part >= 0) or dh;  dx = dres + rstd * dn * gamma - rstd^3 * x * <dn gamma, x> / dim
//   dgated = dx * sigmoid(1 - g_b) when g_part >= 0 (the gradient of the gated branch that produced x)
// dres is the residual branch's gradient.
template <int V>
__global__ __launch_bounds__(kThreads) void norm_bwd_kernel(const float* __restrict__ dh, const float* __restrict__ x,
                                                            const float* __restrict__ rstd,
                                                            const float* __restrict__ gamma,
                                                            const float* __restrict__ modv, int sc_part, int S, int dim,
                                                            int rows, const float* __restrict__ dres,
                                                            float* __restrict__ dx, int g_part,
                                                            float* __restrict__ dgated, bf16* __restrict__ du_x,
                                                            const float* __restrict__ dsc_x,
                                                            bf16* __restrict__ du_g, const float* __restrict__ dsc_g) {
    const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int64_t base = (int64_t)row * dim;
    const float* mv = modv ? modv + (int64_t)(row / S) * 6 * dim : nullptr;
    const float r = rstd[row];
    // the residual gradient is loaded with the row's other operands (one memory round trip)
    float4 dg[V], xv[V], dr[V];
    float dot = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
        const int c = 4 * (lane + 64 * k);
        dg[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        xv[k] = dg[k];
        dr[k] = dg[k];
        if (c < dim) {
            dg[k] = ld4(dh + base + c);
            xv[k] = ld4(x + base + c);
            dr[k] = ld4(dres + base + c);
        }
    }
#pragma unroll
    for (int k = 0; k < V; ++k) {
        const int c = 4 * (lane + 64 * k);
        if (c >= dim) continue;
        if (sc_part >= 0) dg[k] = map4(dg[k], ld4(mv + sc_part * dim + c), [](float d, float s) { return d * (1.0f + s); });
        dg[k] = map4(dg[k], ld4(gamma + c), [](float d, float g) { return d * g; });
        dot += dot4(dg[k], xv[k]);
    }
    dot = wave_sum(dot);
    const float k3 = r * r * r * dot / dim;
#pragma unroll
    for (int k = 0; k < V; ++k) {
        const int c = 4 * (lane + 64 * k);
        if (c >= dim) continue;
        const float4 t = map4(dg[k], xv[k], [r, k3](float d, float xx) { return r * d - k3 * xx; });
        const float4 o = map4(dr[k], t, [](float a, float b) { return a + b; });
        st4(dx + base + c, o);
        if (du_x) st_du4(du_x + base + c, o, dsc_x, c);
        if (g_part >= 0) {
            const float4 gd = map4(o, ld4(mv + g_part * dim + c), [](float d, float g) { return d * sigmoidf_(1.0f - g); });
            if (du_g) st_du4(du_g + base + c, gd, dsc_g, c);
            else st4(dgated + base + c, gd);
        }
    }
}

// Column partial sums per sample over a chunk of rows. mode 0 (norm modulation):
//   p0 = sum dh * x * rstd * gamma (d sc),  p1 = sum dh (d sh)
// mode 1 (gate g, s = sigmoid(1 - g)):  p0 = -sum dout * y * s (1 - s)
// part layout [B][nchunk][2][dim]. With counters, the last chunk of a (column block, sample) to
// arrive adds the chunk sums, in chunk order, into dssg (see colred_sum_kernel); else that kernel
// does it.
__global__ __launch_bounds__(kThreads) void colred_kernel(int mode, const float* __restrict__ a,
                                                          const float* __restrict__ x, const float* __restrict__ rstd,
                                                          const float* __restrict__ gamma, const float* __restrict__ modv,
                                                          int g_part, int S, int dim, int chunk, float* __restrict__ part,
                                                          int part0, float* __restrict__ dssg, int* __restrict__ counters) {
    const int c = blockIdx.x * kThreads + threadIdx.x;
    const int ch = blockIdx.y, b = blockIdx.z, nch = gridDim.y;
    const bool ok = c < dim;
    const int t0 = ch * chunk, t1 = min(S, t0 + chunk);
    float p0 = 0.f, p1 = 0.f;
    if (ok) {
        const float gm = mode == 0 ? gamma[c] : 0.f;
        int t = t0;
        for (; t + 4 <= t1; t += 4) {   // four independent rows in flight
            float av[4], xv[4], rs[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t n = (int64_t)b * S + t + u;
                av[u] = a[n * dim + c];
                xv[u] = x[n * dim + c];
                rs[u] = mode == 0 ? rstd[n] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (mode == 0) {
                    p0 += av[u] * xv[u] * rs[u] * gm;
                    p1 += av[u];
                } else {
                    p0 += av[u] * xv[u];
                }
            }
        }
        for (; t < t1; ++t) {
            const int64_t n = (int64_t)b * S + t;
            const float av = a[n * dim + c];
            if (mode == 0) {
                p0 += av * x[n * dim + c] * rstd[n] * gm;
                p1 += av;
            } else {
                p0 += av * x[n * dim + c];
            }
        }
        if (mode == 1) {
            const float s = sigmoidf_(1.0f - modv[((int64_t)b * 6 + g_part) * dim + c]);
            p0 *= -s * (1.0f - s);
        }
        float* o = part + (((int64_t)b * nch + ch) * 2) * dim;
        if (counters) {   // read back by the last chunk to arrive in this launch
            st_coherent(o + c, p0);
            st_coherent(o + dim + c, p1);
        } else {
            o[c] = p0;
            o[dim + c] = p1;
        }
    }
    if (!counters) return;
    __shared__ int s_last;
    if (!arrive_last(&counters[blockIdx.z * gridDim.x + blockIdx.x], nch, &s_last)) return;
    if (ok) {
        // chunk sums in chunk order (as colred_sum_kernel adds them)
        const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
            part, (short)0, (int)((int64_t)gridDim.z * nch * 2 * dim * 4), 0x00020000);
        const uint32_t base = (uint32_t)(((int64_t)b * nch * 2 * dim + c) * 4);
        const uint32_t off[2] = {base, base + (uint32_t)dim * 4u};
        float sum[2];
        coherent_split_sums(rp, off, (uint32_t)(2 * dim * 4), nch, sum);
        dssg[((int64_t)b * 6 + part0) * dim + c] += sum[0];
        if (mode == 0) dssg[((int64_t)b * 6 + part0 + 1) * dim + c] += sum[1];
    }
}

// dssg[b][part0][c] += sum_ch part[b][ch][0][c]; (mode 0) dssg[b][part0+1][c] += sum part[..][1][c]
__global__ __launch_bounds__(kThreads) void colred_sum_kernel(const float* __restrict__ part, int nch, int dim, int B,
                                                              int part0, int two, float* __restrict__ dssg) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= (int64_t)B * dim) return;
    const int b = (int)(i / dim), c = (int)(i % dim);
    float s0 = 0.f, s1 = 0.f;
    for (int ch = 0; ch < nch; ++ch) {
        const float* o = part + (((int64_t)b * nch + ch) * 2) * dim;
        s0 += o[c];
        s1 += o[dim + c];
    }
    dssg[((int64_t)b * 6 + part0) * dim + c] += s0;
    if (two) dssg[((int64_t)b * 6 + part0 + 1) * dim + c] += s1;
}

// ---------------------------------------------------------------- gate, swiglu (4 elements per thread)
// out = x + y * sigmoid(1 - g_b); n4 = rows * dim / 4 (< 2^31)
__global__ void gate_res_kernel(const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ modv,
                                int g_part, int S, int dim, int n4, float* __restrict__ out) {
    const int i4 = blockIdx.x * kThreads + threadIdx.x;
    if (i4 >= n4) return;
    const unsigned e = 4u * (unsigned)i4, row = e / (unsigned)dim, c = e - row * (unsigned)dim;
    const float4 g = ld4(modv + ((int64_t)(row / (unsigned)S) * 6 + g_part) * dim + c);
    const float4 xv = ld4(x + e), yv = ld4(y + e);
    st4(out + e, make_float4(xv.x + yv.x * sigmoidf_(1.0f - g.x), xv.y + yv.y * sigmoidf_(1.0f - g.y),
                             xv.z + yv.z * sigmoidf_(1.0f - g.z), xv.w + yv.w * sigmoidf_(1.0f - g.w)));
}

// dy = dout * sigmoid(1 - g_b) (du: written as the consuming linear's dU); n4 = rows * dim / 4 (< 2^31)
__global__ void gate_bwd_kernel(const float* __restrict__ dout, const float* __restrict__ modv, int g_part, int S, int dim,
                                int n4, float* __restrict__ dy, bf16* __restrict__ du, const float* __restrict__ dsc) {
    const int i4 = blockIdx.x * kThreads + threadIdx.x;
    if (i4 >= n4) return;
    const unsigned e = 4u * (unsigned)i4, row = e / (unsigned)dim, c = e - row * (unsigned)dim;
    const float4 g = ld4(modv + ((int64_t)(row / (unsigned)S) * 6 + g_part) * dim + c);
    const float4 v = map4(ld4(dout + e), g, [](float d, float gg) { return d * sigmoidf_(1.0f - gg); });
    if (du) st_du4(du + e, v, dsc, c);
    else st4(dy + e, v);
}

// g[n][c] = F[n][c] * silu(F[n][I + c]); n4 = rows * I / 4 (< 2^31)
__global__ void swiglu_fwd_kernel(const float* __restrict__ F, int I, int n4, bf16* __restrict__ g) {
    const int i4 = blockIdx.x * kThreads + threadIdx.x;
    if (i4 >= n4) return;
    const unsigned e = 4u * (unsigned)i4, row = e / (unsigned)I, c = e - row * (unsigned)I;
    const float* f = F + (int64_t)row * 2 * I + c;
    st4(g + e, map4(ld4(f), ld4(f + I), [](float val, float glu) { return val * glu * swiglu_sigmoid(glu); }));
}

// dF from F or its bf16 copy (du: written as the FFN up-projection's dU, scale over its 2I columns)
template <class FT>
__global__ void swiglu_bwd_kernel(const float* __restrict__ dg, const FT* __restrict__ F, int I, int n4,
                                  float* __restrict__ dF, bf16* __restrict__ du, const float* __restrict__ dsc) {
    const int i4 = blockIdx.x * kThreads + threadIdx.x;
    if (i4 >= n4) return;
    const unsigned e = 4u * (unsigned)i4, row = e / (unsigned)I, c = e - row * (unsigned)I;
    const int64_t o = (int64_t)row * 2 * I + c;
    const float4 val = ldx4(F + o), glu = ldx4(F + o + I), d = ld4(dg + e);
    float4 dv, dgl;
    swiglu_bwd4(val, glu, d, dv, dgl);   // the same function as the down-projection's dX epilogue
    if (du) {
        store_du4(du + o, dv, dsc, c);
        store_du4(du + o + I, dgl, dsc, (int64_t)I + c);
    } else {
        st4(dF + o, dv);
        st4(dF + o + I, dgl);
    }
}

// ---------------------------------------------------------------- inpaint local add (src/dit.h:244-254)
// y[b][S - T + t] += le[b][t] (the T latent rows of each sample; the memory rows get nothing), and
// its backward: dle[b][t] = dx[b][S - T + t]; 4 columns per thread (dim % 4 == 0)
__global__ void local_add_kernel(const float* __restrict__ le, int S, int T, int dim, int n4, float* __restrict__ y) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n4) return;
    const int q = dim / 4, row = i / q, b = row / T, t = row - b * T;
    float4* dst = reinterpret_cast<float4*>(y + ((int64_t)b * S + (S - T) + t) * dim) + (i - row * q);
    const float4 a = reinterpret_cast<const float4*>(le)[i], c = *dst;
    *dst = make_float4(c.x + a.x, c.y + a.y, c.z + a.z, c.w + a.w);
}

__global__ void local_grad_kernel(const float* __restrict__ dx, int S, int T, int dim, int n4, float* __restrict__ dle) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n4) return;
    const int q = dim / 4, row = i / q, b = row / T, t = row - b * T;
    reinterpret_cast<float4*>(dle)[i] =
        reinterpret_cast<const float4*>(dx + ((int64_t)b * S + (S - T) + t) * dim)[i - row * q];
}

// ---------------------------------------------------------------- q/k-norm + RoPE prep
// RoPE table of one sequence length: tab[t][i] = cos(theta), tab[t][half + i] = sin(theta),
// theta = t * base^(-2i/rope), i < half = rope/2 (pairs (i, i + half) of NEOX rotation)
__global__ void rope_table_kernel(int S, int rope, float base, float* __restrict__ tab) {
    const int half = rope >> 1;
    const int idx = blockIdx.x * kThreads + threadIdx.x;
    if (idx >= S * half) return;
    const int t = idx / half, i = idx - t * half;
    const float th = (float)t * powf(base, -2.0f * (float)i / (float)rope);
    float sn, cs;
    sincosf(th, &sn, &cs);
    tab[t * rope + i] = cs;
    tab[t * rope + half + i] = sn;
}

struct PrepPart {
    bf16* out;            // [B*H][Sx][64]
    const float* gamma;   // [64]; null: plain copy (v)
    int rope;
};
struct PrepArgs {
    const float* in;      // [B*Sx][ldin] (parts*dim used)
    int parts, Sx, H, dim, rope_dims;
    float eps;
    const float* tab;     // RoPE table [Sx][rope_dims] (parts with rope only)
    PrepPart p[5];
    float* rstd;          // [B*Sx][H][parts]
    int64_t ldin;         // row stride of in (parts*dim when 0)
};

// items = rows * H (< 2^31); every part's loads are issued before any is used
__global__ __launch_bounds__(kThreads) void prep_fwd_kernel(PrepArgs a, int items) {
    const int item = blockIdx.x * (kThreads / 16) + (threadIdx.x >> 4);
    if (item >= items) return;   // whole 16-lane groups leave together
    const int d0 = 4 * (threadIdx.x & 15);
    const int row = item / a.H, h = item - row * a.H;
    const int b = row / a.Sx, t = row - b * a.Sx;
    const int64_t ho = (((int64_t)b * a.H + h) * a.Sx + t) * HD + d0;
    const float* src = a.in + (int64_t)row * (a.ldin ? a.ldin : (int64_t)a.parts * a.dim) + h * HD + d0;
    // every load (inputs, norm weights, the token's RoPE row) before the first store, so the row
    // costs one memory round trip
    float4 x[5], gm[5], cs, sn;
    bool any_rope = false;
#pragma unroll
    for (int k = 0; k < 5; ++k) {
        if (k >= a.parts) break;
        x[k] = ld4(src + (int64_t)k * a.dim);
        gm[k] = a.p[k].gamma ? ld4(a.p[k].gamma + d0) : make_float4(0.f, 0.f, 0.f, 0.f);
        any_rope |= a.p[k].gamma && a.p[k].rope;
    }
    if (any_rope) rope_tab4(d0, a.rope_dims, a.tab + (int64_t)t * a.rope_dims, cs, sn);
#pragma unroll
    for (int k = 0; k < 5; ++k) {
        if (k >= a.parts) break;
        float4 y = x[k];
        if (a.p[k].gamma) {
            const float r = head_norm_rope4(y, gm[k], a.p[k].rope != 0, d0, a.rope_dims, a.eps, cs, sn);
            if (d0 == 0) a.rstd[(int64_t)item * a.parts + k] = r;
        }
        st4(a.p[k].out + ho, y);
    }
}

struct PrepBwdPart {
    const float* dy;      // [B*H][Sx][64] f32
    const float* gamma;
    int rope;
};
struct PrepBwdArgs {
    const float* in;      // forward input [B*Sx][ldin] (pre-norm values; parts*dim used)
    int parts, Sx, H, dim, rope_dims;
    const float* tab;
    PrepBwdPart p[5];
    const float* rstd;
    float* din;           // [B*Sx][parts*dim]
    bf16* du;             // instead of din: the input projection's dU [B*Sx][parts*dim]
    const float* dsc;     // its column scale (null: 1)
    int64_t ldin;         // row stride of in (parts*dim when 0)
    const bf16* inb;      // instead of in: its bf16 copy [B*Sx][parts*dim]
};

__global__ __launch_bounds__(kThreads) void prep_bwd_kernel(PrepBwdArgs a, int items) {
    const int item = blockIdx.x * (kThreads / 16) + (threadIdx.x >> 4);
    if (item >= items) return;
    const int d0 = 4 * (threadIdx.x & 15);
    const int row = item / a.H, h = item - row * a.H;
    const int b = row / a.Sx, t = row - b * a.Sx;
    const int64_t ho = (((int64_t)b * a.H + h) * a.Sx + t) * HD + d0;
    const int64_t xo = (int64_t)row * a.parts * a.dim + h * HD + d0;
    const int64_t xi = (int64_t)row * (a.ldin ? a.ldin : (int64_t)a.parts * a.dim) + h * HD + d0;
    // every load (gradients, inputs, norm weights and rstd, the token's RoPE row) before the first
    // store, so the row costs one memory round trip
    float4 g[5], x[5], gmv[5], cs, sn;
    float rsv[5];
    bool any_rope = false;
#pragma unroll
    for (int k = 0; k < 5; ++k) {
        if (k >= a.parts) break;
        g[k] = ld4(a.p[k].dy + ho);
        if (a.p[k].gamma) {
            x[k] = a.inb ? ld4b(a.inb + xi + (int64_t)k * a.dim) : ld4(a.in + xi + (int64_t)k * a.dim);
            gmv[k] = ld4(a.p[k].gamma + d0);
            rsv[k] = a.rstd[(int64_t)item * a.parts + k];
            any_rope |= a.p[k].rope != 0;
        }
    }
    if (any_rope) rope_tab4(d0, a.rope_dims, a.tab + (int64_t)t * a.rope_dims, cs, sn);
#pragma unroll
    for (int k = 0; k < 5; ++k) {
        if (k >= a.parts) break;
        float4 gv = g[k];
        if (a.p[k].gamma) {
            if (a.p[k].rope) rope4_cs(gv, d0, a.rope_dims, cs, sn, -1.0f);
            const float4 gm = gmv[k];
            const float r = rsv[k];
            const float dot = group16_sum(dot4(map4(gv, gm, [](float u, float w) { return u * w; }), x[k]));
            const float c3 = r * r * r * dot / HD;
            const float4 gg = map4(gv, gm, [r](float u, float w) { return r * u * w; });
            gv = map4(gg, x[k], [c3](float u, float xx) { return u - c3 * xx; });
        }
        if (a.du) st_du4(a.du + xo + (int64_t)k * a.dim, gv, a.dsc, (int64_t)k * a.dim + h * HD + d0);
        else st4(a.din + xo + (int64_t)k * a.dim, gv);
    }
}

}  // namespace

// ------------------------------------------------------------------------------------ objects
namespace {

void target_dims(const sa3k_block_config& c, int t, int64_t& in, int64_t& out) {
    const int64_t d = c.dim, I = c.inner;
    const int64_t ins[NT] = {d, d, d, d, d, d, I};
    const int64_t outs[NT] = {5 * d, d, 2 * d, 3 * d, d, 2 * I, d};
    in = ins[t];
    out = outs[t];
}

inline unsigned nblk(int64_t n) { return (unsigned)ceil_div(n, kThreads); }
inline unsigned nwave_blk(int64_t items) { return (unsigned)ceil_div(items, kThreads / 64); }
inline unsigned ngroup16_blk(int64_t items) { return (unsigned)ceil_div(items, kThreads / 16); }

// the row kernels keep ceil(dim / 256) float4 per lane
constexpr int kMaxRowV = 8;
template <class F>
void with_row_v(int dim, F&& f) {
    switch (ceil_div(dim, 256)) {
        case 1: f(std::integral_constant<int, 1>{}); break;
        case 2: f(std::integral_constant<int, 2>{}); break;
        case 3: f(std::integral_constant<int, 3>{}); break;
        case 4: f(std::integral_constant<int, 4>{}); break;
        case 5: f(std::integral_constant<int, 5>{}); break;
        case 6: f(std::integral_constant<int, 6>{}); break;
        case 7: f(std::integral_constant<int, 7>{}); break;
        case 8: f(std::integral_constant<int, 8>{}); break;
        default: sa3k_throw(SA3K_ERR_UNSUPPORTED, "dim above 2048");
    }
}

// launch a kernel of this file on the context stream under a profiler scope
template <class... KArgs, class... Args>
void launch(sa3k_ctx* ctx, const char* name, void (*kernel)(KArgs...), dim3 grid, Args&&... args) {
    KernelScope ks(ctx, name);
    launch_k(ctx, true, kernel, grid, dim3(kThreads), 0, std::forward<Args>(args)...);
    SA3K_LAUNCHED();
}

// per-sample column reductions into dssg (deterministic: fixed chunking and summation order); they
// feed nothing else in the block, so they run on the second stream when it is usable (the block
// backward joins it at its end)
void colred(sa3k_ctx* ctx, sa3k_block_ws* w, int mode, const float* a, const float* x, const float* rstd,
            const float* gamma, int g_part, int part0) {
    const bool side = side_usable(ctx);
    if (side) side_fork(ctx);
    OnSide os(ctx, side);
    const int chunk = (int)ceil_div(w->S, w->part_chunks);
    const int64_t ctrs = nblk(w->dim) * (int64_t)w->B;
    int* counters = tn_counters(ctx, ctrs, kFuseColred);
    launch(ctx, "blk_colred", colred_kernel, dim3(nblk(w->dim), (unsigned)w->part_chunks, (unsigned)w->B), mode, a, x,
           rstd, gamma, (const float*)w->modv, g_part, w->S, w->dim, chunk, w->part, part0, w->dssg, counters);
    if (!counters)
        launch(ctx, "blk_colred", colred_sum_kernel, dim3(nblk((int64_t)w->B * w->dim)), (const float*)w->part,
               w->part_chunks, w->dim, w->B, part0, (int)(mode == 0), w->dssg);
}

}  // namespace

namespace sa3k {

void block_free(sa3k_ctx* ctx, sa3k_block* b) {
    if (!b) return;
    for (int t = 0; t < NT; ++t) {
        if (b->L[t]) sa3k_lin_destroy(ctx, b->L[t]);
        if (b->W[t]) sa3k_weight_destroy(ctx, b->W[t]);
        if (b->bias[t]) (void)hipFree(b->bias[t]);
        if (b->bnsq[t]) (void)hipFree(b->bnsq[t]);
    }
    for (float* p : {b->ssg, b->pre_g, b->cross_g, b->ff_g, b->sq_g, b->sk_g, b->cq_g, b->ck_g})
        if (p) (void)hipFree(p);
    delete b;
}

sa3k_block* block_build(sa3k_ctx* ctx, const sa3k_block_config& cfg, int weight_type, const void* const* W,
                        const float* const* bias, const float* const* vecs, int on_device, int rank,
                        int64_t max_tokens, int64_t max_ctx) {
    SA3K_REQUIRE(cfg.head_dim == HD && cfg.dim == cfg.heads * HD, "dim must be heads * 64");
    // the q/k prep keeps 4 dims per lane: rotation pairs (i, i + rope/2) then sit in the same
    // component of two lanes
    SA3K_REQUIRE(cfg.rope_dims > 0 && cfg.rope_dims <= HD && cfg.rope_dims % 8 == 0, "rope_dims must be a multiple of 8");
    SA3K_REQUIRE(cfg.dim <= 256 * kMaxRowV, "dim above 2048");
    SA3K_REQUIRE(cfg.inner > 0 && cfg.inner % 4 == 0 && cfg.window >= 0, "inner / window");
    SA3K_REQUIRE(max_tokens > 0 && max_ctx > 0, "token budgets must be positive");
    sa3k_block* b = new sa3k_block();
    b->cfg = cfg;
    b->rank = rank;
    b->max_tokens = max_tokens;
    b->max_ctx = max_ctx;
    try {
        for (int t = 0; t < NT; ++t) {
            int64_t in, o;
            target_dims(cfg, t, in, o);
            SA3K_REQUIRE(W[t] != nullptr, "missing block weight");
            chk(ctx, sa3k_weight_create(ctx, weight_type, in, o, W[t], on_device, &b->W[t]));
            chk(ctx, sa3k_lin_create(ctx, b->W[t], rank, SA3K_PREC_BF16, t == 3 ? max_ctx : max_tokens, &b->L[t]));
            static const char* const kTags[7] = {"qkv", "out", "cross.q", "cross.kv", "cross.out", "ff.proj", "ff.out"};
            lin_set_tag(b->L[t], kTags[t]);
            b->bnsq[t] = dalloc<float>((size_t)o);
            chk(ctx, sa3k_weight_row_norm_sq(ctx, b->W[t], 1e-12f, b->bnsq[t]));
            if (bias && bias[t]) {
                b->bias[t] = dalloc<float>((size_t)o);
                SA3K_HIP(hipMemcpyAsync(b->bias[t], bias[t], o * 4, hipMemcpyDefault, ctx->stream));
                sa3k_note_main(ctx);
            }
        }
        const size_t dim = cfg.dim;
        const size_t len[8] = {6 * dim, dim, dim, dim, HD, HD, HD, HD};
        float** dst[8] = {&b->ssg, &b->pre_g, &b->cross_g, &b->ff_g, &b->sq_g, &b->sk_g, &b->cq_g, &b->ck_g};
        for (int i = 0; i < 8; ++i) {
            SA3K_REQUIRE(vecs[i] != nullptr, "missing block vector");
            *dst[i] = dalloc<float>(len[i]);
            SA3K_HIP(hipMemcpyAsync(*dst[i], vecs[i], len[i] * 4, hipMemcpyDefault, ctx->stream));
            sa3k_note_main(ctx);
        }
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
    } catch (...) {
        block_free(ctx, b);
        throw;
    }
    return b;
}

void block_ws_free(sa3k_block_ws* w) {
    if (!w) return;
    for (void* p : w->allocs) (void)hipFree(p);
    delete w;
}

sa3k_block_ws* block_ws_build(const sa3k_block_config& cfg, int B, int S, int Ctx, const sa3k_block_ws* share,
                              int act_bf16, size_t* count_bytes) {
    SA3K_REQUIRE(B > 0 && S > 0 && Ctx > 0, "bad workspace shape");
    SA3K_REQUIRE(!share || (share->B == B && share->S == S && share->Ctx == Ctx && share->dim == cfg.dim &&
                            share->inner == cfg.inner && share->H == cfg.heads),
                 "shared scratch comes from a workspace of another shape");
    SA3K_REQUIRE(!share || share->act_bf16 == act_bf16, "shared scratch comes from a workspace of another layout");
    sa3k_block_ws* w = new sa3k_block_ws();
    w->act_bf16 = act_bf16;
    w->B = B; w->S = S; w->Ctx = Ctx; w->dim = cfg.dim; w->H = cfg.heads; w->inner = cfg.inner;
    try {
        const size_t N = (size_t)B * S, NC = (size_t)B * Ctx, D = cfg.dim, I = cfg.inner, H = cfg.heads;
        const size_t BHS = (size_t)B * H * S * HD, BHC = (size_t)B * H * Ctx * HD, BHq = (size_t)B * H * S;
        // count_bytes: only add up the bytes the workspace would allocate (every pointer stays null)
        auto F32 = [&](size_t n) -> float* {
            if (count_bytes) { *count_bytes += n * sizeof(float); return nullptr; }
            float* p = dalloc<float>(n); w->allocs.push_back(p); return p;
        };
        auto B16 = [&](size_t n) -> bf16* {
            if (count_bytes) { *count_bytes += n * sizeof(bf16); return nullptr; }
            bf16* p = dalloc<bf16>(n); w->allocs.push_back(p); return p;
        };
        w->x = nullptr; w->ctxf = nullptr; w->dssg = nullptr;
        w->modv = F32((size_t)B * 6 * D);
        const bool fcopy = (act_bf16 & 1) != 0, qcopy = (act_bf16 & 2) != 0;
        w->rs_a = F32(N); w->h = B16(N * D);
        w->qkvb = qcopy ? B16(N * 5 * D) : nullptr;
        w->qkv = qcopy ? nullptr : F32(N * 5 * D);
        w->q1 = B16(BHS); w->k1 = B16(BHS); w->q2 = B16(BHS); w->k2 = B16(BHS); w->v = B16(BHS);
        w->rq = F32(N * H * 5);
        w->o = B16(N * D); w->o1 = B16(BHS); w->o2 = B16(BHS); w->l1 = F32(BHq); w->l2 = F32(BHq);
        w->y = F32(N * D); w->x1 = F32(N * D); w->rs_c = F32(N); w->hc = B16(N * D);
        w->qfb = qcopy ? B16(N * 2 * D) : nullptr;
        w->qf = qcopy ? nullptr : F32(N * 2 * D);
        w->kv = F32(NC * 3 * D);
        w->cq1 = B16(BHS); w->cq2 = B16(BHS); w->ck1 = B16(BHC); w->ck2 = B16(BHC); w->cv = B16(BHC);
        w->rcq = F32(N * H * 2); w->rck = F32(NC * H * 3);
        w->oc = B16(N * D); w->co1 = B16(BHS); w->co2 = B16(BHS); w->cl1 = F32(BHq); w->cl2 = F32(BHq);
        w->x2 = F32(N * D); w->rs_f = F32(N); w->fin = B16(N * D);
        w->Fb = fcopy ? B16(N * 2 * I) : nullptr;
        w->F = fcopy ? nullptr : F32(N * 2 * I);
        w->g = B16(N * I); w->yf = F32(N * D);
        w->rope_tab = F32((size_t)S * HD);
        w->part_chunks = (int)std::max<int64_t>(1, std::min<int64_t>(32, ceil_div(S, 32)));
        // dfin and dx1 are read by second-stream column reductions that may still run while the next
        // block's backward (resident activations, late join) writes the shared scratch: per workspace
        w->dfin = F32(N * D);
        w->dx1 = F32(N * D);
        // the f32 outputs that only the forward reads: shared scratch like the backward's
        if (qcopy) {
            w->qkv = share ? share->qkv : F32(N * 5 * D);
            w->qf = share ? share->qf : F32(N * 2 * D);
        }
        if (fcopy) w->F = share ? share->F : F32(N * 2 * I);
        if (share) {
            w->yc = share->yc;
            w->dg = share->dg; w->dx2 = share->dx2; w->doc = share->doc; w->dhc = share->dhc;
            w->dob = share->dob; w->dh = share->dh;
            w->dOh = share->dOh; w->dn = share->dn;
            w->dq1 = share->dq1; w->dk1 = share->dk1; w->dq2 = share->dq2; w->dk2 = share->dk2; w->dv = share->dv;
            w->part = share->part;
        } else {
            w->yc = F32(N * D);
            // the adapted linears' output gradients go straight into their dU buffers (lin_du)
            w->dg = F32(N * I); w->dx2 = F32(N * D); w->doc = F32(N * D); w->dhc = F32(N * D);
            w->dob = F32(N * D); w->dh = F32(N * D);
            w->dOh = B16(BHS); w->dn = F32(2 * BHq);
            const size_t BHK = std::max(BHS, BHC);   // dK/dV of self (S keys) and cross (Ctx keys)
            w->dq1 = F32(BHS); w->dk1 = F32(BHK); w->dq2 = F32(BHS); w->dk2 = F32(BHK); w->dv = F32(BHK);
            w->part = F32((size_t)B * w->part_chunks * 2 * D);
        }
    } catch (...) {
        block_ws_free(w);
        throw;
    }
    if (count_bytes) {
        block_ws_free(w);
        return nullptr;
    }
    return w;
}

void block_prepare(sa3k_ctx* ctx, sa3k_block* b, const float* const* A, const float* const* Bm,
                   const float* const* mag, float scale, int dora) {
    SA3K_REQUIRE(b && A && Bm && (!dora || mag), "null adapter arrays");
    for (int t = 0; t < NT; ++t)
        chk(ctx, sa3k_lin_prepare(ctx, b->L[t], A[t], Bm[t], scale, dora, dora ? mag[t] : nullptr,
                                  dora ? b->bnsq[t] : nullptr));
}

}  // namespace sa3k

extern "C" {

SA3K_API int sa3k_block_create(sa3k_ctx* ctx, const sa3k_block_config* cfg, const sa3k_block_weights* wts, int rank,
                               int64_t max_tokens, int64_t max_ctx_tokens, sa3k_block** out) {
    return sa3k_guard(ctx, "sa3k_block_create", [&] {
        SA3K_REQUIRE(cfg && wts && out, "null pointer");
        *out = nullptr;
        const float* vecs[8] = {wts->ssg, wts->pre_g, wts->cross_g, wts->ff_g, wts->sq_g, wts->sk_g, wts->cq_g, wts->ck_g};
        *out = block_build(ctx, *cfg, wts->weight_type, wts->W, wts->bias, vecs, 0, rank, max_tokens, max_ctx_tokens);
    });
}

SA3K_API int sa3k_block_destroy(sa3k_ctx* ctx, sa3k_block* b) {
    return sa3k_guard(ctx, "sa3k_block_destroy", [&] {
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
        block_free(ctx, b);
    });
}

SA3K_API int sa3k_block_base_norm_sq(sa3k_ctx* ctx, const sa3k_block* b, int target, const float** nsq) {
    return sa3k_guard(ctx, "sa3k_block_base_norm_sq", [&] {
        SA3K_REQUIRE(b && nsq && target >= 0 && target < NT, "bad target");
        *nsq = b->bnsq[target];
    });
}

SA3K_API int sa3k_block_ws_create(sa3k_ctx* ctx, const sa3k_block_config* cfg, int B, int S, int Ctx,
                                  sa3k_block_ws** out) {
    return sa3k_guard(ctx, "sa3k_block_ws_create", [&] {
        SA3K_REQUIRE(cfg && out, "null pointer");
        *out = block_ws_build(*cfg, B, S, Ctx, nullptr, ctx->act_bf16);
    });
}

SA3K_API int sa3k_block_ws_destroy(sa3k_ctx* ctx, sa3k_block_ws* w) {
    return sa3k_guard(ctx, "sa3k_block_ws_destroy", [&] {
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
        block_ws_free(w);
    });
}

SA3K_API int sa3k_block_prepare(sa3k_ctx* ctx, sa3k_block* b, const float* const* A, const float* const* Bm,
                                const float* const* mag, float scale, int dora) {
    return sa3k_guard(ctx, "sa3k_block_prepare", [&] { block_prepare(ctx, b, A, Bm, mag, scale, dora); });
}

}  // extern "C"

void sa3k::block_forward(sa3k_ctx* ctx, sa3k_block* b, sa3k_block_ws* w, const float* x, const float* context,
                         const float* gcond, float* out) {
    {
        SA3K_REQUIRE(b && w && x && context && gcond && out, "null pointer");
        SA3K_REQUIRE(w->dim == b->cfg.dim && w->inner == b->cfg.inner, "workspace shape differs from the block");
        const sa3k_block_config& c = b->cfg;
        const int B = w->B, S = w->S, Ctx = w->Ctx, D = c.dim, H = c.heads, I = c.inner;
        const int64_t N = (int64_t)B * S, NC = (int64_t)B * Ctx;
        SA3K_REQUIRE(N <= b->max_tokens && NC <= b->max_ctx, "workspace exceeds the block's token budget");
        const float scale = 1.0f / sqrtf((float)HD);
        w->x = x;
        w->ctxf = context;
        const float* mv = w->modv;
        // the rank products of merged linears (read by this block's backward only) run on the second
        // stream beside the main products; joined at the end unless a caller joins
        const bool join_here = ctx->side_defer == 0;
        const uint64_t forks0 = ctx->side_forks;
        SideDeferScope defer(ctx);
        auto arm = [&] { if (side_usable(ctx)) fork_arm(ctx); };   // the next kernel records the fork
        // element-wise kernels index with 32-bit ints
        SA3K_REQUIRE(N * 2 * I < ((int64_t)1 << 31) && N * H * 5 < ((int64_t)1 << 31), "too many tokens");
        if (w->rope_tab_dims != c.rope_dims || w->rope_tab_base != c.rope_base) {
            launch(ctx, "blk_rope_table", rope_table_kernel, dim3(nblk((int64_t)S * c.rope_dims / 2)), S, c.rope_dims,
                   c.rope_base, w->rope_tab);
            w->rope_tab_dims = c.rope_dims;
            w->rope_tab_base = c.rope_base;
        }
        // xo = x [+ y [* sigmoid(1 - g)]], h = rms_norm(xo) * gamma [* (1 + sc) + sh]
        auto resnorm = [&](const float* xin, const float* yin, int g_part, float* xo, const float* gamma, int sc_part,
                           bf16* h, float* rs) {
            with_row_v(D, [&](auto v) {
                launch(ctx, "blk_norm_fwd", resnorm_fwd_kernel<decltype(v)::value>, dim3(nwave_blk(N)), xin, yin,
                       g_part, xo, gamma, mv, sc_part, S, D, (int)N, c.norm_eps, h, rs);
            });
        };
        launch(ctx, "blk_modv", modv_kernel, dim3(nblk((int64_t)B * 6 * D)), (const float*)b->ssg, gcond,
               (int64_t)B * 6 * D, 6 * D, w->modv);
        // self attention
        arm();
        resnorm(x, nullptr, -1, nullptr, b->pre_g, 0, w->h, w->rs_a);
        // q|k|v|qd|kd heads: normed, rotated and head-major from the projection's epilogue where its
        // tiles allow, else by the prep kernel
        const HeadPrep hs{5, S, H, D, c.rope_dims, c.qk_eps, w->rope_tab, {w->q1, w->k1, w->v, w->q2, w->k2},
                          {b->sq_g, b->sk_g, nullptr, b->sq_g, b->sk_g}, {1, 1, 0, 1, 1}, w->rq};
        if (!lin_forward_headprep(ctx, b->L[0], w->h, N, w->qkv, w->qkvb, hs)) {
            PrepArgs ps{w->qkv, 5, S, H, D, c.rope_dims, c.qk_eps, w->rope_tab,
                        {{w->q1, b->sq_g, 1}, {w->k1, b->sk_g, 1}, {w->v, nullptr, 0}, {w->q2, b->sq_g, 1}, {w->k2, b->sk_g, 1}},
                        w->rq};
            launch(ctx, "blk_prep_fwd", prep_fwd_kernel, dim3(ngroup16_blk(N * H)), ps, (int)(N * H));
        }
        arm();
        attn_forward(ctx, w->q1, w->k1, w->q2, w->k2, w->v, B, H, S, S, c.window, scale, w->o, w->o1, w->o2, w->l1, w->l2);
        chk(ctx, sa3k_lin_forward(ctx, b->L[1], SA3K_TYPE_BF16, w->o, N, nullptr, w->y));
        // cross attention: x1 = x + y * sigmoid(1 - g_a), hc = rms_norm(x1) * cross_g
        arm();
        resnorm(x, w->y, 2, w->x1, b->cross_g, -1, w->hc, w->rs_c);
        const HeadPrep hq{2, S, H, D, c.rope_dims, c.qk_eps, nullptr, {w->cq1, w->cq2}, {b->cq_g, b->cq_g}, {0, 0}, w->rcq};
        const bool q_done = lin_forward_headprep(ctx, b->L[2], w->hc, N, w->qf, w->qfb, hq);
        if (!w->kv_ext) chk(ctx, sa3k_lin_forward(ctx, b->L[3], SA3K_TYPE_F32, context, NC, nullptr, w->kv));
        const float* kv = w->kv_ext ? w->kv_ext : w->kv;
        const int64_t kv_ld = w->kv_ext ? w->kv_ld : 0;
        if (!q_done) {
            PrepArgs pq{w->qf, 2, S, H, D, c.rope_dims, c.qk_eps, nullptr,
                        {{w->cq1, b->cq_g, 0}, {w->cq2, b->cq_g, 0}, {}, {}, {}}, w->rcq};
            launch(ctx, "blk_prep_fwd", prep_fwd_kernel, dim3(ngroup16_blk(N * H)), pq, (int)(N * H));
        }
        PrepArgs pk{kv, 3, Ctx, H, D, c.rope_dims, c.qk_eps, nullptr,
                    {{w->ck1, b->ck_g, 0}, {w->ck2, b->ck_g, 0}, {w->cv, nullptr, 0}, {}, {}}, w->rck, kv_ld};
        launch(ctx, "blk_prep_fwd", prep_fwd_kernel, dim3(ngroup16_blk(NC * H)), pk, (int)(NC * H));
        arm();
        attn_forward(ctx, w->cq1, w->ck1, w->cq2, w->ck2, w->cv, B, H, S, Ctx, 0, scale, w->oc, w->co1, w->co2, w->cl1, w->cl2);
        chk(ctx, sa3k_lin_forward(ctx, b->L[4], SA3K_TYPE_BF16, w->oc, N, nullptr, w->yc));
        if (w->ladd) {   // inpaint local add: yc += [0; le] (x2 below then carries it)
            SA3K_REQUIRE(w->ladd_T > 0 && w->ladd_T <= S, "local conditioning frames exceed the sequence");
            const int n4 = (int)((int64_t)B * w->ladd_T * D / 4);
            launch(ctx, "blk_local", local_add_kernel, dim3(nblk(n4)), w->ladd, S, w->ladd_T, D, n4, w->yc);
        }
        // feed-forward: x2 = x1 + yc, fin = rms_norm(x2) * ff_g * (1 + sc_f) + sh_f
        arm();
        resnorm(w->x1, w->yc, -1, w->x2, b->ff_g, 3, w->fin, w->rs_f);
        // g = val * silu(glu): from the up-projection's epilogue where its tiles allow, else here
        if (!lin_forward_swiglu(ctx, b->L[5], w->fin, N, b->bias[5], w->F, w->Fb, w->g)) {
            arm();
            launch(ctx, "blk_swiglu", swiglu_fwd_kernel, dim3(nblk(N * I / 4)), (const float*)w->F, I, (int)(N * I / 4), w->g);
        }
        chk(ctx, sa3k_lin_forward(ctx, b->L[6], SA3K_TYPE_BF16, w->g, N, b->bias[6], w->yf));
        launch(ctx, "blk_gate", gate_res_kernel, dim3(nblk(N * D / 4)), (const float*)w->x2, (const float*)w->yf, mv, 5,
               S, D, (int)(N * D / 4), out);
        if (join_here) side_join_since(ctx, forks0);
    }
}

void sa3k::block_backward(sa3k_ctx* ctx, sa3k_block* b, sa3k_block_ws* w, const float* dout, float* dx,
                          float* dcontext, float* dgcond, float* const* dA, float* const* dB, float* const* dm,
                          bool late_join) {
    {
        SA3K_REQUIRE(b && w && dout && dx && dcontext && dgcond && dA && dB, "null pointer");
        SA3K_REQUIRE(w->x != nullptr, "backward needs a preceding forward on this workspace");
        const sa3k_block_config& c = b->cfg;
        const int B = w->B, S = w->S, Ctx = w->Ctx, D = c.dim, H = c.heads, I = c.inner;
        const int64_t N = (int64_t)B * S, NC = (int64_t)B * Ctx;
        const float scale = 1.0f / sqrtf((float)HD);
        float* dmt[NT];
        for (int t = 0; t < NT; ++t) dmt[t] = dm ? dm[t] : nullptr;
        const float* mv = w->modv;
        w->dssg = dgcond;   // the column reductions add each of the 6 modulation parts once
        // work forked to the second stream (column reductions, cross K/V projection backward, dA
        // partial sums) reads activations and scratch that the next block reuses: join at the end
        SideDeferScope defer(ctx);
        const int64_t nq = (int64_t)B * H * S;
        // dx = dres + norm backward (dh); dgated = dx * sigmoid(1 - g) when g_part >= 0
        // lx / lg: the linear whose dU is dxo / the gated branch's gradient (written as that dU)
        auto norm_bwd = [&](const float* dh, const float* xin, const float* rs, const float* gamma, int sc_part,
                            const float* dres, float* dxo, int g_part, sa3k_lin* lx, sa3k_lin* lg) {
            with_row_v(D, [&](auto v) {
                launch(ctx, "blk_norm_bwd", norm_bwd_kernel<decltype(v)::value>, dim3(nwave_blk(N)), dh, xin, rs, gamma,
                       mv, sc_part, S, D, (int)N, dres, dxo, g_part, (float*)nullptr, lx ? lin_du(lx) : nullptr,
                       lx ? lin_du_scale(lx) : nullptr, lg ? lin_du(lg) : nullptr, lg ? lin_du_scale(lg) : nullptr);
            });
        };
        // out = x2 + yf * s_f (its kernel records the fork of the column reduction that follows)
        if (side_usable(ctx)) fork_arm(ctx);
        // Each adapted linear's output gradient is written by its producer as the linear's bf16 dU
        // (lin_du), which its backward reads (lin_backward_du): no f32 dY round trip.
        launch(ctx, "blk_gate", gate_bwd_kernel, dim3(nblk(N * D / 4)), dout, mv, 5, S, D, (int)(N * D / 4),
               (float*)nullptr, lin_du(b->L[6]), lin_du_scale(b->L[6]));
        colred(ctx, w, 1, dout, w->yf, nullptr, nullptr, 5, 5);
        // the FFN down-projection's dX product writes the up-projection's dU (the SwiGLU backward)
        // from its epilogue where its tiles allow (epi_fuse bit 3; dG itself is then not written)
        int sw_done = 0;
        DxEpi se;
        if ((ctx->epi_fuse & 8) && w->Fb) {
            se.sb = SwiBwd{w->Fb, lin_du(b->L[5]), lin_du_scale(b->L[5]), I};
            se.done = &sw_done;
        }
        lin_backward_du(ctx, b->L[6], SA3K_TYPE_BF16, w->g, N, w->dg, 0, dA[6], dB[6], dmt[6], &se);
        if (!sw_done) {
            if (w->Fb)
                launch(ctx, "blk_swiglu", swiglu_bwd_kernel<bf16>, dim3(nblk(N * I / 4)), (const float*)w->dg,
                       (const bf16*)w->Fb, I, (int)(N * I / 4), (float*)nullptr, lin_du(b->L[5]),
                       lin_du_scale(b->L[5]));
            else
                launch(ctx, "blk_swiglu", swiglu_bwd_kernel<float>, dim3(nblk(N * I / 4)), (const float*)w->dg,
                       (const float*)w->F, I, (int)(N * I / 4), (float*)nullptr, lin_du(b->L[5]),
                       lin_du_scale(b->L[5]));
        }
        lin_backward_du(ctx, b->L[5], SA3K_TYPE_BF16, w->fin, N, w->dfin, 0, dA[5], dB[5], dmt[5]);
        colred(ctx, w, 0, w->dfin, w->x2, w->rs_f, b->ff_g, 0, 3);
        norm_bwd(w->dfin, w->x2, w->rs_f, b->ff_g, 3, dout, w->dx2, -1, b->L[4], nullptr);
        if (w->dladd) {   // the local add's gradient: the latent rows of dx2
            SA3K_REQUIRE(w->ladd_T > 0 && w->ladd_T <= S, "local conditioning frames exceed the sequence");
            const int n4 = (int)((int64_t)B * w->ladd_T * D / 4);
            launch(ctx, "blk_local", local_grad_kernel, dim3(nblk(n4)), (const float*)w->dx2, S, w->ladd_T, D, n4,
                   w->dladd);
        }
        // x2 = x1 + yc
        // the out-projections' dX products write the attention backward's dOh and row dots from
        // their epilogues where their tiles allow (epi_fuse bit 2; dO itself is then not written)
        int dot_done = 0;
        DxEpi adc;
        if (ctx->epi_fuse & 4) {
            adc.ad = AttnDot{w->co1, w->co2, w->dOh, w->dn, w->dn + nq, H, S};
            adc.done = &dot_done;
        }
        lin_backward_du(ctx, b->L[4], SA3K_TYPE_BF16, w->oc, N, w->doc, 0, dA[4], dB[4], dmt[4], &adc);
        attn_backward(ctx, w->cq1, w->ck1, w->cq2, w->ck2, w->cv, w->co1, w->co2, w->cl1, w->cl2, w->doc, B, H, S, Ctx, 0,
                      scale, w->dOh, w->dn, w->dn + nq, w->dq1, w->dk1, w->dq2, w->dk2, w->dv, dot_done != 0);
        PrepBwdArgs bq{w->qf, 2, S, H, D, c.rope_dims, nullptr,
                       {{w->dq1, b->cq_g, 0}, {w->dq2, b->cq_g, 0}, {}, {}, {}}, w->rcq, nullptr,
                       lin_du(b->L[2]), lin_du_scale(b->L[2]), 0, w->qfb};
        launch(ctx, "blk_prep_bwd", prep_bwd_kernel, dim3(ngroup16_blk(N * H)), bq, (int)(N * H));
        PrepBwdArgs bk{w->kv_ext ? w->kv_ext : w->kv, 3, Ctx, H, D, c.rope_dims, nullptr,
                       {{w->dk1, b->ck_g, 0}, {w->dk2, b->ck_g, 0}, {w->dv, nullptr, 0}, {}, {}}, w->rck, nullptr,
                       lin_du(b->L[3]), lin_du_scale(b->L[3]), w->kv_ext ? w->kv_ld : 0};
        if (side_usable(ctx)) fork_arm(ctx);   // recorded by the next kernel, for the K/V projection
        launch(ctx, "blk_prep_bwd", prep_bwd_kernel, dim3(ngroup16_blk(NC * H)), bk, (int)(NC * H));
        {   // the context K/V projection (Ctx tokens, small kernels) beside the query projection
            const bool side = side_usable(ctx);
            if (side) side_fork(ctx);
            OnSide os(ctx, side);
            lin_backward_du(ctx, b->L[3], SA3K_TYPE_F32, w->ctxf, NC, dcontext, 1, dA[3], dB[3], dmt[3]);
        }
        lin_backward_du(ctx, b->L[2], SA3K_TYPE_BF16, w->hc, N, w->dhc, 0, dA[2], dB[2], dmt[2]);
        // x1 = x + y * s_a: dy = dx1 * s_a comes out of the same pass (which records the fork of
        // the column reduction that follows)
        if (side_usable(ctx)) fork_arm(ctx);
        norm_bwd(w->dhc, w->x1, w->rs_c, b->cross_g, -1, w->dx2, w->dx1, 2, nullptr, b->L[1]);
        colred(ctx, w, 1, w->dx1, w->y, nullptr, nullptr, 2, 2);
        dot_done = 0;
        DxEpi ads;
        if (ctx->epi_fuse & 4) {
            ads.ad = AttnDot{w->o1, w->o2, w->dOh, w->dn, w->dn + nq, H, S};
            ads.done = &dot_done;
        }
        lin_backward_du(ctx, b->L[1], SA3K_TYPE_BF16, w->o, N, w->dob, 0, dA[1], dB[1], dmt[1], &ads);
        attn_backward(ctx, w->q1, w->k1, w->q2, w->k2, w->v, w->o1, w->o2, w->l1, w->l2, w->dob, B, H, S, S, c.window,
                      scale, w->dOh, w->dn, w->dn + nq, w->dq1, w->dk1, w->dq2, w->dk2, w->dv, dot_done != 0);
        PrepBwdArgs bs{w->qkv, 5, S, H, D, c.rope_dims, w->rope_tab,
                       {{w->dq1, b->sq_g, 1}, {w->dk1, b->sk_g, 1}, {w->dv, nullptr, 0}, {w->dq2, b->sq_g, 1}, {w->dk2, b->sk_g, 1}},
                       w->rq, nullptr, lin_du(b->L[0]), lin_du_scale(b->L[0]), 0, w->qkvb};
        launch(ctx, "blk_prep_bwd", prep_bwd_kernel, dim3(ngroup16_blk(N * H)), bs, (int)(N * H));
        // the previous block's last second-stream work (late_join) reads w->dh, written next
        if (ctx->block_tail_pending) {
            SA3K_HIP(hipStreamWaitEvent(ctx->main_stream, ctx->block_tail_ev, 0));
            ctx->block_tail_pending = false;
        }
        lin_backward_du(ctx, b->L[0], SA3K_TYPE_BF16, w->h, N, w->dh, 0, dA[0], dB[0], dmt[0]);
        colred(ctx, w, 0, w->dh, w->x, w->rs_a, b->pre_g, 0, 0);
        norm_bwd(w->dh, w->x, w->rs_a, b->pre_g, 0, w->dx1, dx, -1, nullptr, nullptr);
        if (side_usable(ctx)) {
            if (late_join) {   // the column reduction and dA sums of this block finish beside the next block
                SA3K_HIP(hipEventRecord(ctx->block_tail_ev, ctx->side_stream));
                ctx->block_tail_pending = true;
            } else {
                side_join(ctx);
            }
        }
        w->dssg = nullptr;
    }
}

extern "C" {

SA3K_API int sa3k_block_forward(sa3k_ctx* ctx, sa3k_block* b, sa3k_block_ws* w, const float* x, const float* context,
                                const float* gcond, float* out) {
    return sa3k_guard(ctx, "sa3k_block_forward", [&] { block_forward(ctx, b, w, x, context, gcond, out); });
}

SA3K_API int sa3k_block_backward(sa3k_ctx* ctx, sa3k_block* b, sa3k_block_ws* w, const float* dout, float* dx,
                                 float* dcontext, float* dgcond, float* const* dA, float* const* dB, float* const* dm) {
    return sa3k_guard(ctx, "sa3k_block_backward",
                      [&] { block_backward(ctx, b, w, dout, dx, dcontext, dgcond, dA, dB, dm); });
}

}  // extern "C"
