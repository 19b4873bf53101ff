// Composed adapter chains over a frozen (f32 / f16 / bf16 / Q8_0) base for inference: the
// reference's build_functional_lora (src/lora.h:372-622) and the chain branch of dit_lin
// (src/dit.h:108-117).
//
// Merging adapters 1..M into the base one after another (apply_loras) equals
//     y = c0 (.) (W x) + sum_k s_k B'_k (A_k x),   s_k = (alpha_k / rank_k) * strength_k,
// where walking the chain every dora-rows adapter j multiplies the base coefficient b and the
// coefficients g_k of the residuals k <= j by its row scale d_j = m_j / ||V_j row||, with
//     ||V_j row||^2 = b^2 nsq0 + sum_{k<=j} 2 s_k g_k b T2_k + sum_{k,l<=j} s_k s_l g_k g_l G_kl,
//     nsq0 = sum_in W^2 + in 1e-12,  T2_k = rowsum((W A_k^T) * B_k),  G_kl = rowsum(B_k * (B_l A_l A_k^T)),
// and finally c0 = b and B'_k = g_k (.) B_k. All of it depends on the frozen base and adapters only,
// so it is computed once per chain, in double precision:
//   chain_gram_kernel   the Gram matrix of the stacked adapter A rows (one workgroup per entry);
//   chain_fold_kernel   one workgroup per output row: the row's nsq0 and W A_k^T products with the
//                       base decoded from its stored type, then the chain walk -> c0[o], B'[o][:].
// The forward is two GEMMs: H = X [s_1 A_1; ...; s_M A_M]^T (every residual's rank-r input at once),
// then the base product over the stored weight (bf16 working copy, or f16 / Q8_0 decoded on its way
// into LDS) with c0 applied to its accumulators before the rank segment H [B'_1 .. B'_M]^T is added
// (the GEMM's prescale mode), and the bias. A total rank above one K tile (64) adds the rank term
// as a third GEMM accumulating into the output instead of as the base product's second segment.
#include "lora.h"

#include <cmath>
#include <vector>

using namespace sa3k;

namespace {

constexpr int kThreads = 256;
constexpr int kMaxChain = 32;    // adapters in one chain
constexpr int kMaxRank = 512;    // total rank of the active adapters
constexpr int kSegRank = 64;     // up to this total rank the rank term rides on the base product

struct ChainArgs {
    int n;                       // active adapters
    int R;                       // total rank
    const float* A[kMaxChain];   // [rank][in]
    const float* B[kMaxChain];   // [out][rank]
    const float* mag[kMaxChain]; // [out] (dora)
    int rank[kMaxChain];
    int col0[kMaxChain];         // first stacked row / column of the adapter
    int dora[kMaxChain];
    float scale[kMaxChain];
};

__device__ inline int adapter_of(const ChainArgs& c, int a) {
    int k = 0;
    while (k + 1 < c.n && a >= c.col0[k + 1]) ++k;
    return k;
}

__device__ inline const float* a_row(const ChainArgs& c, int a, int64_t in) {
    const int k = adapter_of(c, a);
    return c.A[k] + (int64_t)(a - c.col0[k]) * in;
}

// decoded element i of row o of the forward layout, from the stored type
__device__ inline float w_elem(const sa3k_weight& w, int64_t o, int64_t i) {
    const int64_t idx = o * w.in + i;
    switch (w.type) {
        case SA3K_TYPE_F32: return static_cast<const float*>(w.w)[idx];
        case SA3K_TYPE_F16: return (float)static_cast<const _Float16*>(w.w)[idx];
        case SA3K_TYPE_BF16: return (float)static_cast<const bf16*>(w.w)[idx];
        default:   // Q8_0 planes: f16 scale per 32 inputs times the int8 quant
            return (float)static_cast<const _Float16*>(w.ws)[o * (w.in / 32) + (i >> 5)] *
                   (float)static_cast<const int8_t*>(w.w)[idx];
    }
}

__device__ inline double block_sum(double v, double* sh) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    double s = 0.0;
    for (int w = 0; w < kThreads / 64; ++w) s += sh[w];
    return s;
}

// gram[a][b] = A_row(a) . A_row(b) over the stacked rows, double
__global__ __launch_bounds__(kThreads) void chain_gram_kernel(ChainArgs c, int64_t in, double* __restrict__ gram) {
    __shared__ double sh[kThreads / 64];
    const int a = blockIdx.x / c.R, b = blockIdx.x % c.R;
    const float* ra = a_row(c, a, in);
    const float* rb = a_row(c, b, in);
    double acc = 0.0;
    for (int64_t i = threadIdx.x; i < in; i += kThreads) acc += (double)ra[i] * rb[i];
    const double s = block_sum(acc, sh);
    if (threadIdx.x == 0) gram[blockIdx.x] = s;
}

// Ac [Rp][in] = bf16(s_k A_k) stacked, zero rows past R
__global__ __launch_bounds__(kThreads) void chain_stack_a_kernel(ChainArgs c, int64_t in, int Rp, bf16* __restrict__ Ac) {
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (idx >= (int64_t)Rp * in) return;
    const int a = (int)(idx / in);
    const int64_t i = idx - (int64_t)a * in;
    float v = 0.0f;
    if (a < c.R) {
        const int k = adapter_of(c, a);
        v = c.scale[k] * c.A[k][(int64_t)(a - c.col0[k]) * in + i];
    }
    Ac[idx] = (bf16)v;
}

// One workgroup per output row o: nsq0, P[a] = W[o] . A_row(a), the per-adapter terms T2_k and
// G_kl (one thread each), then the chain walk (one thread) and the folded row (all threads).
__global__ __launch_bounds__(kThreads) void chain_fold_kernel(sa3k_weight w, ChainArgs c, const double* __restrict__ gram,
                                                              int Rp, float* __restrict__ c0, float* __restrict__ Bp,
                                                              bf16* __restrict__ Bc) {
    __shared__ double sh[kThreads / 64];
    __shared__ double P[kMaxRank];
    __shared__ double T2[kMaxChain], G[kMaxChain][kMaxChain], g[kMaxChain];
    __shared__ double bsh;
    const int64_t o = blockIdx.x, in = w.in;
    double nsq0 = 0.0;
    for (int64_t i = threadIdx.x; i < in; i += kThreads) {
        const double v = w_elem(w, o, i);
        nsq0 += v * v;
    }
    nsq0 = block_sum(nsq0, sh) + (double)in * 1e-12;
    for (int a = 0; a < c.R; ++a) {
        const float* ra = a_row(c, a, in);
        double acc = 0.0;
        for (int64_t i = threadIdx.x; i < in; i += kThreads) acc += (double)w_elem(w, o, i) * ra[i];
        const double s = block_sum(acc, sh);
        if (threadIdx.x == 0) P[a] = s;
    }
    __syncthreads();
    // per-row quantities in double: T2_k = P_k . B_k[o], G_kl = B_k[o] . (gram_kl B_l[o])
    for (int t = threadIdx.x; t < c.n * (c.n + 1); t += kThreads) {
        if (t < c.n) {
            const int k = t;
            double v = 0.0;
            for (int j = 0; j < c.rank[k]; ++j) v += P[c.col0[k] + j] * (double)c.B[k][o * c.rank[k] + j];
            T2[k] = v;
            g[k] = 1.0;
        } else {
            const int k = (t - c.n) / c.n, l = (t - c.n) % c.n;
            double acc = 0.0;
            for (int j = 0; j < c.rank[k]; ++j) {
                const double* gr = gram + (int64_t)(c.col0[k] + j) * c.R + c.col0[l];
                double gb = 0.0;
                for (int i = 0; i < c.rank[l]; ++i) gb += gr[i] * (double)c.B[l][o * c.rank[l] + i];
                acc += (double)c.B[k][o * c.rank[k] + j] * gb;
            }
            G[k][l] = acc;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {   // the walk: each dora-rows adapter rescales the base and every residual so far
        double b = 1.0;
        for (int j = 0; j < c.n; ++j) {
            if (!c.dora[j]) continue;
            double nsq = b * b * nsq0;
            for (int k = 0; k <= j; ++k) nsq += 2.0 * (double)c.scale[k] * g[k] * b * T2[k];
            for (int k = 0; k <= j; ++k)
                for (int l = 0; l <= j; ++l) nsq += (double)c.scale[k] * c.scale[l] * g[k] * g[l] * G[k][l];
            const double d = (double)c.mag[j][o] / sqrt(nsq);
            b *= d;
            for (int k = 0; k <= j; ++k) g[k] *= d;
        }
        bsh = b;
        c0[o] = (float)b;
    }
    __syncthreads();
    for (int a = threadIdx.x; a < Rp; a += kThreads) {
        if (a < c.R) {
            const int k = adapter_of(c, a), j = a - c.col0[k];
            const float v = (float)(g[k] * (double)c.B[k][o * c.rank[k] + j]);
            Bp[o * c.R + a] = v;
            Bc[o * Rp + a] = (bf16)v;
        } else {
            Bc[o * Rp + a] = (bf16)0.0f;
        }
    }
}

__global__ __launch_bounds__(kThreads) void chain_cvt_kernel(const float* __restrict__ x, bf16* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) y[i] = (bf16)x[i];
}

template <class T>
T* dalloc(size_t n) {
    void* p = nullptr;
    SA3K_HIP(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)));
    return static_cast<T*>(p);
}

}  // namespace

struct sa3k_lora_chain {
    const sa3k_weight* W = nullptr;
    int64_t max_tokens = 0;
    int R = 0, Rp = 0;               // total active rank, padded to a multiple of 8
    bool dora = false;               // some active adapter is dora-rows (c0 != 1)
    float* c0 = nullptr;             // [out]
    float* Bp = nullptr;             // [out][R] folded B' (f32)
    bf16* Bc = nullptr;              // [out][Rp] folded B' (bf16, zero columns past R)
    bf16* Ac = nullptr;              // [Rp][in] s_k A_k stacked (bf16, zero rows past R)
    bf16* Xb = nullptr;              // [max_tokens][in] bf16 copy of an f32 input
    bf16* Hc = nullptr;              // [max_tokens][Rp]
};

namespace {

void free_chain(sa3k_lora_chain* c) {
    for (void* p : {(void*)c->c0, (void*)c->Bp, (void*)c->Bc, (void*)c->Ac, (void*)c->Xb, (void*)c->Hc})
        if (p) (void)hipFree(p);
    delete c;
}

}  // namespace

extern "C" {

SA3K_API int sa3k_lora_chain_create(sa3k_ctx* ctx, const sa3k_weight* W, int n_adapters,
                                    const sa3k_chain_adapter* adapters, int64_t max_tokens, sa3k_lora_chain** out) {
    return sa3k_guard(ctx, "sa3k_lora_chain_create", [&] {
        SA3K_REQUIRE(W && out && (n_adapters == 0 || adapters), "null pointer");
        SA3K_REQUIRE(n_adapters >= 0 && n_adapters <= kMaxChain, "a chain holds at most 32 adapters");
        SA3K_REQUIRE(max_tokens > 0, "max_tokens must be positive");
        *out = nullptr;
        ChainArgs a{};
        bool dora = false;
        for (int i = 0; i < n_adapters; ++i) {
            const sa3k_chain_adapter& x = adapters[i];
            SA3K_REQUIRE(x.rank > 0 && x.A && x.B && (!x.dora || x.magnitude), "adapter needs rank > 0, A, B (and magnitude)");
            if (x.strength == 0.0f) continue;   // the identity, as in the merge path
            a.A[a.n] = x.A;
            a.B[a.n] = x.B;
            a.mag[a.n] = x.magnitude;
            a.rank[a.n] = x.rank;
            a.col0[a.n] = a.R;
            a.dora[a.n] = x.dora ? 1 : 0;
            a.scale[a.n] = x.alpha / (float)x.rank * x.strength;
            a.R += x.rank;
            dora = dora || x.dora;
            ++a.n;
        }
        SA3K_REQUIRE(a.R <= kMaxRank, "the active adapters' ranks add up to more than 512");
        sa3k_lora_chain* c = new sa3k_lora_chain();
        c->W = W;
        c->max_tokens = max_tokens;
        c->R = a.R;
        // a rank segment of the base product takes up to one K tile (8-column steps); a longer rank
        // term is its own GEMM, whose K runs in whole 64-column tiles
        c->Rp = a.R <= kSegRank ? (int)ceil_div(a.R, 8) * 8 : (int)ceil_div(a.R, 64) * 64;
        c->dora = dora;
        try {
            const int64_t in = W->in, outd = W->out;
            c->Xb = dalloc<bf16>((size_t)(max_tokens * in));
            if (a.n > 0) {
                c->c0 = dalloc<float>((size_t)outd);
                c->Bp = dalloc<float>((size_t)(outd * a.R));
                c->Bc = dalloc<bf16>((size_t)(outd * c->Rp));
                c->Ac = dalloc<bf16>((size_t)(c->Rp * in));
                c->Hc = dalloc<bf16>((size_t)(max_tokens * c->Rp));
                double* gram = dalloc<double>((size_t)(a.R * a.R));
                {
                    KernelScope ks(ctx, "chain_fold");
                    chain_gram_kernel<<<(unsigned)(a.R * a.R), kThreads, 0, ctx->stream>>>(a, in, gram);
                    SA3K_LAUNCHED();
                    chain_stack_a_kernel<<<(unsigned)ceil_div(c->Rp * in, kThreads), kThreads, 0, ctx->stream>>>(
                        a, in, c->Rp, c->Ac);
                    SA3K_LAUNCHED();
                    chain_fold_kernel<<<(unsigned)outd, kThreads, 0, ctx->stream>>>(*W, a, gram, c->Rp, c->c0, c->Bp, c->Bc);
                    SA3K_LAUNCHED();
                }
                SA3K_HIP(hipStreamSynchronize(ctx->stream));
                SA3K_HIP(hipFree(gram));
            }
        } catch (...) {
            free_chain(c);
            throw;
        }
        *out = c;
    });
}

SA3K_API int sa3k_lora_chain_destroy(sa3k_ctx* ctx, sa3k_lora_chain* chain) {
    return sa3k_guard(ctx, "sa3k_lora_chain_destroy", [&] {
        if (!chain) return;
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
        free_chain(chain);
    });
}

SA3K_API int sa3k_lora_chain_constants(sa3k_ctx* ctx, const sa3k_lora_chain* chain, float* base_scale, float* Bp,
                                       int* total_rank) {
    return sa3k_guard(ctx, "sa3k_lora_chain_constants", [&] {
        SA3K_REQUIRE(chain, "null chain");
        if (total_rank) *total_rank = chain->R;
        if (chain->R == 0) return;
        const int64_t outd = chain->W->out;
        if (base_scale)
            SA3K_HIP(hipMemcpyAsync(base_scale, chain->c0, sizeof(float) * outd, hipMemcpyDeviceToDevice, ctx->stream));
        if (Bp)
            SA3K_HIP(hipMemcpyAsync(Bp, chain->Bp, sizeof(float) * outd * chain->R, hipMemcpyDeviceToDevice, ctx->stream));
        sa3k_note_main(ctx);
    });
}

SA3K_API int sa3k_lora_chain_forward(sa3k_ctx* ctx, sa3k_lora_chain* chain, int x_type, const void* X, int64_t N,
                                     const float* bias, float* Y) {
    return sa3k_guard(ctx, "sa3k_lora_chain_forward", [&] {
        SA3K_REQUIRE(chain && X && Y, "null pointer");
        SA3K_REQUIRE(N > 0 && N <= chain->max_tokens, "token count out of range");
        SA3K_REQUIRE(x_type == SA3K_TYPE_F32 || x_type == SA3K_TYPE_BF16, "X must be f32 or bf16");
        const sa3k_weight* W = chain->W;
        const void* xb = X;
        if (x_type == SA3K_TYPE_F32) {
            const int64_t n = N * W->in;
            KernelScope ks(ctx, "chain_cvt_x");
            chain_cvt_kernel<<<(unsigned)ceil_div(n, kThreads), kThreads, 0, ctx->stream>>>(static_cast<const float*>(X),
                                                                                          chain->Xb, n);
            SA3K_LAUNCHED();
            xb = chain->Xb;
        }
        if (chain->R > 0) {   // H = X [s_k A_k]^T for every residual at once
            GemmDesc h;
            h.prec = SA3K_PREC_BF16; h.a_src = SRC_BF16; h.b_src = SRC_BF16;
            h.A = xb; h.lda = W->in; h.B = chain->Ac; h.ldb = W->in;
            h.M = N; h.N = chain->Rp; h.K = W->in;
            h.Cb = chain->Hc; h.ldcb = chain->Rp;
            gemm_run(ctx, h, "chain_h");
        }
        GemmDesc g;
        g.prec = SA3K_PREC_BF16; g.a_src = SRC_BF16;
        weight_fwd_operand(W, g);
        g.A = xb; g.lda = W->in;
        g.M = N; g.N = W->out; g.K = W->in;
        const bool seg = chain->R > 0 && chain->Rp <= kSegRank;
        if (seg) {
            g.A2 = chain->Hc; g.lda2 = chain->Rp; g.B2 = chain->Bc; g.ldb2 = chain->Rp; g.K2 = chain->Rp;
            if (chain->dora) {
                g.colscale = chain->c0;
                g.prescale = 1;
            }
        } else if (chain->R > 0 && chain->dora) {
            g.colscale = chain->c0;   // y = c0 (.) (W x) + bias, the rank term added below
        }
        g.bias = bias;
        g.C = Y; g.ldc = W->out;
        gemm_run(ctx, g, "chain_main");
        if (chain->R > 0 && !seg) {   // y += H [B'_1 .. B'_M]^T
            GemmDesc r;
            r.prec = SA3K_PREC_BF16; r.a_src = SRC_BF16; r.b_src = SRC_BF16;
            r.A = chain->Hc; r.lda = chain->Rp; r.B = chain->Bc; r.ldb = chain->Rp;
            r.M = N; r.N = W->out; r.K = chain->Rp;
            r.C = Y; r.ldc = W->out; r.accumulate = 1;
            gemm_run(ctx, r, "chain_rank");
        }
    });
}

}  // extern "C"
