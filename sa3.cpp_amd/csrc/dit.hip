// C4: the DiT rectified-flow training step on one GPU, device-resident end to end.
//
// Reference: run_train_dit_accumulate_ckpt (src/train_loop.h:309-441) over the segmented graphs of
// src/train_ckpt.h (F: forward storing block boundaries; T: tail + loss + dL/dx_depth; B_l:
// recompute block l and backprop it, in reverse; H: head backward against dL/dx_0 and the summed
// context/gcond gradients), then train_apply_accumulated_adamw (src/train_loop.h:173-211). The
// reference reads every gradient back to the host and sums the shared context/gcond gradients
// there; here gradients accumulate in one flat device arena and never leave the GPU, and the
// fused clip + AdamW (adamw.hip) updates that arena in place.
//
// Activation schedule: with recompute = 1 the checkpointed schedule above (one block workspace;
// every block but the last is recomputed before its backward). With recompute = 0 every block
// keeps its forward activations in its own workspace (about 0.9 GB per block at batch 2 x 1088
// tokens x 1536), which removes the recompute forward: the MI355X's 288 GB hold all 24. Both
// schedules run the same kernels on the same values, so their gradients are bitwise identical.
//
// Head (dit_head, src/dit.h:286-312) and tail (dit_tail, src/dit.h:316-325) run as adapted linears
// plus the small kernels below; tokens are batch-major ([B][S][dim], S = mem_tokens + T).
#include "block.h"
#include "lora.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

using namespace sa3k;

namespace {

constexpr int kThreads = 256;

void chk(sa3k_ctx* ctx, int rc) {
    if (rc != SA3K_OK) sa3k_throw(rc, ctx->last_error);
}

template <class T>
T* dalloc(size_t n) {
    void* p = nullptr;
    SA3K_HIP(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)));
    return static_cast<T*>(p);
}

inline unsigned nblk(int64_t n) { return (unsigned)ceil_div(n, kThreads); }

template <class... KArgs, class... Args>
void launch(sa3k_ctx* ctx, const char* name, void (*kernel)(KArgs...), dim3 grid, Args&&... args) {
    KernelScope ks(ctx, name);
    kernel<<<grid, kThreads, 0, ctx->stream>>>(std::forward<Args>(args)...);
    SA3K_LAUNCHED();
}

// ---------------------------------------------------------------- counter-based random numbers
// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC 2011)
__device__ inline uint4 philox4x32(uint4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t lo0 = 0xD2511F53u * c.x, hi0 = __umulhi(0xD2511F53u, c.x);
        const uint32_t lo1 = 0xCD9E8D57u * c.z, hi1 = __umulhi(0xCD9E8D57u, c.z);
        c = make_uint4(hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0);
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return c;
}

__device__ inline float u01(uint32_t x) { return ((float)(x >> 8) + 0.5f) * (1.0f / 16777216.0f); }   // (0, 1)

template <class T>
__device__ inline void store_as(void* dst, int64_t i, float v) {
    static_cast<T*>(dst)[i] = (T)v;
}

// dst[i] = mean + sd * N(0,1) (Box-Muller on one Philox block per 4 elements); type f32/f16/bf16
__global__ void init_normal_kernel(void* dst, int type, int64_t n, uint64_t seed, uint32_t stream, float mean, float sd) {
    const int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (q * 4 >= n) return;
    const uint4 r = philox4x32(make_uint4((uint32_t)q, (uint32_t)(q >> 32), stream, 0x5a3c0de1u), (uint32_t)seed,
                               (uint32_t)(seed >> 32));
    const float ra = sqrtf(-2.0f * logf(u01(r.x))), rb = sqrtf(-2.0f * logf(u01(r.z)));
    const float th_a = 6.28318530717958648f * u01(r.y), th_b = 6.28318530717958648f * u01(r.w);
    const float z[4] = {ra * cosf(th_a), ra * sinf(th_a), rb * cosf(th_b), rb * sinf(th_b)};
    for (int e = 0; e < 4; ++e) {
        const int64_t i = q * 4 + e;
        if (i >= n) break;
        const float v = mean + sd * z[e];
        if (type == SA3K_TYPE_F16) store_as<_Float16>(dst, i, v);
        else if (type == SA3K_TYPE_BF16) store_as<bf16>(dst, i, v);
        else store_as<float>(dst, i, v);
    }
}

// dst[i] = U(lo, hi)
__global__ void init_uniform_kernel(float* dst, int64_t n, uint64_t seed, uint32_t stream, float lo, float hi) {
    const int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (q * 4 >= n) return;
    const uint4 r = philox4x32(make_uint4((uint32_t)q, (uint32_t)(q >> 32), stream, 0x0a0b0c0du), (uint32_t)seed,
                               (uint32_t)(seed >> 32));
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
    for (int e = 0; e < 4; ++e) {
        const int64_t i = q * 4 + e;
        if (i < n) dst[i] = lo + (hi - lo) * u01(w[e]);
    }
}

__global__ void fill_kernel(float* dst, int64_t n, float v) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) dst[i] = v;
}

// ---------------------------------------------------------------- head / tail element-wise ops
// ExpoFourierFeatures (expo_features, src/sa3_pipeline.h:57-67): [cos | sin](2 pi t f_i)
__global__ void expo_kernel(const float* __restrict__ t, int B, int dim, float lmin, float lmax, float* __restrict__ tf) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    const int half = dim / 2;
    if (i >= B * half) return;
    const int b = i / half, k = i - b * half;
    const float ramp = half > 1 ? (float)k / (float)(half - 1) : 0.0f;
    const float f = expf(ramp * (lmax - lmin) + lmin);
    const float arg = t[b] * f * 6.28318530717958648f;
    tf[(int64_t)b * dim + k] = cosf(arg);
    tf[(int64_t)b * dim + half + k] = sinf(arg);
}

__global__ void silu_kernel(const float* __restrict__ h, int64_t n, float* __restrict__ a) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) a[i] = h[i] / (1.0f + expf(-h[i]));
}

// dh = da * silu'(h), silu'(z) = s(z) (1 + z (1 - s(z)))
__global__ void silu_bwd_kernel(const float* __restrict__ da, const float* __restrict__ h, int64_t n,
                                float* __restrict__ dh) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const float z = h[i], s = 1.0f / (1.0f + expf(-z));
    dh[i] = da[i] * s * (1.0f + z * (1.0f - s));
}

__global__ void copy_kernel(const float* __restrict__ a, int64_t n, float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) out[i] = a[i];
}

__global__ void add_kernel(const float* __restrict__ a, const float* __restrict__ b, int64_t n, float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

// x0[b][s] = s < mem ? memory_tokens[s] : xi[b][s - mem]
__global__ void concat_mem_kernel(const float* __restrict__ mem_tok, const float* __restrict__ xi, int B, int T, int mem,
                                  int dim, float* __restrict__ x0) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int S = mem + T;
    if (i >= (int64_t)B * S * dim) return;
    const int c = (int)(i % dim);
    const int64_t row = i / dim;
    const int b = (int)(row / S), s = (int)(row % S);
    x0[i] = s < mem ? mem_tok[(int64_t)s * dim + c] : xi[((int64_t)b * T + s - mem) * dim + c];
}

// out[b][f] = x[b][mem + f]  (drop the memory tokens)
__global__ void gather_frames_kernel(const float* __restrict__ x, int B, int T, int mem, int dim, float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= (int64_t)B * T * dim) return;
    const int c = (int)(i % dim);
    const int64_t row = i / dim;
    const int b = (int)(row / T), f = (int)(row % T);
    out[i] = x[((int64_t)b * (mem + T) + mem + f) * dim + c];
}

// dx[b][s] = s < mem ? 0 : dxt[b][s - mem]
__global__ void scatter_frames_kernel(const float* __restrict__ dxt, int B, int T, int mem, int dim, float* __restrict__ dx) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int S = mem + T;
    if (i >= (int64_t)B * S * dim) return;
    const int c = (int)(i % dim);
    const int64_t row = i / dim;
    const int b = (int)(row / S), s = (int)(row % S);
    dx[i] = s < mem ? 0.0f : dxt[((int64_t)b * T + s - mem) * dim + c];
}

// Velocity MSE (src/train_dit.h:174-184) per sample, over frames [f0, f1) of sample b:
// part = sum (v - tgt)^2 * w (double), dv = 2 (v - tgt) w, w = loss_weight[b][f] or 1/(io*T)
__global__ __launch_bounds__(kThreads) void mse_kernel(const float* __restrict__ v, const float* __restrict__ tgt,
                                                       const float* __restrict__ lw, int T, int io, int chunk,
                                                       double* __restrict__ part, float* __restrict__ dv) {
    __shared__ double sh[kThreads / 64];
    const int ch = blockIdx.x, b = blockIdx.y, nch = gridDim.x;
    const int f0 = ch * chunk, f1 = min(T, f0 + chunk);
    const double wu = 1.0 / ((double)io * T);
    double acc = 0.0;
    for (int64_t k = (int64_t)f0 * io + threadIdx.x; k < (int64_t)f1 * io; k += kThreads) {
        const int f = (int)(k / io);
        const int64_t i = (int64_t)b * T * io + k;
        const double w = lw ? (double)lw[(int64_t)b * T + f] : wu;
        const double d = (double)v[i] - (double)tgt[i];
        acc += d * d * w;
        dv[i] = (float)(2.0 * d * w);
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) part[(int64_t)b * nch + ch] = sh[0] + sh[1] + sh[2] + sh[3];
}

__global__ void mse_sum_kernel(const double* __restrict__ part, int nch, int B, double* __restrict__ loss) {
    const int b = blockIdx.x * kThreads + threadIdx.x;
    if (b >= B) return;
    double s = 0.0;
    for (int k = 0; k < nch; ++k) s += part[(int64_t)b * nch + k];
    loss[b] = s;
}

// ---------------------------------------------------------------- inpaint local conditioning
// local.0 takes local_dim inputs (1 + io: the mask and the masked latents, src/train_inpaint.h:
// 165-194), which the MFMA products take in whole 64-column steps: its weight, its A and its input
// are kept with kp = local_dim rounded up to 64 columns, the extra columns zero. They add exact
// zeros to every product, and their dA columns are zero (dA = (s B^T dU)^T X plus DoRA terms in
// W_eff, all of which vanish on a zero column).
template <class E>
__global__ void pad_cols_kernel(const E* __restrict__ src, int64_t rows, int64_t cols, int64_t ld, E* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= rows * ld) return;
    const int64_t r = i / ld, c = i - r * ld;
    dst[i] = c < cols ? src[r * cols + c] : E(0);
}

// A of block y's local.0 from the arena ([rank][cols] at off[y]) into dst[y] ([rank][ld])
__global__ void pad_a_kernel(const float* __restrict__ p, const int64_t* __restrict__ off, int rank, int cols, int ld,
                             float* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= (int64_t)rank * ld) return;
    const int64_t r = i / ld, c = i - r * ld;
    dst[(int64_t)blockIdx.y * rank * ld + i] = c < cols ? p[off[blockIdx.y] + r * cols + c] : 0.0f;
}

// g[rank][cols] += src[rank][ld] over the first cols columns; src is cleared for the next backward
__global__ void fold_a_kernel(float* __restrict__ src, int rank, int cols, int ld, float* __restrict__ g) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= (int64_t)rank * ld) return;
    const int64_t r = i / ld, c = i - r * ld;
    if (c < cols) g[r * cols + c] += src[i];
    src[i] = 0.0f;
}

// ---------------------------------------------------------------- model description
enum HeadIdx { H_PRE_CONV, H_PROJ_IN, H_TIME0, H_TIME2, H_GLOBAL0, H_GLOBAL2, H_GCE0, H_GCE2, H_COND0, H_COND2,
               H_PROJ_OUT, H_POST_CONV, H_N };
const char* const kHeadNames[H_N] = {"pre_conv", "proj_in", "time_embed.0", "time_embed.2", "global_embed.0",
                                     "global_embed.2", "gce.0", "gce.2", "cond_embed.0", "cond_embed.2", "proj_out",
                                     "post_conv"};
const char* const kBlockTargets[7] = {"self.qkv", "self.out", "cross.q", "cross.kv", "cross.out", "ff.proj", "ff.out"};
const char* const kLocalNames[2] = {"local.0", "local.2"};
const char* const kBlockVecs[8] = {"ssg", "pre_norm.gamma", "cross_norm.gamma", "ff_norm.gamma", "self.q_norm.gamma",
                                   "self.k_norm.gamma", "cross.q_norm.gamma", "cross.k_norm.gamma"};

struct Tensor {
    std::string name;
    int64_t rows = 0, cols = 0;   // cols = 1 for vectors
    int type = SA3K_TYPE_F32;
    int kind = 0;                 // 0 weight, 1 bias, 2 ssg, 3 gamma, 4 memory tokens
    void* raw = nullptr;          // device storage until setup (weights) / for the whole life (others)
    size_t bytes() const {
        const int64_t n = rows * cols;
        if (type == SA3K_TYPE_Q8_0) return (size_t)(n / 32) * 34;
        return (size_t)n * (type == SA3K_TYPE_F32 ? 4 : 2);
    }
};

struct Target {
    std::string name;
    int64_t in = 0, out = 0, off_a = -1, off_b = -1, off_m = -1;
    sa3k_lin* lin = nullptr;
    const float* bnsq = nullptr;
    const float* a_src = nullptr;   // the A the adapted linear reads when it is not the arena's (padded)
};

}  // namespace

struct sa3k_dit {
    sa3k_dit_config cfg{};
    int wtype = SA3K_TYPE_F16;
    std::vector<Tensor> tensors;
    std::map<std::string, int> index;
    bool ready = false;
    sa3k_dit_train tr{};
    int S = 0;
    float scale = 1.0f;
    // frozen model
    std::vector<sa3k_block*> blocks;
    sa3k_weight* hw[H_N] = {};
    sa3k_lin* hl[H_N] = {};
    float* hbnsq[H_N] = {};
    const float* hbias[H_N] = {};
    bool hf32[H_N] = {};            // head linear i computes in f32 (refreshed by its own prepare)
    bool group_pending = false;     // the grouped refresh is running on the second stream
    const float* memtok = nullptr;
    // adapters
    std::vector<Target> targets;    // sorted by name
    int head_target[H_N];           // index into targets or -1
    std::vector<int> block_target;  // [depth*7]
    float *p = nullptr, *g = nullptr, *m = nullptr, *v = nullptr;
    int64_t n_params = 0;
    bool dirty = true;
    int count = 0;
    LinGroup* group = nullptr;      // every adapted bf16 linear, refreshed together
    LinGroup* hgroup = nullptr;     // the adapted f32 head / tail linears, refreshed together
    LinStack* kvs = nullptr;        // the blocks' context K/V projections as one product (or null)
    // inpaint local conditioning (cfg.local_dim > 0): per block local.0 (local_dim -> dim, its
    // input padded to kp columns) and local.2 (dim -> dim), both with biases, adapted in the full
    // scope; index 2 l + k
    int kp = 0;
    std::vector<sa3k_weight*> lw;
    std::vector<sa3k_lin*> ll;
    std::vector<float*> lbnsq;
    std::vector<const float*> lbias;
    std::vector<int> local_target;  // index into targets or -1
    float* lA = nullptr;            // [depth][rank][kp] local.0's A, the arena's rows padded
    float* ldA = nullptr;           // [rank][kp] local.0's dA of one backward, padded
    int64_t* lA_off = nullptr;      // [depth] arena offsets of local.0's A
    const float* local_in = nullptr;  // bound conditioning [B][T][local_dim] (device) or null
    float* lc = nullptr;            // [B*T][kp] the padded conditioning of the current step
    std::vector<float*> lh, la, le;   // [depth] x [B*T][dim]: local.0 output, its silu, local.2 output
    std::vector<float*> dle;        // [depth] x [B*T][dim]: each block's local-add gradient
    float *dla = nullptr, *dlh = nullptr;   // [B*T][dim] backward scratch
    std::vector<hipEvent_t> lev;    // [depth] block l's local MLP output is ready (second stream)
    // activations
    std::vector<sa3k_block_ws*> ws;
    std::vector<float*> xs;
    std::vector<void*> bufs;
    float *tf, *te_h, *te_a, *te, *ge_h, *ge_a, *ge, *gsum, *gce_h, *gce_a, *gcond, *ce_h, *ce_a, *context;
    float *xp, *xi, *xt, *v0, *vel, *dv, *dv0, *dxt, *dxa, *dxb, *dctx, *dgcond, *dxi, *dxp, *da, *dh, *dg, *dca, *dch;
    double *loss_part, *loss;
    int loss_chunks = 1;
    // HIP graphs of the accumulate step (index 1: with the adapter prepare, 0: without), keyed by
    // the input pointers they were captured with. Off by default: a replay runs the captured
    // second-stream branches one after another, the eager step runs them beside the main stream.
    bool use_graph = false, warm = false;
    hipGraphExec_t gexec[2] = {nullptr, nullptr};
    const void* gkey[2][7] = {};
};

namespace {

void add_tensor(sa3k_dit* d, const std::string& name, int64_t rows, int64_t cols, int kind) {
    Tensor t;
    t.name = name;
    t.rows = rows;
    t.cols = cols;
    t.kind = kind;
    t.type = kind == 0 ? d->wtype : SA3K_TYPE_F32;
    d->index[name] = (int)d->tensors.size();
    d->tensors.push_back(t);
}

void describe(sa3k_dit* d) {
    const sa3k_dit_config& c = d->cfg;
    const int64_t D = c.dim, io = c.io, I = c.inner;
    add_tensor(d, "dit.memory_tokens", c.mem_tokens, D, 4);
    add_tensor(d, "dit.pre_conv.weight", io, io, 0);
    add_tensor(d, "dit.proj_in.weight", D, io, 0);
    add_tensor(d, "dit.proj_out.weight", io, D, 0);
    add_tensor(d, "dit.post_conv.weight", io, io, 0);
    add_tensor(d, "dit.time_embed.0.weight", D, c.time_dim, 0);
    add_tensor(d, "dit.time_embed.0.bias", D, 1, 1);
    add_tensor(d, "dit.time_embed.2.weight", D, D, 0);
    add_tensor(d, "dit.time_embed.2.bias", D, 1, 1);
    add_tensor(d, "dit.global_embed.0.weight", D, c.cond_dim, 0);
    add_tensor(d, "dit.global_embed.2.weight", D, D, 0);
    add_tensor(d, "dit.gce.0.weight", D, D, 0);
    add_tensor(d, "dit.gce.0.bias", D, 1, 1);
    add_tensor(d, "dit.gce.2.weight", 6 * D, D, 0);
    add_tensor(d, "dit.gce.2.bias", 6 * D, 1, 1);
    add_tensor(d, "dit.cond_embed.0.weight", D, c.cond_dim, 0);
    add_tensor(d, "dit.cond_embed.2.weight", D, D, 0);
    const int64_t outs[7] = {5 * D, D, 2 * D, 3 * D, D, 2 * I, D};
    const int64_t ins[7] = {D, D, D, D, D, D, I};
    for (int l = 0; l < c.depth; ++l) {
        const std::string p = "dit." + std::to_string(l) + ".";
        for (int t = 0; t < 7; ++t) add_tensor(d, p + kBlockTargets[t] + ".weight", outs[t], ins[t], 0);
        add_tensor(d, p + "ff.proj.bias", 2 * I, 1, 1);
        add_tensor(d, p + "ff.out.bias", D, 1, 1);
        add_tensor(d, p + "ssg", 6 * D, 1, 2);
        for (int k = 1; k < 8; ++k) add_tensor(d, p + kBlockVecs[k], k <= 3 ? D : 64, 1, 3);
    }
    if (c.local_dim > 0)
        for (int l = 0; l < c.depth; ++l) {
            const std::string p = "dit." + std::to_string(l) + ".";
            add_tensor(d, p + "local.0.weight", D, c.local_dim, 0);
            add_tensor(d, p + "local.0.bias", D, 1, 1);
            add_tensor(d, p + "local.2.weight", D, D, 0);
            add_tensor(d, p + "local.2.bias", D, 1, 1);
        }
}

Tensor& tensor(sa3k_dit* d, const std::string& name) {
    auto it = d->index.find(name);
    SA3K_REQUIRE(it != d->index.end(), "unknown tensor " + name);
    return d->tensors[it->second];
}

void free_dit(sa3k_ctx* ctx, sa3k_dit* d) {
    if (!d) return;
    for (sa3k_block_ws* w : d->ws) block_ws_free(w);
    for (sa3k_block* b : d->blocks) block_free(ctx, b);
    for (int i = 0; i < H_N; ++i) {
        if (d->hl[i]) sa3k_lin_destroy(ctx, d->hl[i]);
        if (d->hw[i]) sa3k_weight_destroy(ctx, d->hw[i]);
        if (d->hbnsq[i]) (void)hipFree(d->hbnsq[i]);
    }
    for (hipEvent_t e : d->lev)
        if (e) (void)hipEventDestroy(e);
    for (size_t i = 0; i < d->ll.size(); ++i) {
        if (d->ll[i]) sa3k_lin_destroy(ctx, d->ll[i]);
        if (d->lw[i]) sa3k_weight_destroy(ctx, d->lw[i]);
        if (d->lbnsq[i]) (void)hipFree(d->lbnsq[i]);
    }
    for (Tensor& t : d->tensors)
        if (t.raw) (void)hipFree(t.raw);
    for (void* p : d->bufs) (void)hipFree(p);
    for (hipGraphExec_t e : d->gexec)
        if (e) (void)hipGraphExecDestroy(e);
    lin_group_free(d->group);
    lin_group_free(d->hgroup);
    lin_stack_free(d->kvs);
    for (float* p : {d->p, d->g, d->m, d->v})
        if (p) (void)hipFree(p);
    delete d;
}

float* fbuf(sa3k_dit* d, size_t n) {
    float* p = dalloc<float>(n);
    d->bufs.push_back(p);
    return p;
}

void fill(sa3k_ctx* ctx, float* p, int64_t n, float v) {
    launch(ctx, "dit_fill", fill_kernel, dim3(nblk(n)), p, n, v);
}

// ---------------------------------------------------------------- setup
void setup(sa3k_ctx* ctx, sa3k_dit* d, const sa3k_dit_train& tr) {
    const sa3k_dit_config& c = d->cfg;
    SA3K_REQUIRE(!d->ready, "the model is already set up");
    SA3K_REQUIRE(tr.rank >= 8 && tr.rank <= 32 && tr.rank % 8 == 0, "rank must be 8, 16, 24 or 32");
    SA3K_REQUIRE(tr.scope == SA3K_SCOPE_CORE || tr.scope == SA3K_SCOPE_FULL, "unknown scope");
    SA3K_REQUIRE(tr.batch > 0 && tr.frames > 0 && tr.ctx_tokens > 0, "batch / frames / ctx_tokens must be positive");
    for (const Tensor& t : d->tensors) SA3K_REQUIRE(t.raw != nullptr, "tensor not set: " + t.name);
    d->tr = tr;
    d->S = c.mem_tokens + tr.frames;
    d->scale = tr.alpha / (float)tr.rank;
    const int B = tr.batch, T = tr.frames, Ctx = tr.ctx_tokens, S = d->S;
    const int64_t N = (int64_t)B * S, NT = (int64_t)B * T, NC = (int64_t)B * Ctx;
    // blocks
    sa3k_block_config bc{c.dim, c.heads, c.head_dim, c.inner, c.rope_dims, c.window, c.rope_base, c.norm_eps, c.qk_eps};
    for (int l = 0; l < c.depth; ++l) {
        const std::string p = "dit." + std::to_string(l) + ".";
        const void* W[7];
        const float* bias[7] = {};
        const float* vecs[8];
        for (int t = 0; t < 7; ++t) W[t] = tensor(d, p + kBlockTargets[t] + ".weight").raw;
        bias[5] = static_cast<const float*>(tensor(d, p + "ff.proj.bias").raw);
        bias[6] = static_cast<const float*>(tensor(d, p + "ff.out.bias").raw);
        for (int k = 0; k < 8; ++k) vecs[k] = static_cast<const float*>(tensor(d, p + kBlockVecs[k]).raw);
        d->blocks.push_back(block_build(ctx, bc, d->wtype, W, bias, vecs, 1, tr.rank, N, NC));
    }
    // head / tail linears
    const int64_t head_tokens[H_N] = {NT, NT, B, B, B, B, B, B, NC, NC, NT, NT};
    for (int i = 0; i < H_N; ++i) {
        Tensor& t = tensor(d, std::string("dit.") + kHeadNames[i] + ".weight");
        chk(ctx, sa3k_weight_create(ctx, d->wtype, t.cols, t.rows, t.raw, 1, &d->hw[i]));
        const int r = tr.scope == SA3K_SCOPE_FULL ? tr.rank : 0;
        // The head and tail sit at both ends of every gradient chain: the conditioning linears see
        // B or B*Ctx tokens (nothing averages their rounding) and feed every block's modulation,
        // and proj_in / proj_out carry the whole residual stream's gradient. They run on f32 MFMA
        // (a fraction of a percent of the update's work) over an f32 or f16 base.
        d->hf32[i] = ctx->head_f32 && (d->wtype == SA3K_TYPE_F32 || d->wtype == SA3K_TYPE_F16);
        chk(ctx, sa3k_lin_create(ctx, d->hw[i], r, d->hf32[i] ? SA3K_PREC_F32 : SA3K_PREC_BF16, head_tokens[i],
                                 &d->hl[i]));
        lin_set_tag(d->hl[i], "head");
        if (r && tr.dora) {
            d->hbnsq[i] = dalloc<float>((size_t)t.rows);
            chk(ctx, sa3k_weight_row_norm_sq(ctx, d->hw[i], 1e-12f, d->hbnsq[i]));
        }
        auto it = d->index.find(std::string("dit.") + kHeadNames[i] + ".bias");
        d->hbias[i] = it != d->index.end() ? static_cast<const float*>(d->tensors[it->second].raw) : nullptr;
    }
    // inpaint local conditioning: local.0 over kp padded input columns, local.2; adapters in the
    // full scope (the core scope drops local.{0,2}, src/train_lora.h:85-89)
    if (c.local_dim > 0) {
        d->kp = (int)ceil_div(c.local_dim, 64) * 64;
        const int r = tr.scope == SA3K_SCOPE_FULL ? tr.rank : 0;
        const size_t nl = (size_t)2 * c.depth;
        d->lw.assign(nl, nullptr); d->ll.assign(nl, nullptr); d->lbnsq.assign(nl, nullptr); d->lbias.assign(nl, nullptr);
        for (int l = 0; l < c.depth; ++l)
            for (int k = 0; k < 2; ++k) {
                const size_t i = (size_t)2 * l + k;
                const std::string stem = "dit." + std::to_string(l) + "." + kLocalNames[k];
                Tensor& t = tensor(d, stem + ".weight");
                const void* src = t.raw;
                void* padded = nullptr;
                int64_t in = t.cols;
                if (k == 0 && d->kp != t.cols) {
                    const int64_t n = t.rows * d->kp;
                    if (d->wtype == SA3K_TYPE_F32) {
                        padded = dalloc<float>((size_t)n);
                        launch(ctx, "dit_local", pad_cols_kernel<uint32_t>, dim3(nblk(n)), (const uint32_t*)t.raw,
                               t.rows, t.cols, (int64_t)d->kp, (uint32_t*)padded);
                    } else {
                        padded = dalloc<uint16_t>((size_t)n);
                        launch(ctx, "dit_local", pad_cols_kernel<uint16_t>, dim3(nblk(n)), (const uint16_t*)t.raw,
                               t.rows, t.cols, (int64_t)d->kp, (uint16_t*)padded);
                    }
                    src = padded;
                    in = d->kp;
                }
                const int rc = sa3k_weight_create(ctx, d->wtype, in, t.rows, src, 1, &d->lw[i]);
                if (padded) {
                    (void)hipStreamSynchronize(ctx->stream);
                    (void)hipFree(padded);
                }
                chk(ctx, rc);
                chk(ctx, sa3k_lin_create(ctx, d->lw[i], r, SA3K_PREC_BF16, NT, &d->ll[i]));
                lin_set_tag(d->ll[i], "local");
                if (r && tr.dora) {   // base_norm_sq over the stored local_dim columns (eps counts them)
                    d->lbnsq[i] = dalloc<float>((size_t)t.rows);
                    chk(ctx, sa3k_row_norms(ctx, d->wtype, t.cols, t.rows, t.raw, 1, 1e-12f, d->lbnsq[i]));
                }
                d->lbias[i] = static_cast<const float*>(tensor(d, stem + ".bias").raw);
            }
    }
    d->memtok = static_cast<const float*>(tensor(d, "dit.memory_tokens").raw);
    SA3K_HIP(hipStreamSynchronize(ctx->stream));
    // the weights and the block vectors now live in the sa3k_weight / sa3k_block objects; the head
    // and local biases and the memory tokens are read in place, and local.0's stored (unpadded)
    // weight stays for its row norms over local_dim columns
    for (Tensor& t : d->tensors)
        if ((t.kind == 0 || t.kind == 2 || t.kind == 3) && t.name.find(".local.0.weight") == std::string::npos) {
            (void)hipFree(t.raw);
            t.raw = nullptr;
        }
    // adapter targets in the reference's order (sorted weight names)
    struct Ref { std::string name; sa3k_lin* lin; const float* bnsq; int64_t in, out; int head; int block; int local; };
    std::vector<Ref> refs;
    const int64_t outs[7] = {5 * (int64_t)c.dim, c.dim, 2 * (int64_t)c.dim, 3 * (int64_t)c.dim, c.dim,
                             2 * (int64_t)c.inner, c.dim};
    const int64_t ins[7] = {c.dim, c.dim, c.dim, c.dim, c.dim, c.dim, c.inner};
    for (int l = 0; l < c.depth; ++l)
        for (int t = 0; t < 7; ++t)
            refs.push_back({"dit." + std::to_string(l) + "." + kBlockTargets[t] + ".weight", d->blocks[l]->L[t],
                            d->blocks[l]->bnsq[t], ins[t], outs[t], -1, l * 7 + t, -1});
    if (tr.scope == SA3K_SCOPE_FULL)
        for (int i = 0; i < H_N; ++i) {
            const Tensor& t = tensor(d, std::string("dit.") + kHeadNames[i] + ".weight");
            refs.push_back({t.name, d->hl[i], d->hbnsq[i], t.cols, t.rows, i, -1, -1});
        }
    if (tr.scope == SA3K_SCOPE_FULL)
        for (size_t i = 0; i < d->ll.size(); ++i) {   // the arena keeps local.0's A at local_dim columns
            const Tensor& t = tensor(d, "dit." + std::to_string(i / 2) + "." + kLocalNames[i % 2] + ".weight");
            refs.push_back({t.name, d->ll[i], d->lbnsq[i], t.cols, t.rows, -1, -1, (int)i});
        }
    std::sort(refs.begin(), refs.end(), [](const Ref& a, const Ref& b) { return a.name < b.name; });
    for (int i = 0; i < H_N; ++i) d->head_target[i] = -1;
    d->block_target.assign((size_t)c.depth * 7, -1);
    d->local_target.assign(d->ll.size(), -1);
    int64_t off = 0;
    for (const Ref& r : refs) {
        Target t;
        t.name = r.name; t.in = r.in; t.out = r.out; t.lin = r.lin; t.bnsq = r.bnsq;
        t.off_a = off; off += (int64_t)tr.rank * r.in;
        t.off_b = off; off += r.out * tr.rank;
        if (tr.dora) { t.off_m = off; off += r.out; }
        if (r.head >= 0) d->head_target[r.head] = (int)d->targets.size();
        if (r.block >= 0) d->block_target[r.block] = (int)d->targets.size();
        if (r.local >= 0) d->local_target[r.local] = (int)d->targets.size();
        d->targets.push_back(t);
    }
    d->n_params = off;
    d->p = dalloc<float>(off); d->g = dalloc<float>(off); d->m = dalloc<float>(off); d->v = dalloc<float>(off);
    fill(ctx, d->p, off, 0.0f); fill(ctx, d->g, off, 0.0f); fill(ctx, d->m, off, 0.0f); fill(ctx, d->v, off, 0.0f);
    // activations
    const int64_t D = c.dim, io = c.io;
    d->tf = fbuf(d, (size_t)B * c.time_dim);
    d->te_h = fbuf(d, B * D); d->te_a = fbuf(d, B * D); d->te = fbuf(d, B * D);
    d->ge_h = fbuf(d, B * D); d->ge_a = fbuf(d, B * D); d->ge = fbuf(d, B * D); d->gsum = fbuf(d, B * D);
    d->gce_h = fbuf(d, B * D); d->gce_a = fbuf(d, B * D); d->gcond = fbuf(d, 6 * B * D);
    d->ce_h = fbuf(d, NC * D); d->ce_a = fbuf(d, NC * D); d->context = fbuf(d, NC * D);
    d->xp = fbuf(d, NT * io); d->xi = fbuf(d, NT * D);
    for (int l = 0; l <= c.depth; ++l) d->xs.push_back(fbuf(d, N * D));
    d->xt = fbuf(d, NT * D); d->v0 = fbuf(d, NT * io); d->vel = fbuf(d, NT * io);
    d->dv = fbuf(d, NT * io); d->dv0 = fbuf(d, NT * io); d->dxt = fbuf(d, NT * D);
    d->dxa = fbuf(d, N * D); d->dxb = fbuf(d, N * D); d->dctx = fbuf(d, NC * D); d->dgcond = fbuf(d, 6 * B * D);
    d->dxi = fbuf(d, NT * D); d->dxp = fbuf(d, NT * io);
    d->da = fbuf(d, 6 * B * D); d->dh = fbuf(d, 6 * B * D); d->dg = fbuf(d, B * D);
    d->dca = fbuf(d, NC * D); d->dch = fbuf(d, NC * D);
    if (c.local_dim > 0) {
        d->lev.assign((size_t)c.depth, nullptr);
        for (hipEvent_t& e : d->lev) SA3K_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        d->lc = fbuf(d, (size_t)NT * d->kp);
        for (int l = 0; l < c.depth; ++l) {
            d->lh.push_back(fbuf(d, NT * D));
            d->la.push_back(fbuf(d, NT * D));
            d->le.push_back(fbuf(d, NT * D));
        }
        if (tr.scope == SA3K_SCOPE_FULL) {
            for (int l = 0; l < c.depth; ++l) d->dle.push_back(fbuf(d, NT * D));
            d->dla = fbuf(d, NT * D); d->dlh = fbuf(d, NT * D);
            d->lA = fbuf(d, (size_t)c.depth * tr.rank * d->kp);
            d->ldA = fbuf(d, (size_t)tr.rank * d->kp);
            fill(ctx, d->ldA, (int64_t)tr.rank * d->kp, 0.0f);
            std::vector<int64_t> offs((size_t)c.depth);
            for (int l = 0; l < c.depth; ++l) {
                Target& t0 = d->targets[d->local_target[(size_t)2 * l]];
                offs[l] = t0.off_a;
                t0.a_src = d->lA + (int64_t)l * tr.rank * d->kp;
            }
            int64_t* od = dalloc<int64_t>(offs.size());
            d->bufs.push_back(od);
            SA3K_HIP(hipMemcpyAsync(od, offs.data(), offs.size() * sizeof(int64_t), hipMemcpyHostToDevice, ctx->stream));
            sa3k_note_main(ctx);
            d->lA_off = od;
        }
    }
    d->loss_chunks = (int)std::min<int64_t>(64, ceil_div(T, 16));
    double* lp = dalloc<double>((size_t)B * d->loss_chunks);
    d->bufs.push_back(lp);
    d->loss_part = lp;
    double* ls = dalloc<double>((size_t)B);
    d->bufs.push_back(ls);
    d->loss = ls;
    if (ctx->kv_stack && c.depth > 1) {
        // every block projects the same context to its cross-attention K/V: one product over the
        // stacked merged weights (set up before the refresh group, which then writes into it)
        std::vector<sa3k_lin*> kl;
        for (sa3k_block* b : d->blocks) kl.push_back(b->L[3]);
        d->kvs = lin_stack_create(ctx, kl.data(), (int)kl.size());
    }
    {
        std::vector<sa3k_lin*> lins;
        std::vector<const float*> A, Bm, mag, bnsq;
        std::vector<bool> f32_lin(d->targets.size(), false);
        for (int i = 0; i < H_N; ++i)
            if (d->head_target[i] >= 0 && d->hf32[i]) f32_lin[(size_t)d->head_target[i]] = true;
        std::vector<sa3k_lin*> hlins;
        std::vector<const float*> hA, hBm, hmag, hbnsq;
        for (size_t k = 0; k < d->targets.size(); ++k) {
            const Target& t = d->targets[k];
            const bool f32 = f32_lin[k];   // the f32 head linears form a group of their own
            (f32 ? hlins : lins).push_back(t.lin);
            (f32 ? hA : A).push_back(t.a_src ? t.a_src : d->p + t.off_a);
            (f32 ? hBm : Bm).push_back(d->p + t.off_b);
            (f32 ? hmag : mag).push_back(tr.dora ? d->p + t.off_m : nullptr);
            (f32 ? hbnsq : bnsq).push_back(tr.dora ? t.bnsq : nullptr);
        }
        d->group = lin_group_create(ctx, lins.data(), (int)lins.size(), A.data(), Bm.data(), mag.data(), bnsq.data(),
                                    d->scale, tr.dora);
        if (!hlins.empty())
            d->hgroup = lin_group_create(ctx, hlins.data(), (int)hlins.size(), hA.data(), hBm.data(), hmag.data(),
                                         hbnsq.data(), d->scale, tr.dora);
        for (int i = 0; i < H_N; ++i)
            if (d->head_target[i] < 0)
                chk(ctx, sa3k_lin_prepare(ctx, d->hl[i], nullptr, nullptr, d->scale, 0, nullptr, nullptr));
        for (size_t i = 0; i < d->ll.size(); ++i)
            if (d->local_target[i] < 0)
                chk(ctx, sa3k_lin_prepare(ctx, d->ll[i], nullptr, nullptr, d->scale, 0, nullptr, nullptr));
    }
    const int nws = tr.recompute ? 1 : c.depth;
    for (int l = 0; l < nws; ++l)
        d->ws.push_back(block_ws_build(bc, B, S, Ctx, l == 0 ? nullptr : d->ws[0], ctx->act_bf16));
    SA3K_HIP(hipStreamSynchronize(ctx->stream));
    d->ready = true;
    d->dirty = true;
}

void prepare(sa3k_ctx* ctx, sa3k_dit* d) {
    if (!d->dirty) return;
    KernelScope ks(ctx, "dit_prepare");
    // The grouped bf16 refresh streams every block weight (HBM-bound, the whole chip); the f32 head
    // linears' refresh is a few short launches. With both, the bf16 group goes to the second stream
    // and the heads' refresh and forwards run beside it on the main stream; forward() joins before
    // the first product that reads a member of the bf16 group.
    const bool side = d->hgroup && ctx->prep_side && side_usable(ctx);
    if (side) side_fork(ctx);
    {
        OnSide os(ctx, side);
        if (d->lA)   // local.0's A at kp columns for its padded product
            launch(ctx, "dit_local", pad_a_kernel, dim3(nblk((int64_t)d->tr.rank * d->kp), (unsigned)d->cfg.depth),
                   (const float*)d->p, (const int64_t*)d->lA_off, d->tr.rank, d->cfg.local_dim, d->kp, d->lA);
        lin_group_prepare(ctx, d->group);
    }
    d->group_pending = side;
    if (d->hgroup) lin_group_prepare(ctx, d->hgroup);   // the f32 head linears: two-segment refresh
    d->dirty = false;
}

// the main stream waits for the grouped refresh when prepare() left it on the second stream
void join_group(sa3k_ctx* ctx, sa3k_dit* d) {
    if (!d->group_pending) return;
    side_join(ctx);
    d->group_pending = false;
}

void lin_fwd(sa3k_ctx* ctx, sa3k_dit* d, int i, const float* X, int64_t N, float* Y) {
    chk(ctx, sa3k_lin_forward(ctx, d->hl[i], SA3K_TYPE_F32, X, N, d->hbias[i], Y));
}

// backward of head linear i: dX (nullable) written or added; adapter gradients added
void lin_bwd(sa3k_ctx* ctx, sa3k_dit* d, int i, const float* X, int64_t N, const float* dY, float* dX, int acc) {
    const int ti = d->head_target[i];
    float *dA = nullptr, *dB = nullptr, *dm = nullptr;
    if (ti >= 0) {
        const Target& tg = d->targets[ti];
        dA = d->g + tg.off_a;
        dB = d->g + tg.off_b;
        dm = d->tr.dora ? d->g + tg.off_m : nullptr;
    } else if (!dX) {
        return;
    }
    chk(ctx, sa3k_lin_backward(ctx, d->hl[i], SA3K_TYPE_F32, X, N, dY, dX, acc, dA, dB, dm));
}

void mlp_fwd(sa3k_ctx* ctx, sa3k_dit* d, int i0, const float* x, int64_t N, float* h, float* a, float* y) {
    const int64_t n = N * d->cfg.dim;
    lin_fwd(ctx, d, i0, x, N, h);
    launch(ctx, "dit_silu", silu_kernel, dim3(nblk(n)), (const float*)h, n, a);
    lin_fwd(ctx, d, i0 + 1, a, N, y);
}

// mlp backward from dy; dx (nullable) written
void mlp_bwd(sa3k_ctx* ctx, sa3k_dit* d, int i0, const float* x, int64_t N, const float* h, const float* a,
             const float* dy, float* dx) {
    const int64_t n = N * d->cfg.dim;
    // the context MLP has scratch of its own: its backward runs beside the modulation chain's
    float* da = i0 == H_COND0 ? d->dca : d->da;
    float* dh = i0 == H_COND0 ? d->dch : d->dh;
    lin_bwd(ctx, d, i0 + 1, a, N, dy, da, 0);
    launch(ctx, "dit_silu", silu_bwd_kernel, dim3(nblk(n)), (const float*)da, h, n, dh);
    lin_bwd(ctx, d, i0, x, N, dh, dx, 0);
}

// block l's context K/V: its columns of the stacked product's output, or its own projection
void bind_kv(sa3k_dit* d, sa3k_block_ws* w, int l) {
    w->kv_ext = d->kvs ? lin_stack_y(d->kvs) + (int64_t)l * 3 * d->cfg.dim : nullptr;
    w->kv_ld = d->kvs ? lin_stack_ld(d->kvs) : 0;
}

// block l's inpaint local add: its MLP's output when conditioning is bound, and the gradient
// buffer when the local linears carry adapters
void bind_local(sa3k_dit* d, sa3k_block_ws* w, int l) {
    const bool on = d->local_in != nullptr;
    w->ladd = on ? d->le[l] : nullptr;
    w->dladd = on && !d->dle.empty() &&
                       (d->local_target[(size_t)2 * l] >= 0 || d->local_target[(size_t)2 * l + 1] >= 0)
                   ? d->dle[l] : nullptr;
    w->ladd_T = d->tr.frames;
}

// le = local.2(silu(local.0(local_cond))), both with biases (src/dit.h:246-249)
void local_fwd(sa3k_ctx* ctx, sa3k_dit* d, int l) {
    const int64_t NT = (int64_t)d->tr.batch * d->tr.frames, n = NT * d->cfg.dim;
    chk(ctx, sa3k_lin_forward(ctx, d->ll[(size_t)2 * l], SA3K_TYPE_F32, d->lc, NT, d->lbias[(size_t)2 * l], d->lh[l]));
    launch(ctx, "dit_local", silu_kernel, dim3(nblk(n)), (const float*)d->lh[l], n, d->la[l]);
    chk(ctx, sa3k_lin_forward(ctx, d->ll[(size_t)2 * l + 1], SA3K_TYPE_F32, d->la[l], NT, d->lbias[(size_t)2 * l + 1],
                              d->le[l]));
}

// the local MLP's backward from dle[l] (written by block l's backward): adapter gradients only (the
// conditioning is data); local.0's dA comes out at kp columns and is folded into the arena
void local_bwd(sa3k_ctx* ctx, sa3k_dit* d, int l) {
    const int64_t NT = (int64_t)d->tr.batch * d->tr.frames, n = NT * d->cfg.dim;
    auto grads = [&](size_t i, float** dA, float** dB, float** dm) {
        const int ti = d->local_target[i];
        *dA = *dB = *dm = nullptr;
        if (ti < 0) return;
        const Target& tg = d->targets[ti];
        *dA = d->g + tg.off_a;
        *dB = d->g + tg.off_b;
        *dm = d->tr.dora ? d->g + tg.off_m : nullptr;
    };
    float *dA, *dB, *dm;
    grads((size_t)2 * l + 1, &dA, &dB, &dm);
    chk(ctx, sa3k_lin_backward(ctx, d->ll[(size_t)2 * l + 1], SA3K_TYPE_F32, d->la[l], NT, d->dle[l], d->dla, 0, dA, dB,
                               dm));
    if (d->local_target[(size_t)2 * l] < 0) return;
    launch(ctx, "dit_local", silu_bwd_kernel, dim3(nblk(n)), (const float*)d->dla, (const float*)d->lh[l], n, d->dlh);
    grads((size_t)2 * l, &dA, &dB, &dm);
    chk(ctx, sa3k_lin_backward(ctx, d->ll[(size_t)2 * l], SA3K_TYPE_F32, d->lc, NT, d->dlh, nullptr, 0, d->ldA, dB, dm));
    launch(ctx, "dit_local", fold_a_kernel, dim3(nblk((int64_t)d->tr.rank * d->kp)), d->ldA, d->tr.rank,
           d->cfg.local_dim, d->kp, dA);
}

// head + blocks + tail forward: velocity in d->vel
void forward(sa3k_ctx* ctx, sa3k_dit* d, const float* x_t, const float* t, const float* cross, const float* glob) {
    const sa3k_dit_config& c = d->cfg;
    const int B = d->tr.batch, T = d->tr.frames, Ctx = d->tr.ctx_tokens, S = d->S;
    const int64_t NT = (int64_t)B * T, NC = (int64_t)B * Ctx, D = c.dim;
    prepare(ctx, d);
    // the rank products of merged linears run on the second stream, read by the backward only: one
    // join at the end (per block under recompute, whose blocks share one workspace)
    const bool join_here = ctx->side_defer == 0;
    const uint64_t forks0 = ctx->side_forks;
    SideDeferScope defer(ctx);
    // The head: three chains of short dependent launches that meet at the first block. The context
    // MLP and the x path run on the third stream beside the modulation chain (gcond = gce(ge + te))
    // on the main stream; both wait on little but memory latency, the more so beside the grouped
    // refresh, so two chains in flight take about as long as the longer one.
    const bool quick = ctx->head_quick && side_usable(ctx);
    if (quick) quick_fork(ctx);   // the head linears' refresh is complete
    {
        OnQuick oq(ctx, quick);
        mlp_fwd(ctx, d, H_COND0, cross, NC, d->ce_h, d->ce_a, d->context);
        lin_fwd(ctx, d, H_PRE_CONV, x_t, NT, d->xp);
        launch(ctx, "dit_head", add_kernel, dim3(nblk(NT * c.io)), (const float*)d->xp, x_t, NT * c.io, d->xp);
        lin_fwd(ctx, d, H_PROJ_IN, d->xp, NT, d->xi);
        launch(ctx, "dit_head", concat_mem_kernel, dim3(nblk((int64_t)B * S * D)), d->memtok, (const float*)d->xi, B,
               T, c.mem_tokens, (int)D, d->xs[0]);
    }
    launch(ctx, "dit_head", expo_kernel, dim3(nblk((int64_t)B * (c.time_dim / 2))), t, B, c.time_dim,
           logf(c.time_min_freq), logf(c.time_max_freq), d->tf);
    mlp_fwd(ctx, d, H_TIME0, d->tf, B, d->te_h, d->te_a, d->te);
    mlp_fwd(ctx, d, H_GLOBAL0, glob, B, d->ge_h, d->ge_a, d->ge);
    launch(ctx, "dit_head", add_kernel, dim3(nblk(B * D)), (const float*)d->ge, (const float*)d->te, (int64_t)B * D,
           d->gsum);
    mlp_fwd(ctx, d, H_GCE0, d->gsum, B, d->gce_h, d->gce_a, d->gcond);   // dim -> dim -> 6 dim
    if (quick) quick_join(ctx);
    join_group(ctx, d);   // every product from here on reads a member of the grouped refresh
    if (d->kvs) lin_stack_forward(ctx, d->kvs, d->context, NC);   // every block's context K/V
    // the inpaint conditioning, zero-padded to local.0's kp input columns; every block's local MLP
    // depends on it alone, so they run on the second stream and block l waits for its own MLP only:
    // all of them up front, or under recompute, where every block joins the second stream at its
    // end, one block ahead (block l's MLP beside block l - 1)
    const bool local_side = d->local_in && side_usable(ctx);
    auto local_ahead = [&](int l0, int l1) {
        if (local_side) side_fork(ctx);
        OnSide os(ctx, local_side);
        for (int l = l0; l < l1; ++l) {
            local_fwd(ctx, d, l);
            if (local_side) SA3K_HIP(hipEventRecord(d->lev[l], ctx->side_stream));
        }
    };
    if (d->local_in) {
        launch(ctx, "dit_local", pad_cols_kernel<float>, dim3(nblk(NT * d->kp)), d->local_in, NT,
               (int64_t)c.local_dim, (int64_t)d->kp, d->lc);
        local_ahead(0, d->tr.recompute ? 1 : c.depth);
    }
    // blocks
    for (int l = 0; l < c.depth; ++l) {
        bind_kv(d, d->ws[d->tr.recompute ? 0 : l], l);
        bind_local(d, d->ws[d->tr.recompute ? 0 : l], l);
        if (d->local_in && d->tr.recompute && l + 1 < c.depth) local_ahead(l + 1, l + 2);
        if (local_side) SA3K_HIP(hipStreamWaitEvent(ctx->main_stream, d->lev[l], 0));
        block_forward(ctx, d->blocks[l], d->ws[d->tr.recompute ? 0 : l], d->xs[l], d->context, d->gcond, d->xs[l + 1]);
        if (d->tr.recompute) side_join_since(ctx, forks0);
    }
    // tail
    launch(ctx, "dit_tail", gather_frames_kernel, dim3(nblk(NT * D)), (const float*)d->xs[c.depth], B, T, c.mem_tokens,
           (int)D, d->xt);
    lin_fwd(ctx, d, H_PROJ_OUT, d->xt, NT, d->v0);
    lin_fwd(ctx, d, H_POST_CONV, d->v0, NT, d->vel);
    launch(ctx, "dit_tail", add_kernel, dim3(nblk(NT * c.io)), (const float*)d->vel, (const float*)d->v0, NT * c.io,
           d->vel);
    if (join_here) side_join_since(ctx, forks0);
}

// per-sample velocity MSE of the last forward into d->loss, and its seed gradient into d->dv
void loss_and_seed(sa3k_ctx* ctx, sa3k_dit* d, const float* target, const float* lw) {
    const int B = d->tr.batch, T = d->tr.frames;
    const int chunk = (int)ceil_div(T, d->loss_chunks);
    launch(ctx, "dit_loss", mse_kernel, dim3((unsigned)d->loss_chunks, (unsigned)B), (const float*)d->vel, target, lw, T,
           d->cfg.io, chunk, d->loss_part, d->dv);
    launch(ctx, "dit_loss", mse_sum_kernel, dim3(1), (const double*)d->loss_part, d->loss_chunks, B, d->loss);
}

void accumulate_body(sa3k_ctx* ctx, sa3k_dit* d, const float* x_t, const float* target, const float* t,
                     const float* cross, const float* glob, const float* lw) {
    const sa3k_dit_config& c = d->cfg;
    const int B = d->tr.batch, T = d->tr.frames, S = d->S;
    const int64_t NT = (int64_t)B * T, NC = (int64_t)B * d->tr.ctx_tokens, D = c.dim;
    KernelScope ks(ctx, "dit_step");
    forward(ctx, d, x_t, t, cross, glob);
    loss_and_seed(ctx, d, target, lw);
    // tail backward: v = post_conv(v0) + v0, v0 = proj_out(x_depth[mem:])
    launch(ctx, "dit_tail", copy_kernel, dim3(nblk(NT * c.io)), (const float*)d->dv, NT * c.io, d->dv0);
    lin_bwd(ctx, d, H_POST_CONV, d->v0, NT, d->dv, d->dv0, 1);
    lin_bwd(ctx, d, H_PROJ_OUT, d->xt, NT, d->dv0, d->dxt, 0);
    launch(ctx, "dit_tail", scatter_frames_kernel, dim3(nblk((int64_t)B * S * D)), (const float*)d->dxt, B, T,
           c.mem_tokens, (int)D, d->dxa);
    // blocks in reverse
    fill(ctx, d->dctx, NC * D, 0.0f);
    fill(ctx, d->dgcond, 6 * B * D, 0.0f);
    float* dcur = d->dxa;
    float* dnext = d->dxb;
    // a block's local MLP backward reads block l's own buffers only, so it runs on the second stream
    // beside the next blocks; under recompute it is enqueued after the next block's recomputed
    // forward, whose join at its end would otherwise wait for it
    auto local_back = [&](int l) {
        const bool side = side_usable(ctx);
        if (side) side_fork(ctx);
        OnSide os(ctx, side);
        local_bwd(ctx, d, l);
    };
    int local_pending = -1;
    for (int l = c.depth - 1; l >= 0; --l) {
        sa3k_block_ws* w = d->ws[d->tr.recompute ? 0 : l];
        bind_kv(d, w, l);
        bind_local(d, w, l);
        if (d->tr.recompute && l != c.depth - 1)   // the last block's activations are still in place
            block_forward(ctx, d->blocks[l], w, d->xs[l], d->context, d->gcond, d->xs[l + 1]);
        if (local_pending >= 0) local_back(local_pending);
        local_pending = -1;
        float* dA[7];
        float* dB[7];
        float* dm[7];
        for (int t = 0; t < 7; ++t) {
            const Target& tg = d->targets[d->block_target[(size_t)l * 7 + t]];
            dA[t] = d->g + tg.off_a;
            dB[t] = d->g + tg.off_b;
            dm[t] = d->tr.dora ? d->g + tg.off_m : nullptr;
        }
        // resident activations: a block's last second-stream work may run on beside the next block
        block_backward(ctx, d->blocks[l], w, dcur, dnext, d->dctx, d->dgcond, dA, dB, d->tr.dora ? dm : nullptr,
                       ctx->late_join && !d->tr.recompute);
        if (w->dladd) {
            if (d->tr.recompute) local_pending = l;
            else local_back(l);
        }
        std::swap(dcur, dnext);
    }
    if (local_pending >= 0) local_back(local_pending);
    if (side_usable(ctx)) side_join(ctx);   // the head reads dgcond; AdamW reads every dA
    ctx->block_tail_pending = false;
    // head backward (only adapter gradients are wanted: the inputs are data). Three independent
    // chains of short launches: the modulation chain (gcond = gce(ge + te)) on the second stream,
    // the x path and the context MLP on the main stream beside it (their own forks held back).
    if (d->tr.scope == SA3K_SCOPE_FULL) {
        const bool two = side_usable(ctx);
        if (two) side_fork(ctx);   // dgcond, dctx and the first block's dx are complete
        {
            OnSide os(ctx, two);
            lin_bwd(ctx, d, H_GCE2, d->gce_a, B, d->dgcond, d->da, 0);
            launch(ctx, "dit_silu", silu_bwd_kernel, dim3(nblk(B * D)), (const float*)d->da, (const float*)d->gce_h,
                   (int64_t)B * D, d->dh);
            lin_bwd(ctx, d, H_GCE0, d->gsum, B, d->dh, d->dg, 0);
            mlp_bwd(ctx, d, H_GLOBAL0, glob, B, d->ge_h, d->ge_a, d->dg, nullptr);
            mlp_bwd(ctx, d, H_TIME0, d->tf, B, d->te_h, d->te_a, d->dg, nullptr);
        }
        {
            SideHeld hold(ctx, two);
            // the context MLP on the third stream beside the x path
            const bool quick = two && ctx->head_quick;
            if (quick) quick_fork(ctx);
            {
                OnQuick oq(ctx, quick);
                mlp_bwd(ctx, d, H_COND0, cross, NC, d->ce_h, d->ce_a, d->dctx, nullptr);
            }
            launch(ctx, "dit_head", gather_frames_kernel, dim3(nblk(NT * D)), (const float*)dcur, B, T, c.mem_tokens,
                   (int)D, d->dxi);
            lin_bwd(ctx, d, H_PROJ_IN, d->xp, NT, d->dxi, d->dxp, 0);
            lin_bwd(ctx, d, H_PRE_CONV, x_t, NT, d->dxp, nullptr, 0);
            if (quick) quick_join(ctx);
        }
        if (two) side_join(ctx);   // AdamW reads every gradient
    }
}

// Capture the accumulate step into a graph (prepare included when the adapters changed). On a
// capture failure the graphs are switched off and the step runs eagerly.
bool capture(sa3k_ctx* ctx, sa3k_dit* d, int gi, const void* const* key, const float* x_t, const float* target,
             const float* t, const float* cross, const float* glob, const float* lw) {
    if (d->gexec[gi]) {
        SA3K_HIP(hipGraphExecDestroy(d->gexec[gi]));
        d->gexec[gi] = nullptr;
    }
    hipGraph_t g = nullptr;
    SA3K_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    ctx->tail_ev = nullptr;   // a fork armed before the capture would wait on uncaptured work
    try {
        accumulate_body(ctx, d, x_t, target, t, cross, glob, lw);
    } catch (...) {
        ctx->capturing = false;
        // bring the other streams back into the capture (best effort: a stream that never joined
        // it refuses), so that ending it leaves no stream capturing
        for (hipStream_t st : {ctx->side_stream, ctx->quick_stream}) {
            if (!st) continue;
            hipEvent_t e = side_event(ctx);
            if (hipEventRecord(e, st) == hipSuccess) (void)hipStreamWaitEvent(ctx->stream, e, 0);
        }
        (void)hipStreamEndCapture(ctx->stream, &g);
        if (g) (void)hipGraphDestroy(g);
        (void)hipGetLastError();
        d->use_graph = false;
        return false;
    }
    ctx->capturing = false;
    SA3K_HIP(hipStreamEndCapture(ctx->stream, &g));
    const hipError_t e = hipGraphInstantiate(&d->gexec[gi], g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    SA3K_HIP(e);
    for (int k = 0; k < 7; ++k) d->gkey[gi][k] = key[k];
    return true;
}

void accumulate(sa3k_ctx* ctx, sa3k_dit* d, const float* x_t, const float* target, const float* t, const float* cross,
                const float* glob, const float* lw, double* loss_out) {
    const int B = d->tr.batch;
    const bool graph = d->use_graph && d->warm && !ctx->prof_on;
    bool launched = false;
    if (graph) {
        const int gi = d->dirty ? 1 : 0;
        const void* key[7] = {x_t, target, t, cross, glob, lw, d->local_in};
        bool have = d->gexec[gi] != nullptr;
        for (int k = 0; k < 7 && have; ++k) have = d->gkey[gi][k] == key[k];
        if (!have) have = capture(ctx, d, gi, key, x_t, target, t, cross, glob, lw);
        if (have) {
            SA3K_HIP(hipGraphLaunch(d->gexec[gi], ctx->stream));
            d->dirty = false;
            launched = true;
        }
    }
    if (!launched) {
        accumulate_body(ctx, d, x_t, target, t, cross, glob, lw);
        d->warm = true;   // the split-K workspace has its final size: later steps can be captured
    }
    d->count += B;
    if (loss_out) {
        SA3K_HIP(hipMemcpyAsync(loss_out, d->loss, sizeof(double) * B, hipMemcpyDeviceToHost, ctx->stream));
        sa3k_note_main(ctx);
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
    }
}

}  // namespace

extern "C" {

SA3K_API int sa3k_dit_create(sa3k_ctx* ctx, const sa3k_dit_config* cfg, int weight_type, sa3k_dit** out) {
    return sa3k_guard(ctx, "sa3k_dit_create", [&] {
        SA3K_REQUIRE(cfg && out, "null pointer");
        *out = nullptr;
        SA3K_REQUIRE(weight_type == SA3K_TYPE_F32 || weight_type == SA3K_TYPE_F16 || weight_type == SA3K_TYPE_BF16,
                     "weight type must be f32, f16 or bf16");
        SA3K_REQUIRE(cfg->head_dim == 64 && cfg->dim == cfg->heads * 64, "dim must be heads * 64");
        SA3K_REQUIRE(cfg->depth > 0 && cfg->mem_tokens >= 0 && cfg->time_dim % 2 == 0 && cfg->time_dim >= 4,
                     "depth / mem_tokens / time_dim");
        for (int v : {cfg->io, cfg->dim, cfg->cond_dim, cfg->time_dim, cfg->inner})
            SA3K_REQUIRE(v > 0 && v % 64 == 0, "io, dim, cond_dim, time_dim and inner must be multiples of 64");
        SA3K_REQUIRE(cfg->local_dim >= 0, "local_dim must be 0 (no inpaint conditioning) or positive");
        sa3k_dit* d = new sa3k_dit();
        d->cfg = *cfg;
        d->wtype = weight_type;
        if (const char* e = std::getenv("SA3K_DIT_GRAPH")) d->use_graph = std::atoi(e) != 0;
        try {
            describe(d);
            for (Tensor& t : d->tensors) SA3K_HIP(hipMalloc(&t.raw, t.bytes()));
        } catch (...) {
            free_dit(ctx, d);
            throw;
        }
        *out = d;
    });
}

SA3K_API int sa3k_dit_destroy(sa3k_ctx* ctx, sa3k_dit* dit) {
    return sa3k_guard(ctx, "sa3k_dit_destroy", [&] {
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
        free_dit(ctx, dit);
    });
}

SA3K_API int sa3k_dit_tensor_count(sa3k_ctx* ctx, const sa3k_dit* dit, int* count) {
    return sa3k_guard(ctx, "sa3k_dit_tensor_count", [&] {
        SA3K_REQUIRE(dit && count, "null pointer");
        *count = (int)dit->tensors.size();
    });
}

SA3K_API int sa3k_dit_tensor_info(sa3k_ctx* ctx, const sa3k_dit* dit, int i, char* name, int name_len, int64_t* rows,
                                  int64_t* cols, int* type) {
    return sa3k_guard(ctx, "sa3k_dit_tensor_info", [&] {
        SA3K_REQUIRE(dit && i >= 0 && i < (int)dit->tensors.size(), "bad tensor index");
        const Tensor& t = dit->tensors[i];
        if (name && name_len > 0) {
            SA3K_REQUIRE((int)t.name.size() < name_len, "name buffer too small");
            std::memcpy(name, t.name.c_str(), t.name.size() + 1);
        }
        if (rows) *rows = t.rows;
        if (cols) *cols = t.cols;
        if (type) *type = t.type;
    });
}

SA3K_API int sa3k_dit_set_tensor(sa3k_ctx* ctx, sa3k_dit* dit, const char* name, const void* data, int64_t bytes) {
    return sa3k_guard(ctx, "sa3k_dit_set_tensor", [&] {
        SA3K_REQUIRE(dit && name && data, "null pointer");
        SA3K_REQUIRE(!dit->ready, "tensors are fixed once the model is set up");
        Tensor& t = tensor(dit, name);
        SA3K_REQUIRE(bytes == (int64_t)t.bytes(), "byte count differs from the tensor's size: " + t.name);
        SA3K_HIP(hipMemcpyAsync(t.raw, data, t.bytes(), hipMemcpyDefault, ctx->stream));
        sa3k_note_main(ctx);
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
    });
}

SA3K_API int sa3k_dit_init_random(sa3k_ctx* ctx, sa3k_dit* dit, uint64_t seed, float w_sd) {
    return sa3k_guard(ctx, "sa3k_dit_init_random", [&] {
        SA3K_REQUIRE(dit, "null pointer");
        SA3K_REQUIRE(!dit->ready, "tensors are fixed once the model is set up");
        uint32_t stream = 1;
        for (Tensor& t : dit->tensors) {
            const int64_t n = t.rows * t.cols;
            float mean = 0.0f, sd = w_sd;
            if (t.kind == 1) sd = 0.02f;
            else if (t.kind == 2) sd = 0.1f;
            else if (t.kind == 3) { mean = 1.0f; sd = 0.1f; }
            else if (t.kind == 4) sd = 1.0f;
            launch(ctx, "dit_init", init_normal_kernel, dim3(nblk(ceil_div(n, 4))), t.raw, t.type, n, seed, stream++,
                   mean, sd);
        }
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
    });
}

SA3K_API int sa3k_dit_weight_row_norms(sa3k_ctx* ctx, sa3k_dit* dit, const char* name, int mode, float eps,
                                       float* out) {
    return sa3k_guard(ctx, "sa3k_dit_weight_row_norms", [&] {
        SA3K_REQUIRE(dit && name && out && (mode == 0 || mode == 1), "bad arguments");
        Tensor& t = tensor(dit, name);
        SA3K_REQUIRE(t.kind == 0, "not a 2-D weight: " + t.name);
        if (t.raw) {   // the stored tensor (before setup; local.0 keeps it, its built weight is padded)
            chk(ctx, sa3k_row_norms(ctx, t.type, t.cols, t.rows, t.raw, mode, eps, out));
            return;
        }
        // after setup: the built weight objects (the raw storage is released at setup)
        const sa3k_weight* w = nullptr;
        for (int l = 0; l < dit->cfg.depth && !w; ++l)
            for (int k = 0; k < 7; ++k)
                if (t.name == "dit." + std::to_string(l) + "." + kBlockTargets[k] + ".weight") w = dit->blocks[l]->W[k];
        for (int h = 0; h < H_N && !w; ++h)
            if (t.name == std::string("dit.") + kHeadNames[h] + ".weight") w = dit->hw[h];
        for (size_t k = 0; k < dit->lw.size() && !w; ++k)
            if (t.name == "dit." + std::to_string(k / 2) + "." + kLocalNames[k % 2] + ".weight") w = dit->lw[k];
        SA3K_REQUIRE(w != nullptr, "weight not found: " + t.name);
        chk(ctx, mode == 0 ? sa3k_weight_row_norms(ctx, w, out) : sa3k_weight_row_norm_sq(ctx, w, eps, out));
    });
}

SA3K_API int sa3k_dit_setup(sa3k_ctx* ctx, sa3k_dit* dit, const sa3k_dit_train* train) {
    return sa3k_guard(ctx, "sa3k_dit_setup", [&] {
        SA3K_REQUIRE(dit && train, "null pointer");
        setup(ctx, dit, *train);
    });
}

SA3K_API int sa3k_dit_resident_bytes(sa3k_ctx* ctx, const sa3k_dit* dit, const sa3k_dit_train* train,
                                     size_t* bytes) {
    return sa3k_guard(ctx, "sa3k_dit_resident_bytes", [&] {
        SA3K_REQUIRE(dit && train && bytes, "null pointer");
        SA3K_REQUIRE(train->batch > 0 && train->frames > 0 && train->ctx_tokens > 0, "batch / frames / ctx_tokens");
        const sa3k_dit_config& c = dit->cfg;
        const sa3k_block_config bc{c.dim, c.heads, c.head_dim, c.inner, c.rope_dims, c.window, c.rope_base,
                                   c.norm_eps, c.qk_eps};
        // the resident schedule keeps depth workspaces where the recompute schedule keeps one; every
        // workspace after the first shares its backward scratch with the first
        sa3k_block_ws shape{};
        shape.B = train->batch; shape.S = c.mem_tokens + train->frames; shape.Ctx = train->ctx_tokens;
        shape.dim = c.dim; shape.inner = c.inner; shape.H = c.heads;
        size_t per = 0;
        shape.act_bf16 = ctx->act_bf16;
        block_ws_build(bc, shape.B, shape.S, shape.Ctx, &shape, ctx->act_bf16, &per);
        *bytes = per * (size_t)(c.depth - 1);
    });
}

SA3K_API int sa3k_dit_arena(sa3k_ctx* ctx, sa3k_dit* dit, int which, float** ptr, int64_t* n) {
    return sa3k_guard(ctx, "sa3k_dit_arena", [&] {
        SA3K_REQUIRE(dit && dit->ready, "the model is not set up");
        SA3K_REQUIRE(which >= 0 && which <= 3, "which: 0 params, 1 grads, 2 m, 3 v");
        float* const a[4] = {dit->p, dit->g, dit->m, dit->v};
        if (ptr) *ptr = a[which];
        if (n) *n = dit->n_params;
    });
}

SA3K_API int sa3k_dit_target_count(sa3k_ctx* ctx, const sa3k_dit* dit, int* count) {
    return sa3k_guard(ctx, "sa3k_dit_target_count", [&] {
        SA3K_REQUIRE(dit && dit->ready && count, "the model is not set up");
        *count = (int)dit->targets.size();
    });
}

SA3K_API int sa3k_dit_target_info(sa3k_ctx* ctx, const sa3k_dit* dit, int i, char* name, int name_len, int64_t* in,
                                  int64_t* out, int64_t* off_a, int64_t* off_b, int64_t* off_m) {
    return sa3k_guard(ctx, "sa3k_dit_target_info", [&] {
        SA3K_REQUIRE(dit && dit->ready && i >= 0 && i < (int)dit->targets.size(), "bad target index");
        const Target& t = dit->targets[i];
        if (name && name_len > 0) {
            SA3K_REQUIRE((int)t.name.size() < name_len, "name buffer too small");
            std::memcpy(name, t.name.c_str(), t.name.size() + 1);
        }
        if (in) *in = t.in;
        if (out) *out = t.out;
        if (off_a) *off_a = t.off_a;
        if (off_b) *off_b = t.off_b;
        if (off_m) *off_m = t.off_m;
    });
}

SA3K_API int sa3k_dit_adapters_init(sa3k_ctx* ctx, sa3k_dit* dit, uint64_t seed, float b_sd) {
    return sa3k_guard(ctx, "sa3k_dit_adapters_init", [&] {
        SA3K_REQUIRE(dit && dit->ready, "the model is not set up");
        const int r = dit->tr.rank;
        uint32_t stream = 1u << 20;
        for (size_t i = 0; i < dit->targets.size(); ++i) {
            const Target& t = dit->targets[i];
            const float bound = 1.0f / sqrtf((float)t.in);
            launch(ctx, "dit_init", init_uniform_kernel, dim3(nblk(ceil_div((int64_t)r * t.in, 4))), dit->p + t.off_a,
                   (int64_t)r * t.in, seed, stream++, -bound, bound);
            if (b_sd > 0.0f)
                launch(ctx, "dit_init", init_normal_kernel, dim3(nblk(ceil_div(t.out * r, 4))), (void*)(dit->p + t.off_b),
                       (int)SA3K_TYPE_F32, t.out * r, seed, stream++, 0.0f, b_sd);
            else
                fill(ctx, dit->p + t.off_b, t.out * r, 0.0f);
            if (dit->tr.dora) {
                // the target's base weight: a block projection or a head/tail linear
                const sa3k_weight* w = nullptr;
                for (int l = 0; l < dit->cfg.depth && !w; ++l)
                    for (int k = 0; k < 7; ++k)
                        if (dit->block_target[(size_t)l * 7 + k] == (int)i) w = dit->blocks[l]->W[k];
                for (int h = 0; h < H_N && !w; ++h)
                    if (dit->head_target[h] == (int)i) w = dit->hw[h];
                for (size_t k = 0; k < dit->ll.size() && !w; ++k)   // local.0 padded: zero columns add nothing
                    if (dit->local_target[k] == (int)i) w = dit->lw[k];
                SA3K_REQUIRE(w != nullptr, "target without a weight");
                chk(ctx, sa3k_weight_row_norms(ctx, w, dit->p + t.off_m));
            }
        }
        fill(ctx, dit->g, dit->n_params, 0.0f);
        fill(ctx, dit->m, dit->n_params, 0.0f);
        fill(ctx, dit->v, dit->n_params, 0.0f);
        dit->count = 0;
        dit->dirty = true;
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
    });
}

SA3K_API int sa3k_dit_adapters_changed(sa3k_ctx* ctx, sa3k_dit* dit) {
    return sa3k_guard(ctx, "sa3k_dit_adapters_changed", [&] {
        SA3K_REQUIRE(dit, "null pointer");
        dit->dirty = true;
    });
}

SA3K_API int sa3k_dit_accumulate(sa3k_ctx* ctx, sa3k_dit* dit, const float* x_t, const float* target, const float* t,
                                 const float* cross, const float* glob, const float* loss_weight, double* loss_out) {
    return sa3k_guard(ctx, "sa3k_dit_accumulate", [&] {
        SA3K_REQUIRE(dit && dit->ready, "the model is not set up");
        SA3K_REQUIRE(x_t && target && t && cross && glob, "training step inputs are empty");
        accumulate(ctx, dit, x_t, target, t, cross, glob, loss_weight, loss_out);
    });
}

SA3K_API int sa3k_dit_apply_adamw(sa3k_ctx* ctx, sa3k_dit* dit, const sa3k_adamw_params* hp, int step,
                                  double* grad_norm_out) {
    return sa3k_guard(ctx, "sa3k_dit_apply_adamw", [&] {
        SA3K_REQUIRE(dit && dit->ready && hp, "the model is not set up");
        SA3K_REQUIRE(dit->count > 0, "no accumulated gradients");   // src/train_loop.h:176-179
        chk(ctx, sa3k_adamw_clip(ctx, dit->p, dit->g, dit->m, dit->v, dit->n_params, hp, step, dit->count,
                                 grad_norm_out));
        fill(ctx, dit->g, dit->n_params, 0.0f);
        dit->count = 0;
        dit->dirty = true;
    });
}

SA3K_API int sa3k_dit_set_local(sa3k_ctx* ctx, sa3k_dit* dit, const float* local) {
    return sa3k_guard(ctx, "sa3k_dit_set_local", [&] {
        SA3K_REQUIRE(dit && dit->ready, "the model is not set up");
        SA3K_REQUIRE(!local || dit->cfg.local_dim > 0, "the model has no local-conditioning linears (local_dim 0)");
        dit->local_in = local;
    });
}

SA3K_API int sa3k_dit_set_graphs(sa3k_ctx* ctx, sa3k_dit* dit, int on) {
    return sa3k_guard(ctx, "sa3k_dit_set_graphs", [&] {
        SA3K_REQUIRE(dit, "null pointer");
        dit->use_graph = on != 0;
        for (hipGraphExec_t& e : dit->gexec)
            if (e) {
                SA3K_HIP(hipGraphExecDestroy(e));
                e = nullptr;
            }
    });
}

SA3K_API int sa3k_dit_get_graphs(sa3k_ctx* ctx, sa3k_dit* dit, int* on) {
    return sa3k_guard(ctx, "sa3k_dit_get_graphs", [&] {
        SA3K_REQUIRE(dit && on, "null pointer");
        *on = dit->use_graph ? 1 : 0;
    });
}

SA3K_API int sa3k_dit_eval_loss(sa3k_ctx* ctx, sa3k_dit* dit, const float* x_t, const float* target, const float* t,
                                const float* cross, const float* glob, const float* loss_weight, double* loss_out) {
    return sa3k_guard(ctx, "sa3k_dit_eval_loss", [&] {
        SA3K_REQUIRE(dit && dit->ready, "the model is not set up");
        SA3K_REQUIRE(x_t && target && t && cross && glob, "evaluation inputs are empty");
        SA3K_REQUIRE(loss_out != nullptr, "loss_out is null");
        forward(ctx, dit, x_t, t, cross, glob);
        loss_and_seed(ctx, dit, target, loss_weight);
        SA3K_HIP(hipMemcpyAsync(loss_out, dit->loss, sizeof(double) * dit->tr.batch, hipMemcpyDeviceToHost,
                                ctx->stream));
        sa3k_note_main(ctx);
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
    });
}

SA3K_API int sa3k_dit_forward(sa3k_ctx* ctx, sa3k_dit* dit, const float* x_t, const float* t, const float* cross,
                              const float* glob, float* velocity) {
    return sa3k_guard(ctx, "sa3k_dit_forward", [&] {
        SA3K_REQUIRE(dit && dit->ready, "the model is not set up");
        SA3K_REQUIRE(x_t && t && cross && glob && velocity, "null pointer");
        forward(ctx, dit, x_t, t, cross, glob);
        const int64_t n = (int64_t)dit->tr.batch * dit->tr.frames * dit->cfg.io;
        SA3K_HIP(hipMemcpyAsync(velocity, dit->vel, sizeof(float) * n, hipMemcpyDeviceToDevice, ctx->stream));
        sa3k_note_main(ctx);
    });
}

}  // extern "C"
