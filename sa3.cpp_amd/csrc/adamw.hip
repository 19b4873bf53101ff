// K6: fused mean + global-L2-clip + AdamW over one flat f32 arena of adapter parameters.
//
// Reference semantics: train_average_and_clip (src/train_loop.h:147-171) followed by
// adamw_update_vector (src/train_optimizer.h:42-66) for every tensor, as sequenced by
// train_apply_accumulated_adamw (src/train_loop.h:173-211). The element update repeats the
// reference's float expression tree operation by operation; this file is compiled with
// -ffp-contract=off so no multiply-add is fused, and HIP's float '/' and sqrtf are IEEE
// correctly rounded, so every element is bit-identical to the host loop given the same clip scale.
//
// Two launches, both HBM-bound (32 bytes of traffic per parameter in total):
//   pass 1  reads g once: per-block double partial sums of (g*inv)^2 (deterministic order)
//   pass 2  every block re-reduces the same partials in the same order (so all blocks agree on
//           norm and scale without a third launch), then streams p, g, m, v -> p, m, v.
// Pass 2 moves p, m and v with non-temporal loads and stores: its 24 bytes per parameter then
// neither evict the gradients that pass 1 just brought into the memory-side cache nor leave dirty
// lines that the next pass 1 must wait behind (measured at 48M parameters: pass 1 63 -> 30 us).
#include "sa3k_internal.h"

#include <cmath>

namespace {

constexpr int kThreads = 256;
constexpr int kSumBlocks = 1024;
// float4 groups in flight per thread and iteration of the update pass (12 16-byte loads): measured
// on MI355X at 48M parameters, 2 / 3 / 4 groups 247 / 239 / 253 us
constexpr int kAdamwGroups = 3;

__device__ inline double block_sum_double(double v, double* sh) {
    // wave64 butterfly, then the 4 wave results in a fixed order
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    double t = 0.0;
    if (threadIdx.x == 0) {
        for (int w = 0; w < kThreads / 64; ++w) t += sh[w];
        sh[kThreads / 64] = t;
    }
    __syncthreads();
    t = sh[kThreads / 64];
    __syncthreads();
    return t;
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void adamw_sumsq_kernel(const float* __restrict__ g, int64_t n,
                                                                float inv, int avg,
                                                                double* __restrict__ partials) {
    __shared__ double sh[kThreads / 64 + 1];
    double acc = 0.0;
    const int64_t tid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    if (VEC) {
        const int64_t n4 = n >> 2;
        const float4* g4 = reinterpret_cast<const float4*>(g);
        auto add = [&](float4 x) {
            if (avg) { x.x = x.x * inv; x.y = x.y * inv; x.z = x.z * inv; x.w = x.w * inv; }
            acc += (double)x.x * x.x;
            acc += (double)x.y * x.y;
            acc += (double)x.z * x.z;
            acc += (double)x.w * x.w;
        };
        // Each block streams one contiguous chunk, eight 16-byte loads in flight per thread one
        // block-width (4 KiB) apart, the last batch guarded per lane; summed in index order.
        constexpr int U = 8;
        const int64_t chunk = (n4 + gridDim.x - 1) / gridDim.x;
        const int64_t beg = (int64_t)blockIdx.x * chunk, end = min(n4, beg + chunk);
        for (int64_t i = beg + threadIdx.x; i < end; i += U * kThreads) {
            float4 x[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t j = i + u * kThreads;
                x[u] = j < end ? g4[j] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) add(x[u]);
        }
        for (int64_t i = (n4 << 2) + tid; i < n; i += stride) {
            float x = g[i];
            if (avg) x = x * inv;
            acc += (double)x * x;
        }
    } else {
        for (int64_t i = tid; i < n; i += stride) {
            float x = g[i];
            if (avg) x = x * inv;
            acc += (double)x * x;
        }
    }
    const double s = block_sum_double(acc, sh);
    if (threadIdx.x == 0) partials[blockIdx.x] = s;
}

typedef float f32x4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ldnt4(const float4* p) {
    const f32x4v v = __builtin_nontemporal_load(reinterpret_cast<const f32x4v*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void stnt4(float4* p, float4 v) {
    __builtin_nontemporal_store(f32x4v{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4v*>(p));
}

struct AdamwScalars {
    float inv;        // 1/count (used when avg)
    int avg;          // count > 1
    float clip;       // grad_clip (<= 0: off)
    float lr, b1, b2, omb1, omb2, eps, wd;
    float b1c, b2c;   // 1 - powf(beta, step), computed on the host like the reference
};

__device__ inline float adamw_elem(float p, float g, float& m, float& v, const AdamwScalars& s,
                                   float scale, int do_clip) {
    if (s.avg) g = g * s.inv;
    if (do_clip) g = g * scale;
    const float mm = s.b1 * m + s.omb1 * g;
    const float vv = s.b2 * v + s.omb2 * g * g;
    m = mm;
    v = vv;
    const float mh = mm / s.b1c;
    const float vh = vv / s.b2c;
    return p - s.lr * (mh / (sqrtf(vh) + s.eps) + s.wd * p);
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void adamw_update_kernel(
    float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m, float* __restrict__ v,
    int64_t n, AdamwScalars s, const double* __restrict__ partials, int n_partials,
    double* __restrict__ result) {
    __shared__ double sh[kThreads / 64 + 1];
    // identical reduction in every block: thread t sums partials t, t+256, ... in order
    double acc = 0.0;
    for (int i = threadIdx.x; i < n_partials; i += kThreads) acc += partials[i];
    const double sumsq = block_sum_double(acc, sh);
    const double norm = sqrt(sumsq);
    int do_clip = 0;
    float scale = 1.0f;
    if (s.clip > 0.0f && norm > (double)s.clip) {
        scale = (float)((double)s.clip / (norm + 1e-6));
        do_clip = 1;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        result[0] = norm;
        result[1] = (double)scale;
    }
    const int64_t tid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    if (VEC) {
        const int64_t n4 = n >> 2;
        float4* p4 = reinterpret_cast<float4*>(p);
        const float4* g4 = reinterpret_cast<const float4*>(g);
        float4* m4 = reinterpret_cast<float4*>(m);
        float4* v4 = reinterpret_cast<float4*>(v);
        auto upd = [&](int64_t i, float4 pp, float4 gg, float4 mm, float4 vv) {
            pp.x = adamw_elem(pp.x, gg.x, mm.x, vv.x, s, scale, do_clip);
            pp.y = adamw_elem(pp.y, gg.y, mm.y, vv.y, s, scale, do_clip);
            pp.z = adamw_elem(pp.z, gg.z, mm.z, vv.z, s, scale, do_clip);
            pp.w = adamw_elem(pp.w, gg.w, mm.w, vv.w, s, scale, do_clip);
            stnt4(p4 + i, pp);
            stnt4(m4 + i, mm);
            stnt4(v4 + i, vv);
        };
        // each block updates one contiguous chunk, two float4 groups (one block-width apart) per
        // iteration: eight 16-byte loads in flight per thread. p, m, v are streamed with
        // non-temporal loads and stores, so the gradients the sum-of-squares pass just read can
        // stay in the memory-side cache for this pass
        const int64_t chunk = (n4 + gridDim.x - 1) / gridDim.x;
        const int64_t beg = (int64_t)blockIdx.x * chunk, end = min(n4, beg + chunk);
        int64_t i = beg + threadIdx.x;
        constexpr int U = kAdamwGroups;
        for (; i + (U - 1) * kThreads < end; i += U * kThreads) {
            float4 pp[U], gg[U], mm[U], vv[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t j = i + u * kThreads;
                pp[u] = ldnt4(p4 + j); gg[u] = g4[j]; mm[u] = ldnt4(m4 + j); vv[u] = ldnt4(v4 + j);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) upd(i + u * kThreads, pp[u], gg[u], mm[u], vv[u]);
        }
        for (; i < end; i += kThreads) upd(i, p4[i], g4[i], m4[i], v4[i]);
        for (int64_t i = (n4 << 2) + tid; i < n; i += stride) {
            float mm = m[i], vv = v[i];
            p[i] = adamw_elem(p[i], g[i], mm, vv, s, scale, do_clip);
            m[i] = mm;
            v[i] = vv;
        }
    } else {
        for (int64_t i = tid; i < n; i += stride) {
            float mm = m[i], vv = v[i];
            p[i] = adamw_elem(p[i], g[i], mm, vv, s, scale, do_clip);
            m[i] = mm;
            v[i] = vv;
        }
    }
}

// train_average_and_clip in place: g := g*inv (count > 1), then g := g*scale when clipping
__global__ __launch_bounds__(kThreads) void average_clip_kernel(float* __restrict__ g, int64_t n, float inv, int avg,
                                                                 float clip, const double* __restrict__ partials,
                                                                 int n_partials, double* __restrict__ result) {
    __shared__ double sh[kThreads / 64 + 1];
    double acc = 0.0;
    for (int i = threadIdx.x; i < n_partials; i += kThreads) acc += partials[i];
    const double norm = sqrt(block_sum_double(acc, sh));
    int do_clip = 0;
    float scale = 1.0f;
    if (clip > 0.0f && norm > (double)clip) {
        scale = (float)((double)clip / (norm + 1e-6));
        do_clip = 1;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        result[0] = norm;
        result[1] = (double)scale;
    }
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        float x = g[i];
        if (avg) x = x * inv;
        if (do_clip) x = x * scale;
        g[i] = x;
    }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace

extern "C" {

SA3K_API int sa3k_adamw_clip(sa3k_ctx* ctx, float* param, const float* grad, float* m, float* v,
                             int64_t n, const sa3k_adamw_params* hp, int step, int count,
                             double* grad_norm_out) {
    return sa3k_guard(ctx, "sa3k_adamw_clip", [&] {
        SA3K_REQUIRE(hp != nullptr, "hyper-parameters are null");
        SA3K_REQUIRE(step > 0, "AdamW step must be positive");
        SA3K_REQUIRE(count > 0, "cannot apply empty gradient batch");
        SA3K_REQUIRE(n >= 0, "negative element count");
        SA3K_REQUIRE(n == 0 || (param && grad && m && v), "null arena pointer");
        AdamwScalars s;
        s.avg = count > 1 ? 1 : 0;
        s.inv = 1.0f / (float)count;
        s.clip = hp->grad_clip;
        s.lr = hp->learning_rate;
        s.b1 = hp->beta1;
        s.b2 = hp->beta2;
        s.omb1 = 1.0f - hp->beta1;
        s.omb2 = 1.0f - hp->beta2;
        s.eps = hp->eps;
        s.wd = hp->weight_decay;
        s.b1c = 1.0f - std::pow(hp->beta1, (float)step);
        s.b2c = 1.0f - std::pow(hp->beta2, (float)step);
        const bool vec = aligned16(param) && aligned16(grad) && aligned16(m) && aligned16(v);
        const int64_t work = vec ? ceil_div(n, 4) : n;
        const int nb1 = (int)std::max<int64_t>(1, std::min<int64_t>(kSumBlocks, ceil_div(work, kThreads)));
        const int nb2 = (int)std::max<int64_t>(1, std::min<int64_t>(8192, ceil_div(work, kThreads * 2)));
        {
            KernelScope ks(ctx, "adamw_sumsq");
            if (vec)
                adamw_sumsq_kernel<true><<<nb1, kThreads, 0, ctx->stream>>>(grad, n, s.inv, s.avg, ctx->adamw_partials);
            else
                adamw_sumsq_kernel<false><<<nb1, kThreads, 0, ctx->stream>>>(grad, n, s.inv, s.avg, ctx->adamw_partials);
            SA3K_LAUNCHED();
        }
        {
            KernelScope ks(ctx, "adamw_update");
            if (vec)
                adamw_update_kernel<true><<<nb2, kThreads, 0, ctx->stream>>>(param, grad, m, v, n, s,
                                                                             ctx->adamw_partials, nb1, ctx->adamw_result);
            else
                adamw_update_kernel<false><<<nb2, kThreads, 0, ctx->stream>>>(param, grad, m, v, n, s,
                                                                              ctx->adamw_partials, nb1, ctx->adamw_result);
            SA3K_LAUNCHED();
        }
        if (grad_norm_out) {
            double r[2];
            SA3K_HIP(hipMemcpyAsync(r, ctx->adamw_result, sizeof r, hipMemcpyDeviceToHost, ctx->stream));
            sa3k_note_main(ctx);
            SA3K_HIP(hipStreamSynchronize(ctx->stream));
            *grad_norm_out = r[0];
        }
    });
}

SA3K_API int sa3k_average_and_clip(sa3k_ctx* ctx, float* grad, int64_t n, int count, float grad_clip,
                                   double* grad_norm_out) {
    return sa3k_guard(ctx, "sa3k_average_and_clip", [&] {
        SA3K_REQUIRE(count > 0, "cannot apply empty gradient batch");
        SA3K_REQUIRE(n >= 0 && (n == 0 || grad), "bad arena");
        const int avg = count > 1 ? 1 : 0;
        const float inv = 1.0f / (float)count;
        const bool vec = aligned16(grad);
        const int64_t work = vec ? ceil_div(n, 4) : n;
        const int nb1 = (int)std::max<int64_t>(1, std::min<int64_t>(kSumBlocks, ceil_div(work, kThreads)));
        const int nb2 = (int)std::max<int64_t>(1, std::min<int64_t>(8192, ceil_div(n, kThreads * 2)));
        {
            KernelScope ks(ctx, "adamw_sumsq");
            if (vec) adamw_sumsq_kernel<true><<<nb1, kThreads, 0, ctx->stream>>>(grad, n, inv, avg, ctx->adamw_partials);
            else adamw_sumsq_kernel<false><<<nb1, kThreads, 0, ctx->stream>>>(grad, n, inv, avg, ctx->adamw_partials);
            SA3K_LAUNCHED();
        }
        {
            KernelScope ks(ctx, "average_clip");
            average_clip_kernel<<<nb2, kThreads, 0, ctx->stream>>>(grad, n, inv, avg, grad_clip, ctx->adamw_partials, nb1,
                                                                  ctx->adamw_result);
            SA3K_LAUNCHED();
        }
        if (grad_norm_out) {
            double r[2];
            SA3K_HIP(hipMemcpyAsync(r, ctx->adamw_result, sizeof r, hipMemcpyDeviceToHost, ctx->stream));
            sa3k_note_main(ctx);
            SA3K_HIP(hipStreamSynchronize(ctx->stream));
            *grad_norm_out = r[0];
        }
    });
}

SA3K_API int sa3k_adamw_clip_scale(sa3k_ctx* ctx, double* norm_out, float* scale_out) {
    return sa3k_guard(ctx, "sa3k_adamw_clip_scale", [&] {
        double r[2];
        SA3K_HIP(hipMemcpyAsync(r, ctx->adamw_result, sizeof r, hipMemcpyDeviceToHost, ctx->stream));
        sa3k_note_main(ctx);
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
        if (norm_out) *norm_out = r[0];
        if (scale_out) *scale_out = (float)r[1];
    });
}

}  // extern "C"
