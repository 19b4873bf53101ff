// oracle: optimizer and clip — TEST INFRASTRUCTURE ONLY (see oracle.h).
// Float loops restated from the reference host code; compiled with -ffp-contract=off so that no
// multiply-add is fused (the reference's x86-64 build does not fuse them either).
#include "oracle.h"

#include <algorithm>
#include <cmath>

extern "C" {

// src/train_optimizer.h:20-27 (InverseLR closed form, double math, float result)
float orc_inverse_lr(float base_lr, int step0, float inv_gamma, float power, float warmup, float final_lr) {
    const double n = (double)step0;
    const double wf = (warmup > 0.0f) ? (1.0 - std::pow((double)warmup, n + 1.0)) : 1.0;
    const double lr_mult = std::pow(1.0 + n / (double)inv_gamma, -(double)power);
    return (float)(wf * std::max((double)final_lr, (double)base_lr * lr_mult));
}

// src/train_optimizer.h:42-66
int orc_adamw_update_vector(float* param, const float* grad, float* m, float* v, int64_t n,
                            float lr, float b1, float b2, float eps, float wd, int step) {
    if (step <= 0) return 1;
    const float b1_corr = 1.0f - std::pow(b1, (float)step);
    const float b2_corr = 1.0f - std::pow(b2, (float)step);
    for (int64_t i = 0; i < n; ++i) {
        const float g = grad[i];
        m[i] = b1 * m[i] + (1.0f - b1) * g;
        v[i] = b2 * v[i] + (1.0f - b2) * g * g;
        const float mh = m[i] / b1_corr;
        const float vh = v[i] / b2_corr;
        param[i] -= lr * (mh / (std::sqrt(vh) + eps) + wd * param[i]);
    }
    return 0;
}

// src/train_loop.h:147-171, over one arena that holds the tensors in the reference's visit order
void orc_average_and_clip(float* grad, int64_t n, int count, float grad_clip, double* norm_out,
                          float* scale_out) {
    if (count > 1) {
        const float inv = 1.0f / (float)count;
        for (int64_t i = 0; i < n; ++i) grad[i] *= inv;
    }
    double sumsq = 0.0;
    for (int64_t i = 0; i < n; ++i) sumsq += (double)grad[i] * grad[i];
    const double norm = std::sqrt(sumsq);
    if (norm_out) *norm_out = norm;
    float scale = 1.0f;
    if (grad_clip > 0.0f && norm > (double)grad_clip) {
        scale = (float)((double)grad_clip / (norm + 1e-6));
        for (int64_t i = 0; i < n; ++i) grad[i] *= scale;
    }
    if (scale_out) *scale_out = scale;
}

// src/train_loop.h:173-211 (one step increment, average + clip, then AdamW per tensor; the
// per-tensor split does not change any element's arithmetic, so one call covers the arena)
int orc_apply_accumulated_adamw(float* param, float* grad, float* m, float* v, int64_t n,
                                float lr, float b1, float b2, float eps, float wd, float clip,
                                int step, int count, double* norm_out, float* scale_out) {
    if (count <= 0) return 1;
    orc_average_and_clip(grad, n, count, clip, norm_out, scale_out);
    return orc_adamw_update_vector(param, grad, m, v, n, lr, b1, b2, eps, wd, step);
}

}  // extern "C"
