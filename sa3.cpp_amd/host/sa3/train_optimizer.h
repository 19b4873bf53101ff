// train_optimizer.h - AdamW for native SA3 LoRA training, the interface of the reference's
// src/train_optimizer.h:20-66 (same names, fields, defaults, argument meaning and bool/err
// convention); the update itself runs on the GPU (sa3k_adamw_clip), bit-identical to the
// reference's host float loop.
#pragma once

#include "sa3k_host.h"

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <string>
#include <vector>

namespace sa3 {

// InverseLR learning-rate schedule (src/train_optimizer.h:11-27), step0 = 0-indexed optimizer step:
//   lr = (1 - warmup^(step0+1)) * max(final_lr, base_lr * (1 + step0/inv_gamma)^(-power))
// evaluated in double and returned as float; warmup 0 disables the warmup factor. A scalar of the
// host schedule, not GPU work.
inline float inverse_lr(float base_lr, int step0, float inv_gamma, float power, float warmup, float final_lr) {
    const double n = (double)step0;
    const double warm = warmup > 0.0f ? 1.0 - std::pow((double)warmup, n + 1.0) : 1.0;
    const double mult = std::pow(1.0 + n / (double)inv_gamma, -(double)power);
    return (float)(warm * std::max((double)final_lr, (double)base_lr * mult));
}

struct TrainAdamWParams {
    float learning_rate = 1.0e-4f;
    float beta1 = 0.9f;
    float beta2 = 0.999f;
    float eps = 1.0e-8f;
    float weight_decay = 0.0f;
    float grad_clip = 0.0f;   // global gradient-norm clip; 0 = off (reference training uses 1.0)
};

struct TrainAdamWTensorState {
    std::vector<float> m;
    std::vector<float> v;
};

// One AdamW step of one tensor (src/train_optimizer.h:42-66): rejects a size mismatch and
// step <= 0 with err; zero-initialises a moment state of the wrong size; no clip, no averaging.
inline bool adamw_update_vector(std::vector<float>& param, const std::vector<float>& grad,
                                TrainAdamWTensorState& state, const TrainAdamWParams& hp, int step,
                                std::string& err) {
    if (param.size() != grad.size()) {
        err = "AdamW parameter/gradient size mismatch";
        return false;
    }
    if (step <= 0) {
        err = "AdamW step must be positive";
        return false;
    }
    if (state.m.size() != param.size()) state.m.assign(param.size(), 0.0f);
    if (state.v.size() != param.size()) state.v.assign(param.size(), 0.0f);
    if (param.empty()) return true;
    sa3k_ctx* ctx = sa3k_default_ctx(err);
    if (!ctx) return false;
    const size_t n = param.size();
    DeviceF32 buf;   // [p | g | m | v]
    if (!buf.alloc(ctx, 4 * n, err) || !buf.upload(param.data(), n, 0, err) || !buf.upload(grad.data(), n, n, err) ||
        !buf.upload(state.m.data(), n, 2 * n, err) || !buf.upload(state.v.data(), n, 3 * n, err))
        return false;
    sa3k_adamw_params p{hp.learning_rate, hp.beta1, hp.beta2, hp.eps, hp.weight_decay, 0.0f};
    float* b = buf.get();
    if (sa3k_adamw_clip(ctx, b, b + n, b + 2 * n, b + 3 * n, (int64_t)n, &p, step, 1, nullptr) != SA3K_OK)
        return sa3k_fail(ctx, err);
    return buf.download(param.data(), n, 0, err) && buf.download(state.m.data(), n, 2 * n, err) &&
           buf.download(state.v.data(), n, 3 * n, err);
}

}  // namespace sa3
