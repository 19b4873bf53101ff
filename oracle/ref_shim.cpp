// TEST INFRASTRUCTURE ONLY: a C-ABI shim over the reference's own std-only headers, compiled from
// where they lie (reference src/train_optimizer.h, src/train_diffusion.h, src/train_inpaint.h) by
// `make -C oracle ref` into oracle/_ref/libsa3ref.so. Tests and fixture scripts load it as the
// checker of the oracle and of the host mirror; nothing in the product links it. The headers need
// only the C++ standard library; the rest of the reference (ggml graphs) is not built.
#include "train_optimizer.h"
#include "train_diffusion.h"
#include "train_inpaint.h"

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

extern "C" {

float ref_inverse_lr(float base_lr, int step0, float inv_gamma, float power, float warmup, float final_lr) {
    return sa3::inverse_lr(base_lr, step0, inv_gamma, power, warmup, final_lr);
}

// sa3::adamw_update_vector on one tensor, state m/v in and out; returns 0 on success
int ref_adamw_update_vector(float* param, const float* grad, float* m, float* v, int64_t n, float lr, float b1,
                            float b2, float eps, float wd, int step) {
    std::vector<float> p(param, param + n), g(grad, grad + n);
    sa3::TrainAdamWTensorState st;
    st.m.assign(m, m + n);
    st.v.assign(v, v + n);
    sa3::TrainAdamWParams hp;
    hp.learning_rate = lr;
    hp.beta1 = b1;
    hp.beta2 = b2;
    hp.eps = eps;
    hp.weight_decay = wd;
    std::string err;
    if (!sa3::adamw_update_vector(p, g, st, hp, step, err)) return 1;
    std::memcpy(param, p.data(), n * sizeof(float));
    std::memcpy(m, st.m.data(), n * sizeof(float));
    std::memcpy(v, st.v.data(), n * sizeof(float));
    return 0;
}

// `count` draws of sa3::TrainDiffusionSampler(seed, mode).sample(z) in a row: t[count],
// noise/x_t/v [count][n]; then the serialized state after the draws into state (NUL-terminated,
// truncated to state_len); returns 0 on success
int ref_diffusion_samples(uint64_t seed, const char* mode, const float* z, int64_t n, int count, float* t,
                          float* noise, float* x_t, float* v, char* state, int state_len) {
    sa3::TrainDiffusionSampler s(seed, mode);
    std::vector<float> zz(z, z + n);
    for (int k = 0; k < count; ++k) {
        sa3::TrainDiffusionSample o;
        std::string err;
        if (!s.sample(zz, o, err)) return 1;
        t[k] = o.t;
        std::memcpy(noise + (int64_t)k * n, o.noise.data(), n * sizeof(float));
        std::memcpy(x_t + (int64_t)k * n, o.x_t.data(), n * sizeof(float));
        std::memcpy(v + (int64_t)k * n, o.velocity_target.data(), n * sizeof(float));
    }
    if (state && state_len > 0) {
        const std::string st = s.serialize_state();
        std::strncpy(state, st.c_str(), (size_t)state_len - 1);
        state[state_len - 1] = 0;
    }
    return 0;
}

// `count` masks of sa3::generate_inpaint_mask from one std::mt19937_64(seed): masks [count][frames],
// types [count]
void ref_inpaint_masks(uint64_t seed, int frames, int real_len, const double* probs, int n_probs, int count,
                       int mask_padding, int max_mask_segments, int max_spans, double ratio_lo, double ratio_hi,
                       const double* span_w, int n_span_w, float* masks, int* types) {
    std::mt19937_64 rng(seed);
    const std::vector<double> p(probs, probs + n_probs), w(span_w, span_w + n_span_w);
    for (int k = 0; k < count; ++k) {
        sa3::InpaintMaskType ty;
        const std::vector<float> m = sa3::generate_inpaint_mask(frames, real_len, p, rng, ty, mask_padding != 0,
                                                                max_mask_segments, max_spans, ratio_lo, ratio_hi, w);
        std::memcpy(masks + (int64_t)k * frames, m.data(), (size_t)frames * sizeof(float));
        types[k] = (int)ty;
    }
}

// sa3::build_train_inpaint: local [frames][local_dim], weight [frames][io], counts {n_gen, n_ctx}
void ref_build_train_inpaint(const float* z, const float* mask, int io, int frames, int local_dim,
                             float mask_loss_weight, int mask_padding_attention, float* local, float* weight,
                             int* counts) {
    const std::vector<float> zz(z, z + (int64_t)io * frames), mm(mask, mask + frames);
    const sa3::TrainInpaint r = sa3::build_train_inpaint(zz, mm, io, frames, local_dim, mask_loss_weight,
                                                         mask_padding_attention != 0);
    std::memcpy(local, r.local.data(), r.local.size() * sizeof(float));
    std::memcpy(weight, r.loss_weight.data(), r.loss_weight.size() * sizeof(float));
    counts[0] = r.n_gen;
    counts[1] = r.n_ctx;
}

}  // extern "C"
