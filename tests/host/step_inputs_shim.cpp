// C-ABI shim over the host mirror's step-input producers (sa3/train_diffusion.h, sa3/train_inpaint.h,
// sa3/dist_shift.h), compiled by tests/test_host_step_inputs.py and loaded with ctypes. Same call
// shapes as the reference shim (oracle/ref_shim.cpp) so the two can be compared value for value.
#include "sa3/dist_shift.h"
#include "sa3/train_diffusion.h"
#include "sa3/train_inpaint.h"

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

extern "C" {

int host_diffusion_samples(uint64_t seed, const char* mode, const float* z, int64_t n, int count, float* t,
                           float* noise, float* x_t, float* v, char* state, int state_len) {
    sa3::TrainDiffusionSampler s(seed, mode);
    const std::vector<float> zz(z, z + n);
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

// draw_t + sample_at with a warped t, and a save/restore in the middle: returns 0 when the restored
// sampler continues the sequence exactly and sample_at reproduces sample
int host_diffusion_continuation(uint64_t seed, const char* mode, const float* z, int64_t n) {
    const std::vector<float> zz(z, z + n);
    std::string err;
    sa3::TrainDiffusionSampler a(seed, mode), b(seed, mode);
    sa3::TrainDiffusionSample sa, sb;
    if (!a.sample(zz, sa, err) || !b.sample_at(zz, b.draw_t(), sb, err)) return 1;
    if (sa.t != sb.t || sa.noise != sb.noise || sa.x_t != sb.x_t) return 2;
    const std::string st = a.serialize_state();
    sa3::TrainDiffusionSampler c(seed + 1, mode);
    if (!c.restore_state(st, err)) return 3;
    if (!a.sample(zz, sa, err) || !c.sample(zz, sb, err)) return 4;
    if (sa.t != sb.t || sa.noise != sb.noise) return 5;
    sa3::TrainDiffusionSample e;
    if (a.sample({}, e, err)) return 6;   // empty latent rejected
    if (c.restore_state("not a state", err)) return 7;
    return 0;
}

double host_norm_icdf(double p) { return sa3::sa3_norm_icdf(p); }
double host_norm_cdf(double x) { return sa3::sa3_norm_cdf(x); }

void host_inpaint_masks(uint64_t seed, int frames, int real_len, const double* probs, int n_probs, int count,
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

void host_build_train_inpaint(const float* z, const float* mask, int io, int frames, int local_dim,
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

float host_dist_shift_warp(const char* type, float t, int seq_len, float p1, float p2, float p3, float p4) {
    return sa3::dist_shift_warp(type, t, seq_len, p1, p2, p3, p4);
}

void host_dist_shift_defaults(const char* type, float* p) {
    sa3::dist_shift_defaults(type, p[0], p[1], p[2], p[3]);
}

void host_expo_features(float t, float* out, int dim, float min_f, float max_f) {
    std::vector<float> v;
    sa3::expo_features(t, v, dim, min_f, max_f);
    std::memcpy(out, v.data(), v.size() * sizeof(float));
}

}  // extern "C"
