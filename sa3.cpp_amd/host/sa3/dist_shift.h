// dist_shift.h - the step-schedule helpers of the reference's src/sa3_pipeline.h:57-118 that a
// training step uses: expo_features (the timestep's Fourier features) and dist_shift_warp /
// dist_shift_defaults (the distribution shift applied to a drawn t before noising). Same names,
// arguments and float arithmetic. The DiT step computes the timestep features on the device from
// t (sa3k_dit_accumulate); the host version here is the same function for callers that need it.
#pragma once

#include <algorithm>
#include <cmath>
#include <string>
#include <vector>

namespace sa3 {

// dim features of t: out[i] = cos(2 pi t f_i), out[dim/2 + i] = sin(2 pi t f_i), with the dim/2
// frequencies f_i log-spaced from min_f to max_f (f_0 = min_f alone when dim/2 == 1)
inline void expo_features(float t, std::vector<float>& out, int dim, float min_f, float max_f) {
    const int half = dim / 2;
    const float log_lo = std::log(min_f), log_hi = std::log(max_f);
    constexpr float two_pi = 6.28318530717958648f;
    out.resize((size_t)dim);
    for (int i = 0; i < half; ++i) {
        const float frac = half > 1 ? (float)i / (float)(half - 1) : 0.0f;
        const float arg = t * std::exp(frac * (log_hi - log_lo) + log_lo) * two_pi;
        out[(size_t)i] = std::cos(arg);
        out[(size_t)(half + i)] = std::sin(arg);
    }
}

// Warp of one t in (0,1) for a sequence of seq_len latent frames. type and (p1..p4):
//   "LogSNR" (anchor_length, anchor_logsnr, rate, logsnr_end): the log-SNR runs linearly in t from
//            logsnr_end down to anchor_logsnr - rate log2(seq_len / anchor_length); t' =
//            sigmoid(-logsnr)
//   "Flux"   (min_length, max_length, alpha_min, alpha_max): alpha interpolated log-linearly in
//            log(seq_len clamped to [min, max]); t' = alpha t / (1 + (alpha - 1) t); parameters
//            that would take a log of a non-positive value leave t unchanged
//   "Full"   (base_shift, max_shift, min_length, max_length): mu = -(base + (max - base) x) with x
//            the clamped length's position in [min, max]; t' = 1 - e^mu / (e^mu + t / (1 - t));
//            an empty or negative length range leaves t unchanged
//   anything else ("None"): t unchanged
inline float dist_shift_warp(const std::string& type, float t, int seq_len, float p1, float p2, float p3, float p4) {
    const float len = (float)seq_len;
    if (type == "LogSNR") {
        const float start = p2 - p3 * std::log2(len / p1);
        const float logsnr = p4 - t * (p4 - start);
        return 1.0f / (1.0f + std::exp(logsnr));
    }
    if (type == "Flux") {
        const float lo = p1, hi = p2, a_lo = p3, a_hi = p4;
        if (lo <= 0.0f || hi <= 0.0f || hi < lo || a_lo <= 0.0f || a_hi <= 0.0f) return t;
        const float clamped = std::min(std::max(len, lo), hi);
        const float log_lo = std::log(lo);
        float log_hi = std::log(hi);
        if (log_hi == log_lo) log_hi += 1e-8f;   // equal bounds: a constant alpha
        const float x = (std::log(clamped) - log_lo) / (log_hi - log_lo);
        const float la = std::log(std::max(a_lo, 1e-8f)), lb = std::log(std::max(a_hi, 1e-8f));
        const float alpha = std::exp(la + x * (lb - la));
        return alpha * t / (1.0f + (alpha - 1.0f) * t);
    }
    if (type == "Full") {
        const float base = p1, top = p2, lo = p3, hi = p4;
        if (hi <= lo || hi <= 0.0f || lo < 0.0f) return t;
        const float clamped = std::min(std::max(len, lo), hi);
        const float mu = -(base + (top - base) * (clamped - lo) / (hi - lo));
        const float em = std::exp(mu);
        return 1.0f - em / (em + t / (1.0f - t));
    }
    return t;
}

// the (p1..p4) a type uses when none are given: the configurations the model ships with
inline void dist_shift_defaults(const std::string& type, float& p1, float& p2, float& p3, float& p4) {
    if (type == "Flux") {
        p1 = 256.0f, p2 = 4096.0f, p3 = 6.93f, p4 = 6.93f;
    } else if (type == "Full") {
        p1 = 0.5f, p2 = 1.15f, p3 = 256.0f, p4 = 4096.0f;
    } else if (type == "None") {
        p1 = p2 = p3 = p4 = 0.0f;
    } else {   // LogSNR
        p1 = 2000.0f, p2 = -6.2f, p3 = 0.0f, p4 = 2.0f;
    }
}

}  // namespace sa3
