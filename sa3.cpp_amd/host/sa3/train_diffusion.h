// train_diffusion.h - the rectified-flow step inputs of the reference's src/train_diffusion.h:12-125:
// TrainDiffusionSample, TrainDiffusionSampler (timestep draw "uniform" / "trunc_logit_normal",
// noising, velocity target, state save/restore) and the normal CDF / inverse CDF it uses. Same
// names, fields, argument meaning and bool/err convention.
//
// The sampler is host code on purpose: a training trajectory is the reference's only if t and the
// noise come from the same generator in the same order (std::mt19937_64 with the standard library's
// uniform_real_distribution<float> and normal_distribution<float>, drawn per element in latent
// order), and one sample is 64 x 1024 floats, uploaded with the step's other inputs. The DiT step
// itself (sa3k_dit_accumulate) takes x_t, the velocity target and t.
#pragma once

#include <algorithm>
#include <cmath>
#include <random>
#include <sstream>
#include <string>
#include <vector>

namespace sa3 {

struct TrainDiffusionSample {
    float t = 0.0f;
    std::vector<float> noise;
    std::vector<float> x_t;              // [io, T] (ggml order: T rows of io)
    std::vector<float> velocity_target;  // [io, T]
};

// Phi(x) = erfc(-x / sqrt 2) / 2, with 1/sqrt 2 as the nearest double (a multiply, not a divide)
inline double sa3_norm_cdf(double x) { return 0.5 * std::erfc(-x * 0.70710678118654752440); }

// Phi^-1(p) by P. J. Acklam's rational approximation (relative error below 1.15e-9): a central
// rational function on [0.02425, 0.97575] and a tail function in sqrt(-2 ln p) outside it, the
// upper tail by symmetry. p <= 0 gives -1e9 and p >= 1 gives 1e9.
inline double sa3_norm_icdf(double p) {
    if (p <= 0.0) return -1e9;
    if (p >= 1.0) return 1e9;
    // Acklam's published coefficients: central numerator a, denominator b; tail numerator c,
    // denominator d (evaluated by Horner's rule, highest order first)
    static const double a[6] = {-3.969683028665376e+01, 2.209460984245205e+02, -2.759285104469687e+02,
                                1.383577518672690e+02,  -3.066479806614716e+01, 2.506628277459239e+00};
    static const double b[5] = {-5.447609879822406e+01, 1.615858368580409e+02, -1.556989798598866e+02,
                                6.680131188771972e+01,  -1.328068155288572e+01};
    static const double c[6] = {-7.784894002430293e-03, -3.223964580411365e-01, -2.400758277161838e+00,
                                -2.549732539343734e+00, 4.374664141464968e+00,  2.938163982698783e+00};
    static const double d[4] = {7.784695709041462e-03, 3.224671290700398e-01, 2.445134137142996e+00,
                                3.754408661907416e+00};
    auto horner = [](const double* k, int n, double x) {
        double y = k[0];
        for (int i = 1; i < n; ++i) y = y * x + k[i];
        return y;
    };
    auto tail = [&](double q) { return horner(c, 6, q) / (horner(d, 4, q) * q + 1.0); };
    constexpr double p_low = 0.02425;
    if (p < p_low) return tail(std::sqrt(-2.0 * std::log(p)));
    if (p > 1.0 - p_low) return -tail(std::sqrt(-2.0 * std::log(1.0 - p)));
    const double q = p - 0.5, r = q * q;
    return horner(a, 6, r) * q / (horner(b, 5, r) * r + 1.0);
}

class TrainDiffusionSampler {
public:
    explicit TrainDiffusionSampler(unsigned long long seed, const std::string& mode = "uniform")
        : engine_(seed), mode_(mode) {}

    // one draw of t, then the noising of z at it
    bool sample(const std::vector<float>& z, TrainDiffusionSample& out, std::string& err) {
        return sample_at(z, draw_t(), out, err);
    }

    // the noising at a given t (the caller may warp a drawn t first):
    //   noise_i ~ N(0,1) in element order, x_t = (1 - t) z + t noise, velocity target = noise - z
    bool sample_at(const std::vector<float>& z, float t, TrainDiffusionSample& out, std::string& err) {
        if (z.empty()) {
            err = "latent vector is empty";
            return false;
        }
        const size_t n = z.size();
        out.t = t;
        out.noise.assign(n, 0.0f);
        out.x_t.assign(n, 0.0f);
        out.velocity_target.assign(n, 0.0f);
        const float keep = 1.0f - t;
        for (size_t i = 0; i < n; ++i) {
            const float e = gauss_(engine_);
            out.noise[i] = e;
            out.x_t[i] = keep * z[i] + t * e;
            out.velocity_target[i] = e - z[i];
        }
        return true;
    }

    // "uniform": t ~ U(0,1). "trunc_logit_normal": a logit-normal t truncated below at 0.075 and
    // rescaled to [0,1], then flipped (t -> 1 - t): u = Phi(e) for e ~ N(0,1) is mapped into
    // [Phi(logit 0.075), 1], clamped to [1e-7, 1 - 1e-7], pushed through sigmoid(Phi^-1(.)).
    float draw_t() {
        if (mode_ != "trunc_logit_normal") return unit_(engine_);
        constexpr double left = 0.075;
        const double lower = sa3_norm_cdf(std::log(left / (1.0 - left)));
        const double u = sa3_norm_cdf((double)gauss_(engine_));
        double p = lower + (1.0 - lower) * u;
        p = std::min(std::max(p, 1e-7), 1.0 - 1e-7);
        const double s = 1.0 / (1.0 + std::exp(-sa3_norm_icdf(p)));
        return (float)(1.0 - (s - left) / (1.0 - left));
    }

    // the engine and both distributions (normal_distribution keeps a cached second variate), in
    // the standard stream format, so a restored sampler continues the same sequence
    std::string serialize_state() const {
        std::ostringstream os;
        os << engine_ << '\n' << unit_ << '\n' << gauss_;
        return os.str();
    }

    bool restore_state(const std::string& state, std::string& err) {
        std::istringstream is(state);
        std::mt19937_64 engine;
        std::uniform_real_distribution<float> unit;
        std::normal_distribution<float> gauss;
        if (!(is >> engine >> unit >> gauss)) {
            err = "invalid diffusion sampler state";
            return false;
        }
        engine_ = engine;
        unit_ = unit;
        gauss_ = gauss;
        return true;
    }

private:
    std::mt19937_64 engine_;
    std::string mode_;
    std::uniform_real_distribution<float> unit_{0.0f, 1.0f};
    std::normal_distribution<float> gauss_{0.0f, 1.0f};
};

}  // namespace sa3
