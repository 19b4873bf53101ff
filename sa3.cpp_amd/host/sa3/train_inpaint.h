// train_inpaint.h - the inpainting-mask step inputs of the reference's src/train_inpaint.h:25-194:
// InpaintMaskType, generate_inpaint_mask (mask type drawn from a probability vector, then random
// segments / full / causal prefix / random spans over the latent frames, padding masked) and
// build_train_inpaint (the local conditioning [mask | z * mask] and the per-position loss weight).
// Same names, arguments, defaults and results.
//
// Host code for the same reason as the diffusion sampler: the masks are the reference's only if
// they are drawn from the same std::mt19937_64 with the same standard-library distributions in the
// same order, so every draw below (its distribution, bounds and position in the sequence) follows
// the reference step by step. A mask is one float per latent frame. The loss weight is what
// sa3k_dit_accumulate takes as its per-position weight; the local conditioning feeds the DiT's
// dit.local.* linears, which the device DiT does not carry (run_train_dit_accumulate rejects an
// inpaint sample).
#pragma once

#include <algorithm>
#include <functional>
#include <numeric>
#include <random>
#include <utility>
#include <vector>

namespace sa3 {

enum class InpaintMaskType { RandomSegments = 0, FullMask = 1, Causal = 2, RandomSpans = 3 };

namespace inpaint_detail {

// integer uniform on [lo, hi] (hi < lo gives lo without a draw)
inline int draw_int(std::mt19937_64& g, int lo, int hi) {
    return hi < lo ? lo : std::uniform_int_distribution<int>(lo, hi)(g);
}
// real uniform on [lo, hi)
inline double draw_real(std::mt19937_64& g, double lo = 0.0, double hi = 1.0) {
    return std::uniform_real_distribution<double>(lo, hi)(g);
}
// index drawn with probability proportional to w (all-zero weights: uniform index)
inline int draw_weighted(const std::vector<double>& w, std::mt19937_64& g) {
    const double total = std::accumulate(w.begin(), w.end(), 0.0);
    if (total <= 0.0) return draw_int(g, 0, (int)w.size() - 1);
    const double u = draw_real(g) * total;
    double run = 0.0;
    for (size_t i = 0; i < w.size(); ++i) {
        run += w[i];
        if (u < run) return (int)i;
    }
    return (int)w.size() - 1;
}

// 1..max_spans non-overlapping spans zeroed in mask[0, real_len), covering about a ratio drawn from
// U(ratio_lo, ratio_hi) of the real frames
inline void zero_random_spans(std::vector<float>& mask, int real_len, std::mt19937_64& g, int max_spans,
                              double ratio_lo, double ratio_hi, const std::vector<double>& span_count_w) {
    if (real_len == 0) return;
    const int want = std::max(1, (int)(draw_real(g, ratio_lo, ratio_hi) * real_len));
    // how many spans: weights over 1..max_spans (default 4:2:1:1, padded with the last weight)
    std::vector<double> w = span_count_w.empty() ? std::vector<double>{4, 2, 1, 1} : span_count_w;
    w.resize((size_t)max_spans, w.empty() ? 1.0 : w.back());
    const int spans = std::min(draw_weighted(w, g) + 1, real_len);
    if (spans <= 0) return;
    // span lengths: a random split of `want`, each at least 1, fixed up to sum to `want` where the
    // minimum of 1 allows (surplus to the first span, deficit taken from the front), longest first
    std::vector<double> share((size_t)spans);
    double share_sum = 0.0;
    for (double& x : share) share_sum += (x = draw_real(g));
    if (share_sum <= 0.0) share_sum = 1.0;
    std::vector<int> len((size_t)spans);
    for (int i = 0; i < spans; ++i) len[(size_t)i] = std::max(1, (int)(share[(size_t)i] / share_sum * want));
    int gap = want - std::accumulate(len.begin(), len.end(), 0);
    if (gap > 0) len[0] += gap;
    for (int i = 0; gap < 0 && i < spans; ++i) {
        const int cut = std::min(-gap, len[(size_t)i] - 1);
        len[(size_t)i] -= cut;
        gap += cut;
    }
    std::sort(len.begin(), len.end(), std::greater<int>());
    // placement: up to 50 random starts per span, then the first free start from the left
    std::vector<std::pair<int, int>> taken;
    auto is_free = [&](int b, int e) {
        for (const auto& s : taken)
            if (s.first < e && b < s.second) return false;
        return true;
    };
    auto take = [&](int b, int e) {
        taken.emplace_back(b, e);
        std::fill(mask.begin() + b, mask.begin() + e, 0.0f);
    };
    for (int l : len) {
        l = std::min(l, real_len);
        if (l <= 0) continue;
        const int last = real_len - l;
        bool placed = false;
        for (int tries = 0; tries < 50 && !placed; ++tries) {
            const int b = draw_int(g, 0, last);
            if (is_free(b, b + l)) {
                take(b, b + l);
                placed = true;
            }
        }
        for (int b = 0; !placed && b <= last; ++b)
            if (is_free(b, b + l)) {
                take(b, b + l);
                placed = true;
            }
    }
}

}  // namespace inpaint_detail

// A frame mask (1 keep / 0 generate) over `frames`, of which the first real_len are not padding.
// probs: 3 weights over {segments, full, causal} or 4 adding {random spans}.
inline std::vector<float> generate_inpaint_mask(int frames, int real_len, const std::vector<double>& probs,
                                                std::mt19937_64& rng, InpaintMaskType& type_out,
                                                bool mask_padding = true, int max_mask_segments = 10,
                                                int max_spans = 4, double mask_ratio_lo = 0.2,
                                                double mask_ratio_hi = 1.0,
                                                const std::vector<double>& span_count_weights = {}) {
    using namespace inpaint_detail;
    std::vector<float> mask((size_t)frames, 1.0f);
    const int pick = draw_weighted(probs, rng);
    static const InpaintMaskType kinds[4] = {InpaintMaskType::RandomSegments, InpaintMaskType::FullMask,
                                             InpaintMaskType::Causal, InpaintMaskType::RandomSpans};
    const InpaintMaskType type = kinds[pick];   // pick < 3 unless probs has 4 entries
    type_out = type;
    if (type == InpaintMaskType::FullMask) {
        std::fill(mask.begin(), mask.end(), 0.0f);
        return mask;
    }
    if (real_len == 0) return mask;
    switch (type) {
        case InpaintMaskType::RandomSegments: {
            const int count = draw_int(rng, 1, max_mask_segments);
            const int longest = std::max(1, real_len / count);
            for (int k = 0; k < count; ++k) {
                const int l = draw_int(rng, 1, longest);
                if (real_len < l) continue;
                const int b = draw_int(rng, 0, real_len - l);
                std::fill(mask.begin() + b, mask.begin() + b + l, 0.0f);
            }
            break;
        }
        case InpaintMaskType::RandomSpans:
            zero_random_spans(mask, real_len, rng, max_spans, mask_ratio_lo, mask_ratio_hi, span_count_weights);
            break;
        case InpaintMaskType::Causal: {
            const int keep = draw_int(rng, 0, real_len);   // context [0, keep), generate [keep, real_len)
            std::fill(mask.begin() + keep, mask.begin() + real_len, 0.0f);
            break;
        }
        default:
            break;
    }
    if (mask_padding) std::fill(mask.begin() + real_len, mask.end(), 0.0f);   // padding is no context
    return mask;
}

// Host-built inpainting inputs for one training step.
struct TrainInpaint {
    std::vector<float> local;        // [local_dim * frames], idx = t*local_dim + ch (ch0=mask, ch1..io=z*mask)
    std::vector<float> loss_weight;  // [io * frames],        idx = t*io + c   (per-frame, broadcast over c)
    InpaintMaskType type = InpaintMaskType::FullMask;
    int n_gen = 0, n_ctx = 0;
};

// Local conditioning and loss weight from the clean latent z ([frames][io]) and a frame mask.
// Weights make the loss a mean over the generated positions: with mask_padding_attention every
// generated position weighs 1 / (io n_gen + 1e-8) and context positions 0; without it, context
// positions count mask_loss_weight times as much in a joint mean,
//   w_gen = 1 / D, w_ctx = mask_loss_weight / D, D = io n_gen + mask_loss_weight io n_ctx + 1e-8.
inline TrainInpaint build_train_inpaint(const std::vector<float>& z, const std::vector<float>& mask, int io,
                                        int frames, int local_dim, float mask_loss_weight,
                                        bool mask_padding_attention = true) {
    TrainInpaint r;
    r.local.assign((size_t)local_dim * frames, 0.0f);
    r.loss_weight.assign((size_t)io * frames, 0.0f);
    for (int t = 0; t < frames; ++t) {
        const float m = mask[(size_t)t];
        float* row = r.local.data() + (size_t)t * local_dim;
        row[0] = m;
        for (int c = 0; c < io; ++c) row[1 + c] = z[(size_t)t * io + c] * m;
        (m > 0.5f ? r.n_ctx : r.n_gen) += 1;
    }
    const float gen_positions = (float)io * (float)r.n_gen;
    float w_gen = 0.0f, w_ctx = 0.0f;
    if (mask_padding_attention) {
        w_gen = 1.0f / (gen_positions + 1e-8f);
    } else {
        const float denom = gen_positions + mask_loss_weight * (float)io * (float)r.n_ctx + 1e-8f;
        w_gen = 1.0f / denom;
        w_ctx = mask_loss_weight / denom;
    }
    for (int t = 0; t < frames; ++t)
        std::fill(r.loss_weight.begin() + (size_t)t * io, r.loss_weight.begin() + (size_t)(t + 1) * io,
                  mask[(size_t)t] > 0.5f ? w_ctx : w_gen);
    return r;
}

}  // namespace sa3
