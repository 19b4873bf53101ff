// train_lora.h - trainable LoRA / DoRA adapter state, the interface of the reference's
// src/train_lora.h:17-273 for the two adapter families of this path (lora, dora-rows). Target
// enumeration, scopes, initialisation and the state layout follow the reference; the row norms
// that seed the DoRA magnitudes run on the GPU.
#pragma once

#include "dit_model.h"

#include <algorithm>
#include <cctype>
#include <cmath>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

namespace sa3 {

struct TrainLoraTarget {
    std::string weight_name;
    std::string stem;
    int64_t in = 0;
    int64_t out = 0;
};

struct TrainLoraParam {
    TrainLoraTarget target;
    std::vector<float> lora_A;      // [rank, in] host row-major by rank
    std::vector<float> lora_B;      // [out, rank]
    std::vector<float> U;           // -xs families (not implemented here): stay empty
    std::vector<float> V;
    std::vector<float> M_xs;
    std::vector<float> magnitude;   // dora-rows [out]
    std::vector<float> magnitude_r; // bora (not implemented here): stays empty
    std::vector<float> magnitude_c;
};

struct TrainLoraState {
    std::string adapter_type = "lora";
    int rank = 0;
    float alpha = 1.0f;
    std::vector<TrainLoraParam> params;
    // This build only (no reference counterpart): set while a training graph in device-resident
    // mode (train_dit.h) holds newer values of `params` than these host vectors, i.e. after an
    // AdamW update that ran there; device_read copies them into a state of the same layout.
    // train_state_to_host (train_loop.h) refreshes the vectors; the checkpoint writers read through
    // train_lora_host_view. Host code must not change `params` while this is set.
    const void* device_newer = nullptr;
    bool (*device_read)(const void* graph, TrainLoraState& into, std::string& err) = nullptr;
    // Bumped by the functions of this build that change the host vectors of an existing state
    // (train_restore_adapter_values): a device-resident graph holding an older edit uploads again.
    // Code that changes the vectors itself calls upload_train_lora_state.
    uint64_t host_edits = 0;
};

// The values of `s` as host vectors: `s` itself, or (device-newer) a copy filled from the device
// into `tmp`.
inline bool train_lora_host_view(const TrainLoraState& s, TrainLoraState& tmp, const TrainLoraState*& view,
                                 std::string& err) {
    view = &s;
    if (!s.device_newer) return true;
    tmp = s;
    tmp.device_newer = nullptr;
    if (!s.device_read || !s.device_read(s.device_newer, tmp, err)) return false;
    view = &tmp;
    return true;
}

// Which weights get an adapter (src/train_lora.h:53-97): "full" = every 2-D dit.*.weight, "core" =
// the 7 per-block projections (dit.<N>.*, no local.*); include/exclude are substring filters.
struct TrainLoraScope {
    std::string name = "full";
    std::vector<std::string> include;
    std::vector<std::string> exclude;
};

inline bool train_lora_scope_known(const std::string& s) { return s == "full" || s == "core"; }

namespace detail {
inline bool ends_with(const std::string& s, const std::string& suffix) {
    return s.size() >= suffix.size() && std::equal(suffix.rbegin(), suffix.rend(), s.rbegin());
}
inline bool contains_any(const std::string& s, const std::vector<std::string>& parts) {
    return std::any_of(parts.begin(), parts.end(),
                       [&](const std::string& p) { return s.find(p) != std::string::npos; });
}
}  // namespace detail

// A per-block tensor is named "dit.<block index>.<rest>": a non-empty run of decimal digits right
// after the "dit." prefix, closed by a dot (src/train_lora.h:64-75).
inline bool train_lora_is_block_weight(const std::string& name) {
    constexpr size_t kPrefix = 4;   // "dit."
    const size_t digits_end = name.find_first_not_of("0123456789", kPrefix);
    return digits_end != std::string::npos && digits_end > kPrefix && name[digits_end] == '.';
}

// Scope rules (src/train_lora.h:77-97): "core" keeps only per-block tensors and drops the inpaint
// local-conditioning branch; then a non-empty include list needs one matching substring, and any
// matching exclude substring drops the weight.
inline bool train_lora_target_selected(const std::string& name, const TrainLoraScope& scope) {
    const bool in_scope = scope.name != "core" ||
                          (train_lora_is_block_weight(name) && name.find(".local.") == std::string::npos);
    const bool included = scope.include.empty() || detail::contains_any(name, scope.include);
    return in_scope && included && !detail::contains_any(name, scope.exclude);
}

// The adapter targets (src/train_lora.h:99-121): every 2-D tensor named dit.*.weight that the scope
// selects, with in = ne0 and out = ne1, in ascending order of weight name (which fixes the order of
// the trained state and of the optimizer moments).
inline std::vector<TrainLoraTarget> enumerate_train_lora_targets(const DitModel& dit, const TrainLoraScope& scope = {}) {
    static const std::string kSuffix = ".weight";
    std::vector<TrainLoraTarget> targets;
    for (const std::string& name : dit.tensor_names()) {
        const bool candidate = name.compare(0, 4, "dit.") == 0 && detail::ends_with(name, kSuffix) &&
                               dit.is_2d(name) && train_lora_target_selected(name, scope);
        if (!candidate || dit.ne0(name) <= 0 || dit.ne1(name) <= 0) continue;
        TrainLoraTarget t;
        t.weight_name = name;
        t.stem = name.substr(0, name.size() - kSuffix.size());
        t.in = dit.ne0(name);
        t.out = dit.ne1(name);
        targets.push_back(std::move(t));
    }
    std::sort(targets.begin(), targets.end(),
              [](const TrainLoraTarget& a, const TrainLoraTarget& b) { return a.weight_name < b.weight_name; });
    return targets;
}

// Row norms of a host weight W [out][in] (the reference's ggml_tensor argument, src/train_lora.h:
// 141-174): double accumulation on the GPU; train_row_norm_sq adds in*eps. The reference returns
// ones / in*eps for a missing tensor (a short vector here); a failing GPU throws.
inline std::vector<float> train_row_norms_impl(const std::vector<float>& w, int64_t in, int64_t out, int mode,
                                               float eps) {
    std::vector<float> r((size_t)out, mode == 0 ? 1.0f : (float)((double)in * eps));
    if (w.size() < (size_t)(in * out)) return r;
    std::string err;
    sa3k_ctx* ctx = sa3k_default_ctx(err);
    DeviceF32 dw, dn;
    if (!ctx || !dw.alloc(ctx, w.size(), err) || !dw.upload(w.data(), w.size(), 0, err) ||
        !dn.alloc(ctx, (size_t)out, err))
        throw std::runtime_error("train_row_norms: " + err);
    if (sa3k_row_norms(ctx, SA3K_TYPE_F32, in, out, dw.get(), mode, eps, dn.get()) != SA3K_OK)
        throw std::runtime_error(std::string("train_row_norms: ") + sa3k_last_error(ctx));
    if (!dn.download(r.data(), r.size(), 0, err)) throw std::runtime_error("train_row_norms: " + err);
    return r;
}
inline std::vector<float> train_row_norms(const std::vector<float>& w, int64_t in, int64_t out) {
    return train_row_norms_impl(w, in, out, 0, 0.0f);
}
inline std::vector<float> train_row_norm_sq(const std::vector<float>& w, int64_t in, int64_t out, float eps) {
    return train_row_norms_impl(w, in, out, 1, eps);
}
// ... and of a model weight by name (decoded from its stored type)
inline std::vector<float> train_row_norms(const DitModel& dit, const std::string& weight_name) {
    std::vector<float> out;
    std::string err;
    if (!dit.row_norms(weight_name, 0, 0.0f, out, err)) throw std::runtime_error("train_row_norms: " + err);
    return out;
}
inline std::vector<float> train_row_norm_sq(const DitModel& dit, const std::string& weight_name, float eps) {
    std::vector<float> out;
    std::string err;
    if (!dit.row_norms(weight_name, 1, eps, out, err)) throw std::runtime_error("train_row_norm_sq: " + err);
    return out;
}

// init_train_lora_state (src/train_lora.h:205-273) for "lora" and "dora-rows": A ~ Kaiming-uniform
// U(-1/sqrt(in), 1/sqrt(in)) drawn from std::mt19937_64(seed) in target order (the reference's
// stream, so the same seed gives the same A), B = 0, dora magnitude = row norms of W.
inline bool init_train_lora_state(const DitModel& dit, const std::vector<TrainLoraTarget>& targets,
                                  const std::string& adapter_type, int rank, float alpha, unsigned long long seed,
                                  TrainLoraState& out, std::string& err) {
    if (rank <= 0) {
        err = "rank must be positive";
        return false;
    }
    if (adapter_type != "lora" && adapter_type != "dora-rows") {
        err = "adapter type " + adapter_type + " is not implemented (lora, dora-rows)";
        return false;
    }
    out = TrainLoraState{};
    out.adapter_type = adapter_type;
    out.rank = rank;
    out.alpha = alpha;
    std::mt19937_64 rng(seed);
    for (const TrainLoraTarget& t : targets) {
        if (rank > t.in || rank > t.out) {
            err = "rank is infeasible for target " + t.stem;
            return false;
        }
        TrainLoraParam p;
        p.target = t;
        p.lora_A.resize((size_t)rank * t.in);
        p.lora_B.assign((size_t)t.out * rank, 0.0f);
        const float bound = 1.0f / std::sqrt((float)t.in);
        std::uniform_real_distribution<float> kaiming(-bound, bound);
        for (float& v : p.lora_A) v = kaiming(rng);
        if (adapter_type == "dora-rows") {
            if (!dit.row_norms(t.weight_name, 0, 0.0f, p.magnitude, err)) return false;
        }
        out.params.push_back(std::move(p));
    }
    return true;
}

}  // namespace sa3
