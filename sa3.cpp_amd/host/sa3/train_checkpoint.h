// train_checkpoint.h - adapter checkpoints, the interface of the reference's
// src/train_checkpoint.h:38-173 (write_train_lora_gguf, load_train_lora_gguf): an inference-ready
// "sa3-lora" GGUF adapter with the reference's metadata keys, tensor names and shapes (the contract
// of docs/lora_checkpoint_contract.md), written and read by gguf_io.h instead of ggml's gguf code.
//
//   metadata: general.architecture = "sa3-lora", general.name, lora.adapter_type, lora.rank (u32),
//             lora.alpha (f32), lora.n_targets (u32)
//   tensors (f32, per target in state order, the non-empty ones):
//     <stem>.lora_A ne = [in, rank]     <stem>.lora_B ne = [rank, out]
//     <stem>.U      ne = [rank, out]    <stem>.V      ne = [rank, in]    <stem>.M_xs ne = [rank, rank]
//     <stem>.magnitude / .magnitude_r / .magnitude_c  ne = [length]
// Reading groups tensors by stem (targets come back sorted by stem, as the reference's std::map
// gives them), takes in from lora_A / V and out from lora_B / U, defaults a missing
// lora.adapter_type to "lora", and requires lora.rank and lora.alpha.
#pragma once

#include "gguf_io.h"
#include "train_lora.h"

#include <map>
#include <string>
#include <vector>

namespace sa3 {

inline bool write_train_lora_gguf(const TrainLoraState& state_in, const std::string& out_path, std::string& err) {
    TrainLoraState synced;   // device-resident training: the newest values, read from the device
    const TrainLoraState* view = nullptr;
    if (!train_lora_host_view(state_in, synced, view, err)) return false;
    const TrainLoraState& state = *view;
    if (state.rank <= 0 || state.params.empty()) {
        err = "cannot write empty LoRA checkpoint";
        return false;
    }
    gguf::Writer w;
    w.set_str("general.architecture", "sa3-lora");
    w.set_str("general.name", "sa3 native trained adapter");
    w.set_str("lora.adapter_type", state.adapter_type);
    w.set_u32("lora.rank", (uint32_t)state.rank);
    w.set_f32("lora.alpha", state.alpha);
    w.set_u32("lora.n_targets", (uint32_t)state.params.size());
    const int64_t r = state.rank;
    for (const TrainLoraParam& p : state.params) {
        const std::string& s = p.target.stem;
        const int64_t in = p.target.in, out = p.target.out;
        auto add = [&](const char* kind, const std::vector<float>& v, std::vector<int64_t> ne) {
            if (!v.empty()) w.add_f32(s + kind, ne, v);
        };
        add(".lora_A", p.lora_A, {in, r});
        add(".lora_B", p.lora_B, {r, out});
        add(".U", p.U, {r, out});
        add(".V", p.V, {r, in});
        add(".M_xs", p.M_xs, {r, r});
        add(".magnitude", p.magnitude, {(int64_t)p.magnitude.size()});
        add(".magnitude_r", p.magnitude_r, {(int64_t)p.magnitude_r.size()});
        add(".magnitude_c", p.magnitude_c, {(int64_t)p.magnitude_c.size()});
    }
    std::string werr;
    if (!w.write(out_path, werr)) {
        err = "failed to write " + out_path + " (" + werr + ")";
        return false;
    }
    return true;
}

inline bool load_train_lora_gguf(const std::string& path, TrainLoraState& state, std::string& err) {
    gguf::Reader g;
    if (!g.open(path, err)) return false;
    state = TrainLoraState{};
    const gguf::Value* type = g.find("lora.adapter_type");
    const gguf::Value* rank = g.find("lora.rank");
    const gguf::Value* alpha = g.find("lora.alpha");
    if (!rank || rank->type != gguf::kU32) {
        err = "key not found or not u32: lora.rank";
        return false;
    }
    if (!alpha || alpha->type != gguf::kF32) {
        err = "key not found or not f32: lora.alpha";
        return false;
    }
    state.adapter_type = type && type->type == gguf::kString ? type->s : "lora";
    state.rank = (int)rank->u;
    state.alpha = (float)alpha->f;
    static const char* const kinds[] = {".lora_A", ".lora_B", ".U", ".V", ".M_xs",
                                        ".magnitude", ".magnitude_r", ".magnitude_c"};
    std::map<std::string, TrainLoraParam> by_stem;
    for (const gguf::TensorInfo& t : g.tensors()) {
        std::string kind;
        for (const char* k : kinds) {
            const size_t n = std::char_traits<char>::length(k);
            if (t.name.size() > n && t.name.compare(t.name.size() - n, n, k) == 0) {
                kind = k;
                break;
            }
        }
        if (kind.empty()) continue;
        const std::string stem = t.name.substr(0, t.name.size() - kind.size());
        TrainLoraParam& p = by_stem[stem];
        p.target.stem = stem;
        p.target.weight_name = stem + ".weight";
        std::vector<float>* dst = nullptr;
        if (kind == ".lora_A") {
            p.target.in = t.ne.empty() ? 0 : t.ne[0];
            dst = &p.lora_A;
        } else if (kind == ".lora_B") {
            p.target.out = t.ne.size() > 1 ? t.ne[1] : 0;
            dst = &p.lora_B;
        } else if (kind == ".U") {
            p.target.out = t.ne.size() > 1 ? t.ne[1] : 0;
            dst = &p.U;
        } else if (kind == ".V") {
            p.target.in = t.ne.size() > 1 ? t.ne[1] : 0;
            dst = &p.V;
        } else if (kind == ".M_xs") {
            dst = &p.M_xs;
        } else if (kind == ".magnitude") {
            dst = &p.magnitude;
        } else if (kind == ".magnitude_r") {
            dst = &p.magnitude_r;
        } else {
            dst = &p.magnitude_c;
        }
        if (!g.read(t, *dst, err)) return false;
    }
    for (auto& kv : by_stem) state.params.push_back(std::move(kv.second));
    if (state.params.empty()) {
        err = "no adapter tensors found in " + path;
        return false;
    }
    return true;
}

}  // namespace sa3
