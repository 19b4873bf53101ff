// train_resume.h - exact trainer continuation: the interface of the reference's
// src/train_resume.h:23-538 for the parts that carry the training state of this path.
//
//   TrainResumeProgress            the data pipeline's cursor and RNG states, as caller-provided
//                                  strings and arrays (their producers are outside this build)
//   write_train_state_gguf         the "sa3-trainer-state" sidecar: optimizer step, progress and the
//   load_train_state_gguf          AdamW moments optimizer.<stem>.<kind>.m / .v of every trained vector
//   write_train_checkpoint_pair    adapter-step-N.gguf + trainer-state-step-N.gguf, both written to
//                                  temporaries and published by rename, the state last (its presence
//                                  marks a complete pair); existing checkpoints are never overwritten
//   train_resolve_resume_pair, train_checkpoint_step_from_name, train_latest_checkpoint_step,
//   train_restore_adapter_values, train_resume_file_fingerprint (FNV-1a 64 of the adapter file's
//   bytes), train_validate_resume_adapter_fingerprint, train_validate_resume_compatibility,
//   train_serialize_random_state / train_restore_random_state
//
// The sidecar's metadata keys, value types and tensor names are the reference's (a state written by
// one continues in the other). The compatibility fingerprint's producer hashes the trainer's CLI
// configuration and dataset manifest (src/train_resume.h:256-298), which are not part of this
// path: callers pass their own string, compared as the reference compares it.
#pragma once

#include "gguf_io.h"
#include "train_checkpoint.h"
#include "train_loop.h"

#include <cstdio>
#include <filesystem>
#include <limits>
#include <map>
#include <sstream>
#include <string>
#include <vector>

namespace sa3 {

struct TrainResumeProgress {
    uint64_t epoch = 0;
    uint64_t next_sample = 0;
    std::vector<uint64_t> order;
    std::string adapter_file;
    std::string adapter_fingerprint;
    std::string compatibility;
    std::string shuffle_rng;
    std::string crop_rng;
    std::string cfg_rng;
    std::string prompt_rng;
    std::string inpaint_rng;
    std::string diffusion_rng;
};

// A standard-library random engine's state as its stream text (the engines' own format), and back.
template <typename Engine>
inline std::string train_serialize_random_state(const Engine& engine) {
    std::ostringstream s;
    s << engine;
    return s.str();
}

template <typename Engine>
inline bool train_restore_random_state(const std::string& text, Engine& engine, const char* name, std::string& err) {
    std::istringstream s(text);
    Engine e;
    if (!(s >> e)) {
        err = std::string("invalid ") + name + " random state";
        return false;
    }
    engine = e;
    return true;
}

namespace detail {
inline const std::string kAdapterPrefix = "adapter-step-";
inline const std::string kStatePrefix = "trainer-state-step-";

inline bool starts_with(const std::string& s, const std::string& p) { return s.compare(0, p.size(), p) == 0; }
}  // namespace detail

// Either file of a pair names the other: adapter-step-N.gguf <-> trainer-state-step-N.gguf in the
// same directory.
inline bool train_resolve_resume_pair(const std::string& input, std::string& adapter_path, std::string& state_path,
                                      std::string& err) {
    namespace fs = std::filesystem;
    const fs::path p(input);
    const std::string file = p.filename().string();
    if (p.extension() == ".gguf") {
        if (detail::starts_with(file, detail::kAdapterPrefix)) {
            adapter_path = p.string();
            state_path = (p.parent_path() / (detail::kStatePrefix + file.substr(detail::kAdapterPrefix.size()))).string();
            return true;
        }
        if (detail::starts_with(file, detail::kStatePrefix)) {
            state_path = p.string();
            adapter_path = (p.parent_path() / (detail::kAdapterPrefix + file.substr(detail::kStatePrefix.size()))).string();
            return true;
        }
    }
    err = "--resume expects adapter-step-N.gguf or trainer-state-step-N.gguf";
    return false;
}

// N of "trainer-state-step-N.gguf" (decimal, fits an int), else -1.
inline int train_checkpoint_step_from_name(const std::string& name) {
    static const std::string suffix = ".gguf";
    const size_t lo = detail::kStatePrefix.size();
    if (!detail::starts_with(name, detail::kStatePrefix) || name.size() <= lo + suffix.size() ||
        name.compare(name.size() - suffix.size(), suffix.size(), suffix) != 0)
        return -1;
    long long step = 0;
    for (size_t i = lo; i < name.size() - suffix.size(); ++i) {
        const char ch = name[i];
        if (ch < '0' || ch > '9') return -1;
        step = 10 * step + (ch - '0');
        if (step > std::numeric_limits<int>::max()) return -1;
    }
    return (int)step;
}

// The highest step among the trainer-state files of a directory (-1 when there is none).
inline int train_latest_checkpoint_step(const std::string& directory) {
    namespace fs = std::filesystem;
    std::error_code ec;
    int latest = -1;
    for (fs::directory_iterator it(directory, ec), end; !ec && it != end; it.increment(ec))
        if (it->is_regular_file(ec)) latest = std::max(latest, train_checkpoint_step_from_name(it->path().filename().string()));
    return latest;
}

// Copy a reloaded adapter's values into the state the current model expects (its targets, order and
// shapes), checking family, rank, alpha, the target set and every vector's length.
inline bool train_restore_adapter_values(TrainLoraState& expected, const TrainLoraState& loaded, std::string& err) {
    if (loaded.adapter_type != expected.adapter_type || loaded.rank != expected.rank || loaded.alpha != expected.alpha) {
        err = "resume adapter type/rank/alpha does not match the current training configuration";
        return false;
    }
    std::map<std::string, const TrainLoraParam*> loaded_by_stem;
    for (const TrainLoraParam& p : loaded.params)
        if (!loaded_by_stem.emplace(p.target.stem, &p).second) {
            err = "duplicate resume adapter target: " + p.target.stem;
            return false;
        }
    if (loaded_by_stem.size() != expected.params.size()) {
        err = "resume adapter target count does not match the current model";
        return false;
    }
    for (TrainLoraParam& dst : expected.params) {
        const auto it = loaded_by_stem.find(dst.target.stem);
        if (it == loaded_by_stem.end()) {
            err = "resume adapter is missing target: " + dst.target.stem;
            return false;
        }
        const TrainLoraParam& src = *it->second;
        const std::pair<std::vector<float>*, const std::vector<float>*> parts[] = {
            {&dst.lora_A, &src.lora_A}, {&dst.lora_B, &src.lora_B}, {&dst.U, &src.U}, {&dst.V, &src.V},
            {&dst.M_xs, &src.M_xs}, {&dst.magnitude, &src.magnitude}, {&dst.magnitude_r, &src.magnitude_r},
            {&dst.magnitude_c, &src.magnitude_c}};
        static const char* const kinds[] = {"lora_A", "lora_B", "U", "V", "M_xs", "magnitude", "magnitude_r",
                                            "magnitude_c"};
        for (size_t k = 0; k < 8; ++k) {
            if (parts[k].first->size() != parts[k].second->size()) {
                err = "resume adapter tensor shape mismatch: " + dst.target.stem + "." + kinds[k];
                return false;
            }
            *parts[k].first = *parts[k].second;
        }
    }
    expected.device_newer = nullptr;   // the restored values are the newest; a holding graph uploads them
    expected.host_edits += 1;
    return true;
}

// 64-bit FNV-1a (offset basis 14695981039346656037, prime 1099511628211) over bytes.
inline uint64_t train_resume_fnv1a(uint64_t hash, const void* data, size_t size) {
    const unsigned char* p = static_cast<const unsigned char*>(data);
    for (size_t i = 0; i < size; ++i) hash = (hash ^ p[i]) * UINT64_C(1099511628211);
    return hash;
}

// "fnv1a64:" + 16 lowercase hex digits of the FNV-1a hash of the file's bytes; "" and err on failure.
inline std::string train_resume_file_fingerprint(const std::string& path, std::string& err) {
    std::FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) {
        err = "cannot fingerprint checkpoint file: " + path;
        return {};
    }
    uint64_t h = UINT64_C(14695981039346656037);
    std::vector<unsigned char> buf((size_t)1 << 20);
    size_t got = 0;
    while ((got = std::fread(buf.data(), 1, buf.size(), f)) > 0) h = train_resume_fnv1a(h, buf.data(), got);
    const bool bad = std::ferror(f) != 0;
    std::fclose(f);
    if (bad) {
        err = "failed while fingerprinting checkpoint file: " + path;
        return {};
    }
    char text[32];
    std::snprintf(text, sizeof text, "fnv1a64:%016llx", (unsigned long long)h);
    return text;
}

inline bool train_validate_resume_adapter_fingerprint(const std::string& path, const std::string& expected,
                                                      std::string& err) {
    const std::string actual = train_resume_file_fingerprint(path, err);
    if (actual.empty()) return false;
    if (actual != expected) {
        err = "resume adapter does not match its trainer-state sidecar";
        return false;
    }
    return true;
}

inline bool train_validate_resume_compatibility(const std::string& saved, const std::string& current,
                                                std::string& err) {
    if (saved == current) return true;
    err = "resume checkpoint is incompatible with the current model, dataset, or training settings";
    return false;
}

namespace detail {

// Every trained vector's AdamW moments in the reference's visit order (per target: lora_A, lora_B,
// M_xs, magnitude, magnitude_r, magnitude_c; empty vectors have none), with the sidecar's names.
struct MomentRef {
    std::string base;                   // optimizer.<stem>.<kind>
    const std::vector<float>* param;
    int kind;                           // index into the six per-target vectors
    size_t i;                           // target
};

template <class Loop>   // TrainLoopState or const TrainLoopState
inline auto& moment_states(Loop& loop, int kind) {
    switch (kind) {
        case 0: return loop.A_state;
        case 1: return loop.B_state;
        case 2: return loop.mxs_state;
        case 3: return loop.mag_state;
        case 4: return loop.mag_r_state;
        default: return loop.mag_c_state;
    }
}

inline std::vector<MomentRef> moment_refs(const TrainLoraState& lora) {
    static const char* const kinds[6] = {"lora_A", "lora_B", "M_xs", "magnitude", "magnitude_r", "magnitude_c"};
    std::vector<MomentRef> refs;
    for (size_t i = 0; i < lora.params.size(); ++i) {
        const TrainLoraParam& p = lora.params[i];
        const std::vector<float>* vecs[6] = {&p.lora_A, &p.lora_B, &p.M_xs, &p.magnitude, &p.magnitude_r, &p.magnitude_c};
        for (int k = 0; k < 6; ++k)
            if (!vecs[k]->empty()) refs.push_back({"optimizer." + p.target.stem + "." + kinds[k], vecs[k], k, i});
    }
    return refs;
}

inline bool state_string(const gguf::Reader& g, const char* key, std::string& out, std::string& err) {
    const gguf::Value* v = g.find(key);
    if (!v || v->type != gguf::kString) {
        err = std::string("trainer state is missing string metadata: ") + key;
        return false;
    }
    out = v->s;
    return true;
}

inline bool state_u64(const gguf::Reader& g, const char* key, uint64_t& out, std::string& err) {
    const gguf::Value* v = g.find(key);
    if (!v || v->type != gguf::kU64) {
        err = std::string("trainer state is missing integer metadata: ") + key;
        return false;
    }
    out = v->u;
    return true;
}

}  // namespace detail

// write_train_state_gguf (src/train_resume.h:336-381)
inline bool write_train_state_gguf(const TrainLoraState& lora_in, const TrainLoopState& loop_in,
                                   const TrainResumeProgress& progress, const std::string& out_path, std::string& err) {
    // device-resident training: the newest values, read from the device
    TrainLoraState lora_synced;
    TrainLoopState loop_synced;
    const TrainLoraState* lv = nullptr;
    const TrainLoopState* pv = nullptr;
    if (!train_lora_host_view(lora_in, lora_synced, lv, err) || !train_loop_host_view(loop_in, loop_synced, pv, err))
        return false;
    const TrainLoraState& lora = *lv;
    const TrainLoopState& loop = *pv;
    if (loop.step <= 0 || progress.order.empty() || progress.next_sample > progress.order.size()) {
        err = "cannot write invalid trainer continuation state";
        return false;
    }
    const std::vector<detail::MomentRef> refs = detail::moment_refs(lora);
    for (const detail::MomentRef& r : refs) {
        const std::vector<TrainAdamWTensorState>& st = detail::moment_states(loop, r.kind);
        if (st.size() != lora.params.size() || st[r.i].m.size() != r.param->size() ||
            st[r.i].v.size() != r.param->size()) {
            err = "optimizer state is incomplete for " + r.base.substr(10);   // past "optimizer."
            return false;
        }
    }
    gguf::Writer w;
    w.set_str("general.architecture", "sa3-trainer-state");
    w.set_str("general.name", "sa3 native trainer continuation state");
    w.set_u32("trainer.state_version", 1);
    w.set_u64("trainer.step", (uint64_t)loop.step);
    w.set_u64("trainer.epoch", progress.epoch);
    w.set_u64("trainer.next_sample", progress.next_sample);
    w.set_u32("trainer.n_targets", (uint32_t)lora.params.size());
    w.set_str("trainer.adapter_file", progress.adapter_file);
    w.set_str("trainer.adapter_fingerprint", progress.adapter_fingerprint);
    w.set_str("trainer.compatibility", progress.compatibility);
    w.set_str("trainer.rng.shuffle", progress.shuffle_rng);
    w.set_str("trainer.rng.crop", progress.crop_rng);
    w.set_str("trainer.rng.cfg", progress.cfg_rng);
    w.set_str("trainer.rng.prompt", progress.prompt_rng);
    w.set_str("trainer.rng.inpaint", progress.inpaint_rng);
    w.set_str("trainer.rng.diffusion", progress.diffusion_rng);
    w.set_arr_u64("trainer.order", progress.order);
    std::vector<std::string> stems;
    for (const TrainLoraParam& p : lora.params) stems.push_back(p.target.stem);
    w.set_arr_str("trainer.targets", stems);
    for (const detail::MomentRef& r : refs) {
        const TrainAdamWTensorState& st = detail::moment_states(loop, r.kind)[r.i];
        w.add_f32(r.base + ".m", {(int64_t)st.m.size()}, st.m);
        w.add_f32(r.base + ".v", {(int64_t)st.v.size()}, st.v);
    }
    std::string werr;
    if (!w.write(out_path, werr)) {
        err = "failed to write " + out_path;
        return false;
    }
    return true;
}

// load_train_state_gguf (src/train_resume.h:394-502): `lora` gives the expected targets (their order
// must match the sidecar's) and which vectors have moments.
inline bool load_train_state_gguf(const std::string& path, const TrainLoraState& lora, TrainLoopState& loop,
                                  TrainResumeProgress& progress, std::string& err) {
    gguf::Reader g;
    if (!g.open(path, err)) return false;
    std::string arch;
    if (!detail::state_string(g, "general.architecture", arch, err)) return false;
    if (arch != "sa3-trainer-state") {
        err = "not an sa3 trainer-state GGUF: " + path;
        return false;
    }
    const gguf::Value* version = g.find("trainer.state_version");
    if (!version || version->type != gguf::kU32 || version->u != 1) {
        err = "unsupported trainer-state version";
        return false;
    }
    uint64_t step = 0;
    if (!detail::state_u64(g, "trainer.step", step, err) || !detail::state_u64(g, "trainer.epoch", progress.epoch, err) ||
        !detail::state_u64(g, "trainer.next_sample", progress.next_sample, err))
        return false;
    if (step > (uint64_t)std::numeric_limits<int>::max()) {
        err = "trainer state step out of range";
        return false;
    }
    const std::pair<const char*, std::string*> strings[] = {
        {"trainer.adapter_file", &progress.adapter_file}, {"trainer.adapter_fingerprint", &progress.adapter_fingerprint},
        {"trainer.compatibility", &progress.compatibility}, {"trainer.rng.shuffle", &progress.shuffle_rng},
        {"trainer.rng.crop", &progress.crop_rng},           {"trainer.rng.cfg", &progress.cfg_rng},
        {"trainer.rng.prompt", &progress.prompt_rng},       {"trainer.rng.inpaint", &progress.inpaint_rng},
        {"trainer.rng.diffusion", &progress.diffusion_rng}};
    for (const auto& s : strings)
        if (!detail::state_string(g, s.first, *s.second, err)) return false;
    const gguf::Value* order = g.find("trainer.order");
    if (!order || order->type != gguf::kArray || order->arr_type != gguf::kU64) {
        err = "trainer state is missing the dataset order";
        return false;
    }
    progress.order = order->au;
    if (progress.order.empty() || progress.next_sample > progress.order.size()) {
        err = "trainer state has an invalid dataset cursor";
        return false;
    }
    const gguf::Value* targets = g.find("trainer.targets");
    if (!targets || targets->type != gguf::kArray || targets->arr_type != gguf::kString ||
        targets->as.size() != lora.params.size()) {
        err = "trainer state target inventory does not match the adapter";
        return false;
    }
    for (size_t i = 0; i < lora.params.size(); ++i)
        if (targets->as[i] != lora.params[i].target.stem) {
            err = "trainer state target order does not match the current model";
            return false;
        }
    loop = TrainLoopState{};
    loop.step = (int)step;
    const size_t n = lora.params.size();
    for (auto* s : {&loop.A_state, &loop.B_state, &loop.mxs_state, &loop.mag_state, &loop.mag_r_state, &loop.mag_c_state})
        s->resize(n);
    std::map<std::string, const gguf::TensorInfo*> by_name;
    for (const gguf::TensorInfo& t : g.tensors()) by_name[t.name] = &t;
    for (const detail::MomentRef& r : detail::moment_refs(lora)) {
        const auto m = by_name.find(r.base + ".m"), v = by_name.find(r.base + ".v");
        if (m == by_name.end() || v == by_name.end()) {
            err = "trainer state is missing optimizer tensors for " + r.base;
            return false;
        }
        TrainAdamWTensorState& st = detail::moment_states(loop, r.kind)[r.i];
        if (!g.read(*m->second, st.m, err) || !g.read(*v->second, st.v, err)) return false;
        if (st.m.size() != r.param->size() || st.v.size() != r.param->size()) {
            err = "trainer optimizer tensor shape mismatch for " + r.base;
            return false;
        }
    }
    return true;
}

// write_train_checkpoint_pair (src/train_resume.h:504-538): the adapter and its trainer state as an
// immutable pair. Both go to ".tmp" files first; the adapter is published (renamed) first and the
// state last, so a state file marks a complete pair.
inline bool write_train_checkpoint_pair(const TrainLoraState& lora, const TrainLoopState& loop,
                                        TrainResumeProgress progress, const std::string& adapter_path,
                                        const std::string& state_path, std::string& err) {
    namespace fs = std::filesystem;
    if (fs::exists(adapter_path) || fs::exists(state_path)) {
        err = "refusing to overwrite an existing immutable training checkpoint at step " + std::to_string(loop.step) +
              "; resume the latest checkpoint or choose --out";
        return false;
    }
    progress.adapter_file = fs::path(adapter_path).filename().string();
    const std::string adapter_tmp = adapter_path + ".tmp", state_tmp = state_path + ".tmp";
    std::error_code ec;
    auto drop_temps = [&] {
        fs::remove(adapter_tmp, ec);
        fs::remove(state_tmp, ec);
    };
    drop_temps();
    if (!write_train_lora_gguf(lora, adapter_tmp, err)) {
        drop_temps();
        return false;
    }
    progress.adapter_fingerprint = train_resume_file_fingerprint(adapter_tmp, err);
    if (progress.adapter_fingerprint.empty() || !write_train_state_gguf(lora, loop, progress, state_tmp, err)) {
        drop_temps();
        return false;
    }
    fs::rename(adapter_tmp, adapter_path, ec);
    if (ec) {
        err = "failed to publish adapter checkpoint: " + ec.message();
        drop_temps();
        return false;
    }
    fs::rename(state_tmp, state_path, ec);
    if (ec) {
        err = "adapter was written, but trainer state could not be published: " + ec.message();
        fs::remove(state_tmp, ec);
        return false;
    }
    return true;
}

}  // namespace sa3
