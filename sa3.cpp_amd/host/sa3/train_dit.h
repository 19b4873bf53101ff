// train_dit.h - the DiT training graph of the reference's src/train_dit.h:30-218 (TrainDitGraph,
// build_train_dit_forward_graph, free_train_dit_graph) over the device-resident DiT step: building
// the "graph" sets the model up for one sample of `frames` latent frames and `ctx_len` context
// tokens, lays the adapters out in the arena in the reference's target order, and allocates the
// step inputs. The rectified-flow sample and the conditioning keep the reference's host structs
// (src/train_diffusion.h:12-17, src/train_conditioning.h:16-22); the sample comes from
// TrainDiffusionSampler (train_diffusion.h), the conditioning's producer (text encoder) is outside
// this build.
#pragma once

#include "train_diffusion.h"
#include "train_lora.h"

#include <stdexcept>
#include <string>
#include <vector>

namespace sa3 {

struct TrainConditioning {
    std::vector<float> cross;   // [cond_dim, ctx_len] (ggml order)
    std::vector<float> global;  // [cond_dim]
    int cond_dim = 0;
    int ctx_len = 0;
    int token_count = 0;
};

namespace detail {

// What a training "graph" of this build holds: the device model in one activation schedule, its
// adapter arena (one slot per target, in the order of TrainLoraState::params) and the device
// buffers of one sample's inputs. TrainDitGraph (monolithic) and TrainDitCkpt (checkpointed) are
// both this; they differ in the schedule the model is set up with.
struct DitDeviceStep {
    struct Slot {   // one adapted target in the arena
        int64_t off_a = 0, off_b = 0, off_m = -1, n_a = 0, n_b = 0, n_m = 0;
    };
    DitModel* model = nullptr;
    int frames = 0, cond_dim = 0, ctx_len = 0;
    float* params = nullptr;   // device adapter arena (owned by the model)
    float* grads = nullptr;
    int64_t n_params = 0;
    std::vector<Slot> slots;   // aligned with TrainLoraState::params
    DeviceF32 x, target, t, cross, global;
    // inpaint graphs (src/train_dit.h:83-87): the local conditioning [frames][local_dim] and the
    // per-frame loss weight [frames] of the last sample
    bool inpaint = false;
    DeviceF32 local, loss_weight;
    // Device-resident training (this build; set device_resident before the first step). The
    // reference uploads the adapters and reads every gradient back per sample, and runs AdamW on
    // host vectors (src/train_loop.h:42-73, :173-211). In this mode the adapter values, the
    // gradient sums of the accumulation window and the AdamW moments stay in the model's arenas
    // between calls: run_train_dit_accumulate[_ckpt] uploads a state only when the arena does not
    // already hold it and adds the sample's gradients into a device accumulator (f32, as
    // train_accum_add does on the host), train_apply_accumulated_adamw updates the arena in place,
    // and the host vectors are refreshed by train_state_to_host and read through by the checkpoint
    // writers (TrainLoraState::device_newer). Same values bit for bit as the round-trip path.
    bool device_resident = false;
    const void* held = nullptr;       // the TrainLoraState whose values the params arena holds
    uint64_t held_edits = 0;          // its host_edits at the upload
    DeviceF32 acc;                    // the accumulation window's gradient sums
    void* newer_state = nullptr;      // a TrainLoraState / TrainLoopState newer here than on the host
    void* newer_loop = nullptr;
    bool (*release)(DitDeviceStep& step, std::string& err) = nullptr;   // copies those back
};

// Set `dit` up for one sample of `frames` latent frames and `ctx_len` context tokens with the
// adapters of `lora` (a scope this build runs: every block projection, with or without the 12
// head/tail linears) in the given schedule (recompute = 1: the checkpointed one), and fill `out`.
// A model is set up once.
inline bool setup_dit_step(DitModel& dit, const DitConfig& dc, const TrainLoraState& lora, int frames, int cond_dim,
                           int ctx_len, int recompute, DitDeviceStep& out, std::string& err, bool inpaint) {
    if (frames <= 0 || cond_dim <= 0 || ctx_len <= 0) {
        err = "invalid DiT training graph dimensions";
        return false;
    }
    if (inpaint && dc.local_dim <= 0) {
        err = "inpainting requested but DiT has no local-cond weights (dit.local_dim <= 0)";
        return false;
    }
    if (cond_dim != dc.cond_dim) {
        err = "conditioning width differs from the model's cond_dim";
        return false;
    }
    if (lora.adapter_type != "lora" && lora.adapter_type != "dora-rows") {
        err = "adapter type " + lora.adapter_type + " is not implemented (lora, dora-rows)";
        return false;
    }
    bool all_blocks = true;
    for (const TrainLoraParam& p : lora.params) all_blocks = all_blocks && train_lora_is_block_weight(p.target.weight_name);
    const int scope = all_blocks ? SA3K_SCOPE_CORE : SA3K_SCOPE_FULL;
    sa3k_ctx* ctx = dit.ctx();
    sa3k_dit_train tr{lora.rank, lora.alpha, lora.adapter_type == "dora-rows" ? 1 : 0, scope, 1, frames, ctx_len,
                      recompute};
    if (sa3k_dit_setup(ctx, dit.handle(), &tr) != SA3K_OK) return sa3k_fail(ctx, err);
    out.model = &dit;
    out.frames = frames;
    out.cond_dim = cond_dim;
    out.ctx_len = ctx_len;
    out.slots.clear();
    int nt = 0;
    if (sa3k_dit_target_count(ctx, dit.handle(), &nt) != SA3K_OK) return sa3k_fail(ctx, err);
    if ((size_t)nt != lora.params.size()) {
        err = "the adapter targets are not a scope this build runs (core or full)";
        return false;
    }
    char name[256];
    for (int i = 0; i < nt; ++i) {
        int64_t in = 0, o = 0;
        DitDeviceStep::Slot s;
        if (sa3k_dit_target_info(ctx, dit.handle(), i, name, (int)sizeof name, &in, &o, &s.off_a, &s.off_b, &s.off_m) !=
            SA3K_OK)
            return sa3k_fail(ctx, err);
        if (lora.params[i].target.weight_name != name) {
            err = std::string("adapter target order differs from the model's: ") + name;
            return false;
        }
        s.n_a = (int64_t)lora.rank * in;
        s.n_b = o * lora.rank;
        s.n_m = s.off_m >= 0 ? o : 0;
        out.slots.push_back(s);
    }
    if (sa3k_dit_arena(ctx, dit.handle(), 0, &out.params, &out.n_params) != SA3K_OK ||
        sa3k_dit_arena(ctx, dit.handle(), 1, &out.grads, nullptr) != SA3K_OK)
        return sa3k_fail(ctx, err);
    const size_t nx = (size_t)dc.io * frames;
    out.inpaint = inpaint;
    if (inpaint && !(out.local.alloc(ctx, (size_t)dc.local_dim * frames, err) &&
                     out.loss_weight.alloc(ctx, (size_t)frames, err)))
        return false;
    return out.x.alloc(ctx, nx, err) && out.target.alloc(ctx, nx, err) && out.t.alloc(ctx, 1, err) &&
           out.cross.alloc(ctx, (size_t)cond_dim * ctx_len, err) && out.global.alloc(ctx, (size_t)cond_dim, err);
}

}  // namespace detail

// The monolithic training graph (src/train_dit.h:30-48): every block keeps its forward activations.
struct TrainDitGraph : detail::DitDeviceStep {};

namespace detail {
// Before a graph goes away: the values only it holds (device-resident training) go back to the
// host state and loop objects.
inline void release_device_step(DitDeviceStep& g) {
    std::string err;
    if (g.release && !g.release(g, err)) throw std::runtime_error("freeing a device-resident training graph: " + err);
}
}  // namespace detail

inline void free_train_dit_graph(TrainDitGraph& g) {
    detail::release_device_step(g);
    g = TrainDitGraph{};
}

// build_train_dit_forward_graph (src/train_dit.h:57-218): the model's adapters are those of `lora`.
inline bool build_train_dit_forward_graph(DitModel& dit, const DitConfig& dc, const TrainLoraState& lora, int frames,
                                          int cond_dim, int ctx_len, TrainDitGraph& out, std::string& err,
                                          bool inpaint = false) {
    free_train_dit_graph(out);
    return detail::setup_dit_step(dit, dc, lora, frames, cond_dim, ctx_len, 0, out, err, inpaint);
}

}  // namespace sa3
