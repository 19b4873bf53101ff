// train_ckpt.h - the gradient-checkpointed DiT training schedule of the reference's
// src/train_ckpt.h:73-474 (TrainDitCkpt, build_train_dit_ckpt, free_train_dit_ckpt), the path
// sa3-train takes by default (src/train_config.h:77, tools/sa3-train.cpp:574-632).
//
// The reference decomposes one step into graphs F (forward, storing the block inputs), T (tail and
// loss, forward + backward), B_l for l = depth-1 .. 0 (recompute block l from its stored input and
// backpropagate) and H (head backward), so only one block's activations are alive at a time. Here
// the device DiT runs that same schedule inside one call when it is set up with recompute = 1: the
// block boundaries stay on the device, every block but the last is recomputed right before its
// backward, and the context / adaLN-signal gradients are summed on the device instead of on the
// host. What the reference keeps per graph - which adapter targets the tail, each block and the
// head own - is kept here as the same index lists, so a caller that reads gradients per segment
// finds them where the reference's does.
#pragma once

#include "train_dit.h"

#include <cstdlib>
#include <string>
#include <vector>

namespace sa3 {

// The segment that owns an adapter target stem (src/train_ckpt.h:48-61): the block index for
// dit.<l>.*, -2 for the tail linears (proj_out, post_conv), -1 for every other head linear.
inline int train_ckpt_segment(const std::string& stem, int depth) {
    if (stem == "dit.proj_out" || stem == "dit.post_conv") return -2;
    if (train_lora_is_block_weight(stem + ".")) {
        long long l = 0;
        for (size_t i = 4; i < stem.size() && stem[i] != '.' && l < depth; ++i) l = 10 * l + (stem[i] - '0');
        if (l < depth) return (int)l;
    }
    return -1;
}

struct TrainDitCkpt : detail::DitDeviceStep {
    int depth = 0;
    // the device schedule build_train_dit_ckpt chose: 1 recompute every block before its backward
    // (the reference's), 0 keep every block's activations (when they fit; the same results bit for
    // bit, one forward per block less)
    int recompute = 1;
    std::vector<size_t> tail_param_idx;                // targets of the tail graph (T)
    std::vector<std::vector<size_t>> block_param_idx;  // per block l: the targets of B_l
    std::vector<size_t> head_param_idx;                // targets of the head graph (H)
};

inline void free_train_dit_ckpt(TrainDitCkpt& ck) {
    detail::release_device_step(ck);
    ck = TrainDitCkpt{};
}

// build_train_dit_ckpt (src/train_ckpt.h:143-474): set `dit` up in the checkpointed schedule for
// one sample of `frames` frames and `ctx_len` context tokens with the adapters of `lora`, and group
// the targets by segment. The model must not have been set up before (a model runs one schedule).
inline bool build_train_dit_ckpt(DitModel& dit, const DitConfig& dc, const TrainLoraState& lora, int frames,
                                 int cond_dim, int ctx_len, TrainDitCkpt& out, std::string& err, bool inpaint = false) {
    free_train_dit_ckpt(out);
    // The reference checkpoints to fit 8 GB GPUs. The activations of every block are kept when they
    // fit the device with room to spare (a quarter more plus 16 GiB for the weights' working copies,
    // the arenas and the shared scratch): the recompute forward is then skipped.
    int recompute = 1;
    {
        sa3k_ctx* ctx = dit.ctx();
        const bool dora = lora.adapter_type == "dora-rows";
        sa3k_dit_train tr{lora.rank, lora.alpha, dora ? 1 : 0, SA3K_SCOPE_FULL, 1, frames, ctx_len, 0};
        size_t need = 0, free_b = 0, total_b = 0;
        if (frames > 0 && ctx_len > 0 && sa3k_dit_resident_bytes(ctx, dit.handle(), &tr, &need) == SA3K_OK &&
            sa3k_device_memory(ctx, &free_b, &total_b) == SA3K_OK && free_b > need + need / 4 + ((size_t)16 << 30))
            recompute = 0;
        // SA3K_CKPT_RECOMPUTE=1 keeps the reference's checkpointed schedule, 0 forces the resident one
        if (const char* e = std::getenv("SA3K_CKPT_RECOMPUTE")) recompute = std::atoi(e) != 0 ? 1 : 0;
    }
    if (!detail::setup_dit_step(dit, dc, lora, frames, cond_dim, ctx_len, recompute, out, err, inpaint)) {
        free_train_dit_ckpt(out);
        return false;
    }
    out.depth = dc.depth;
    out.recompute = recompute;
    out.block_param_idx.assign((size_t)dc.depth, {});
    for (size_t i = 0; i < lora.params.size(); ++i) {
        const int seg = train_ckpt_segment(lora.params[i].target.stem, dc.depth);
        if (seg == -2) out.tail_param_idx.push_back(i);
        else if (seg == -1) out.head_param_idx.push_back(i);
        else out.block_param_idx[(size_t)seg].push_back(i);
    }
    return true;
}

}  // namespace sa3
