// train_loop.h - the training-step helpers of the reference's src/train_loop.h:21-476 over the
// GPU: loop/accumulator state, averaging + global clip, the accumulated AdamW update, one
// micro-batch of the DiT step in the monolithic or the checkpointed schedule
// (run_train_dit_accumulate, run_train_dit_accumulate_ckpt), the one-sample update
// (run_train_dit_step) and the evaluation loss (run_eval_dit_loss). Names, fields, argument meaning and the
// bool/err convention are the reference's; the arithmetic runs through the sa3k C ABI.
//
// Difference of signature: the reference's first argument of run_train_dit_accumulate[_ckpt],
// run_train_dit_step and run_eval_dit_loss is the ggml backend; here the graph carries its device
// (sa3k) context, so that argument is gone.
#pragma once

#include "train_ckpt.h"
#include "train_diffusion.h"
#include "train_dit.h"
#include "train_inpaint.h"
#include "train_optimizer.h"

#include <string>
#include <vector>

namespace sa3 {

struct TrainLoopState {
    int step = 0;
    std::vector<TrainAdamWTensorState> A_state;
    std::vector<TrainAdamWTensorState> B_state;
    std::vector<TrainAdamWTensorState> mxs_state;
    std::vector<TrainAdamWTensorState> mag_state;
    std::vector<TrainAdamWTensorState> mag_r_state;
    std::vector<TrainAdamWTensorState> mag_c_state;
    // This build only: set while a device-resident training graph holds newer AdamW moments than
    // these host vectors (TrainLoraState::device_newer has the rules); device_read fills a loop
    // state with them.
    const void* device_newer = nullptr;
    bool (*device_read)(const void* graph, TrainLoopState& into, std::string& err) = nullptr;
};

struct TrainLoraGradAccum {
    int count = 0;
    std::vector<std::vector<float>> A;
    std::vector<std::vector<float>> B;
    std::vector<std::vector<float>> mxs;
    std::vector<std::vector<float>> mag;
    std::vector<std::vector<float>> mag_r;
    std::vector<std::vector<float>> mag_c;
    // This build only: the device-resident training graph whose accumulator holds this window's
    // sums (the host vectors then stay empty)
    const void* device = nullptr;
};

// The values of `loop` as host vectors: `loop` itself, or (device-newer) a copy filled from the
// device into `tmp`.
inline bool train_loop_host_view(const TrainLoopState& loop, TrainLoopState& tmp, const TrainLoopState*& view,
                                 std::string& err) {
    view = &loop;
    if (!loop.device_newer) return true;
    tmp = loop;
    tmp.device_newer = nullptr;
    if (!loop.device_read || !loop.device_read(loop.device_newer, tmp, err)) return false;
    view = &tmp;
    return true;
}

inline void train_accum_add(std::vector<float>& dst, const std::vector<float>& grad) {
    if (dst.empty()) dst.assign(grad.size(), 0.0f);
    for (size_t i = 0; i < grad.size(); ++i) dst[i] += grad[i];
}

inline void train_clear_accum(TrainLoraGradAccum& accum) { accum = TrainLoraGradAccum{}; }

namespace detail {

// every accumulated vector in the reference's visit order (A, B, mxs, mag, mag_r, mag_c per target)
inline std::vector<std::vector<float>*> accum_vectors(TrainLoraGradAccum& a) {
    std::vector<std::vector<float>*> v;
    for (size_t i = 0; i < a.A.size(); ++i)
        for (auto* g : {&a.A[i], &a.B[i], &a.mxs[i], &a.mag[i], &a.mag_r[i], &a.mag_c[i]}) v.push_back(g);
    return v;
}

inline size_t total_size(const std::vector<std::vector<float>*>& v) {
    size_t n = 0;
    for (auto* x : v) n += x->size();
    return n;
}

// ---- device-resident training (DitDeviceStep::device_resident)

// the params arena in the state layout of the graph's slots
inline bool read_state_from(const DitDeviceStep& st, TrainLoraState& into, std::string& err) {
    if (into.params.size() != st.slots.size()) {
        err = "adapter state does not match the training graph's targets";
        return false;
    }
    sa3k_ctx* ctx = st.model->ctx();
    for (size_t i = 0; i < st.slots.size(); ++i) {
        const DitDeviceStep::Slot& sl = st.slots[i];
        TrainLoraParam& q = into.params[i];
        q.lora_A.resize((size_t)sl.n_a);
        q.lora_B.resize((size_t)sl.n_b);
        if (sl.off_m >= 0) q.magnitude.resize((size_t)sl.n_m);
        if (sa3k_download(ctx, q.lora_A.data(), st.params + sl.off_a, (size_t)sl.n_a * 4) != SA3K_OK ||
            sa3k_download(ctx, q.lora_B.data(), st.params + sl.off_b, (size_t)sl.n_b * 4) != SA3K_OK ||
            (sl.off_m >= 0 &&
             sa3k_download(ctx, q.magnitude.data(), st.params + sl.off_m, (size_t)sl.n_m * 4) != SA3K_OK))
            return sa3k_fail(ctx, err);
    }
    return true;
}

// the moment arenas (m, v) of the graph and their slots' vectors in a loop state
inline bool moment_arenas(const DitDeviceStep& st, float** m, float** v, std::string& err) {
    sa3k_ctx* ctx = st.model->ctx();
    if (sa3k_dit_arena(ctx, st.model->handle(), 2, m, nullptr) != SA3K_OK ||
        sa3k_dit_arena(ctx, st.model->handle(), 3, v, nullptr) != SA3K_OK)
        return sa3k_fail(ctx, err);
    return true;
}

inline bool read_loop_from(const DitDeviceStep& st, TrainLoopState& into, std::string& err) {
    float *m = nullptr, *v = nullptr;
    if (!moment_arenas(st, &m, &v, err)) return false;
    sa3k_ctx* ctx = st.model->ctx();
    const size_t np = st.slots.size();
    for (auto* x : {&into.A_state, &into.B_state, &into.mag_state}) x->resize(np);
    for (size_t i = 0; i < np; ++i) {
        const DitDeviceStep::Slot& sl = st.slots[i];
        const struct { TrainAdamWTensorState* s; int64_t off, n; } parts[3] = {
            {&into.A_state[i], sl.off_a, sl.n_a}, {&into.B_state[i], sl.off_b, sl.n_b}, {&into.mag_state[i], sl.off_m, sl.n_m}};
        for (const auto& p : parts) {
            if (p.off < 0) continue;
            p.s->m.resize((size_t)p.n);
            p.s->v.resize((size_t)p.n);
            if (sa3k_download(ctx, p.s->m.data(), m + p.off, (size_t)p.n * 4) != SA3K_OK ||
                sa3k_download(ctx, p.s->v.data(), v + p.off, (size_t)p.n * 4) != SA3K_OK)
                return sa3k_fail(ctx, err);
        }
    }
    return true;
}

// a loop's host moments into the graph's moment arenas (zeros where a vector is missing, as the
// round-trip path starts them)
inline bool write_loop_to(const DitDeviceStep& st, const TrainLoopState& loop, std::string& err) {
    float *m = nullptr, *v = nullptr;
    if (!moment_arenas(st, &m, &v, err)) return false;
    sa3k_ctx* ctx = st.model->ctx();
    if (sa3k_memset(ctx, m, 0, (size_t)st.n_params * 4) != SA3K_OK ||
        sa3k_memset(ctx, v, 0, (size_t)st.n_params * 4) != SA3K_OK)
        return sa3k_fail(ctx, err);
    const size_t np = st.slots.size();
    for (size_t i = 0; i < np; ++i) {
        const DitDeviceStep::Slot& sl = st.slots[i];
        const struct { const std::vector<TrainAdamWTensorState>* s; int64_t off, n; } parts[3] = {
            {&loop.A_state, sl.off_a, sl.n_a}, {&loop.B_state, sl.off_b, sl.n_b}, {&loop.mag_state, sl.off_m, sl.n_m}};
        for (const auto& p : parts) {
            if (p.off < 0 || i >= p.s->size()) continue;
            const TrainAdamWTensorState& ts = (*p.s)[i];
            if (ts.m.size() == (size_t)p.n && sa3k_upload(ctx, m + p.off, ts.m.data(), (size_t)p.n * 4) != SA3K_OK)
                return sa3k_fail(ctx, err);
            if (ts.v.size() == (size_t)p.n && sa3k_upload(ctx, v + p.off, ts.v.data(), (size_t)p.n * 4) != SA3K_OK)
                return sa3k_fail(ctx, err);
        }
    }
    return true;
}

inline bool read_state_cb(const void* g, TrainLoraState& into, std::string& err) {
    return read_state_from(*static_cast<const DitDeviceStep*>(g), into, err);
}
inline bool read_loop_cb(const void* g, TrainLoopState& into, std::string& err) {
    return read_loop_from(*static_cast<const DitDeviceStep*>(g), into, err);
}

// the graph goes away: the state and loop whose newest values it holds get them back
inline bool release_cb(DitDeviceStep& st, std::string& err) {
    if (auto* s = static_cast<TrainLoraState*>(st.newer_state); s && s->device_newer == &st) {
        if (!read_state_from(st, *s, err)) return false;
        s->device_newer = nullptr;
    }
    if (auto* l = static_cast<TrainLoopState*>(st.newer_loop); l && l->device_newer == &st) {
        if (!read_loop_from(st, *l, err)) return false;
        l->device_newer = nullptr;
    }
    st.newer_state = st.newer_loop = nullptr;
    return true;
}

}  // namespace detail

// This build only: copy the newest values of a device-resident training run back into the host
// vectors of `lora` (and `loop`, when given). A no-op for values the host already holds.
inline bool train_state_to_host(TrainLoraState& lora, TrainLoopState* loop, std::string& err) {
    if (lora.device_newer) {
        if (!lora.device_read || !lora.device_read(lora.device_newer, lora, err)) return false;
        lora.device_newer = nullptr;
    }
    if (loop && loop->device_newer) {
        if (!loop->device_read || !loop->device_read(loop->device_newer, *loop, err)) return false;
        loop->device_newer = nullptr;
    }
    return true;
}

// train_average_and_clip (src/train_loop.h:147-171): mean over the window (count > 1), then scale
// every vector so the global L2 norm is <= grad_clip; grad_norm_out gets the pre-clip norm.
inline void train_average_and_clip(TrainLoraGradAccum& accum, const TrainAdamWParams& hp,
                                   double* grad_norm_out = nullptr) {
    if (accum.device) {   // device-resident: the window's sums are on the device
        auto& st = *static_cast<detail::DitDeviceStep*>(const_cast<void*>(accum.device));
        sa3k_ctx* ctx = st.model->ctx();
        double norm = 0.0;
        if (sa3k_average_and_clip(ctx, st.acc.get(), st.n_params, accum.count > 0 ? accum.count : 1, hp.grad_clip,
                                  &norm) != SA3K_OK)
            throw std::runtime_error(std::string("train_average_and_clip: ") + sa3k_last_error(ctx));
        if (grad_norm_out) *grad_norm_out = norm;
        return;
    }
    auto vecs = detail::accum_vectors(accum);
    const size_t n = detail::total_size(vecs);
    std::string err;
    sa3k_ctx* ctx = sa3k_default_ctx(err);
    DeviceF32 g;
    if (!ctx || !g.alloc(ctx, n, err)) throw std::runtime_error("train_average_and_clip: " + err);
    size_t off = 0;
    for (auto* x : vecs) {
        if (!g.upload(x->data(), x->size(), off, err)) throw std::runtime_error("train_average_and_clip: " + err);
        off += x->size();
    }
    double norm = 0.0;
    if (sa3k_average_and_clip(ctx, g.get(), (int64_t)n, accum.count > 0 ? accum.count : 1, hp.grad_clip, &norm) !=
        SA3K_OK)
        throw std::runtime_error(std::string("train_average_and_clip: ") + sa3k_last_error(ctx));
    if (grad_norm_out) *grad_norm_out = norm;
    off = 0;
    for (auto* x : vecs) {
        if (!g.download(x->data(), x->size(), off, err)) throw std::runtime_error("train_average_and_clip: " + err);
        off += x->size();
    }
}

// train_apply_accumulated_adamw (src/train_loop.h:173-211): loop.step += 1, mean + global clip,
// AdamW on every trained vector, accumulator cleared. One fused pass over all vectors on the GPU
// (sa3k_adamw_clip), bit-identical to the reference's per-vector host loops.
inline bool train_apply_accumulated_adamw(TrainLoraState& state, TrainLoraGradAccum& accum, TrainLoopState& loop,
                                          const TrainAdamWParams& hp, std::string& err,
                                          double* grad_norm_out = nullptr) {
    if (accum.count <= 0) {
        err = "cannot apply empty gradient batch";
        return false;
    }
    if (accum.device) {   // device-resident: AdamW over the graph's arenas, in place
        auto& st = *static_cast<detail::DitDeviceStep*>(const_cast<void*>(accum.device));
        sa3k_ctx* ctx = st.model->ctx();
        if (st.held != &state) {
            err = "the accumulator's training graph holds another adapter state";
            return false;
        }
        if (loop.device_newer && loop.device_newer != &st) {
            err = "the loop state's moments are newer on another training graph (train_state_to_host first)";
            return false;
        }
        if (loop.device_newer != &st && !detail::write_loop_to(st, loop, err)) return false;
        float *m = nullptr, *v = nullptr;
        if (!detail::moment_arenas(st, &m, &v, err)) return false;
        loop.step += 1;
        sa3k_adamw_params p{hp.learning_rate, hp.beta1, hp.beta2, hp.eps, hp.weight_decay, hp.grad_clip};
        double norm = 0.0;
        if (sa3k_adamw_clip(ctx, st.params, st.acc.get(), m, v, st.n_params, &p, loop.step, accum.count, &norm) !=
                SA3K_OK ||
            sa3k_dit_adapters_changed(ctx, st.model->handle()) != SA3K_OK)
            return sa3k_fail(ctx, err);
        if (grad_norm_out) *grad_norm_out = norm;
        state.device_newer = &st;
        state.device_read = detail::read_state_cb;
        loop.device_newer = &st;
        loop.device_read = detail::read_loop_cb;
        st.newer_state = &state;
        st.newer_loop = &loop;
        st.release = detail::release_cb;
        train_clear_accum(accum);
        return true;
    }
    if (state.device_newer || loop.device_newer) {
        err = "adapter or optimizer state is newer on a device-resident training graph (train_state_to_host first)";
        return false;
    }
    loop.step += 1;
    const size_t np = state.params.size();
    for (auto* s : {&loop.A_state, &loop.B_state, &loop.mxs_state, &loop.mag_state, &loop.mag_r_state,
                    &loop.mag_c_state})
        s->resize(np);
    for (auto* a : {&accum.A, &accum.B, &accum.mxs, &accum.mag, &accum.mag_r, &accum.mag_c}) a->resize(np);
    // the trained vectors, their gradients and moments, in visit order
    struct Slot { std::vector<float>* p; std::vector<float>* g; TrainAdamWTensorState* st; };
    std::vector<Slot> slots;
    for (size_t i = 0; i < np; ++i) {
        TrainLoraParam& q = state.params[i];
        const Slot s[6] = {{&q.lora_A, &accum.A[i], &loop.A_state[i]},      {&q.lora_B, &accum.B[i], &loop.B_state[i]},
                           {&q.M_xs, &accum.mxs[i], &loop.mxs_state[i]},     {&q.magnitude, &accum.mag[i], &loop.mag_state[i]},
                           {&q.magnitude_r, &accum.mag_r[i], &loop.mag_r_state[i]},
                           {&q.magnitude_c, &accum.mag_c[i], &loop.mag_c_state[i]}};
        for (const Slot& x : s) {
            if (x.p->empty()) continue;
            if (x.g->size() != x.p->size()) {
                err = "AdamW parameter/gradient size mismatch";
                return false;
            }
            if (x.st->m.size() != x.p->size()) x.st->m.assign(x.p->size(), 0.0f);
            if (x.st->v.size() != x.p->size()) x.st->v.assign(x.p->size(), 0.0f);
            slots.push_back(x);
        }
    }
    size_t n = 0;
    for (const Slot& x : slots) n += x.p->size();
    sa3k_ctx* ctx = sa3k_default_ctx(err);
    if (!ctx) return false;
    DeviceF32 buf;   // [p | g | m | v], each n long
    if (!buf.alloc(ctx, 4 * n, err)) return false;
    size_t off = 0;
    for (const Slot& x : slots) {
        const size_t k = x.p->size();
        if (!buf.upload(x.p->data(), k, off, err) || !buf.upload(x.g->data(), k, n + off, err) ||
            !buf.upload(x.st->m.data(), k, 2 * n + off, err) || !buf.upload(x.st->v.data(), k, 3 * n + off, err))
            return false;
        off += k;
    }
    sa3k_adamw_params p{hp.learning_rate, hp.beta1, hp.beta2, hp.eps, hp.weight_decay, hp.grad_clip};
    float* b = buf.get();
    double norm = 0.0;
    if (sa3k_adamw_clip(ctx, b, b + n, b + 2 * n, b + 3 * n, (int64_t)n, &p, loop.step, accum.count, &norm) != SA3K_OK)
        return sa3k_fail(ctx, err);
    if (grad_norm_out) *grad_norm_out = norm;
    off = 0;
    for (const Slot& x : slots) {
        const size_t k = x.p->size();
        if (!buf.download(x.p->data(), k, off, err) || !buf.download(x.st->m.data(), k, 2 * n + off, err) ||
            !buf.download(x.st->v.data(), k, 3 * n + off, err))
            return false;
        off += k;
    }
    train_clear_accum(accum);
    return true;
}

// upload_train_lora_state (src/train_loop.h:42-60): the host adapters into the graph's arena
inline bool upload_train_lora_state(const TrainLoraState& state, detail::DitDeviceStep& graph, std::string& err) {
    if (state.device_newer) {   // device-resident training: its newest values are on a device
        if (state.device_newer == &graph) return true;
        err = "adapter state is newer on another training graph's device (train_state_to_host first)";
        return false;
    }
    if (state.params.size() != graph.slots.size()) {
        err = "adapter state does not match the training graph's targets";
        return false;
    }
    sa3k_ctx* ctx = graph.model->ctx();
    for (size_t i = 0; i < state.params.size(); ++i) {
        const TrainLoraParam& q = state.params[i];
        const TrainDitGraph::Slot& s = graph.slots[i];
        if (q.lora_A.size() != (size_t)s.n_a || q.lora_B.size() != (size_t)s.n_b ||
            (s.off_m >= 0 && q.magnitude.size() != (size_t)s.n_m)) {
            err = "adapter state does not match the training graph: " + q.target.weight_name;
            return false;
        }
        if (sa3k_upload(ctx, graph.params + s.off_a, q.lora_A.data(), q.lora_A.size() * 4) != SA3K_OK ||
            sa3k_upload(ctx, graph.params + s.off_b, q.lora_B.data(), q.lora_B.size() * 4) != SA3K_OK ||
            (s.off_m >= 0 &&
             sa3k_upload(ctx, graph.params + s.off_m, q.magnitude.data(), q.magnitude.size() * 4) != SA3K_OK))
            return sa3k_fail(ctx, err);
    }
    if (sa3k_dit_adapters_changed(ctx, graph.model->handle()) != SA3K_OK) return sa3k_fail(ctx, err);
    graph.held = &state;
    graph.held_edits = state.host_edits;
    return true;
}

namespace detail {
// The state's values into the graph's arena: every call on the round-trip path (the reference's
// per-sample upload); once in device-resident mode, while the arena holds them.
inline bool ensure_state(DitDeviceStep& st, const TrainLoraState& lora, std::string& err) {
    if (st.device_resident && st.held == &lora && st.held_edits == lora.host_edits &&
        (!lora.device_newer || lora.device_newer == &st))
        return true;
    return upload_train_lora_state(lora, st, err);
}
}  // namespace detail

namespace detail {

// The inputs of one sample into the step's device buffers, after the reference's checks.
inline bool upload_step_inputs(DitDeviceStep& st, const TrainDiffusionSample& sample, const TrainConditioning& cond,
                               const DitConfig& dc, const char* empty_msg, std::string& err) {
    if (sample.x_t.empty() || sample.velocity_target.empty() || cond.cross.empty() || cond.global.empty()) {
        err = empty_msg;
        return false;
    }
    const size_t nx = (size_t)dc.io * st.frames;
    if (sample.x_t.size() != nx || sample.velocity_target.size() != nx ||
        cond.cross.size() != (size_t)st.cond_dim * st.ctx_len || cond.global.size() != (size_t)st.cond_dim) {
        err = "training step inputs do not match the graph's dimensions";
        return false;
    }
    return st.x.upload(sample.x_t.data(), nx, 0, err) && st.target.upload(sample.velocity_target.data(), nx, 0, err) &&
           st.t.upload(&sample.t, 1, 0, err) &&
           st.cross.upload(cond.cross.data(), (size_t)st.cond_dim * st.ctx_len, 0, err) &&
           st.global.upload(cond.global.data(), (size_t)st.cond_dim, 0, err);
}

// An inpaint sample's local conditioning and loss weight (src/train_loop.h:239-242). The reference's
// weight is [frames][io] with one value per frame (build_train_inpaint broadcasts it over the
// channels); the device loss takes that per-frame value.
inline bool upload_inpaint(DitDeviceStep& st, const TrainInpaint& in, const DitConfig& dc, std::string& err) {
    const size_t F = (size_t)st.frames, io = (size_t)dc.io;
    if (in.local.size() != (size_t)dc.local_dim * F || in.loss_weight.size() != io * F) {
        err = "inpaint inputs do not match the graph's dimensions";
        return false;
    }
    std::vector<float> w(F);
    for (size_t t = 0; t < F; ++t) {
        w[t] = in.loss_weight[t * io];
        for (size_t c = 1; c < io; ++c)
            if (in.loss_weight[t * io + c] != w[t]) {
                err = "inpaint loss weights must be constant over a frame's channels";
                return false;
            }
    }
    return st.local.upload(in.local.data(), in.local.size(), 0, err) && st.loss_weight.upload(w.data(), F, 0, err);
}

// One sample through the model in whichever schedule it was set up with: forward, velocity MSE,
// backward; this call's gradients are read back and added into accum target by target, in the
// order of `visit` (count += 1).
inline bool accumulate_step(DitDeviceStep& st, const TrainLoraState& lora, TrainLoraGradAccum& accum,
                            const TrainDiffusionSample& sample, const TrainConditioning& cond, const DitConfig& dc,
                            float& loss_out, std::string& err, const TrainInpaint* inpaint,
                            const std::vector<size_t>& visit) {
    if (sample.x_t.empty() || sample.velocity_target.empty() || cond.cross.empty() || cond.global.empty()) {
        err = "training step inputs are empty";
        return false;
    }
    if (st.inpaint != (inpaint != nullptr)) {
        err = "inpaint graph/sample mismatch (local-cond present in one but not the other)";
        return false;
    }
    if (!upload_step_inputs(st, sample, cond, dc, "training step inputs are empty", err)) return false;
    if (inpaint && !upload_inpaint(st, *inpaint, dc, err)) return false;
    if (!ensure_state(st, lora, err)) return false;
    sa3k_ctx* ctx = st.model->ctx();
    if (st.device_resident) {
        // this sample's gradients into the graph's gradient arena, then added into the window's
        // device accumulator (0 + g1 + g2 ... in f32, as train_accum_add sums them on the host)
        if (accum.device != &st && (accum.device || accum.count > 0)) {
            err = "the accumulator holds sums of another graph or of the host path";
            return false;
        }
        if (!st.acc.get() && !st.acc.alloc(ctx, (size_t)st.n_params, err)) return false;
        if (!accum.device && sa3k_memset(ctx, st.acc.get(), 0, (size_t)st.n_params * 4) != SA3K_OK)
            return sa3k_fail(ctx, err);
        if (sa3k_memset(ctx, st.grads, 0, (size_t)st.n_params * 4) != SA3K_OK) return sa3k_fail(ctx, err);
        double loss = 0.0;
        if (sa3k_dit_set_local(ctx, st.model->handle(), st.inpaint ? st.local.get() : nullptr) != SA3K_OK ||
            sa3k_dit_accumulate(ctx, st.model->handle(), st.x.get(), st.target.get(), st.t.get(), st.cross.get(),
                                st.global.get(), st.inpaint ? st.loss_weight.get() : nullptr, &loss) != SA3K_OK ||
            sa3k_vec_add(ctx, st.acc.get(), st.grads, st.n_params) != SA3K_OK)
            return sa3k_fail(ctx, err);
        loss_out = (float)loss;
        accum.device = &st;
        accum.count += 1;
        (void)visit;   // the device accumulator keeps the arena's target order
        return true;
    }
    // this call's gradients alone, then added into the host accumulator like the reference reads
    // them back from its graphs (train_accum_read_subset)
    if (sa3k_memset(ctx, st.grads, 0, (size_t)st.n_params * 4) != SA3K_OK) return sa3k_fail(ctx, err);
    double loss = 0.0;
    if (sa3k_dit_set_local(ctx, st.model->handle(), st.inpaint ? st.local.get() : nullptr) != SA3K_OK ||
        sa3k_dit_accumulate(ctx, st.model->handle(), st.x.get(), st.target.get(), st.t.get(), st.cross.get(),
                            st.global.get(), st.inpaint ? st.loss_weight.get() : nullptr, &loss) != SA3K_OK)
        return sa3k_fail(ctx, err);
    loss_out = (float)loss;
    std::vector<float> g((size_t)st.n_params);
    if (sa3k_download(ctx, g.data(), st.grads, g.size() * 4) != SA3K_OK) return sa3k_fail(ctx, err);
    const size_t np = lora.params.size();
    for (auto* a : {&accum.A, &accum.B, &accum.mxs, &accum.mag, &accum.mag_r, &accum.mag_c}) a->resize(np);
    auto slice = [&](int64_t off, int64_t n) {
        return std::vector<float>(g.begin() + off, g.begin() + off + n);
    };
    for (size_t i : visit) {
        const DitDeviceStep::Slot& s = st.slots[i];
        train_accum_add(accum.A[i], slice(s.off_a, s.n_a));
        train_accum_add(accum.B[i], slice(s.off_b, s.n_b));
        if (s.off_m >= 0) train_accum_add(accum.mag[i], slice(s.off_m, s.n_m));
    }
    accum.count += 1;
    return true;
}

inline std::vector<size_t> all_targets(size_t n) {
    std::vector<size_t> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = i;
    return v;
}

}  // namespace detail

// run_train_dit_accumulate (src/train_loop.h:212-256): one sample through the DiT, velocity MSE,
// and the adapter gradients added into accum (count += 1).
inline bool run_train_dit_accumulate(TrainDitGraph& graph, const TrainLoraState& lora, TrainLoraGradAccum& accum,
                                     const TrainDiffusionSample& sample, const TrainConditioning& cond,
                                     const DitConfig& dc, float& loss_out, std::string& err,
                                     const TrainInpaint* inpaint = nullptr) {
    return detail::accumulate_step(graph, lora, accum, sample, cond, dc, loss_out, err, inpaint,
                                   detail::all_targets(lora.params.size()));
}

// run_train_dit_accumulate_ckpt (src/train_loop.h:309-441): the same step in the checkpointed
// schedule (one block's activations, each block recomputed before its backward). The gradients are
// read back segment by segment in the reference's order: tail (T), blocks depth-1 .. 0 (B_l), head
// (H). Each target belongs to exactly one segment, so the accumulated values are those of
// run_train_dit_accumulate bit for bit.
inline bool run_train_dit_accumulate_ckpt(TrainDitCkpt& ck, const TrainLoraState& lora, TrainLoraGradAccum& accum,
                                          const TrainDiffusionSample& sample, const TrainConditioning& cond,
                                          const DitConfig& dc, float& loss_out, std::string& err,
                                          const TrainInpaint* inpaint = nullptr) {
    std::vector<size_t> visit(ck.tail_param_idx);
    for (int l = ck.depth - 1; l >= 0; --l)
        visit.insert(visit.end(), ck.block_param_idx[(size_t)l].begin(), ck.block_param_idx[(size_t)l].end());
    visit.insert(visit.end(), ck.head_param_idx.begin(), ck.head_param_idx.end());
    if (visit.size() != lora.params.size()) {
        err = "checkpointed graph does not match the adapter state";
        return false;
    }
    return detail::accumulate_step(ck, lora, accum, sample, cond, dc, loss_out, err, inpaint, visit);
}

// run_train_dit_step (src/train_loop.h:443-451): one sample's gradients, then the AdamW update.
inline bool run_train_dit_step(TrainDitGraph& graph, TrainLoraState& lora, TrainLoopState& loop,
                               const TrainAdamWParams& opt, const TrainDiffusionSample& sample,
                               const TrainConditioning& cond, const DitConfig& dc, float& loss_out, std::string& err) {
    TrainLoraGradAccum accum;
    if (!run_train_dit_accumulate(graph, lora, accum, sample, cond, dc, loss_out, err)) return false;
    return train_apply_accumulated_adamw(lora, accum, loop, opt, err);
}

// run_eval_dit_loss (src/train_loop.h:453-476): the loss of one sample under the adapters of
// `lora`, forward only (no gradient is computed or accumulated). The same device kernels as the
// training step compute it, so it equals the loss run_train_dit_accumulate reports.
inline bool run_eval_dit_loss(detail::DitDeviceStep& graph, const TrainLoraState& lora,
                              const TrainDiffusionSample& sample, const TrainConditioning& cond, const DitConfig& dc,
                              float& loss_out, std::string& err) {
    if (!detail::upload_step_inputs(graph, sample, cond, dc, "evaluation inputs are empty", err)) return false;
    if (!detail::ensure_state(graph, lora, err)) return false;
    sa3k_ctx* ctx = graph.model->ctx();
    double loss = 0.0;
    // an inpaint graph evaluates with its last sample's local conditioning and loss weight, as the
    // reference's graph keeps its input tensors
    if (sa3k_dit_set_local(ctx, graph.model->handle(), graph.inpaint ? graph.local.get() : nullptr) != SA3K_OK ||
        sa3k_dit_eval_loss(ctx, graph.model->handle(), graph.x.get(), graph.target.get(), graph.t.get(),
                           graph.cross.get(), graph.global.get(), graph.inpaint ? graph.loss_weight.get() : nullptr,
                           &loss) != SA3K_OK)
        return sa3k_fail(ctx, err);
    loss_out = (float)loss;
    return true;
}

}  // namespace sa3
