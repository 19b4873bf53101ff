// mirror_bench.cpp - the reference trainer's default update sequence (tools/sa3-train.cpp:574-714)
// through the host mirror (host/sa3/*.h), for bench.py's `dit_mirror` workload: a synthetic DiT of
// the benchmark size (24 blocks x 1536, f16 base), the full-scope dora-rows r32 adapters from
// init_train_lora_state, build_train_dit_ckpt, then per update `micro` samples through
// run_train_dit_accumulate_ckpt (one sample per call, as the reference runs them) and
// train_apply_accumulated_adamw. The samples come from TrainDiffusionSampler over random latents
// and are drawn before timing (the data pipeline is not part of the update).
//
// Built by sa3.cpp_amd/build.py into libsa3mirror.so (host code only, over libsa3k.so).
#include "sa3/train_loop.h"

#include <chrono>
#include <cstring>
#include <memory>
#include <random>
#include <string>
#include <vector>

namespace {

struct MirrorRun {
    sa3::DitConfig dc;
    sa3::DitModel model;
    sa3::TrainLoraState lora;
    sa3::TrainDitCkpt graph;
    sa3::TrainLoopState loop;
    sa3::TrainAdamWParams hp;
    sa3::TrainConditioning cond;
    std::vector<sa3::TrainDiffusionSample> samples;
    double last_loss = 0.0, last_norm = 0.0;
};

void copy_err(const std::string& e, char* err, int err_len) {
    if (err && err_len > 0) {
        std::strncpy(err, e.c_str(), (size_t)err_len - 1);
        err[err_len - 1] = '\0';
    }
}

}  // namespace

extern "C" {

// Set the run up: device_resident 0 = the reference's per-sample round trips (upload the adapters,
// read every gradient back, AdamW on host vectors through the device), 1 = this build's
// device-resident mode. Returns an opaque handle or null (message in err).
__attribute__((visibility("default"))) void* sa3m_create(int device_resident, int micro, int frames, char* err,
                                                         int err_len) {
    try {
        std::unique_ptr<MirrorRun> r(new MirrorRun());
        std::string e;
        sa3::DitConfig& dc = r->dc;
        dc.io = 64; dc.dim = 1536; dc.depth = 24; dc.heads = 24; dc.head_dim = 64; dc.cond_dim = 768;
        dc.mem_tokens = 64; dc.rot = 32; dc.time_dim = 256; dc.inner = 6144; dc.window = 256;
        if (!r->model.create(dc, SA3K_TYPE_F16, e) || !r->model.init_random(1234, 0.02f, e)) throw std::runtime_error(e);
        sa3::TrainLoraScope full;
        const std::vector<sa3::TrainLoraTarget> targets = sa3::enumerate_train_lora_targets(r->model, full);
        if (!sa3::init_train_lora_state(r->model, targets, "dora-rows", 32, 32.0f, 99, r->lora, e))
            throw std::runtime_error(e);
        std::mt19937 rng(7);
        std::normal_distribution<float> nd(0.0f, 1.0f);
        for (sa3::TrainLoraParam& p : r->lora.params)
            for (float& b : p.lora_B) b = 0.01f * nd(rng);
        const int ctx_len = 128;
        if (!sa3::build_train_dit_ckpt(r->model, dc, r->lora, frames, dc.cond_dim, ctx_len, r->graph, e))
            throw std::runtime_error(e);
        r->graph.device_resident = device_resident != 0;
        r->cond.cond_dim = dc.cond_dim;
        r->cond.ctx_len = ctx_len;
        r->cond.cross.resize((size_t)dc.cond_dim * ctx_len);
        r->cond.global.resize((size_t)dc.cond_dim);
        for (float& x : r->cond.cross) x = nd(rng);
        for (float& x : r->cond.global) x = nd(rng);
        sa3::TrainDiffusionSampler sampler(5, "trunc_logit_normal");
        r->samples.resize((size_t)micro);
        for (sa3::TrainDiffusionSample& s : r->samples) {
            std::vector<float> z((size_t)dc.io * frames);
            for (float& x : z) x = nd(rng);
            if (!sampler.sample_at(z, sampler.draw_t(), s, e)) throw std::runtime_error(e);
        }
        r->hp.learning_rate = 1e-4f;
        r->hp.weight_decay = 0.01f;
        r->hp.grad_clip = 1.0f;
        return r.release();
    } catch (const std::exception& ex) {
        copy_err(ex.what(), err, err_len);
        return nullptr;
    }
}

// One optimizer update: every sample of the run through the checkpointed graph, then AdamW.
// Returns 0, or 1 with the message in err.
__attribute__((visibility("default"))) int sa3m_update(void* h, char* err, int err_len) {
    MirrorRun* r = static_cast<MirrorRun*>(h);
    try {
        std::string e;
        sa3::TrainLoraGradAccum accum;
        double loss = 0.0;
        for (const sa3::TrainDiffusionSample& s : r->samples) {
            float l = 0.0f;
            if (!sa3::run_train_dit_accumulate_ckpt(r->graph, r->lora, accum, s, r->cond, r->dc, l, e))
                throw std::runtime_error(e);
            loss += l;
        }
        double norm = 0.0;
        if (!sa3::train_apply_accumulated_adamw(r->lora, accum, r->loop, r->hp, e, &norm)) throw std::runtime_error(e);
        r->last_loss = loss / (double)r->samples.size();
        r->last_norm = norm;
        return 0;
    } catch (const std::exception& ex) {
        copy_err(ex.what(), err, err_len);
        return 1;
    }
}

// the schedule build_train_dit_ckpt chose (1 checkpointed, 0 resident), the adapter parameter
// count, and the last update's mean loss and pre-clip gradient norm
__attribute__((visibility("default"))) void sa3m_info(void* h, int* recompute, long long* n_params, double* loss,
                                                      double* norm) {
    const MirrorRun* r = static_cast<const MirrorRun*>(h);
    if (recompute) *recompute = r->graph.recompute;
    if (n_params) *n_params = (long long)r->graph.n_params;
    if (loss) *loss = r->last_loss;
    if (norm) *norm = r->last_norm;
}

__attribute__((visibility("default"))) void sa3m_destroy(void* h) {
    MirrorRun* r = static_cast<MirrorRun*>(h);
    if (!r) return;
    try {
        sa3::free_train_dit_ckpt(r->graph);
    } catch (...) {
    }
    delete r;
}

}  // extern "C"
