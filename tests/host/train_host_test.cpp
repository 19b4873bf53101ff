// Host-interface test of the trainer mirror (sa3.cpp_amd/host/sa3/*.h), in the style of the
// reference's tests/train_optimizer_test.cpp and tests/train_lora_test.cpp. Mode "cpu" checks the
// host-only parts (InverseLR schedule, target scopes); mode "gpu" also runs the device-backed
// parts: AdamW, row norms, adapter init, the DiT training graph and the accumulated update, and
// checks the mirror's packing against the C ABI's own arena path.
#include "sa3/dist_shift.h"
#include "sa3/train_checkpoint.h"
#include "sa3/train_loop.h"
#include "sa3/train_resume.h"

#include <cmath>
#include <filesystem>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

static int fails = 0;
static void expect(bool ok, const char* msg) {
    if (!ok) {
        std::fprintf(stderr, "FAIL: %s\n", msg);
        fails++;
    }
}

static void test_cpu() {
    // InverseLR at base_lr 1e-4, inv_gamma 1e6, power 0.5, warmup 0.995, final_lr 0
    // (tests/train_optimizer_test.cpp:32-44 of the reference)
    struct { int n; float lr; } ref[] = {
        {0, 5.0000000000e-07f},   {1, 9.9749950125e-07f},   {10, 5.3645151961e-06f},  {100, 3.9723855426e-05f},
        {500, 9.1860637497e-05f}, {1000, 9.9288298382e-05f}, {2499, 9.9874922989e-05f},
    };
    for (auto& r : ref) {
        const float got = sa3::inverse_lr(1.0e-4f, r.n, 1.0e6f, 0.5f, 0.995f, 0.0f);
        expect(std::fabs(got - r.lr) / r.lr < 1.0e-5f, "inverse_lr matches the published values");
    }
    expect(std::fabs(sa3::inverse_lr(1.0e-4f, 0, 1.0e6f, 0.5f, 0.0f, 0.0f) - 1.0e-4f) < 1.0e-10f,
           "inverse_lr without warmup: step 0 == base_lr");
    // final_lr is a floor
    expect(sa3::inverse_lr(1.0e-4f, 1000000, 1.0f, 1.0f, 0.0f, 3.0e-5f) == 3.0e-5f, "inverse_lr floor");

    // scopes over names (tests/train_lora_test.cpp:35-61)
    const char* names[] = {"dit.0.self.qkv.weight", "dit.0.cross.kv.weight", "dit.0.local.0.weight",
                           "dit.proj_in.weight"};
    auto count = [&](const sa3::TrainLoraScope& s) {
        int n = 0;
        for (const char* x : names) n += sa3::train_lora_target_selected(x, s) ? 1 : 0;
        return n;
    };
    sa3::TrainLoraScope full, core, only_cross, no_self, core_no_cross;
    core.name = "core";
    only_cross.include = {"cross."};
    no_self.exclude = {"self."};
    core_no_cross.name = "core";
    core_no_cross.exclude = {"cross."};
    expect(count(full) == 4, "full scope keeps all");
    expect(count(core) == 2, "core drops local + non-block");
    expect(count(only_cross) == 1, "include filters");
    expect(count(no_self) == 3, "exclude filters");
    expect(count(core_no_cross) == 1, "scope then exclude");
    expect(sa3::train_lora_is_block_weight("dit.11.ff.out.weight"), "block weight detected");
    expect(!sa3::train_lora_is_block_weight("dit.proj_in.weight"), "non-block detected");
    expect(!sa3::train_lora_is_block_weight("dit.time_embed.0.weight"), "embed is not a block");
    expect(sa3::train_lora_scope_known("core") && !sa3::train_lora_scope_known("attn"), "scope names");
}

// AdamW on the host in float, term by term (the reference's loop, src/train_optimizer.h:55-64)
static void host_adamw(std::vector<float>& p, const std::vector<float>& g, std::vector<float>& m,
                       std::vector<float>& v, const sa3::TrainAdamWParams& hp, int step) {
    const float b1c = 1.0f - std::pow(hp.beta1, (float)step);
    const float b2c = 1.0f - std::pow(hp.beta2, (float)step);
    for (size_t i = 0; i < p.size(); ++i) {
        m[i] = hp.beta1 * m[i] + (1.0f - hp.beta1) * g[i];
        v[i] = hp.beta2 * v[i] + (1.0f - hp.beta2) * g[i] * g[i];
        const float mh = m[i] / b1c, vh = v[i] / b2c;
        p[i] -= hp.learning_rate * (mh / (std::sqrt(vh) + hp.eps) + hp.weight_decay * p[i]);
    }
}

static double max_rel(const std::vector<float>& a, const std::vector<float>& b) {
    double d = 0, s = 0;
    for (size_t i = 0; i < a.size(); ++i) {
        d = std::max(d, std::fabs((double)a[i] - b[i]));
        s = std::max(s, std::fabs((double)b[i]));
    }
    return s > 0 ? d / s : d;
}

// Exact continuation (the reference's tests/train_checkpoint_test.cpp:55-190, its inputs): six
// uninterrupted updates == three, the checkpoint pair written, reloaded into fresh state, three
// more; parameters and both AdamW moments bit for bit. The updates run on the GPU.
static void test_gpu_resume() {
    namespace fs = std::filesystem;
    sa3::TrainLoraState st;
    st.adapter_type = "lora";
    st.rank = 2;
    st.alpha = 4.0f;
    sa3::TrainLoraParam p;
    p.target.weight_name = "dit.0.self.qkv.weight";
    p.target.stem = "dit.0.self.qkv";
    p.target.in = 3;
    p.target.out = 5;
    p.lora_A = {0, 1, 2, 3, 4, 5};
    p.lora_B = {0, 1, 2, 3, 4, 5, 6, 7, 8, 9};
    st.params.push_back(p);
    auto apply_step = [&](sa3::TrainLoraState& state, sa3::TrainLoopState& loop, int update) {
        sa3::TrainLoraGradAccum accum;
        const size_t n = state.params.size();
        accum.count = 1;
        accum.A.resize(n); accum.B.resize(n); accum.mxs.resize(n);
        accum.mag.resize(n); accum.mag_r.resize(n); accum.mag_c.resize(n);
        for (size_t i = 0; i < n; ++i) {
            accum.A[i].resize(state.params[i].lora_A.size());
            accum.B[i].resize(state.params[i].lora_B.size());
            for (size_t j = 0; j < accum.A[i].size(); ++j) accum.A[i][j] = 0.01f * (float)(update + 1) + 0.001f * (float)j;
            for (size_t j = 0; j < accum.B[i].size(); ++j) accum.B[i][j] = -0.02f * (float)(update + 1) + 0.0005f * (float)j;
        }
        sa3::TrainAdamWParams hp;
        hp.learning_rate = 1.0e-3f;
        hp.beta1 = 0.9f;
        hp.beta2 = 0.95f;
        hp.weight_decay = 0.01f;
        std::string e;
        return sa3::train_apply_accumulated_adamw(state, accum, loop, hp, e);
    };
    sa3::TrainLoraState uninterrupted = st, split = st;
    sa3::TrainLoopState u_loop, s_loop;
    for (int i = 0; i < 6; ++i) expect(apply_step(uninterrupted, u_loop, i), "uninterrupted AdamW step");
    for (int i = 0; i < 3; ++i) expect(apply_step(split, s_loop, i), "pre-checkpoint AdamW step");
    std::string err;
    sa3::TrainResumeProgress progress;
    progress.epoch = 2;
    progress.next_sample = 1;
    progress.order = {1, 0};
    progress.compatibility = "test-compatibility";
    std::mt19937_64 rng(12345);
    progress.shuffle_rng = progress.crop_rng = progress.cfg_rng = progress.prompt_rng = progress.inpaint_rng =
        sa3::train_serialize_random_state(rng);
    progress.diffusion_rng = sa3::TrainDiffusionSampler(6789, "trunc_logit_normal").serialize_state();
    const fs::path dir = fs::temp_directory_path() / "sa3_train_host_test_resume";
    fs::remove_all(dir);
    fs::create_directories(dir);
    const fs::path adapter = dir / "adapter-step-3.gguf", state = dir / "trainer-state-step-3.gguf";
    expect(sa3::write_train_checkpoint_pair(split, s_loop, progress, adapter.string(), state.string(), err),
           "write checkpoint pair");
    expect(!sa3::write_train_checkpoint_pair(split, s_loop, progress, adapter.string(), state.string(), err),
           "immutable checkpoint overwrite rejected");
    sa3::TrainLoraState reloaded, continued = st;   // expected targets and shapes from the current model
    sa3::TrainLoopState c_loop;
    sa3::TrainResumeProgress rp;
    expect(sa3::load_train_lora_gguf(adapter.string(), reloaded, err) &&
               sa3::train_restore_adapter_values(continued, reloaded, err) &&
               sa3::load_train_state_gguf(state.string(), continued, c_loop, rp, err),
           "reload the pair");
    expect(c_loop.step == 3 && rp.order == progress.order && rp.next_sample == 1, "step and cursor restored");
    expect(sa3::train_validate_resume_adapter_fingerprint(adapter.string(), rp.adapter_fingerprint, err),
           "adapter matches its sidecar");
    for (int i = 3; i < 6; ++i) expect(apply_step(continued, c_loop, i), "post-resume AdamW step");
    expect(c_loop.step == u_loop.step, "final optimizer step exact");
    expect(continued.params[0].lora_A == uninterrupted.params[0].lora_A &&
               continued.params[0].lora_B == uninterrupted.params[0].lora_B,
           "final adapter parameters exact");
    expect(c_loop.A_state[0].m == u_loop.A_state[0].m && c_loop.A_state[0].v == u_loop.A_state[0].v &&
               c_loop.B_state[0].m == u_loop.B_state[0].m && c_loop.B_state[0].v == u_loop.B_state[0].v,
           "final AdamW moments exact");
    fs::remove_all(dir);
}

static void test_gpu() {
    test_gpu_resume();
    std::string err;
    // ---- AdamW (tests/train_optimizer_test.cpp:17-30) + the float update term by term
    {
        std::vector<float> p = {1.0f, -1.0f}, g = {0.5f, -0.25f};
        sa3::TrainAdamWTensorState st;
        sa3::TrainAdamWParams hp;
        hp.learning_rate = 0.1f;
        hp.weight_decay = 0.01f;
        expect(sa3::adamw_update_vector(p, g, st, hp, 1, err), "adamw update");
        expect(p[0] < 1.0f, "positive grad decreases param");
        expect(p[1] > -1.0f, "negative grad increases param");
        expect(st.m.size() == 2 && st.v.size() == 2, "state initialized");
        std::vector<float> bad = {1.0f};
        expect(!sa3::adamw_update_vector(p, bad, st, hp, 2, err), "size mismatch rejected");
        expect(!sa3::adamw_update_vector(p, g, st, hp, 0, err), "step 0 rejected");

        std::mt19937 rng(5);
        std::normal_distribution<float> nd(0.0f, 1.0f);
        std::vector<float> q(1000), gq(1000), hq, hm(1000, 0.0f), hv(1000, 0.0f);
        for (float& x : q) x = nd(rng);
        hq = q;
        sa3::TrainAdamWTensorState sq;
        for (int step = 1; step <= 3; ++step) {
            for (float& x : gq) x = nd(rng);
            expect(sa3::adamw_update_vector(q, gq, sq, hp, step, err), "adamw continuation");
            host_adamw(hq, gq, hm, hv, hp, step);
        }
        expect(max_rel(q, hq) < 1e-6 && max_rel(sq.m, hm) < 1e-6 && max_rel(sq.v, hv) < 1e-6,
               "adamw continuation matches the float update");
    }
    // ---- row norms of W = 1..32 as [8 rows][4] (tests/train_lora_test.cpp:19-24, :73)
    {
        std::vector<float> w(32);
        for (int i = 0; i < 32; ++i) w[i] = (float)(i + 1);
        std::vector<float> n = sa3::train_row_norms(w, 4, 8), nsq = sa3::train_row_norm_sq(w, 4, 8, 1e-3f);
        expect(n[0] > 5.47f && n[0] < 5.48f, "dora row norm");
        bool ok = true;
        for (int r = 0; r < 8; ++r) {
            double s = 0;
            for (int c = 0; c < 4; ++c) s += (double)w[r * 4 + c] * w[r * 4 + c];
            ok = ok && std::fabs(n[r] - std::sqrt(s)) <= 1e-6 * std::sqrt(s);
            ok = ok && std::fabs(nsq[r] - (s + 4 * 1e-3)) <= 1e-6 * s;
        }
        expect(ok, "row norms and norm_sq match the closed form");
        expect(sa3::train_row_norms(std::vector<float>(), 4, 8) == std::vector<float>(8, 1.0f), "missing tensor: ones");
    }
    // ---- a depth-2 DiT: targets, adapter init, training graph, accumulate, AdamW
    sa3::DitConfig dc;
    dc.io = 64; dc.dim = 128; dc.depth = 2; dc.heads = 2; dc.head_dim = 64; dc.cond_dim = 64; dc.mem_tokens = 4;
    dc.time_dim = 64; dc.inner = 128; dc.window = 0;
    sa3::DitModel dit;
    if (!dit.create(dc, SA3K_TYPE_F32, err)) {
        expect(false, ("dit create: " + err).c_str());
        return;
    }
    expect(dit.init_random(11, 0.05f, err), "dit init");
    // a weight with known rows: W[o][i] = (o*in + i + 1) / 1000
    {
        const std::string name = "dit.1.cross.q.weight";
        const int64_t in = dit.ne0(name), out = dit.ne1(name);
        std::vector<float> w((size_t)(in * out));
        for (size_t i = 0; i < w.size(); ++i) w[i] = (float)(i + 1) / 1000.0f;
        expect(dit.set_tensor(name, w.data(), w.size() * 4, err), "set tensor");
        std::vector<float> n = sa3::train_row_norms(dit, name), ref = sa3::train_row_norms(w, in, out);
        expect(max_rel(n, ref) < 1e-6, "model row norms == host-vector row norms");
    }
    sa3::TrainLoraScope full, core, cross;
    core.name = "core";
    cross.include = {"cross."};
    std::vector<sa3::TrainLoraTarget> targets = sa3::enumerate_train_lora_targets(dit, full);
    expect(targets.size() == 2 * 7 + 12, "full scope: 7 per block + 12 head/tail");
    expect(sa3::enumerate_train_lora_targets(dit, core).size() == 14, "core scope: 7 per block");
    expect(sa3::enumerate_train_lora_targets(dit, cross).size() == 6, "include cross.: q, kv, out per block");
    bool sorted = true;
    for (size_t i = 1; i < targets.size(); ++i) sorted = sorted && targets[i - 1].weight_name < targets[i].weight_name;
    expect(sorted, "targets sorted by weight name");
    expect(targets[0].stem + ".weight" == targets[0].weight_name, "target stem");

    sa3::TrainLoraState st;
    expect(!sa3::init_train_lora_state(dit, targets, "lora", 129, 8.0f, 7, st, err), "infeasible rank rejected");
    expect(!sa3::init_train_lora_state(dit, targets, "bora", 8, 8.0f, 7, st, err), "unimplemented family rejected");
    expect(sa3::init_train_lora_state(dit, targets, "dora-rows", 8, 16.0f, 7, st, err), "init dora rows");
    sa3::TrainLoraState st2;
    expect(sa3::init_train_lora_state(dit, targets, "dora-rows", 8, 16.0f, 7, st2, err) &&
               st2.params[3].lora_A == st.params[3].lora_A,
           "same seed, same A");
    bool shapes = st.params.size() == targets.size();
    for (size_t i = 0; shapes && i < targets.size(); ++i) {
        const sa3::TrainLoraParam& p = st.params[i];
        const float bound = 1.0f / std::sqrt((float)targets[i].in);
        shapes = p.lora_A.size() == (size_t)(8 * targets[i].in) && p.lora_B.size() == (size_t)(8 * targets[i].out) &&
                 p.magnitude.size() == (size_t)targets[i].out;
        for (float a : p.lora_A) shapes = shapes && std::fabs(a) <= bound;
        for (float b : p.lora_B) shapes = shapes && b == 0.0f;
    }
    expect(shapes, "adapter shapes, Kaiming bound, B = 0");

    sa3::TrainDitGraph graph;
    const int frames = 12, ctx_len = 5;
    if (!sa3::build_train_dit_forward_graph(dit, dc, st, frames, dc.cond_dim, ctx_len, graph, err)) {
        expect(false, ("build graph: " + err).c_str());
        return;
    }
    // B ~ small noise so every gradient term is live
    std::mt19937 rng(3);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    for (sa3::TrainLoraParam& p : st.params)
        for (float& b : p.lora_B) b = 0.01f * nd(rng);
    // the step's sample from the rectified-flow sampler: a clean latent, a truncated logit-normal t
    // warped by the LogSNR distribution shift, the noised x_t and the velocity target
    std::vector<float> z((size_t)dc.io * frames);
    for (float& x : z) x = nd(rng);
    sa3::TrainDiffusionSampler sampler(77, "trunc_logit_normal");
    float p1, p2, p3, p4;
    sa3::dist_shift_defaults("LogSNR", p1, p2, p3, p4);
    const float t_warped = sa3::dist_shift_warp("LogSNR", sampler.draw_t(), frames, p1, p2, p3, p4);
    sa3::TrainDiffusionSample s;
    expect(sampler.sample_at(z, t_warped, s, err), "sampler");
    expect(s.t == t_warped && s.t > 0.0f && s.t < 1.0f, "warped t in (0,1)");
    sa3::TrainConditioning c;
    c.cond_dim = dc.cond_dim;
    c.ctx_len = ctx_len;
    c.cross.resize((size_t)dc.cond_dim * ctx_len);
    c.global.resize((size_t)dc.cond_dim);
    for (float& x : c.cross) x = nd(rng);
    for (float& x : c.global) x = nd(rng);

    sa3::TrainLoraGradAccum accum;
    sa3::TrainLoopState loop;
    sa3::TrainAdamWParams hp;
    hp.learning_rate = 1e-3f;
    hp.weight_decay = 0.01f;
    hp.grad_clip = 1.0f;
    expect(!sa3::train_apply_accumulated_adamw(st, accum, loop, hp, err) && err == "cannot apply empty gradient batch",
           "empty batch rejected");
    sa3::TrainDiffusionSample bad = s;
    bad.x_t.pop_back();
    float loss0 = 0.0f, loss1 = 0.0f;
    expect(!sa3::run_train_dit_accumulate(graph, st, accum, bad, c, dc, loss0, err), "input size mismatch rejected");
    {
        std::mt19937_64 mrng(5);
        sa3::InpaintMaskType ty;
        const std::vector<float> mask = sa3::generate_inpaint_mask(frames, frames, {0.1, 0.8, 0.1}, mrng, ty);
        const sa3::TrainInpaint ip = sa3::build_train_inpaint(z, mask, dc.io, frames, dc.io + 1, 1.0f);
        expect(!sa3::run_train_dit_accumulate(graph, st, accum, s, c, dc, loss0, err, &ip) &&
                   err.find("inpaint graph/sample mismatch") == 0,
               "inpaint sample rejected by a graph built without local conditioning");
    }
    expect(sa3::run_train_dit_accumulate(graph, st, accum, s, c, dc, loss0, err), "accumulate 1");
    const sa3::TrainLoraGradAccum once = accum;
    expect(sa3::run_train_dit_accumulate(graph, st, accum, s, c, dc, loss1, err), "accumulate 2");
    expect(std::isfinite(loss0) && loss0 > 0.0f && loss0 == loss1, "loss finite and deterministic");
    expect(accum.count == 2, "two samples counted");
    bool twice = true, live = false;
    for (size_t i = 0; i < accum.A.size(); ++i) {
        for (size_t k = 0; k < accum.A[i].size(); ++k) twice = twice && accum.A[i][k] == 2.0f * once.A[i][k];
        for (size_t k = 0; k < accum.B[i].size(); ++k) twice = twice && accum.B[i][k] == 2.0f * once.B[i][k];
        for (size_t k = 0; k < accum.mag[i].size(); ++k) twice = twice && accum.mag[i][k] == 2.0f * once.mag[i][k];
        for (float g : once.A[i]) live = live || g != 0.0f;
    }
    expect(twice, "two identical samples accumulate exactly twice the gradients");
    expect(live, "A gradients are live");

    // ---- the reference's default path (tools/sa3-train.cpp:574-714): the checkpointed schedule on a
    // second model with the same weights: build_train_dit_ckpt -> the sampler's sample ->
    // run_train_dit_accumulate_ckpt -> train_apply_accumulated_adamw, against the monolithic path
    {
        sa3::DitModel dit2;
        expect(dit2.create(dc, SA3K_TYPE_F32, err) && dit2.init_random(11, 0.05f, err), "second model");
        {
            const std::string name = "dit.1.cross.q.weight";
            std::vector<float> w((size_t)(dit2.ne0(name) * dit2.ne1(name)));
            for (size_t i = 0; i < w.size(); ++i) w[i] = (float)(i + 1) / 1000.0f;
            expect(dit2.set_tensor(name, w.data(), w.size() * 4, err), "second model tensor");
        }
        sa3::TrainDitCkpt ck;
        expect(sa3::build_train_dit_ckpt(dit2, dc, st, frames, dc.cond_dim, ctx_len, ck, err), "build ckpt");
        expect(ck.depth == 2 && ck.tail_param_idx.size() == 2 && ck.head_param_idx.size() == 10 &&
                   ck.block_param_idx.size() == 2 && ck.block_param_idx[0].size() == 7 &&
                   ck.block_param_idx[1].size() == 7,
               "segments: tail 2, blocks 7 each, head 10");
        expect(sa3::train_ckpt_segment("dit.post_conv", 2) == -2 && sa3::train_ckpt_segment("dit.1.ff.out", 2) == 1 &&
                   sa3::train_ckpt_segment("dit.gce.0", 2) == -1 && sa3::train_ckpt_segment("dit.7.ff.out", 2) == -1,
               "segment of a stem");
        sa3::TrainLoraGradAccum acc_ck;
        float loss_ck = 0.0f;
        expect(!sa3::run_train_dit_accumulate_ckpt(ck, st, acc_ck, bad, c, dc, loss_ck, err), "ckpt: bad input rejected");
        expect(sa3::run_train_dit_accumulate_ckpt(ck, st, acc_ck, s, c, dc, loss_ck, err), "accumulate ckpt");
        expect(loss_ck == loss0 && acc_ck.count == 1, "checkpointed loss == monolithic loss");
        bool same = acc_ck.A.size() == once.A.size();
        for (size_t i = 0; same && i < once.A.size(); ++i)
            same = acc_ck.A[i] == once.A[i] && acc_ck.B[i] == once.B[i] && acc_ck.mag[i] == once.mag[i];
        expect(same, "checkpointed gradients == monolithic gradients, bit for bit");
        // the evaluation loss on either schedule is the training step's loss
        float le = 0.0f, le_ck = 0.0f;
        expect(sa3::run_eval_dit_loss(graph, st, s, c, dc, le, err) && le == loss0, "eval loss == accumulate loss");
        expect(sa3::run_eval_dit_loss(ck, st, s, c, dc, le_ck, err) && le_ck == loss0, "eval loss (ckpt)");
        expect(!sa3::run_eval_dit_loss(graph, st, bad, c, dc, le, err), "eval: bad input rejected");
        // one update from each schedule's accumulator, and run_train_dit_step, agree bit for bit
        sa3::TrainLoraState s_mono = st, s_ck = st, s_step = st;
        sa3::TrainLoopState l_mono, l_ck, l_step;
        sa3::TrainLoraGradAccum a_mono = once;
        expect(sa3::train_apply_accumulated_adamw(s_mono, a_mono, l_mono, hp, err) &&
                   sa3::train_apply_accumulated_adamw(s_ck, acc_ck, l_ck, hp, err),
               "adamw from both schedules");
        float l_st = 0.0f;
        expect(sa3::run_train_dit_step(graph, s_step, l_step, hp, s, c, dc, l_st, err) && l_st == loss0 &&
                   l_step.step == 1,
               "run_train_dit_step");
        bool upd = true;
        for (size_t i = 0; upd && i < st.params.size(); ++i)
            upd = s_ck.params[i].lora_A == s_mono.params[i].lora_A && s_ck.params[i].lora_B == s_mono.params[i].lora_B &&
                  s_ck.params[i].magnitude == s_mono.params[i].magnitude &&
                  s_step.params[i].lora_A == s_mono.params[i].lora_A && s_step.params[i].lora_B == s_mono.params[i].lora_B &&
                  s_step.params[i].magnitude == s_mono.params[i].magnitude;
        expect(upd, "updated adapters equal across schedules and run_train_dit_step");
        sa3::free_train_dit_ckpt(ck);
    }

    // ---- inpainting (src/train_dit.h:59-87, src/train_loop.h:212-256): a model with the local
    // conditioning linears (local_dim = 1 + io), its full scope (9 per block + 12), an inpaint
    // sample through the monolithic and the checkpointed graphs (bitwise equal), the mismatch rules
    {
        sa3::DitConfig di = dc;
        di.local_dim = dc.io + 1;
        sa3::TrainDitGraph ig;
        expect(!sa3::build_train_dit_forward_graph(dit, dc, st, frames, dc.cond_dim, ctx_len, ig, err, true) &&
                   err == "inpainting requested but DiT has no local-cond weights (dit.local_dim <= 0)",
               "inpaint graph on a model without local weights rejected");
        sa3::DitModel m1, m2;
        expect(m1.create(di, SA3K_TYPE_F16, err) && m1.init_random(21, 0.05f, err), "inpaint model");
        expect(m2.create(di, SA3K_TYPE_F16, err) && m2.init_random(21, 0.05f, err), "inpaint model 2");
        sa3::TrainLoraScope sfull, score;
        score.name = "core";
        const std::vector<sa3::TrainLoraTarget> it = sa3::enumerate_train_lora_targets(m1, sfull);
        expect(it.size() == 2 * 9 + 12, "full scope with local linears: 9 per block + 12");
        expect(sa3::enumerate_train_lora_targets(m1, score).size() == 14, "core scope drops local.{0,2}");
        sa3::TrainLoraState ist;
        expect(sa3::init_train_lora_state(m1, it, "dora-rows", 8, 16.0f, 9, ist, err), "init inpaint state");
        for (sa3::TrainLoraParam& p : ist.params)
            for (float& b : p.lora_B) b = 0.01f * nd(rng);
        std::mt19937_64 mrng(6);
        sa3::InpaintMaskType ty;
        const std::vector<float> mask = sa3::generate_inpaint_mask(frames, frames, {0.1, 0.8, 0.1}, mrng, ty);
        const sa3::TrainInpaint ip = sa3::build_train_inpaint(z, mask, dc.io, frames, di.local_dim, 1.0f);
        sa3::TrainDitCkpt ick;
        expect(sa3::build_train_dit_forward_graph(m1, di, ist, frames, dc.cond_dim, ctx_len, ig, err, true),
               "inpaint graph");
        expect(sa3::build_train_dit_ckpt(m2, di, ist, frames, dc.cond_dim, ctx_len, ick, err, true), "inpaint ckpt");
        sa3::TrainLoraGradAccum a1, a2;
        float l1 = 0.0f, l2 = 0.0f, le = 0.0f;
        expect(!sa3::run_train_dit_accumulate(ig, ist, a1, s, c, dc, l1, err) &&
                   err.find("inpaint graph/sample mismatch") == 0,
               "inpaint graph without its sample rejected");
        expect(sa3::run_train_dit_accumulate(ig, ist, a1, s, c, di, l1, err, &ip), "inpaint accumulate");
        expect(sa3::run_train_dit_accumulate_ckpt(ick, ist, a2, s, c, di, l2, err, &ip), "inpaint accumulate ckpt");
        expect(std::isfinite(l1) && l1 > 0.0f && l1 == l2, "inpaint loss finite, equal across schedules");
        expect(sa3::run_eval_dit_loss(ig, ist, s, c, di, le, err) && le == l1, "inpaint eval loss == accumulate loss");
        bool same = a1.A.size() == a2.A.size(), local_live = false;
        for (size_t i = 0; same && i < a1.A.size(); ++i) {
            same = a1.A[i] == a2.A[i] && a1.B[i] == a2.B[i] && a1.mag[i] == a2.mag[i];
            if (it[i].weight_name.find(".local.") != std::string::npos)
                for (float g : a1.A[i]) local_live = local_live || g != 0.0f;
        }
        expect(same, "inpaint gradients: checkpointed == monolithic bit for bit");
        expect(local_live, "local-conditioning adapters receive gradients");
        sa3::free_train_dit_ckpt(ick);
    }

    // ---- device-resident training (TrainDitCkpt::device_resident): the reference's default
    // sequence (build_train_dit_ckpt -> per-sample run_train_dit_accumulate_ckpt -> AdamW over
    // the window) with the adapters, the accumulator and the moments kept on the device, against
    // the round-trip path on a second model with the same weights: the same losses, pre-clip norms,
    // adapters and moments bit for bit over three updates of two samples each; the checkpoint pair
    // written from the device-resident state (read through, no explicit sync) is the same bytes;
    // freeing the graph hands the newest values back to the host state
    {
        sa3::DitModel ma, mb;
        expect(ma.create(dc, SA3K_TYPE_F16, err) && ma.init_random(31, 0.05f, err) && mb.create(dc, SA3K_TYPE_F16, err) &&
                   mb.init_random(31, 0.05f, err),
               "resident: two models");
        sa3::TrainLoraState sa, sb;
        expect(sa3::init_train_lora_state(ma, targets, "dora-rows", 8, 16.0f, 13, sa, err), "resident: init");
        for (sa3::TrainLoraParam& q : sa.params)
            for (float& b : q.lora_B) b = 0.01f * nd(rng);
        sb = sa;
        sa3::TrainDitCkpt ca, cb;
        expect(sa3::build_train_dit_ckpt(ma, dc, sa, frames, dc.cond_dim, ctx_len, ca, err) &&
                   sa3::build_train_dit_ckpt(mb, dc, sb, frames, dc.cond_dim, ctx_len, cb, err),
               "resident: build ckpt graphs");
        expect(ca.recompute == 0 && cb.recompute == 0, "the activations fit: the resident schedule is chosen");
        cb.device_resident = true;
        std::vector<sa3::TrainDiffusionSample> samples(2);
        for (int k = 0; k < 2; ++k) {
            std::vector<float> zz((size_t)dc.io * frames);
            for (float& x : zz) x = nd(rng);
            expect(sampler.sample_at(zz, sampler.draw_t(), samples[(size_t)k], err), "resident: sample");
        }
        sa3::TrainLoopState la, lb;
        bool same = true;
        for (int step = 0; step < 3; ++step) {
            sa3::TrainLoraGradAccum aa, ab;
            for (const sa3::TrainDiffusionSample& smp : samples) {
                float lossa = 0.0f, lossb = 0.0f;
                expect(sa3::run_train_dit_accumulate_ckpt(ca, sa, aa, smp, c, dc, lossa, err) &&
                           sa3::run_train_dit_accumulate_ckpt(cb, sb, ab, smp, c, dc, lossb, err),
                       "resident: accumulate");
                same = same && lossa == lossb;
            }
            expect(ab.device == &cb && ab.A.empty() && ab.count == 2, "resident: the window's sums stay on the device");
            double na = 0.0, nb = 0.0;
            expect(sa3::train_apply_accumulated_adamw(sa, aa, la, hp, err, &na) &&
                       sa3::train_apply_accumulated_adamw(sb, ab, lb, hp, err, &nb),
                   "resident: adamw");
            same = same && na == nb && la.step == lb.step && sb.device_newer == &cb;
        }
        expect(same, "resident: losses, norms and steps equal the round-trip path");
        // checkpoint pair from the device-resident state, read through without an explicit sync
        sa3::TrainResumeProgress prog;
        prog.order = {0, 1};
        prog.next_sample = 1;
        const std::string p_ad = "resident_pair.gguf", p_st = "resident_pair.state.gguf";
        auto bytes = [](const std::string& f) {
            std::FILE* h = std::fopen(f.c_str(), "rb");
            std::vector<char> v;
            if (!h) return v;
            char buf[65536];
            size_t k;
            while ((k = std::fread(buf, 1, sizeof buf, h)) > 0) v.insert(v.end(), buf, buf + k);
            std::fclose(h);
            return v;
        };
        std::vector<char> files[2][2];
        for (int k = 0; k < 2; ++k) {
            std::remove(p_ad.c_str());
            std::remove(p_st.c_str());
            expect(k == 0 ? sa3::write_train_checkpoint_pair(sa, la, prog, p_ad, p_st, err)
                          : sa3::write_train_checkpoint_pair(sb, lb, prog, p_ad, p_st, err),
                   "resident: checkpoint pair");
            files[k][0] = bytes(p_ad);
            files[k][1] = bytes(p_st);
        }
        std::remove(p_ad.c_str());
        std::remove(p_st.c_str());
        expect(!files[0][1].empty() && files[0][0] == files[1][0] && files[0][1] == files[1][1],
               "resident: the same adapter and trainer-state files");
        expect(sb.device_newer == &cb && sb.params[0].lora_A != sa.params[0].lora_A,
               "resident: the host vectors are stale until synced");
        sa3::free_train_dit_ckpt(cb);   // hands the newest values back to sb and lb
        bool eq = sb.device_newer == nullptr && lb.device_newer == nullptr && sa.params.size() == sb.params.size();
        for (size_t i = 0; eq && i < sa.params.size(); ++i)
            eq = sa.params[i].lora_A == sb.params[i].lora_A && sa.params[i].lora_B == sb.params[i].lora_B &&
                 sa.params[i].magnitude == sb.params[i].magnitude && la.A_state[i].m == lb.A_state[i].m &&
                 la.A_state[i].v == lb.A_state[i].v && la.B_state[i].m == lb.B_state[i].m &&
                 la.mag_state[i].v == lb.mag_state[i].v;
        expect(eq, "resident: adapters and moments equal the round-trip path bit for bit");
        sa3::free_train_dit_ckpt(ca);
        // the reference's checkpointed schedule on request, bitwise equal to the resident one
        setenv("SA3K_CKPT_RECOMPUTE", "1", 1);
        sa3::DitModel mc;
        sa3::TrainDitCkpt cc;
        expect(mc.create(dc, SA3K_TYPE_F16, err) && mc.init_random(31, 0.05f, err) &&
                   sa3::build_train_dit_ckpt(mc, dc, sa, frames, dc.cond_dim, ctx_len, cc, err) && cc.recompute == 1,
               "recompute schedule on request");
        unsetenv("SA3K_CKPT_RECOMPUTE");
        sa3::DitModel md;
        sa3::TrainDitCkpt cd;
        expect(md.create(dc, SA3K_TYPE_F16, err) && md.init_random(31, 0.05f, err) &&
                   sa3::build_train_dit_ckpt(md, dc, sa, frames, dc.cond_dim, ctx_len, cd, err) && cd.recompute == 0,
               "resident schedule again");
        sa3::TrainLoraGradAccum ac, ad;
        float lc = 0.0f, ld = 0.0f;
        expect(sa3::run_train_dit_accumulate_ckpt(cc, sa, ac, samples[0], c, dc, lc, err) &&
                   sa3::run_train_dit_accumulate_ckpt(cd, sa, ad, samples[0], c, dc, ld, err),
               "accumulate on both schedules");
        bool bit = lc == ld && ac.A.size() == ad.A.size();
        for (size_t i = 0; bit && i < ac.A.size(); ++i) bit = ac.A[i] == ad.A[i] && ac.B[i] == ad.B[i] && ac.mag[i] == ad.mag[i];
        expect(bit, "checkpointed == resident schedule, bit for bit");
        sa3::free_train_dit_ckpt(cc);
        sa3::free_train_dit_ckpt(cd);
    }

    // the C ABI's arena path on the same state: gradients of two accumulate calls, then one
    // sa3k_adamw_clip over the whole arena with count 2 == the mirror's packed update
    sa3k_ctx* ctx = dit.ctx();
    float *mom = nullptr, *var = nullptr;
    sa3k_dit_arena(ctx, dit.handle(), 2, &mom, nullptr);
    sa3k_dit_arena(ctx, dit.handle(), 3, &var, nullptr);
    const size_t n = (size_t)graph.n_params;
    expect(sa3::upload_train_lora_state(st, graph, err), "upload state");
    sa3k_memset(ctx, graph.grads, 0, n * 4);
    sa3k_memset(ctx, mom, 0, n * 4);
    sa3k_memset(ctx, var, 0, n * 4);
    double l2[1];
    expect(sa3k_dit_accumulate(ctx, dit.handle(), graph.x.get(), graph.target.get(), graph.t.get(), graph.cross.get(),
                               graph.global.get(), nullptr, l2) == SA3K_OK &&
               sa3k_dit_accumulate(ctx, dit.handle(), graph.x.get(), graph.target.get(), graph.t.get(),
                                   graph.cross.get(), graph.global.get(), nullptr, l2) == SA3K_OK,
           "arena accumulate");
    std::vector<float> ga(n);
    sa3k_download(ctx, ga.data(), graph.grads, n * 4);
    // the mirror adds per-sample gradients on the host (as the reference reads them back); the
    // arena accumulates in place term by term, so the two sums agree to rounding
    double gworst = 0.0;
    for (size_t i = 0; i < graph.slots.size(); ++i) {
        const sa3::TrainDitGraph::Slot& sl = graph.slots[i];
        gworst = std::max(gworst, max_rel(std::vector<float>(ga.begin() + sl.off_a, ga.begin() + sl.off_a + sl.n_a),
                                          accum.A[i]));
        gworst = std::max(gworst, max_rel(std::vector<float>(ga.begin() + sl.off_b, ga.begin() + sl.off_b + sl.n_b),
                                          accum.B[i]));
        gworst = std::max(gworst, max_rel(std::vector<float>(ga.begin() + sl.off_m, ga.begin() + sl.off_m + sl.n_m),
                                          accum.mag[i]));
    }
    expect(gworst < 1e-6, "mirror accumulator == arena gradients");
    sa3k_adamw_params p{hp.learning_rate, hp.beta1, hp.beta2, hp.eps, hp.weight_decay, hp.grad_clip};
    double norm_abi = 0.0, norm_mirror = 0.0;
    expect(sa3k_adamw_clip(ctx, graph.params, graph.grads, mom, var, (int64_t)n, &p, 1, 2, &norm_abi) == SA3K_OK,
           "arena adamw");
    expect(sa3::train_apply_accumulated_adamw(st, accum, loop, hp, err, &norm_mirror), "mirror adamw");
    expect(loop.step == 1 && accum.count == 0 && accum.A.empty(), "step counted, accumulator cleared");
    expect(std::fabs(norm_abi - norm_mirror) <= 1e-9 * norm_abi, "same pre-clip norm");
    std::vector<float> pa(n), ma(n);
    sa3k_download(ctx, pa.data(), graph.params, n * 4);
    sa3k_download(ctx, ma.data(), mom, n * 4);
    double worst = 0.0;
    for (size_t i = 0; i < graph.slots.size(); ++i) {
        const sa3::TrainDitGraph::Slot& sl = graph.slots[i];
        worst = std::max(worst, max_rel(std::vector<float>(pa.begin() + sl.off_a, pa.begin() + sl.off_a + sl.n_a),
                                        st.params[i].lora_A));
        worst = std::max(worst, max_rel(std::vector<float>(pa.begin() + sl.off_b, pa.begin() + sl.off_b + sl.n_b),
                                        st.params[i].lora_B));
        worst = std::max(worst, max_rel(std::vector<float>(pa.begin() + sl.off_m, pa.begin() + sl.off_m + sl.n_m),
                                        st.params[i].magnitude));
        worst = std::max(worst, max_rel(std::vector<float>(ma.begin() + sl.off_b, ma.begin() + sl.off_b + sl.n_b),
                                        loop.B_state[i].m));
    }
    expect(worst < 1e-6, "mirror AdamW == arena AdamW");

    // a few updates on the fixed sample lower the loss
    float first = 0.0f, last = 0.0f;
    for (int it = 0; it < 6; ++it) {
        float l = 0.0f;
        expect(sa3::run_train_dit_accumulate(graph, st, accum, s, c, dc, l, err), "train accumulate");
        expect(sa3::train_apply_accumulated_adamw(st, accum, loop, hp, err), "train adamw");
        if (it == 0) first = l;
        last = l;
    }
    expect(loop.step == 7, "seven optimizer steps");
    expect(last < first, "loss falls over updates");
    std::printf("loss %.6f -> %.6f over %d steps\n", first, last, loop.step - 1);

    // the trained adapters through an adapter checkpoint: written, read back bit for bit (targets in
    // stem order), and the reloaded state gives the same loss on the same sample
    {
        const std::string path = "train_host_test_adapter.gguf";
        expect(sa3::write_train_lora_gguf(st, path, err), "write adapter checkpoint");
        sa3::TrainLoraState back;
        expect(sa3::load_train_lora_gguf(path, back, err), "load adapter checkpoint");
        std::remove(path.c_str());
        bool same = back.adapter_type == st.adapter_type && back.rank == st.rank && back.alpha == st.alpha &&
                    back.params.size() == st.params.size();
        for (size_t i = 0; same && i < st.params.size(); ++i) {
            const sa3::TrainLoraParam& a = st.params[i];   // targets are already sorted by name
            const sa3::TrainLoraParam& b = back.params[i];
            same = a.target.stem == b.target.stem && a.target.in == b.target.in && a.target.out == b.target.out &&
                   a.lora_A == b.lora_A && a.lora_B == b.lora_B && a.magnitude == b.magnitude;
        }
        expect(same, "checkpoint round trip is bitwise");
        float l_st = 0.0f, l_back = 0.0f;
        sa3::TrainLoraGradAccum scratch;
        expect(sa3::run_train_dit_accumulate(graph, st, scratch, s, c, dc, l_st, err) &&
                   sa3::run_train_dit_accumulate(graph, back, scratch, s, c, dc, l_back, err),
               "accumulate with the reloaded adapters");
        expect(l_st == l_back, "reloaded adapters give the same loss");
    }
    sa3::free_train_dit_graph(graph);
}

int main(int argc, char** argv) {
    const bool gpu = argc > 1 && std::strcmp(argv[1], "gpu") == 0;
    test_cpu();
    if (gpu) test_gpu();
    if (fails) {
        std::fprintf(stderr, "train_host_test: %d failure(s)\n", fails);
        return 1;
    }
    std::printf("train_host_test (%s): ok\n", gpu ? "gpu" : "cpu");
    return 0;
}
