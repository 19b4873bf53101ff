// Adapter checkpoints of the host mirror (sa3/train_checkpoint.h over sa3/gguf_io.h), driven by
// tests/test_adapter_gguf.py:
//   checkpoint_test write <path>   writes the deterministic state below
//   checkpoint_test read <path>    loads a file and prints its summary (one line per target)
//   checkpoint_test errors <dir>   round trip and every rejected input; prints "ok"
//   checkpoint_test bench <path>   times a write and a read of a full-scope DiT adapter
//   checkpoint_test resume <dir>   trainer-state sidecar and checkpoint pair (sa3/train_resume.h) with
//                                  the inputs of the reference's tests/train_checkpoint_test.cpp:18-103,
//                                  synthetic moments in place of its AdamW updates (those run on the
//                                  GPU in tests/host/train_host_test.cpp); prints "ok"
//   checkpoint_test state <path>   writes the deterministic trainer state below (for the format test)
#include "sa3/train_checkpoint.h"
#include "sa3/train_resume.h"

#include <chrono>
#include <filesystem>
#include <fstream>
#include <random>
#include <cmath>
#include <cstdio>
#include <string>
#include <vector>

namespace {

int fails = 0;
void expect(bool ok, const char* what) {
    if (!ok) {
        std::printf("FAIL: %s\n", what);
        ++fails;
    }
}

// value k of tensor `kind` of target `t`: distinct, exactly representable
float val(int t, int kind, size_t k) { return (float)(t * 1000 + kind * 100) + (float)(k % 97) * 0.25f - 7.0f; }

sa3::TrainLoraState make_state() {
    sa3::TrainLoraState st;
    st.adapter_type = "dora-rows";
    st.rank = 4;
    st.alpha = 6.5f;
    const char* stems[3] = {"dit.1.self.qkv", "dit.0.ff.out", "dit.proj_in"};
    const int64_t ins[3] = {16, 24, 8}, outs[3] = {40, 16, 12};
    for (int t = 0; t < 3; ++t) {
        sa3::TrainLoraParam p;
        p.target.stem = stems[t];
        p.target.weight_name = std::string(stems[t]) + ".weight";
        p.target.in = ins[t];
        p.target.out = outs[t];
        p.lora_A.resize((size_t)(st.rank * ins[t]));
        p.lora_B.resize((size_t)(outs[t] * st.rank));
        p.magnitude.resize((size_t)outs[t]);
        for (size_t k = 0; k < p.lora_A.size(); ++k) p.lora_A[k] = val(t, 0, k);
        for (size_t k = 0; k < p.lora_B.size(); ++k) p.lora_B[k] = val(t, 1, k);
        for (size_t k = 0; k < p.magnitude.size(); ++k) p.magnitude[k] = val(t, 5, k);
        st.params.push_back(p);
    }
    return st;
}

// the reference test's adapter (tests/train_checkpoint_test.cpp:21-31)
sa3::TrainLoraState reference_state() {
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
    return st;
}

// a loop state at step 3 with distinct moments for every trained vector
sa3::TrainLoopState synthetic_loop(const sa3::TrainLoraState& st) {
    sa3::TrainLoopState loop;
    loop.step = 3;
    const size_t n = st.params.size();
    for (auto* v : {&loop.A_state, &loop.B_state, &loop.mxs_state, &loop.mag_state, &loop.mag_r_state, &loop.mag_c_state})
        v->resize(n);
    for (size_t i = 0; i < n; ++i) {
        const sa3::TrainLoraParam& p = st.params[i];
        auto fill = [&](sa3::TrainAdamWTensorState& s, size_t len, float base) {
            s.m.resize(len);
            s.v.resize(len);
            for (size_t k = 0; k < len; ++k) {
                s.m[k] = base + 0.125f * (float)k;
                s.v[k] = 1e-6f * (float)(k + 1) + base * 1e-3f;
            }
        };
        fill(loop.A_state[i], p.lora_A.size(), 1.0f + (float)i);
        fill(loop.B_state[i], p.lora_B.size(), -2.0f - (float)i);
        if (!p.magnitude.empty()) fill(loop.mag_state[i], p.magnitude.size(), 0.5f);
    }
    return loop;
}

sa3::TrainResumeProgress reference_progress(std::mt19937_64& rng, sa3::TrainDiffusionSampler& diffusion) {
    sa3::TrainResumeProgress progress;   // tests/train_checkpoint_test.cpp:85-97
    progress.epoch = 2;
    progress.next_sample = 1;
    progress.order = {1, 0};
    progress.compatibility = "test-compatibility";
    progress.shuffle_rng = sa3::train_serialize_random_state(rng);
    progress.crop_rng = progress.shuffle_rng;
    progress.cfg_rng = progress.shuffle_rng;
    progress.prompt_rng = progress.shuffle_rng;
    progress.inpaint_rng = progress.shuffle_rng;
    progress.diffusion_rng = diffusion.serialize_state();
    return progress;
}

int resume_test(const std::string& dir) {
    namespace fs = std::filesystem;
    std::string err;
    const sa3::TrainLoraState st = reference_state();
    const sa3::TrainLoopState loop = synthetic_loop(st);
    std::mt19937_64 rng(12345);
    (void)rng();
    (void)rng();
    sa3::TrainDiffusionSampler diffusion(6789, "trunc_logit_normal");
    const std::vector<float> latent = {0.1f, -0.2f, 0.3f};
    sa3::TrainDiffusionSample first;
    expect(diffusion.sample(latent, first, err), "pre-checkpoint diffusion sample");
    const sa3::TrainResumeProgress progress = reference_progress(rng, diffusion);

    const fs::path pair_dir = fs::path(dir) / "pair";
    fs::remove_all(pair_dir);
    fs::create_directories(pair_dir);
    const fs::path adapter = pair_dir / "adapter-step-3.gguf", state = pair_dir / "trainer-state-step-3.gguf";
    expect(sa3::write_train_checkpoint_pair(st, loop, progress, adapter.string(), state.string(), err), err.c_str());
    expect(!fs::exists(adapter.string() + ".tmp") && !fs::exists(state.string() + ".tmp"), "no temporaries left");
    expect(!sa3::write_train_checkpoint_pair(st, loop, progress, adapter.string(), state.string(), err) &&
               err.find("refusing to overwrite an existing immutable training checkpoint at step 3") == 0,
           "immutable checkpoint overwrite rejected");
    {   // either file of the pair present is enough to refuse
        const fs::path lone = pair_dir / "adapter-step-4.gguf";
        std::ofstream(lone.string()) << "x";
        expect(!sa3::write_train_checkpoint_pair(st, loop, progress, lone.string(),
                                                 (pair_dir / "trainer-state-step-4.gguf").string(), err),
               "a lone adapter file blocks the pair");
        fs::remove(lone);
    }

    std::string ra, rs;
    expect(sa3::train_resolve_resume_pair(adapter.string(), ra, rs, err) && fs::path(rs) == state, "adapter -> state");
    expect(sa3::train_resolve_resume_pair(state.string(), ra, rs, err) && fs::path(ra) == adapter, "state -> adapter");
    expect(!sa3::train_resolve_resume_pair((pair_dir / "x.gguf").string(), ra, rs, err) &&
               err == "--resume expects adapter-step-N.gguf or trainer-state-step-N.gguf",
           "other names rejected");
    expect(sa3::train_checkpoint_step_from_name("trainer-state-step-17.gguf") == 17 &&
               sa3::train_checkpoint_step_from_name("trainer-state-step-.gguf") == -1 &&
               sa3::train_checkpoint_step_from_name("trainer-state-step-1x.gguf") == -1 &&
               sa3::train_checkpoint_step_from_name("trainer-state-step-99999999999.gguf") == -1 &&
               sa3::train_checkpoint_step_from_name("adapter-step-3.gguf") == -1,
           "step from name");
    expect(sa3::train_latest_checkpoint_step(pair_dir.string()) == 3, "latest step in a directory");
    expect(sa3::train_latest_checkpoint_step((pair_dir / "missing").string()) == -1, "latest step: no directory");

    // reload: adapter values into the expected state, then the sidecar
    sa3::TrainLoraState reloaded;
    expect(sa3::load_train_lora_gguf(adapter.string(), reloaded, err), "load adapter");
    sa3::TrainLoraState continued = st;
    for (float& a : continued.params[0].lora_A) a = -1.0f;
    expect(sa3::train_restore_adapter_values(continued, reloaded, err) &&
               continued.params[0].lora_A == st.params[0].lora_A && continued.params[0].lora_B == st.params[0].lora_B,
           "adapter values restored");
    sa3::TrainLoopState back;
    sa3::TrainResumeProgress rp;
    expect(sa3::load_train_state_gguf(state.string(), continued, back, rp, err), err.c_str());
    expect(back.step == 3 && rp.epoch == 2 && rp.next_sample == 1 && rp.order == progress.order,
           "step and dataset cursor restored");
    expect(rp.adapter_file == "adapter-step-3.gguf" && rp.compatibility == progress.compatibility &&
               rp.shuffle_rng == progress.shuffle_rng && rp.diffusion_rng == progress.diffusion_rng &&
               rp.crop_rng == progress.crop_rng && rp.cfg_rng == progress.cfg_rng &&
               rp.prompt_rng == progress.prompt_rng && rp.inpaint_rng == progress.inpaint_rng,
           "progress strings restored");
    expect(back.A_state[0].m == loop.A_state[0].m && back.A_state[0].v == loop.A_state[0].v &&
               back.B_state[0].m == loop.B_state[0].m && back.B_state[0].v == loop.B_state[0].v,
           "moments restored bit for bit");
    const std::string fp = sa3::train_resume_file_fingerprint(adapter.string(), err);
    expect(!fp.empty() && fp == rp.adapter_fingerprint && fp.rfind("fnv1a64:", 0) == 0 && fp.size() == 24,
           "trainer state is bound to the exact adapter file");
    {
        const fs::path tampered = pair_dir / "tampered.gguf";
        fs::copy_file(adapter, tampered);
        std::fstream f(tampered, std::ios::in | std::ios::out | std::ios::binary);
        f.seekg(-1, std::ios::end);
        char byte = 0;
        f.read(&byte, 1);
        byte ^= 1;
        f.seekp(-1, std::ios::end);
        f.write(&byte, 1);
        f.close();
        expect(!sa3::train_validate_resume_adapter_fingerprint(tampered.string(), rp.adapter_fingerprint, err) &&
                   err == "resume adapter does not match its trainer-state sidecar",
               "mismatched adapter/state pair rejected");
        expect(sa3::train_validate_resume_adapter_fingerprint(adapter.string(), rp.adapter_fingerprint, err),
               "matching adapter accepted");
        fs::remove(tampered);
    }
    expect(sa3::train_validate_resume_compatibility(rp.compatibility, progress.compatibility, err), "compatible");
    expect(!sa3::train_validate_resume_compatibility(rp.compatibility, "different", err), "incompatible rejected");
    // the random engines continue exactly
    std::mt19937_64 restored;
    expect(sa3::train_restore_random_state(rp.shuffle_rng, restored, "shuffle", err) && rng() == restored(),
           "random engine continues exactly");
    expect(!sa3::train_restore_random_state(std::string("not a state"), restored, "shuffle", err) &&
               err == "invalid shuffle random state",
           "bad random state rejected");
    sa3::TrainDiffusionSampler restored_diffusion(1, "trunc_logit_normal");
    sa3::TrainDiffusionSample na, nb;
    expect(restored_diffusion.restore_state(rp.diffusion_rng, err) && diffusion.sample(latent, na, err) &&
               restored_diffusion.sample(latent, nb, err) && na.t == nb.t && na.noise == nb.noise,
           "diffusion sampler continues exactly");

    // rejected states
    {
        sa3::TrainLoopState zero = loop;
        zero.step = 0;
        expect(!sa3::write_train_state_gguf(st, zero, progress, (pair_dir / "z.gguf").string(), err) &&
                   err == "cannot write invalid trainer continuation state",
               "step 0 rejected");
        sa3::TrainResumeProgress cursor = progress;
        cursor.next_sample = 3;
        expect(!sa3::write_train_state_gguf(st, loop, cursor, (pair_dir / "z.gguf").string(), err), "cursor past the order");
        sa3::TrainLoopState partial = loop;
        partial.B_state[0].v.pop_back();
        expect(!sa3::write_train_state_gguf(st, partial, progress, (pair_dir / "z.gguf").string(), err) &&
                   err == "optimizer state is incomplete for dit.0.self.qkv.lora_B",
               "incomplete moments rejected");
        sa3::TrainLoraState other = st;
        other.params[0].target.stem = "dit.1.self.qkv";
        expect(!sa3::load_train_state_gguf(state.string(), other, back, rp, err) &&
                   err == "trainer state target order does not match the current model",
               "target order mismatch rejected");
        sa3::TrainLoraState more = st;
        more.params.push_back(st.params[0]);
        expect(!sa3::load_train_state_gguf(state.string(), more, back, rp, err) &&
                   err == "trainer state target inventory does not match the adapter",
               "target count mismatch rejected");
        sa3::TrainLoraState dora = st;
        dora.params[0].magnitude.assign(5, 1.0f);
        expect(!sa3::load_train_state_gguf(state.string(), dora, back, rp, err) &&
                   err.find("trainer state is missing optimizer tensors for optimizer.dit.0.self.qkv.magnitude") == 0,
               "missing moment tensors rejected");
        expect(!sa3::load_train_state_gguf(adapter.string(), st, back, rp, err) &&
                   err.find("not an sa3 trainer-state GGUF") == 0,
               "an adapter file is not a trainer state");
        sa3::TrainLoraState rank3 = reloaded;
        rank3.rank = 3;
        sa3::TrainLoraState tgt = st;
        expect(!sa3::train_restore_adapter_values(tgt, rank3, err) &&
                   err == "resume adapter type/rank/alpha does not match the current training configuration",
               "rank mismatch rejected");
        sa3::TrainLoraState shorter = reloaded;
        shorter.params[0].lora_B.pop_back();
        expect(!sa3::train_restore_adapter_values(tgt, shorter, err) &&
                   err == "resume adapter tensor shape mismatch: dit.0.self.qkv.lora_B",
               "shape mismatch rejected");
    }
    fs::remove_all(pair_dir);
    if (fails) return 1;
    std::printf("checkpoint_test resume: ok\n");
    return 0;
}

double checksum(const std::vector<float>& v) {
    double s = 0.0;
    for (size_t k = 0; k < v.size(); ++k) s += (double)v[k] * (double)(k % 13 + 1);
    return s;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 3) return 2;
    const std::string mode = argv[1], path = argv[2];
    std::string err;
    if (mode == "write") {
        if (!sa3::write_train_lora_gguf(make_state(), path, err)) {
            std::printf("write failed: %s\n", err.c_str());
            return 1;
        }
        std::printf("written\n");
        return 0;
    }
    if (mode == "read") {
        sa3::TrainLoraState st;
        if (!sa3::load_train_lora_gguf(path, st, err)) {
            std::printf("load failed: %s\n", err.c_str());
            return 1;
        }
        std::printf("type=%s rank=%d alpha=%.9g targets=%zu\n", st.adapter_type.c_str(), st.rank, st.alpha,
                    st.params.size());
        for (const sa3::TrainLoraParam& p : st.params)
            std::printf("%s in=%lld out=%lld A=%zu:%.17g B=%zu:%.17g m=%zu:%.17g\n", p.target.stem.c_str(),
                        (long long)p.target.in, (long long)p.target.out, p.lora_A.size(), checksum(p.lora_A),
                        p.lora_B.size(), checksum(p.lora_B), p.magnitude.size(), checksum(p.magnitude));
        return 0;
    }
    if (mode == "bench") {
        // the DiT's full-scope dora-rows rank-32 adapter shapes: per block qkv 1536->7680, out
        // 1536->1536, cross.q 1536->1536, cross.kv 1536->3072, cross.out 1536->1536, ff.proj
        // 1536->12288, ff.out 6144->1536 (24 blocks), plus the 12 head/tail linears (approximated
        // here as 12 x 1536->1536)
        sa3::TrainLoraState big;
        big.adapter_type = "dora-rows";
        big.rank = 32;
        big.alpha = 32.0f;
        const int64_t io[7][2] = {{1536, 7680}, {1536, 1536}, {1536, 1536}, {1536, 3072},
                                  {1536, 1536}, {1536, 12288}, {6144, 1536}};
        size_t floats = 0;
        for (int b = 0; b < 24 + 2; ++b)
            for (int k = 0; k < 7 && !(b >= 24 && k >= 6); ++k) {
                sa3::TrainLoraParam p;
                const int64_t in = b < 24 ? io[k][0] : 1536, out = b < 24 ? io[k][1] : 1536;
                p.target.stem = "dit." + std::to_string(b) + ".t" + std::to_string(k);
                p.target.in = in;
                p.target.out = out;
                p.lora_A.assign((size_t)(32 * in), 0.5f);
                p.lora_B.assign((size_t)(out * 32), 0.25f);
                p.magnitude.assign((size_t)out, 1.0f);
                floats += p.lora_A.size() + p.lora_B.size() + p.magnitude.size();
                big.params.push_back(std::move(p));
            }
        const auto t0 = std::chrono::steady_clock::now();
        if (!sa3::write_train_lora_gguf(big, path, err)) return 1;
        const auto t1 = std::chrono::steady_clock::now();
        sa3::TrainLoraState back;
        if (!sa3::load_train_lora_gguf(path, back, err)) return 1;
        const auto t2 = std::chrono::steady_clock::now();
        const double mb = floats * 4 / 1e6;
        const double w = std::chrono::duration<double>(t1 - t0).count(), r = std::chrono::duration<double>(t2 - t1).count();
        std::printf("adapter %zu targets, %.1f MB: write %.1f ms (%.0f MB/s), read %.1f ms (%.0f MB/s)\n",
                    big.params.size(), mb, w * 1e3, mb / w, r * 1e3, mb / r);
        return back.params.size() == big.params.size() ? 0 : 1;
    }
    if (mode == "resume") return resume_test(path);
    if (mode == "state") {
        // the reference test's adapter at step 3 with synthetic moments and its progress values
        const sa3::TrainLoraState st = reference_state();
        std::mt19937_64 rng(12345);
        sa3::TrainDiffusionSampler diffusion(6789, "trunc_logit_normal");
        sa3::TrainResumeProgress progress = reference_progress(rng, diffusion);
        progress.adapter_file = "adapter-step-3.gguf";
        progress.adapter_fingerprint = "fnv1a64:0123456789abcdef";
        std::string err;
        return sa3::write_train_state_gguf(st, synthetic_loop(st), progress, path, err) ? 0 : 1;
    }
    if (mode != "errors") return 2;
    const std::string dir = path;
    // round trip: values bitwise, targets sorted by stem, in/out from the shapes
    const sa3::TrainLoraState st = make_state();
    expect(sa3::write_train_lora_gguf(st, dir + "/a.gguf", err), "write");
    sa3::TrainLoraState back;
    expect(sa3::load_train_lora_gguf(dir + "/a.gguf", back, err), "load");
    expect(back.adapter_type == "dora-rows" && back.rank == 4 && back.alpha == 6.5f && back.params.size() == 3,
           "metadata");
    const int order[3] = {1, 0, 2};   // dit.0.ff.out < dit.1.self.qkv < dit.proj_in
    for (int i = 0; i < 3 && back.params.size() == 3; ++i) {
        const sa3::TrainLoraParam &a = st.params[(size_t)order[i]], &b = back.params[(size_t)i];
        expect(a.target.stem == b.target.stem && b.target.weight_name == a.target.stem + ".weight", "stem order");
        expect(a.target.in == b.target.in && a.target.out == b.target.out, "in/out from shapes");
        expect(a.lora_A == b.lora_A && a.lora_B == b.lora_B && a.magnitude == b.magnitude, "values bitwise");
        expect(b.U.empty() && b.V.empty() && b.M_xs.empty() && b.magnitude_r.empty(), "absent kinds stay empty");
    }
    // rejected inputs
    expect(!sa3::write_train_lora_gguf(sa3::TrainLoraState{}, dir + "/e.gguf", err) &&
               err == "cannot write empty LoRA checkpoint", "empty state rejected");
    expect(!sa3::write_train_lora_gguf(st, dir + "/no/such/dir/x.gguf", err), "unwritable path rejected");
    expect(!sa3::load_train_lora_gguf(dir + "/missing.gguf", back, err), "missing file rejected");
    {
        std::FILE* f = std::fopen((dir + "/bad.gguf").c_str(), "wb");
        std::fputs("GGML not a gguf", f);
        std::fclose(f);
        expect(!sa3::load_train_lora_gguf(dir + "/bad.gguf", back, err), "bad magic rejected");
    }
    {
        // the valid file cut short (in the header, metadata, tensor infos, the last tensor's data)
        std::FILE* f = std::fopen((dir + "/a.gguf").c_str(), "rb");
        std::vector<char> bytes(1 << 16);
        bytes.resize(std::fread(bytes.data(), 1, bytes.size(), f));
        std::fclose(f);
        bool all = true;
        for (size_t cut : {size_t(3), size_t(20), size_t(100), size_t(200), bytes.size() - 20}) {
            std::FILE* g = std::fopen((dir + "/cut.gguf").c_str(), "wb");
            std::fwrite(bytes.data(), 1, cut, g);
            std::fclose(g);
            all = all && !sa3::load_train_lora_gguf(dir + "/cut.gguf", back, err);
        }
        expect(all, "truncated files rejected");
    }
    {
        sa3::gguf::Writer w;   // adapter metadata but no rank
        w.set_str("general.architecture", "sa3-lora");
        w.set_f32("lora.alpha", 1.0f);
        w.add_f32("x.lora_A", {4, 2}, std::vector<float>(8, 1.0f));
        expect(w.write(dir + "/norank.gguf", err), "write norank");
        expect(!sa3::load_train_lora_gguf(dir + "/norank.gguf", back, err) && err.find("lora.rank") != std::string::npos,
               "missing lora.rank rejected");
    }
    {
        sa3::gguf::Writer w;   // rank and alpha, but no adapter tensors
        w.set_u32("lora.rank", 2);
        w.set_f32("lora.alpha", 1.0f);
        w.add_f32("dit.0.self.qkv.bias", {4}, std::vector<float>(4, 1.0f));
        expect(w.write(dir + "/none.gguf", err), "write none");
        expect(!sa3::load_train_lora_gguf(dir + "/none.gguf", back, err) &&
                   err.find("no adapter tensors found") == 0,
               "no adapter tensors rejected");
    }
    if (fails) return 1;
    std::printf("checkpoint_test: ok\n");
    return 0;
}
