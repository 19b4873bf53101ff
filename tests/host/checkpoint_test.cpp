// Adapter checkpoints of the host mirror (sa3/train_checkpoint.h over sa3/gguf_io.h), driven by
// tests/test_adapter_gguf.py:
//   checkpoint_test write <path>   writes the deterministic state below
//   checkpoint_test read <path>    loads a file and prints its summary (one line per target)
//   checkpoint_test errors <dir>   round trip and every rejected input; prints "ok"
//   checkpoint_test bench <path>   times a write and a read of a full-scope DiT adapter
#include "sa3/train_checkpoint.h"

#include <chrono>
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
