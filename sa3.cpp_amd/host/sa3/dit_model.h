// dit_model.h - the DiT configuration and its named frozen tensors on the GPU: the parts of the
// reference's DitConfig (src/dit.h:20-46) and GgufModel::get/has (src/gguf_model.h:200-276) that the
// training path reads. Tensors keep the GGUF names (dit.<l>.self.qkv.weight, dit.memory_tokens,
// ...); they are filled from host memory or drawn on the device (synthetic models). Reading a GGUF
// file is outside this build.
#pragma once

#include "sa3k_host.h"

#include <map>
#include <string>
#include <vector>

namespace sa3 {

struct DitConfig {
    int io = 256, dim = 1536, depth = 24, heads = 24, head_dim = 64, cond_dim = 768, mem_tokens = 64, rot = 32,
        time_dim = 256, local_dim = 0;
    float rope_base = 10000.0f, norm_eps = 1e-5f, qk_eps = 1e-6f, time_min_freq = 0.5f, time_max_freq = 10000.0f;
    bool differential = true;
    // not DitConfig fields in the reference: the feed-forward width (read there from the
    // ff.proj weight's shape) and this build's self-attention window (0 = dense, the reference)
    int inner = 6144;
    int window = 0;
};

class DitModel {
public:
    DitModel() = default;
    DitModel(const DitModel&) = delete;
    DitModel& operator=(const DitModel&) = delete;
    ~DitModel() { reset(); }

    // weight_type: SA3K_TYPE_F32 / F16 / BF16 storage of the 2-D weights
    bool create(const DitConfig& c, int weight_type, std::string& err) {
        reset();
        if (!c.differential) {
            err = "only the differential DiT (medium family) is implemented";
            return false;
        }
        if (c.local_dim < 0) {
            err = "dit.local_dim must be 0 (no inpaint conditioning) or positive";
            return false;
        }
        ctx_ = sa3k_default_ctx(err);
        if (!ctx_) return false;
        cfg_ = c;
        sa3k_dit_config kc{c.io, c.dim, c.depth, c.heads, c.head_dim, c.cond_dim, c.mem_tokens, c.rot, c.time_dim,
                           c.inner, c.window, c.rope_base, c.norm_eps, c.qk_eps, c.time_min_freq, c.time_max_freq,
                           c.local_dim};
        if (sa3k_dit_create(ctx_, &kc, weight_type, &dit_) != SA3K_OK) return sa3k_fail(ctx_, err);
        int n = 0;
        if (sa3k_dit_tensor_count(ctx_, dit_, &n) != SA3K_OK) return sa3k_fail(ctx_, err);
        char name[256];
        for (int i = 0; i < n; ++i) {
            Info info;
            if (sa3k_dit_tensor_info(ctx_, dit_, i, name, (int)sizeof name, &info.rows, &info.cols, &info.type) != SA3K_OK)
                return sa3k_fail(ctx_, err);
            names_.push_back(name);
            info_[name] = info;
        }
        return true;
    }
    void reset() {
        if (dit_ && ctx_) sa3k_dit_destroy(ctx_, dit_);
        dit_ = nullptr;
        names_.clear();
        info_.clear();
    }

    bool has(const std::string& name) const { return info_.count(name) != 0; }
    // ggml ne order of the reference: ne0 = in (cols), ne1 = out (rows); 1-D tensors have ne1 = 1
    int64_t ne0(const std::string& name) const { return has(name) ? info_.at(name).cols : 0; }
    int64_t ne1(const std::string& name) const { return has(name) ? info_.at(name).rows : 0; }
    bool is_2d(const std::string& name) const { return has(name) && info_.at(name).cols > 1; }
    int type(const std::string& name) const { return has(name) ? info_.at(name).type : -1; }
    const std::vector<std::string>& tensor_names() const { return names_; }

    // elements in the tensor's stored type (f32 / f16 / bf16 bits), host memory
    bool set_tensor(const std::string& name, const void* data, size_t bytes, std::string& err) {
        if (sa3k_dit_set_tensor(ctx_, dit_, name.c_str(), data, (int64_t)bytes) != SA3K_OK) return sa3k_fail(ctx_, err);
        return true;
    }
    bool init_random(unsigned long long seed, float w_sd, std::string& err) {
        if (sa3k_dit_init_random(ctx_, dit_, seed, w_sd) != SA3K_OK) return sa3k_fail(ctx_, err);
        return true;
    }
    // train_row_norms / train_row_norm_sq of a weight (mode 0 / 1), computed on the device
    bool row_norms(const std::string& name, int mode, float eps, std::vector<float>& out, std::string& err) const {
        const int64_t rows = ne1(name);
        DeviceF32 d;
        if (!d.alloc(ctx_, (size_t)rows, err)) return false;
        if (sa3k_dit_weight_row_norms(ctx_, dit_, name.c_str(), mode, eps, d.get()) != SA3K_OK)
            return sa3k_fail(ctx_, err);
        out.resize((size_t)rows);
        return d.download(out.data(), out.size(), 0, err);
    }

    const DitConfig& config() const { return cfg_; }
    sa3k_ctx* ctx() const { return ctx_; }
    sa3k_dit* handle() const { return dit_; }

private:
    struct Info {
        int64_t rows = 0, cols = 0;
        int type = 0;
    };
    sa3k_ctx* ctx_ = nullptr;
    sa3k_dit* dit_ = nullptr;
    DitConfig cfg_;
    std::vector<std::string> names_;
    std::map<std::string, Info> info_;
};

}  // namespace sa3
