// sa3k_host.h - host glue under the train_* headers of this directory: the process-wide sa3k
// context they run on and a small owning device buffer. The headers keep the reference trainer's
// host interface (src/train_optimizer.h, src/train_lora.h, src/train_loop.h, src/train_dit.h) and
// execute its arithmetic through the sa3k C ABI (include/sa3k.h) on the GPU.
#pragma once

#include "sa3k.h"

#include <cstdlib>
#include <string>
#include <vector>

namespace sa3 {

// The context every train_* helper uses: device SA3K_DEVICE (default 0), created on first use and
// kept until the process ends. Returns nullptr (and err) when no GPU or no library is usable; the
// helpers then fail with that message — there is no host fallback.
inline sa3k_ctx* sa3k_default_ctx(std::string& err) {
    static sa3k_ctx* ctx = nullptr;
    static std::string create_err;
    static bool tried = false;
    if (!tried) {
        tried = true;
        const char* dev = std::getenv("SA3K_DEVICE");
        char buf[512] = {0};
        ctx = sa3k_create(dev ? std::atoi(dev) : 0, buf, (int)sizeof buf);
        if (!ctx) create_err = buf[0] ? buf : "sa3k_create failed";
    }
    if (!ctx) err = create_err;
    return ctx;
}

// Record the context's last error into err and return false (for `return sa3k_fail(...)`).
inline bool sa3k_fail(sa3k_ctx* ctx, std::string& err) {
    err = ctx ? sa3k_last_error(ctx) : "no sa3k context";
    return false;
}

// An owning f32 device buffer on a context.
class DeviceF32 {
public:
    DeviceF32() = default;
    DeviceF32(const DeviceF32&) = delete;
    DeviceF32& operator=(const DeviceF32&) = delete;
    DeviceF32(DeviceF32&& o) noexcept : ctx_(o.ctx_), p_(o.p_), n_(o.n_) { o.p_ = nullptr; o.n_ = 0; }
    DeviceF32& operator=(DeviceF32&& o) noexcept {
        if (this != &o) {
            release();
            ctx_ = o.ctx_; p_ = o.p_; n_ = o.n_;
            o.p_ = nullptr; o.n_ = 0;
        }
        return *this;
    }
    ~DeviceF32() { release(); }

    bool alloc(sa3k_ctx* ctx, size_t n, std::string& err) {
        release();
        ctx_ = ctx;
        void* p = nullptr;
        if (sa3k_malloc(ctx, (n ? n : 1) * sizeof(float), &p) != SA3K_OK) return sa3k_fail(ctx, err);
        p_ = static_cast<float*>(p);
        n_ = n;
        return true;
    }
    bool upload(const float* src, size_t n, size_t offset, std::string& err) {
        if (!n) return true;
        if (sa3k_upload(ctx_, p_ + offset, src, n * sizeof(float)) != SA3K_OK) return sa3k_fail(ctx_, err);
        return true;
    }
    bool download(float* dst, size_t n, size_t offset, std::string& err) const {
        if (!n) return true;
        if (sa3k_download(ctx_, dst, p_ + offset, n * sizeof(float)) != SA3K_OK) return sa3k_fail(ctx_, err);
        return true;
    }
    float* get() const { return p_; }
    size_t size() const { return n_; }

private:
    void release() {
        if (p_ && ctx_) sa3k_free(ctx_, p_);
        p_ = nullptr;
        n_ = 0;
    }
    sa3k_ctx* ctx_ = nullptr;
    float* p_ = nullptr;
    size_t n_ = 0;
};

}  // namespace sa3
