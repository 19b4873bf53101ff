// Context, device memory and stream timing for the sa3k C ABI.
#include "sa3k_internal.h"
#include "gemm.h"

#include <algorithm>
#include <cctype>
#include <cstdlib>
#include <cstring>
#include <string>

namespace {
constexpr int kAdamwMaxBlocks = 2048;

void copy_err(char* err, int n, const std::string& m) {
    if (err && n > 0) {
        std::strncpy(err, m.c_str(), (size_t)n - 1);
        err[n - 1] = '\0';
    }
}
}  // namespace

hipEvent_t prof_event(sa3k_ctx* ctx) {
    if (!ctx->prof_pool.empty()) {
        hipEvent_t e = ctx->prof_pool.back();
        ctx->prof_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    SA3K_HIP(hipEventCreate(&e));
    return e;
}

void prof_collect(sa3k_ctx* ctx) {
    if (ctx->prof_pending.empty()) return;
    SA3K_HIP(hipStreamSynchronize(ctx->stream));
    for (const ProfRecord& r : ctx->prof_pending) {
        float ms = 0.0f;
        SA3K_HIP(hipEventElapsedTime(&ms, r.start, r.stop));
        ProfTotal& t = ctx->prof_totals[r.name];
        t.count += 1;
        t.ms += ms;
        t.work += r.work;
        ctx->prof_pool.push_back(r.start);
        ctx->prof_pool.push_back(r.stop);
    }
    ctx->prof_pending.clear();
}

namespace {
// Every tunable of a context, by name: sa3k_set_option / sa3k_get_option / sa3k_option_name.
struct OptionDef {
    const char* name;
    int sa3k_ctx::*field;
    bool flag;   // stored as 0 / 1
};
const OptionDef kOptions[] = {
    {"gemm_split", &sa3k_ctx::gemm_split, true},   {"gemm_fixup", &sa3k_ctx::gemm_fixup, false},
    {"gemm_dma", &sa3k_ctx::gemm_dma, true},       {"gemm_dq", &sa3k_ctx::gemm_dq, false},
    {"gemm_cfg", &sa3k_ctx::gemm_cfg, false},      {"gemm_small", &sa3k_ctx::gemm_small, false},
    {"gemm_nt_store", &sa3k_ctx::gemm_nt_store, true}, {"gemm_skinny", &sa3k_ctx::gemm_skinny, true},
    {"gemm_big", &sa3k_ctx::gemm_big, false},      {"gemm_splits", &sa3k_ctx::gemm_splits, false},
    {"side_stream", &sa3k_ctx::use_side, true},    {"fork_tail", &sa3k_ctx::fork_tail, true},
    {"late_join", &sa3k_ctx::late_join, true},     {"lin_merge", &sa3k_ctx::lin_merge, true},
    {"rank_cols", &sa3k_ctx::rank_cols, false},    {"merge_kn", &sa3k_ctx::merge_kn, true},
    {"tn_fuse", &sa3k_ctx::tn_fuse, false},        {"kv_stack", &sa3k_ctx::kv_stack, true},
    {"attn_fwd32", &sa3k_ctx::attn_fwd32, false},  {"head_f32", &sa3k_ctx::head_f32, true},
    {"prep_side", &sa3k_ctx::prep_side, true},     {"epi_fuse", &sa3k_ctx::epi_fuse, false},
    {"act_bf16", &sa3k_ctx::act_bf16, false},     {"gemm_prio", &sa3k_ctx::gemm_prio, true},
    {"head_quick", &sa3k_ctx::head_quick, true},
};
constexpr int kNumOptions = (int)(sizeof(kOptions) / sizeof(kOptions[0]));

// SA3K_<NAME> in the environment overrides option <name> at context creation (A/B measurements)
void options_from_env(sa3k_ctx* ctx) {
    for (const OptionDef& o : kOptions) {
        std::string env = "SA3K_";
        for (const char* p = o.name; *p; ++p) env += (char)std::toupper((unsigned char)*p);
        if (const char* e = std::getenv(env.c_str())) ctx->*o.field = o.flag ? (std::atoi(e) != 0) : std::atoi(e);
    }
}

const OptionDef& find_option(const char* name) {
    SA3K_REQUIRE(name != nullptr, "null option name");
    for (const OptionDef& o : kOptions)
        if (std::strcmp(o.name, name) == 0) return o;
    sa3k_throw(SA3K_ERR_INVALID, std::string("unknown option ") + name);
    return kOptions[0];   // not reached
}
}  // namespace

namespace {
// dst += src element by element in f32 (the reference's train_accum_add, src/train_loop.h:75-78)
__global__ __launch_bounds__(256) void vec_add_kernel(float* __restrict__ dst, const float* __restrict__ src,
                                                      int64_t n) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i + 4 <= n) {
        float4 a = *reinterpret_cast<const float4*>(dst + i);
        const float4 b = *reinterpret_cast<const float4*>(src + i);
        a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
        *reinterpret_cast<float4*>(dst + i) = a;
    } else {
        for (int64_t k = i; k < n; ++k) dst[k] += src[k];
    }
}

void vec_add(sa3k_ctx* ctx, float* dst, const float* src, int64_t n) {
    const bool al = ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15u) == 0;
    SA3K_REQUIRE(al, "sa3k_vec_add needs 16-byte aligned buffers");
    vec_add_kernel<<<(unsigned)ceil_div(ceil_div(n, 4), 256), 256, 0, ctx->stream>>>(dst, src, n);
    SA3K_LAUNCHED();
}
}  // namespace

extern "C" {

SA3K_API const char* sa3k_version(void) { return "sa3k 0.1 gfx950"; }

SA3K_API sa3k_ctx* sa3k_create(int device, char* err, int err_len) {
    sa3k_ctx* ctx = new (std::nothrow) sa3k_ctx();
    if (!ctx) {
        copy_err(err, err_len, "sa3k_create: out of host memory");
        return nullptr;
    }
    int rc = sa3k_guard(ctx, "sa3k_create", [&] {
        int n = 0;
        SA3K_HIP(hipGetDeviceCount(&n));
        SA3K_REQUIRE(device >= 0 && device < n, "device ordinal out of range");
        ctx->device = device;
        SA3K_HIP(hipSetDevice(device));
        hipDeviceProp_t prop;
        SA3K_HIP(hipGetDeviceProperties(&prop, device));
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            sa3k_throw(SA3K_ERR_UNSUPPORTED,
                       std::string("kernels are built for gfx950, device is ") + prop.gcnArchName);
        // Default-priority stream (non-blocking w.r.t. the null stream).
        SA3K_HIP(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
        ctx->main_stream = ctx->stream;
        SA3K_HIP(hipStreamCreateWithFlags(&ctx->side_stream, hipStreamNonBlocking));
        SA3K_HIP(hipStreamCreateWithFlags(&ctx->quick_stream, hipStreamNonBlocking));
        for (hipEvent_t& e : ctx->side_ev) SA3K_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        SA3K_HIP(hipEventCreateWithFlags(&ctx->block_tail_ev, hipEventDisableTiming));
        options_from_env(ctx);
        SA3K_HIP(hipEventCreate(&ctx->ev_start));
        SA3K_HIP(hipEventCreate(&ctx->ev_stop));
        if (const char* e = std::getenv("SA3K_GEMM_PD")) ctx->gemm_pd = std::atoi(e) == 2 ? 2 : 1;
        if (const char* e = std::getenv("SA3K_GEMM_WGPCU")) ctx->gemm_wg_per_cu = std::max(1, std::atoi(e));
        SA3K_HIP(hipMalloc(&ctx->zero_page, 256));
        SA3K_HIP(hipMemsetAsync(ctx->zero_page, 0, 256, ctx->stream));
        sa3k_note_main(ctx);
        for (int** c : {&ctx->tile_counters, &ctx->tile_counters_side}) {
            SA3K_HIP(hipMalloc(c, sizeof(int) * kMaxFixupTiles));
            SA3K_HIP(hipMemsetAsync(*c, 0, sizeof(int) * kMaxFixupTiles, ctx->stream));
            sa3k_note_main(ctx);
        }
        SA3K_HIP(hipMalloc(&ctx->skinny_counters, sizeof(int) * 2 * kSkinnyMaxTiles));
        SA3K_HIP(hipMemsetAsync(ctx->skinny_counters, 0, sizeof(int) * 2 * kSkinnyMaxTiles, ctx->stream));
        sa3k_note_main(ctx);
        SA3K_HIP(hipMalloc(&ctx->adamw_partials, sizeof(double) * kAdamwMaxBlocks));
        SA3K_HIP(hipMalloc(&ctx->adamw_result, sizeof(double) * 2));
        SA3K_HIP(hipMemsetAsync(ctx->adamw_result, 0, sizeof(double) * 2, ctx->stream));
        sa3k_note_main(ctx);
        // this device's address of the allocation-free GEMM's scratch array
        sa3k::gemm_noalloc_setup(ctx);
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
    });
    if (rc != SA3K_OK) {
        copy_err(err, err_len, ctx->last_error);
        sa3k_destroy(ctx);
        return nullptr;
    }
    return ctx;
}

SA3K_API void sa3k_destroy(sa3k_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->main_stream) (void)hipStreamSynchronize(ctx->main_stream);
    if (ctx->side_stream) (void)hipStreamSynchronize(ctx->side_stream);
    if (ctx->quick_stream) (void)hipStreamSynchronize(ctx->quick_stream);
    if (ctx->adamw_partials) (void)hipFree(ctx->adamw_partials);
    if (ctx->adamw_result) (void)hipFree(ctx->adamw_result);
    if (ctx->gemm_ws) (void)hipFree(ctx->gemm_ws);
    if (ctx->red_ws) (void)hipFree(ctx->red_ws);
    if (ctx->gemm_ws_side) (void)hipFree(ctx->gemm_ws_side);
    if (ctx->red_ws_side) (void)hipFree(ctx->red_ws_side);
    if (ctx->gemm_ws_quick) (void)hipFree(ctx->gemm_ws_quick);
    if (ctx->red_ws_quick) (void)hipFree(ctx->red_ws_quick);
    for (hipEvent_t e : ctx->side_ev)
        if (e) (void)hipEventDestroy(e);
    if (ctx->block_tail_ev) (void)hipEventDestroy(ctx->block_tail_ev);
    if (ctx->zero_page) (void)hipFree(ctx->zero_page);
    if (ctx->tile_counters) (void)hipFree(ctx->tile_counters);
    if (ctx->tile_counters_side) (void)hipFree(ctx->tile_counters_side);
    if (ctx->skinny_counters) (void)hipFree(ctx->skinny_counters);
    for (const ProfRecord& r : ctx->prof_pending) {
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    for (hipEvent_t e : ctx->prof_pool) (void)hipEventDestroy(e);
    if (ctx->ev_start) (void)hipEventDestroy(ctx->ev_start);
    if (ctx->ev_stop) (void)hipEventDestroy(ctx->ev_stop);
    if (ctx->side_stream) (void)hipStreamDestroy(ctx->side_stream);
    if (ctx->quick_stream) (void)hipStreamDestroy(ctx->quick_stream);
    if (ctx->main_stream) (void)hipStreamDestroy(ctx->main_stream);
    delete ctx;
}

SA3K_API const char* sa3k_last_error(const sa3k_ctx* ctx) {
    return ctx ? ctx->last_error.c_str() : "null context";
}

SA3K_API int sa3k_malloc(sa3k_ctx* ctx, size_t bytes, void** out) {
    return sa3k_guard(ctx, "sa3k_malloc", [&] {
        SA3K_REQUIRE(out != nullptr, "out is null");
        *out = nullptr;
        SA3K_HIP(hipSetDevice(ctx->device));
        SA3K_HIP(hipMalloc(out, bytes ? bytes : 1));
    });
}

SA3K_API int sa3k_free(sa3k_ctx* ctx, void* ptr) {
    return sa3k_guard(ctx, "sa3k_free", [&] {
        if (!ptr) return;
        SA3K_HIP(hipSetDevice(ctx->device));
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
        SA3K_HIP(hipFree(ptr));
    });
}

SA3K_API int sa3k_upload(sa3k_ctx* ctx, void* dst, const void* src, size_t bytes) {
    return sa3k_guard(ctx, "sa3k_upload", [&] {
        if (!bytes) return;
        SA3K_REQUIRE(dst && src, "null pointer");
        SA3K_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
        sa3k_note_main(ctx);
        // pageable source: the runtime stages it, but keep the contract simple for callers that
        // reuse the host buffer right away
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
    });
}

SA3K_API int sa3k_download(sa3k_ctx* ctx, void* dst, const void* src, size_t bytes) {
    return sa3k_guard(ctx, "sa3k_download", [&] {
        if (!bytes) return;
        SA3K_REQUIRE(dst && src, "null pointer");
        SA3K_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
        sa3k_note_main(ctx);
        SA3K_HIP(hipStreamSynchronize(ctx->stream));
    });
}

SA3K_API int sa3k_copy_d2d(sa3k_ctx* ctx, void* dst, const void* src, size_t bytes) {
    return sa3k_guard(ctx, "sa3k_copy_d2d", [&] {
        if (!bytes) return;
        SA3K_REQUIRE(dst && src, "null pointer");
        SA3K_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
        sa3k_note_main(ctx);
    });
}

SA3K_API int sa3k_memset(sa3k_ctx* ctx, void* dst, int value, size_t bytes) {
    return sa3k_guard(ctx, "sa3k_memset", [&] {
        if (!bytes) return;
        SA3K_REQUIRE(dst, "null pointer");
        SA3K_HIP(hipMemsetAsync(dst, value, bytes, ctx->stream));
        sa3k_note_main(ctx);
    });
}

SA3K_API int sa3k_device_memory(sa3k_ctx* ctx, size_t* free_bytes, size_t* total_bytes) {
    return sa3k_guard(ctx, "sa3k_device_memory", [&] {
        SA3K_REQUIRE(free_bytes && total_bytes, "null pointer");
        SA3K_HIP(hipMemGetInfo(free_bytes, total_bytes));
    });
}

SA3K_API int sa3k_vec_add(sa3k_ctx* ctx, float* dst, const float* src, int64_t n) {
    return sa3k_guard(ctx, "sa3k_vec_add", [&] {
        SA3K_REQUIRE(n >= 0 && (n == 0 || (dst && src)), "null pointer or negative length");
        if (!n) return;
        vec_add(ctx, dst, src, n);
    });
}

SA3K_API int sa3k_sync(sa3k_ctx* ctx) {
    return sa3k_guard(ctx, "sa3k_sync", [&] {
        SA3K_HIP(hipStreamSynchronize(ctx->side_stream));
        SA3K_HIP(hipStreamSynchronize(ctx->quick_stream));
        SA3K_HIP(hipStreamSynchronize(ctx->main_stream));
    });
}


SA3K_API int sa3k_set_option(sa3k_ctx* ctx, const char* name, int value) {
    return sa3k_guard(ctx, "sa3k_set_option", [&] {
        const OptionDef& o = find_option(name);
        int v = o.flag ? (value != 0) : value;
        if (o.field == &sa3k_ctx::gemm_splits) v = std::max(0, v);
        ctx->*o.field = v;
    });
}

SA3K_API int sa3k_get_option(sa3k_ctx* ctx, const char* name, int* value) {
    return sa3k_guard(ctx, "sa3k_get_option", [&] {
        SA3K_REQUIRE(value != nullptr, "value is null");
        *value = ctx->*find_option(name).field;
    });
}

SA3K_API const char* sa3k_option_name(int index) {
    return index >= 0 && index < kNumOptions ? kOptions[index].name : nullptr;
}

SA3K_API int sa3k_timer_start(sa3k_ctx* ctx) {
    return sa3k_guard(ctx, "sa3k_timer_start",
                      [&] { SA3K_HIP(hipEventRecord(ctx->ev_start, ctx->stream)); });
}

SA3K_API int sa3k_timer_stop(sa3k_ctx* ctx, float* ms) {
    return sa3k_guard(ctx, "sa3k_timer_stop", [&] {
        SA3K_REQUIRE(ms != nullptr, "ms is null");
        SA3K_HIP(hipEventRecord(ctx->ev_stop, ctx->stream));
        SA3K_HIP(hipEventSynchronize(ctx->ev_stop));
        SA3K_HIP(hipEventElapsedTime(ms, ctx->ev_start, ctx->ev_stop));
    });
}

SA3K_API int sa3k_profile_enable(sa3k_ctx* ctx, int on) {
    return sa3k_guard(ctx, "sa3k_profile_enable", [&] {
        prof_collect(ctx);
        ctx->prof_on = on != 0;
    });
}

SA3K_API int sa3k_profile_reset(sa3k_ctx* ctx) {
    return sa3k_guard(ctx, "sa3k_profile_reset", [&] {
        prof_collect(ctx);
        ctx->prof_totals.clear();
    });
}

SA3K_API int sa3k_profile_report(sa3k_ctx* ctx, char* buf, int buf_len) {
    return sa3k_guard(ctx, "sa3k_profile_report", [&] {
        SA3K_REQUIRE(buf && buf_len > 0, "null buffer");
        prof_collect(ctx);
        std::string out;
        char line[256];
        for (const auto& kv : ctx->prof_totals) {
            std::snprintf(line, sizeof line, "%s %lld %.6f %.6e\n", kv.first.c_str(),
                          (long long)kv.second.count, kv.second.ms, kv.second.work);
            out += line;
        }
        SA3K_REQUIRE((int)out.size() < buf_len, "report buffer too small");
        std::memcpy(buf, out.c_str(), out.size() + 1);
    });
}

}  // extern "C"
