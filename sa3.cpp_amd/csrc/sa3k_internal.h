// Internal helpers shared by the sa3k translation units: the context object, error plumbing and
// small device utilities. Not part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <map>
#include <string>
#include <vector>

#include "sa3k.h"

// Per-kernel event timing (off by default): every launch site wraps its launch in a KernelScope,
// which records a start/stop event pair on the context stream while profiling is on.
struct ProfRecord {
    const char* name;
    hipEvent_t start, stop;
    double work;   // algorithmic flops (or bytes) of the launch, 0 when not counted
};
struct ProfTotal {
    int64_t count = 0;
    double ms = 0.0;
    double work = 0.0;
};

constexpr int kSideEvents = 64;
// row tiles (32 rows each) of one skinny-product launch that may split K over workgroups
constexpr int kSkinnyMaxTiles = 8192;

// option tn_fuse: which split reductions their own last split to arrive sums (instead of a
// separate launch): the block's modulation-gradient column sums, the adapted linears' dA sums, and
// the adapted linears' dU column reduction together with its per-row step
constexpr int kFuseColred = 1, kFuseXSum = 2, kFuseRows = 4;

struct sa3k_ctx {
    int device = 0;
    // The stream launches go to: the context's main stream, or, while side work is being enqueued
    // (OnSide below), its second stream. Both have the default priority.
    hipStream_t stream = nullptr;
    hipStream_t main_stream = nullptr;
    hipStream_t side_stream = nullptr;
    hipStream_t quick_stream = nullptr;    // third stream: short branches the main stream joins right away
    hipEvent_t side_ev[kSideEvents] = {};   // fork/join events, reused round-robin
    int side_ev_i = 0;
    int use_side = 1;                      // run independent chains on the second stream
    int side_held = 0;                     // > 0: the second stream is taken by a caller's own chain
    int side_defer = 0;                    // >0: a caller joins the second stream (callees need not)
    int fork_tail = 1;                     // forks recorded by the producer kernel's completion (fork_arm)
    int late_join = 1;                     // a DiT block's last second-stream work may overlap the next block
    int lin_merge = 1;                     // bf16 adapted linears contract W + s B A, refreshed per prepare
    int rank_cols = 1;                     // merged: s X A^T (1) / s dU B (2) as extra GEMM output columns
    int merge_kn = 1;                      // merged: dX reads W_eff [out][in] as a [K][N] operand (no W_eff^T copy)
    hipEvent_t block_tail_ev = nullptr;    // second-stream work of a block backward left running (late_join)
    bool block_tail_pending = false;       // block_tail_ev holds a record not yet waited for
    hipEvent_t tail_ev = nullptr;          // fork event armed for the producer about to launch (fork_arm)
    uint64_t tail_seq = 0;                 // main_seq right after the launch that last recorded tail_ev
    uint64_t main_seq = 0;                 // operations enqueued on the main stream (note_main)
    uint64_t side_synced = ~(uint64_t)0;   // main_seq up to which the second stream already waits
    uint64_t side_forks = 0;               // forks so far (each precedes work enqueued on the second stream)
    std::string last_error;
    hipEvent_t ev_start = nullptr, ev_stop = nullptr;
    bool prof_on = false;
    std::vector<ProfRecord> prof_pending;
    std::vector<hipEvent_t> prof_pool;
    std::map<std::string, ProfTotal> prof_totals;
    // AdamW: per-block partial sums of squares and the {norm, scale} pair of the last update.
    double* adamw_partials = nullptr;     // [kAdamwMaxBlocks]
    double* adamw_result = nullptr;       // [0] = norm, [1] = scale (as double)
    void* gemm_ws = nullptr;              // split-K partial sums (grown on demand)
    size_t gemm_ws_bytes = 0;
    int gemm_pd = 1;                      // GEMM global-load prefetch depth (1 or 2 K tiles)
    int gemm_split = 1;                   // allow split-K
    int gemm_dma = 1;                     // use the DMA-fed kernel for compute-type operands
    int gemm_dq = 1;                      // bf16 products with an f16 / Q8_0 B on the DMA-fed kernel (decoded from LDS)
    int gemm_cfg = 0;                     // DMA kernel tile configuration
    int gemm_nt_store = 1;                // GEMM outputs written with non-temporal stores
    int gemm_skinny = 1;                  // products with <= 32 output columns on the skinny kernel
    int gemm_big = 3;                     // 256 x 256 bf16 tiles: 0 never, 1 where they fill the chip, 2 always,
                                          // 3 as 1 plus every product with K >= 8192 (split over K)
    int gemm_splits = 0;                  // > 0: split-K count of DMA GEMMs that split (for measurement)
    int gemm_small = 4;                   // tile configuration for small grids (0: the default tile + split-K)
    int gemm_prio = 1;                    // DMA GEMMs: wave priority 1 over the MFMA clusters of the K loop
    int gemm_wg_per_cu = 0;               // resident workgroups per CU assumed by the split choice (0: from LDS use)
    void* red_ws = nullptr;              // column-reduction partial sums (grows on demand)
    size_t red_ws_bytes = 0;
    void* gemm_ws_side = nullptr;        // the same two workspaces for work on the second stream
    size_t gemm_ws_side_bytes = 0;
    void* red_ws_side = nullptr;
    size_t red_ws_side_bytes = 0;
    void* gemm_ws_quick = nullptr;       // and on the third stream
    size_t gemm_ws_quick_bytes = 0;
    void* red_ws_quick = nullptr;
    size_t red_ws_quick_bytes = 0;
    int gemm_fixup = 0;                   // split partials summed by the last split (no reduce launch):
                                          // 0 never, 1 always, 2 for small outputs only
    int* tile_counters = nullptr;         // [kMaxFixupTiles] arrival counters, zero between launches
    int* tile_counters_side = nullptr;    // the same for launches on the second stream
    int tn_fuse = kFuseColred | kFuseRows; // split reductions summed in-kernel (bits kFuse*)
    int kv_stack = 1;                     // a DiT's context K/V projections as one stacked product
    int attn_fwd32 = 1;                   // attention forward on 32x32x16 MFMA blocks, 32 queries per wave
    int prep_side = 1;                    // a DiT's bf16 group refresh on the second stream beside the f32 heads'
    int head_f32 = 1;                     // a DiT's head / tail linears on f32 MFMA (f32 / f16 bases)
    int head_quick = 1;                   // a DiT's head chains partly on the third stream
    int epi_fuse = 3;                     // in GEMM epilogues where the tiles allow: 1 the FFN SwiGLU, 2 q/k head prep,
                                          // 4 the attention backward's dOh and row dots, 8 the SwiGLU backward
    int act_bf16 = 1;                     // block backward reads bf16 copies: 1 of the FFN up output, 2 of qkv / qf
    int* skinny_counters = nullptr;       // [2][kSkinnyMaxTiles] the skinny product's split arrivals,
                                          // one half per stream, zero between launches
    bool capturing = false;               // a HIP graph capture is recording the stream
    void* zero_page = nullptr;            // 256 zero bytes
    // This device's address of the file-scope scratch array of the allocation-free GEMM entry
    // point (gemm.hip), looked up once per device when the context is created.
    float* noalloc_scratch = nullptr;
    // While set, the split-K partials of GEMMs on this context go to this fixed buffer of
    // ws_fixed_bytes instead of the growing workspace (a launch that needs more fails).
    float* ws_fixed = nullptr;
    size_t ws_fixed_bytes = 0;
};

// An error that carries an sa3k status code across the internal call chain; every C entry point
// converts it into a return code + ctx->last_error.
struct Sa3kError : std::runtime_error {
    int code;
    Sa3kError(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

inline void sa3k_throw(int code, const std::string& msg) { throw Sa3kError(code, msg); }

#define SA3K_HIP(call)                                                                            \
    do {                                                                                          \
        hipError_t e_ = (call);                                                                   \
        if (e_ != hipSuccess)                                                                     \
            sa3k_throw(e_ == hipErrorOutOfMemory ? SA3K_ERR_NOMEM : SA3K_ERR_DEVICE,              \
                       std::string(#call) + ": " + hipGetErrorString(e_));                        \
    } while (0)

#define SA3K_REQUIRE(cond, msg)                                                                   \
    do {                                                                                          \
        if (!(cond)) sa3k_throw(SA3K_ERR_INVALID, (msg));                                         \
    } while (0)

// Wrap an entry point body: returns SA3K_OK or the code of the first failure, recording the message.
template <class F>
inline int sa3k_guard(sa3k_ctx* ctx, const char* fn, F&& body) {
    if (!ctx) return SA3K_ERR_INVALID;
    try {
        body();
        return SA3K_OK;
    } catch (const Sa3kError& e) {
        ctx->last_error = std::string(fn) + ": " + e.what();
        return e.code;
    } catch (const std::exception& e) {
        ctx->last_error = std::string(fn) + ": " + e.what();
        return SA3K_ERR_DEVICE;
    } catch (...) {
        ctx->last_error = std::string(fn) + ": unknown failure";
        return SA3K_ERR_DEVICE;
    }
}

// Launch-error check after a kernel launch on the context stream.
// after every kernel launch (and, as note_main, after every async copy or fill): checks the launch
// and counts work enqueued on the main stream, so a fork can tell whether the second stream already
// waits for all of it
#define SA3K_LAUNCHED()                   \
    do {                                  \
        SA3K_HIP(hipGetLastError());      \
        sa3k_note_main(ctx);              \
    } while (0)

hipEvent_t prof_event(sa3k_ctx* ctx);
void prof_collect(sa3k_ctx* ctx);

class KernelScope {
public:
    KernelScope(sa3k_ctx* ctx, const char* name, double work = 0.0) : ctx_(ctx) {
        if (!ctx_->prof_on) return;
        rec_.name = name;
        rec_.work = work;
        rec_.start = prof_event(ctx_);
        rec_.stop = prof_event(ctx_);
        (void)hipEventRecord(rec_.start, ctx_->stream);
    }
    ~KernelScope() {
        if (!ctx_->prof_on) return;
        (void)hipEventRecord(rec_.stop, ctx_->stream);
        ctx_->prof_pending.push_back(rec_);
        if (ctx_->prof_pending.size() >= 4096) prof_collect(ctx_);
    }
private:
    sa3k_ctx* ctx_;
    ProfRecord rec_{};
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline void sa3k_note_main(sa3k_ctx* c) {
    if (c->stream == c->main_stream) ++c->main_seq;
}

// ---- a second stream for independent chains of work (e.g. a column reduction beside the GEMM
// that does not need it). Used only while launches go to the main stream and outside profiling
// (per-kernel timing stays serial). Every function that forks joins before it returns, so no side
// work outlives a call.
inline bool side_usable(const sa3k_ctx* c) {
    return c->use_side && !c->side_held && c->side_stream && !c->prof_on && c->stream == c->main_stream;
}
inline hipEvent_t side_event(sa3k_ctx* c) {
    hipEvent_t e = c->side_ev[c->side_ev_i];
    c->side_ev_i = (c->side_ev_i + 1) % kSideEvents;
    return e;
}
// the second stream waits for everything enqueued on the main stream so far (nothing to do when
// nothing was enqueued there since the last fork)
inline void fork_fire(sa3k_ctx* c);
inline void side_fork(sa3k_ctx* c) {
    if (c->tail_ev) return fork_fire(c);   // armed before the producer
    ++c->side_forks;
    if (c->side_synced == c->main_seq) return;
    hipEvent_t e = side_event(c);
    SA3K_HIP(hipEventRecord(e, c->main_stream));
    SA3K_HIP(hipStreamWaitEvent(c->side_stream, e, 0));
    c->side_synced = c->main_seq;
}
// Fork after a producer without a separate event record (a marker packet on the main stream that
// costs ~4.6 us; a kernel's own completion event costs ~0.9 us): fork_arm, then the producer's
// launches through launch_k (the last of them passes last = true and records the armed event at
// its completion), then fork_fire (or side_fork) makes the second stream wait on it. The event is
// used only if the recording launch is the last operation enqueued on the main stream (main_seq);
// otherwise fork_fire records it itself, so a producer that records nothing, or anything enqueued
// after the recording launch, still forks correctly.
template <class T>
struct ident {
    using type = T;
};
template <class... KArgs>
inline void launch_k(sa3k_ctx* c, bool last, void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t shmem,
                     typename ident<KArgs>::type... args) {
    if (last && c->tail_ev && c->stream == c->main_stream) {
        hipExtLaunchKernelGGL(kernel, grid, block, shmem, c->stream, nullptr, c->tail_ev, 0, args...);
        c->tail_seq = c->main_seq + 1;   // main_seq once the caller's SA3K_LAUNCHED() has counted it
    } else {
        kernel<<<grid, block, shmem, c->stream>>>(args...);
    }
}
// Under a graph capture the fork records its own event: the completion event of a launch through
// hipExtLaunchKernelGGL is not part of the capture, and a captured stream may not wait on it.
inline void fork_arm(sa3k_ctx* c) {
    if (!c->fork_tail || c->capturing) return;
    c->tail_ev = side_event(c);
    c->tail_seq = ~(uint64_t)0;
}
inline void fork_fire(sa3k_ctx* c) {
    if (!c->tail_ev) return side_fork(c);   // not armed (fork_tail off)
    ++c->side_forks;
    hipEvent_t e = c->tail_ev;
    c->tail_ev = nullptr;
    if (c->tail_seq != c->main_seq) SA3K_HIP(hipEventRecord(e, c->main_stream));
    SA3K_HIP(hipStreamWaitEvent(c->side_stream, e, 0));
    c->side_synced = c->main_seq;
}
// the main stream waits for everything enqueued on the second stream so far
inline void side_join(sa3k_ctx* c) {
    hipEvent_t e = side_event(c);
    SA3K_HIP(hipEventRecord(e, c->side_stream));
    SA3K_HIP(hipStreamWaitEvent(c->main_stream, e, 0));
}
// ---- a third stream for short branches that the main stream joins right away (attention dQ beside
// dK/dV): joining the second stream instead would also wait for every longer chain queued there
// first (streams run their work in order)
inline void quick_fork(sa3k_ctx* c) {
    hipEvent_t e;
    if (c->tail_ev) {   // armed before the producer: its completion event, unless more work followed
        e = c->tail_ev;
        c->tail_ev = nullptr;
        if (c->tail_seq != c->main_seq) SA3K_HIP(hipEventRecord(e, c->main_stream));
    } else {
        e = side_event(c);
        SA3K_HIP(hipEventRecord(e, c->main_stream));
    }
    SA3K_HIP(hipStreamWaitEvent(c->quick_stream, e, 0));
}
inline void quick_join(sa3k_ctx* c) {
    hipEvent_t e = side_event(c);
    SA3K_HIP(hipEventRecord(e, c->quick_stream));
    SA3K_HIP(hipStreamWaitEvent(c->main_stream, e, 0));
}
// the main stream waits for the second stream if anything was forked since side_forks was `mark`
inline void side_join_since(sa3k_ctx* c, uint64_t mark) {
    if (c->side_forks != mark) side_join(c);
}
// A caller that joins the second stream itself at its end (see SideDeferScope) lets the functions
// it calls leave their side work running; otherwise every forking function joins before returning.
inline void side_join_unless_deferred(sa3k_ctx* c) {
    if (c->side_defer == 0) side_join(c);
}
struct SideDeferScope {
    sa3k_ctx* c;
    explicit SideDeferScope(sa3k_ctx* ctx) : c(ctx) { ++c->side_defer; }
    ~SideDeferScope() { --c->side_defer; }
    SideDeferScope(const SideDeferScope&) = delete;
    SideDeferScope& operator=(const SideDeferScope&) = delete;
};
// launches inside the scope go to the third stream (when `on`)
struct OnQuick {
    sa3k_ctx* c;
    bool on;
    OnQuick(sa3k_ctx* ctx, bool enable) : c(ctx), on(enable) {
        if (on) c->stream = c->quick_stream;
    }
    ~OnQuick() {
        if (on) c->stream = c->main_stream;
    }
    OnQuick(const OnQuick&) = delete;
    OnQuick& operator=(const OnQuick&) = delete;
};
// while held, functions on the main stream fork nothing (a caller runs its own chain on the second
// stream beside them)
struct SideHeld {
    sa3k_ctx* c;
    bool on;
    SideHeld(sa3k_ctx* ctx, bool enable) : c(ctx), on(enable) {
        if (on) ++c->side_held;
    }
    ~SideHeld() {
        if (on) --c->side_held;
    }
    SideHeld(const SideHeld&) = delete;
    SideHeld& operator=(const SideHeld&) = delete;
};
// launches inside the scope go to the second stream (when `on`)
struct OnSide {
    sa3k_ctx* c;
    bool on;
    OnSide(sa3k_ctx* ctx, bool enable) : c(ctx), on(enable) {
        if (on) c->stream = c->side_stream;
    }
    ~OnSide() {
        if (on) c->stream = c->main_stream;
    }
    OnSide(const OnSide&) = delete;
    OnSide& operator=(const OnSide&) = delete;
};

// capacity of sa3k_ctx::tile_counters (tiles of one split-K / split-reduction launch)
constexpr int kMaxFixupTiles = 8192;
// Outputs of at most this many floats are reduced in-kernel under gemm_fixup = 2. (Measured on
// MI355X, even these small in-kernel reductions cost more than the separate launch: the coherent
// partial loads of the last workgroup serialize; 2 stays selectable, 0 is the default.)
constexpr int64_t kSmallFixupElems = (int64_t)1 << 18;

// The arrival counters of in-kernel split reductions launched on the current stream: one array
// per stream, so reductions on the two streams never share a counter (launches on one stream run
// one after another, and the last arrival resets each counter). Null on any other stream.
inline int* stream_counters(const sa3k_ctx* c) {
    if (c->stream == c->main_stream) return c->tile_counters;
    if (c->stream == c->side_stream) return c->tile_counters_side;
    return nullptr;
}
// whether a split reduction over an output of `elems` floats is done by the last split to arrive
inline bool use_fixup(const sa3k_ctx* ctx, int64_t elems, int64_t tiles) {
    if (tiles > kMaxFixupTiles || !stream_counters(ctx)) return false;
    return ctx->gemm_fixup == 1 || (ctx->gemm_fixup == 2 && elems <= kSmallFixupElems);
}
// the counters of a reduction of kind `bit` over `tiles` column tiles summed by its last split to
// arrive, or null: a separate launch sums the partials
inline int* tn_counters(const sa3k_ctx* ctx, int64_t tiles, int bit) {
    if (!(ctx->tn_fuse & bit) || tiles > kMaxFixupTiles) return nullptr;
    return stream_counters(ctx);
}

// The FFN SwiGLU's gate sigmoid(z) = 1 / (1 + e^-z) on the hardware exp2 and reciprocal (within a
// few ulp of the correctly rounded value). The up-projection's GEMM epilogue and the separate
// SwiGLU kernel both use it, so the two paths give the same bits.
__device__ __forceinline__ float swiglu_sigmoid(float z) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.44269504088896341f * z));
}

// Split partial sums handed from one workgroup to another inside a launch ("the last split to
// arrive reduces"): device-coherent (sc1) accesses, so no cache level can hold a stale copy and no
// L2-wide write-back fence is needed. The writer waits for its coherent stores to complete before
// the workgroup barrier that precedes its arrival on the tile counter. On MI355X these uncached
// accesses cost more than the separate reduction launch they replace (a device-scope release
// fence instead writes back a whole L2 per workgroup, costlier still), so the option is off by
// default; it stays selectable and is tested bit-identical to the separate launch.
__device__ __forceinline__ void st_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores_done() { __builtin_amdgcn_s_waitcnt(0x0F70); }   // vmcnt(0)
// The split sums of NE elements of coherent partials: acc[i] = sum over z < S of the float at byte
// offset off[i] + z * zstride of rs, added in z order from zero (the same sums as a sequential
// loop over z), with device-coherent (sc1) buffer loads issued 8 splits x NE elements at a time so
// the reading workgroup waits about ceil(S / 8) memory round trips, not S x NE. The caller gives every
// element it stores a valid offset; the sums of the others are not used.
constexpr int kSc1 = 16;   // buffer intrinsic cache policy: sc1 (device scope)
template <int NE>
__device__ __forceinline__ void coherent_split_sums(__amdgpu_buffer_rsrc_t rs, const uint32_t (&off)[NE],
                                                    uint32_t zstride, int S, float (&acc)[NE]) {
#pragma unroll
    for (int i = 0; i < NE; ++i) acc[i] = 0.f;
    int z = 0;
    for (; z + 8 <= S; z += 8) {
        float v[NE][8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
#pragma unroll
            for (int i = 0; i < NE; ++i)
                v[i][k] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(rs, off[i] + (uint32_t)(z + k) * zstride, 0, kSc1));
#pragma unroll
        for (int i = 0; i < NE; ++i)
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[i] += v[i][k];
    }
    if (z < S) {   // the last S % 8 splits: also in one batch (a loop over them waited once per split)
        const int n = S - z;
        float v[NE][8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (k < n)
#pragma unroll
                for (int i = 0; i < NE; ++i)
                    v[i][k] = __builtin_bit_cast(
                        float, __builtin_amdgcn_raw_buffer_load_b32(rs, off[i] + (uint32_t)(z + k) * zstride, 0, kSc1));
#pragma unroll
        for (int i = 0; i < NE; ++i)
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (k < n) acc[i] += v[i][k];
    }
}
// arrival of this workgroup on counter c of `expected` arrivals; true for the last one, which
// also resets the counter. Every thread must call it (it contains workgroup barriers).
__device__ __forceinline__ bool arrive_last(int* c, int expected, int* s_flag) {
    wait_stores_done();
    __syncthreads();
    if (threadIdx.x == 0) {
        const int prev = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *s_flag = prev == expected - 1;
        if (*s_flag) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return *s_flag != 0;
}
