// K1/K2 GEMM kernels and their host dispatch. See gemm.h for the contract.
#include "gemm.h"

#include <algorithm>
#include <mutex>

namespace sa3k {
namespace {

constexpr int kThreads = 256;
constexpr int kRowBytes = 144;   // 128 bytes of compute-type data + 16 bytes pad per LDS row

typedef _Float16 f16x8 __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef _Float16 f16x4 __attribute__((__vector_size__(4 * sizeof(_Float16))));

struct KParams {
    const void* A; int64_t lda;
    const void* B; int64_t ldb;
    const void* Bs; int64_t ldbs;
    const void* A2; int64_t lda2;
    const void* B2; int64_t ldb2;
    int K2;
    int64_t M, N, K;
    float alpha;
    const float* colscale;
    const float* bias;
    float* C; int64_t ldc; int accumulate;
    bf16* Cb; int64_t ldcb;
    float* U; bf16* Ub; int64_t ldu;
    int64_t Mx;
    const void* Ax; int64_t ldax;
    const void* A2x; int64_t lda2x;
    float* Cx; int64_t ldcx; int accumulate_x;
    bf16* Cbx;
    float* ws;   // split-K partials [splits][M+Mx][N] (null: no split)
    int kps;     // K tiles per split
    int prescale;
};

}  // namespace

// Scratch of sa3k_gemm_nt_noalloc: the split-K partial sums of one GEMM, in device memory that
// the code object itself carries (no hipMalloc at any call). 64 MiB covers every split plan the
// dispatch chooses by itself: a GEMM splits only while its tiles fill fewer than the chip's
// resident slots (512 for 128 x 128 tiles, 256 for 128 x 256 and 256 x 256 ones), so splits x
// tiles x tile floats <= 256 x 65536 = 2^24 (kMaxSplitFloats; the launchers check both factors).
// Every GPU that loads the library holds its own copy until the process ends.
constexpr size_t kNoAllocScratchFloats = (size_t)1 << 24;
static_assert((int64_t)kNoAllocScratchFloats >= kMaxSplitFloats, "the scratch must hold every automatic split plan");
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_dev[kMaxDevices] = {};   // per device: its copy of `scratch`
}  // namespace

void gemm_noalloc_setup(sa3k_ctx* ctx) {
    SA3K_REQUIRE(ctx->device >= 0 && ctx->device < kMaxDevices, "device ordinal beyond the scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    float*& ptr = g_scratch_dev[ctx->device];
    if (!ptr) {
        // the host-side name of the array is only a stand-in: the device address comes from the
        // runtime, with this device current (sa3k_create has selected it)
        void* p = nullptr;
        SA3K_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        SA3K_REQUIRE(p != nullptr, "no device address for the GEMM scratch array");
        ptr = static_cast<float*>(p);
    }
    ctx->noalloc_scratch = ptr;
}

// split-K workspace owned by the context (grows on demand; kernels on one stream use it in turn)
float* gemm_workspace_bytes(sa3k_ctx* ctx, size_t bytes) {
    if (ctx->ws_fixed) {
        // a caller that cannot allocate: the fixed buffer or an error, never a hipMalloc
        if (bytes > ctx->ws_fixed_bytes)
            sa3k_throw(SA3K_ERR_INVALID, "split-K partials need " + std::to_string(bytes) +
                                             " bytes of scratch, more than the " +
                                             std::to_string(ctx->ws_fixed_bytes) + " bytes available");
        return ctx->ws_fixed;
    }
    // one workspace per stream: work on the second and third streams runs beside the main stream's
    const bool side = ctx->stream == ctx->side_stream, quick = ctx->stream == ctx->quick_stream;
    void*& ws = side ? ctx->gemm_ws_side : quick ? ctx->gemm_ws_quick : ctx->gemm_ws;
    size_t& have = side ? ctx->gemm_ws_side_bytes : quick ? ctx->gemm_ws_quick_bytes : ctx->gemm_ws_bytes;
    if (bytes > have) {
        SA3K_REQUIRE(!ctx->capturing, "the split-K workspace cannot grow while a graph is being captured");
        if (ws) {
            SA3K_HIP(hipStreamSynchronize(ctx->stream));
            SA3K_HIP(hipFree(ws));
            ws = nullptr;
            have = 0;
        }
        SA3K_HIP(hipMalloc(&ws, bytes));
        have = bytes;
    }
    return static_cast<float*>(ws);
}

namespace {

__device__ inline uint4 zero4() { return make_uint4(0u, 0u, 0u, 0u); }

__device__ inline uint4 pack8(const float (&f)[8]) {
    bf16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (bf16)f[e];
    return __builtin_bit_cast(uint4, v);
}

template <int SRC>
constexpr int src_bytes() { return SRC == SRC_F32 ? 4 : (SRC == SRC_BF16 || SRC == SRC_F16) ? 2 : 1; }

// 16 bytes of the compute type from element pointer p (CE consecutive K elements of one row) and,
// for Q8_0 sources, scale pointer s (Q8: the row's f16 scale of this 32-block; Q8T: 8 f16 scales).
template <int SRC, bool BF16>
__device__ inline uint4 load_src(const char* p, const char* s) {
    if constexpr (BF16) {
        if constexpr (SRC == SRC_BF16) {
            return *reinterpret_cast<const uint4*>(p);
        } else if constexpr (SRC == SRC_F32) {
            const float4* q = reinterpret_cast<const float4*>(p);
            const float4 a = q[0], b = q[1];
            const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            return pack8(f);
        } else if constexpr (SRC == SRC_F16) {
            const f16x8 h = *reinterpret_cast<const f16x8*>(p);
            float f[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = (float)h[e];
            return pack8(f);
        } else if constexpr (SRC == SRC_Q8) {
            const uint2 q = *reinterpret_cast<const uint2*>(p);
            const float d = (float)*reinterpret_cast<const _Float16*>(s);
            float f[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                f[e] = d * (float)(int8_t)((q.x >> (8 * e)) & 0xff);
                f[4 + e] = d * (float)(int8_t)((q.y >> (8 * e)) & 0xff);
            }
            return pack8(f);
        } else {  // SRC_Q8T
            const uint2 q = *reinterpret_cast<const uint2*>(p);
            const f16x8 d = *reinterpret_cast<const f16x8*>(s);
            float f[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                f[e] = (float)d[e] * (float)(int8_t)((q.x >> (8 * e)) & 0xff);
                f[4 + e] = (float)d[4 + e] * (float)(int8_t)((q.y >> (8 * e)) & 0xff);
            }
            return pack8(f);
        }
    } else {
        if constexpr (SRC == SRC_F32) {
            return *reinterpret_cast<const uint4*>(p);
        } else {  // SRC_F16
            const f16x4 h = *reinterpret_cast<const f16x4*>(p);
            const float4 f = make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
            return __builtin_bit_cast(uint4, f);
        }
    }
}

template <int FM, int FN, bool BF16>
__device__ inline void mma_tile(const char* As, const char* Bs, int wm0, int wn0, int lane,
                                f32x4 (&acc)[FM][FN]) {
    const int r = lane & 15;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int off = s * 64 + (lane >> 4) * 16;
        if constexpr (BF16) {
            bf16x8 af[FM], bfr[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *reinterpret_cast<const bf16x8*>(As + (wm0 + 16 * i + r) * kRowBytes + off);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bfr[j] = *reinterpret_cast<const bf16x8*>(Bs + (wn0 + 16 * j + r) * kRowBytes + off);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        } else {
            f32x4 af[FM], bfr[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *reinterpret_cast<const f32x4*>(As + (wm0 + 16 * i + r) * kRowBytes + off);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bfr[j] = *reinterpret_cast<const f32x4*>(Bs + (wn0 + 16 * j + r) * kRowBytes + off);
            // lane group g holds k = 16s + 4g + e: MFMA e sums the four groups' element e
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][e], bfr[j][e], acc[i][j], 0, 0, 0);
        }
    }
}

// Epilogue of one output element (see gemm.h): rows >= M are the extra rows, stored to Cx.
__device__ inline void epilogue_elem(const KParams& p, int64_t m, int64_t n, float acc) {
    float x = p.alpha * acc;
    if (m >= p.M) {
        if (p.Cbx) {
            p.Cbx[(m - p.M) * p.ldcx + n] = (bf16)x;
            return;
        }
        float* cx = p.Cx + (m - p.M) * p.ldcx + n;
        *cx = p.accumulate_x ? *cx + x : x;
        return;
    }
    if (p.U) p.U[m * p.ldu + n] = x;
    if (p.Ub) p.Ub[m * p.ldu + n] = (bf16)x;
    if (p.colscale && !p.prescale) x = x * p.colscale[n];
    if (p.bias) x = x + p.bias[n];
    if (p.C) {
        if (p.accumulate) p.C[m * p.ldc + n] += x;
        else p.C[m * p.ldc + n] = x;
    }
    if (p.Cb) p.Cb[m * p.ldcb + n] = (bf16)x;
}

// Main kernel. Grid: x = output tiles (padded to a multiple of 8, XCD-remapped), y = K splits.
// Pipeline: K tiles stream through two LDS buffers; global loads run two tiles ahead of the MFMAs
// in two register staging sets (the loop is unrolled by two so the sets stay in registers).
template <int BM, int BN, int WMW, int ASRC, int BSRC, bool BF16, int PD>
__global__ __launch_bounds__(kThreads, 2) void gemm_kernel(KParams p) {
    constexpr int WNW = 4 / WMW;
    constexpr int WTM = BM / WMW, WTN = BN / WNW;
    constexpr int FM = WTM / 16, FN = WTN / 16;
    constexpr int NA = BM * 8 / kThreads, NB = BN * 8 / kThreads;
    constexpr int BKE = BF16 ? 64 : 32;   // elements per K tile
    constexpr int CE = BF16 ? 8 : 4;      // elements per 16-byte chunk
    constexpr int CTSRC = BF16 ? SRC_BF16 : SRC_F32;
    constexpr int CTB = BF16 ? 2 : 4;
    constexpr int AEB = src_bytes<ASRC>(), BEB = src_bytes<BSRC>();
    // per-tile byte advance of the B scale pointer: Q8 one f16 per 32 K; Q8T 8 f16 per chunk row
    constexpr int BSSTR = BSRC == SRC_Q8 ? (BKE / 32) * 2 : BSRC == SRC_Q8T ? BKE * 2 : 0;
    static_assert(NA >= 1 && NB >= 1 && FM >= 1 && FN >= 1, "tile too small");
    __shared__ __attribute__((aligned(16))) char lds[2 * (BM + BN) * kRowBytes];

    // XCD-aware tile order: the grid is padded to a multiple of 8 and consecutive tile ids are
    // given to one XCD (the hardware deals workgroups round-robin over the 8 XCDs), then row tiles
    // are grouped by 8 so neighbouring workgroups share B tiles in that XCD's L2.
    const int64_t Mt = p.M + p.Mx;
    const int tiles_m = (int)((Mt + BM - 1) / BM), tiles_n = (int)((p.N + BN - 1) / BN);
    const int nwg = gridDim.x;
    const int bid = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
    if (bid >= tiles_m * tiles_n) return;
    constexpr int G = 8;
    const int per_group = G * tiles_n;
    const int group = bid / per_group;
    const int first_m = group * G;
    const int gsz = min(tiles_m - first_m, G);
    const int in_g = bid - group * per_group;
    const int tm = first_m + in_g % gsz, tn = in_g / gsz;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave % WMW) * WTM, wn0 = (wave / WMW) * WTN;

    // K range of this split; the second segment (K2) belongs to the last split
    const int KT = (int)(p.K / BKE);
    const int z = blockIdx.y;
    const int kt0 = z * p.kps;
    const int Tm = max(0, min(KT, kt0 + p.kps) - kt0);
    const bool ext = p.K2 > 0 && z == (int)gridDim.y - 1;
    const int T = Tm + (ext ? 1 : 0);
    const int64_t k0 = (int64_t)kt0 * BKE;

    // per-chunk 32-bit byte offsets at the split's first K tile (kNone = zero chunk); main rows
    // index A, extra rows (flag bit) index Ax. Scalar bases + vector offsets keep the address
    // arithmetic out of the loop and the register budget at two waves per SIMD.
    constexpr uint32_t kNone = 0xffffffffu;
    uint32_t aoff[NA];
    uint32_t axmask = 0;
#pragma unroll
    for (int q = 0; q < NA; ++q) {
        const int c = tid + q * kThreads, row = c >> 3, part = c & 7;
        const int64_t gm = m0 + row;
        aoff[q] = kNone;
        if (gm < p.M) {
            aoff[q] = (uint32_t)((gm * p.lda + k0 + part * CE) * AEB);
        } else if (gm < Mt) {
            aoff[q] = (uint32_t)(((gm - p.M) * p.ldax + k0 + part * CE) * CTB);
            axmask |= 1u << q;
        }
    }
    uint32_t boff[NB], bsoff[NB];
#pragma unroll
    for (int q = 0; q < NB; ++q) {
        const int c = tid + q * kThreads, row = c >> 3, part = c & 7;
        const int64_t gn = n0 + row;
        boff[q] = kNone;
        bsoff[q] = 0;
        if (gn < p.N) {
            const int64_t k = k0 + part * CE;
            boff[q] = (uint32_t)((gn * p.ldb + k) * BEB);
            if constexpr (BSRC == SRC_Q8) bsoff[q] = (uint32_t)((gn * p.ldbs + (k >> 5)) * 2);
            if constexpr (BSRC == SRC_Q8T) bsoff[q] = (uint32_t)(((gn >> 5) * p.ldbs + k) * 2);
        }
    }
    const char* Ab = static_cast<const char*>(p.A);
    const char* Axb = static_cast<const char*>(p.Ax);
    const char* Bb = static_cast<const char*>(p.B);
    const char* Bsb = static_cast<const char*>(p.Bs);

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto load = [&](int t, uint4 (&ra)[NA], uint4 (&rb)[NB]) {
        if (t < Tm) {
#pragma unroll
            for (int q = 0; q < NA; ++q) {
                if (aoff[q] == kNone) ra[q] = zero4();
                else if (axmask & (1u << q)) ra[q] = load_src<CTSRC, BF16>(Axb + aoff[q] + t * (BKE * CTB), nullptr);
                else ra[q] = load_src<ASRC, BF16>(Ab + aoff[q] + t * (BKE * AEB), nullptr);
            }
#pragma unroll
            for (int q = 0; q < NB; ++q)
                rb[q] = boff[q] != kNone ? load_src<BSRC, BF16>(Bb + boff[q] + t * (BKE * BEB), Bsb + bsoff[q] + t * BSSTR)
                                         : zero4();
        } else {  // the second segment: one tile of K2 <= BKE elements
#pragma unroll
            for (int q = 0; q < NA; ++q) {
                const int c = tid + q * kThreads, row = c >> 3, part = c & 7;
                const int64_t gm = m0 + row;
                ra[q] = zero4();
                if (part * CE < p.K2) {
                    if (gm < p.M)
                        ra[q] = load_src<CTSRC, BF16>(static_cast<const char*>(p.A2) + (gm * p.lda2 + part * CE) * CTB, nullptr);
                    else if (gm < Mt)
                        ra[q] = load_src<CTSRC, BF16>(static_cast<const char*>(p.A2x) + ((gm - p.M) * p.lda2x + part * CE) * CTB, nullptr);
                }
            }
#pragma unroll
            for (int q = 0; q < NB; ++q) {
                const int c = tid + q * kThreads, row = c >> 3, part = c & 7;
                const int64_t gn = n0 + row;
                rb[q] = (gn < p.N && part * CE < p.K2)
                            ? load_src<CTSRC, BF16>(static_cast<const char*>(p.B2) + (gn * p.ldb2 + part * CE) * CTB, nullptr)
                            : zero4();
            }
        }
    };
    auto store = [&](int buf, const uint4 (&ra)[NA], const uint4 (&rb)[NB]) {
        char* base = lds + buf * (BM + BN) * kRowBytes;
#pragma unroll
        for (int q = 0; q < NA; ++q) {
            const int c = tid + q * kThreads;
            *reinterpret_cast<uint4*>(base + (c >> 3) * kRowBytes + (c & 7) * 16) = ra[q];
        }
#pragma unroll
        for (int q = 0; q < NB; ++q) {
            const int c = tid + q * kThreads;
            *reinterpret_cast<uint4*>(base + (BM + (c >> 3)) * kRowBytes + (c & 7) * 16) = rb[q];
        }
    };
    auto compute = [&](int buf) {
        const char* base = lds + buf * (BM + BN) * kRowBytes;
        mma_tile<FM, FN, BF16>(base, base + BM * kRowBytes, wm0, wn0, lane, acc);
    };
    // prescale: the main segment's sums times colscale[n], before the second segment is added
    auto scale_acc = [&] {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int64_t n = n0 + wn0 + 16 * j + (lane & 15);
            const float c = n < p.N ? p.colscale[n] : 0.f;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[i][j][v] = acc[i][j][v] * c;
        }
    };

    if constexpr (PD == 2) {
        uint4 ra0[NA], rb0[NB], ra1[NA], rb1[NB];
        if (T > 0) load(0, ra0, rb0);
        if (T > 1) load(1, ra1, rb1);
        if (T > 0) store(0, ra0, rb0);
        __syncthreads();
        if (T > 2) load(2, ra0, rb0);
        for (int t = 0; t < T; t += 2) {
            // tile t in LDS buffer 0; tile t+1 in ra1/rb1; tile t+2 in flight into ra0/rb0
            if (p.prescale && t == Tm) scale_acc();
            compute(0);
            if (t + 1 < T) store(1, ra1, rb1);
            __syncthreads();
            if (t + 3 < T) load(t + 3, ra1, rb1);
            if (t + 1 >= T) break;
            if (p.prescale && t + 1 == Tm) scale_acc();
            compute(1);
            if (t + 2 < T) store(0, ra0, rb0);
            __syncthreads();
            if (t + 4 < T) load(t + 4, ra0, rb0);
        }
    } else {
        // one tile of register prefetch: load t+1 while the MFMAs consume tile t
        uint4 ra[NA], rb[NB];
        if (T > 0) {
            load(0, ra, rb);
            store(0, ra, rb);
        }
        __syncthreads();
        for (int t = 0; t < T; ++t) {
            if (t + 1 < T) load(t + 1, ra, rb);
            if (p.prescale && t == Tm) scale_acc();
            compute(t & 1);
            if (t + 1 < T) store((t + 1) & 1, ra, rb);
            __syncthreads();
        }
    }
    if (p.prescale && !ext) scale_acc();   // a split without the second segment

    // lane holds rows 4*(lane/16)+v, column lane%16 of each 16x16 block
    if (p.ws) {  // split-K partial sums, reduced (and epilogued) by gemm_splitk_reduce
        float* w = p.ws + (int64_t)z * Mt * p.N;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int64_t n = n0 + wn0 + 16 * j + (lane & 15);
            if (n >= p.N) continue;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int64_t m = m0 + wm0 + 16 * i + 4 * (lane >> 4) + v;
                    if (m < Mt) w[m * p.N + n] = acc[i][j][v];
                }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int64_t n = n0 + wn0 + 16 * j + (lane & 15);
        if (n >= p.N) continue;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t m = m0 + wm0 + 16 * i + 4 * (lane >> 4) + v;
                if (m < Mt) epilogue_elem(p, m, n, acc[i][j][v]);
            }
    }
}

// sum of the split partials in split order (deterministic), then the epilogue
__global__ __launch_bounds__(kThreads) void gemm_splitk_reduce(KParams p, int splits) {
    const int64_t Mt = p.M + p.Mx;
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (idx >= Mt * p.N) return;
    // eight splits' partials loaded per memory round trip (indices past the last split re-read it
    // and are not added); the sums are added in split order from zero
    const int64_t plane = Mt * p.N;
    float s = 0.f;
    for (int z = 0; z < splits; z += 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = p.ws[(int64_t)min(z + k, splits - 1) * plane + idx];
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (z + k < splits) s += v[k];
    }
    const int64_t m = idx / p.N, n = idx - m * p.N;
    epilogue_elem(p, m, n, s);
}

template <int BM, int BN, int WMW, int ASRC, int BSRC, bool BF16>
void launch(sa3k_ctx* ctx, KParams p) {
    const int64_t tiles = ceil_div(p.M + p.Mx, BM) * ceil_div(p.N, BN);
    const int64_t grid = ceil_div(tiles, 8) * 8;
    const int KT = (int)(p.K / (BF16 ? 64 : 32));
    // split K when the output tiles cannot fill the chip twice over (2 workgroups per CU resident);
    // a product with a handful of output tiles (a few tokens against a long K: the DiT's conditioning
    // linears) splits further, so its B operand streams through many workgroups
    int splits = 1;
    const int64_t max_splits = tiles <= 32 ? 64 : 16;
    if (ctx->gemm_split && tiles < 512 && KT >= 8) splits = (int)std::min<int64_t>({max_splits, KT / 4, std::max<int64_t>(1, 512 / tiles)});
    p.kps = (KT + splits - 1) / std::max(splits, 1);
    if (p.kps == 0) p.kps = 1;
    splits = std::max(1, (KT + p.kps - 1) / p.kps);
    p.ws = nullptr;
    if (splits > 1) {
        const size_t need = (size_t)splits * (size_t)(p.M + p.Mx) * (size_t)p.N * sizeof(float);
        p.ws = gemm_workspace_bytes(ctx, need);
    }
    dim3 g((unsigned)grid, (unsigned)splits);
    {
        static const std::string name = std::string("gemm_decode<") + std::to_string(BM) + "," + std::to_string(BN) +
                                        "," + std::to_string(WMW) + ",a" + std::to_string(ASRC) + ",b" +
                                        std::to_string(BSRC) + (BF16 ? ",bf16>" : ",f32>");
        KernelScope ks(ctx, name.c_str(), 2.0 * (double)(p.M + p.Mx) * (double)p.N * (double)(p.K + p.K2));
        if (ctx->gemm_pd == 2)
            launch_k(ctx, splits == 1, gemm_kernel<BM, BN, WMW, ASRC, BSRC, BF16, 2>, g, dim3(kThreads), 0, p);
        else
            launch_k(ctx, splits == 1, gemm_kernel<BM, BN, WMW, ASRC, BSRC, BF16, 1>, g, dim3(kThreads), 0, p);
        SA3K_LAUNCHED();
    }
    if (splits > 1) {
        KernelScope ks(ctx, "gemm_splitk_reduce");
        launch_k(ctx, true, gemm_splitk_reduce, dim3((unsigned)ceil_div((p.M + p.Mx) * p.N, kThreads)), dim3(kThreads),
                 0, p, splits);
        SA3K_LAUNCHED();
    }
}

template <int ASRC, int BSRC, bool BF16>
void launch_tiles(sa3k_ctx* ctx, const KParams& p) {
    if (p.M + p.Mx <= 32) launch<32, 128, 1, ASRC, BSRC, BF16>(ctx, p);
    else if (p.M + p.Mx <= 64 && p.N > 64) launch<64, 128, 2, ASRC, BSRC, BF16>(ctx, p);
    else if (p.N <= 32) launch<128, 32, 4, ASRC, BSRC, BF16>(ctx, p);
    else if (p.N <= 64) launch<128, 64, 4, ASRC, BSRC, BF16>(ctx, p);
    else launch<128, 128, 2, ASRC, BSRC, BF16>(ctx, p);
}

template <int ASRC, bool BF16>
void launch_b(sa3k_ctx* ctx, const KParams& p, int b_src) {
    if constexpr (BF16) {
        switch (b_src) {
            case SRC_BF16: return launch_tiles<ASRC, SRC_BF16, true>(ctx, p);
            case SRC_F16: return launch_tiles<ASRC, SRC_F16, true>(ctx, p);
            case SRC_F32: return launch_tiles<ASRC, SRC_F32, true>(ctx, p);
            case SRC_Q8: return launch_tiles<ASRC, SRC_Q8, true>(ctx, p);
            case SRC_Q8T: return launch_tiles<ASRC, SRC_Q8T, true>(ctx, p);
        }
    } else {
        switch (b_src) {
            case SRC_F32: return launch_tiles<ASRC, SRC_F32, false>(ctx, p);
            case SRC_F16: return launch_tiles<ASRC, SRC_F16, false>(ctx, p);
        }
    }
    sa3k_throw(SA3K_ERR_UNSUPPORTED, "GEMM B operand type not supported for this precision");
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

void gemm_run(sa3k_ctx* ctx, const GemmDesc& d, const char* prof_name) {
    const bool bf = d.prec == SA3K_PREC_BF16;
    SA3K_REQUIRE(d.prec == SA3K_PREC_BF16 || d.prec == SA3K_PREC_F32, "unknown GEMM precision");
    SA3K_REQUIRE(d.M >= 0 && d.N >= 0 && d.K >= 0, "negative GEMM extent");
    if (d.M == 0 || d.N == 0) return;
    const int bke = bf ? 64 : 32, ce = bf ? 8 : 4;
    SA3K_REQUIRE(d.K % bke == 0, "GEMM K must be a multiple of the K tile (64 bf16 / 32 f32)");
    SA3K_REQUIRE(d.K2 >= 0 && d.K2 <= bke && d.K2 % ce == 0, "GEMM second segment exceeds one K tile");
    SA3K_REQUIRE(d.K > 0 || d.K2 > 0, "GEMM with empty K");
    SA3K_REQUIRE(d.A && d.B && al16(d.A) && al16(d.B), "GEMM operands must be non-null and 16-byte aligned");
    SA3K_REQUIRE(d.K2 == 0 || (d.A2 && d.B2 && al16(d.A2) && al16(d.B2)), "GEMM second segment misaligned");
    SA3K_REQUIRE(d.C || d.Cb || d.U || d.Ub, "GEMM without an output");
    const int a_ce = (d.a_src == SRC_F32) ? 4 : 2;
    SA3K_REQUIRE((d.lda * a_ce) % 16 == 0, "GEMM lda must keep rows 16-byte aligned");
    if (d.b_src == SRC_Q8 || d.b_src == SRC_Q8T) {
        SA3K_REQUIRE(bf && d.Bs, "Q8_0 B operand needs bf16 compute and scales");
        SA3K_REQUIRE(d.ldb % 16 == 0, "Q8_0 quant rows must be 16-byte aligned");
        if (d.b_src == SRC_Q8) SA3K_REQUIRE(d.K % 32 == 0, "Q8_0 K must be a multiple of 32");
        if (d.b_src == SRC_Q8T) SA3K_REQUIRE(d.N % 32 == 0 && d.ldbs % 8 == 0 && al16(d.Bs), "Q8_0 transposed layout misaligned");
    }
    SA3K_REQUIRE(d.Mx >= 0, "negative extra rows");
    SA3K_REQUIRE(d.Mx == 0 || (d.Ax && (d.Cx || d.Cbx) && al16(d.Ax) && (d.K2 == 0 || (d.A2x && al16(d.A2x)))),
                 "GEMM extra rows need Ax, Cx or Cbx (and A2x with a second segment)");
    SA3K_REQUIRE(!d.prescale || (d.colscale && d.Mx == 0 && !d.U && !d.Ub),
                 "GEMM prescale needs colscale and no extra rows or pre-scale copies");
    SA3K_REQUIRE(!d.b_kn || (bf && d.a_src == SRC_BF16 && d.b_src == SRC_BF16 && ctx->gemm_dma && d.K2 == 0 &&
                             !d.prescale && d.N % 8 == 0 && d.ldb >= d.N && (d.ldb * 2) % 16 == 0 &&
                             (d.Nx == 0 || (d.N % 64 == 0 && d.ldbx >= d.Nx))),
                 "a [K][N] B operand needs bf16 operands on the DMA kernel, no second segment, and extra "
                 "columns ([K][Nx], row pitch ldbx) only beside N % 64 == 0");
    SA3K_REQUIRE(d.Nx >= 0, "negative extra columns");
    SA3K_REQUIRE(d.Nx == 0 || (bf && d.a_src == SRC_BF16 && d.b_src == SRC_BF16 && ctx->gemm_dma && d.K2 == 0 &&
                               !d.prescale && d.N % 8 == 0 && d.Nx % 8 == 0 && d.Bx && al16(d.Bx) &&
                               (d.ldbx * 2) % 16 == 0 && d.Cbn && d.ldcn >= d.Nx),
                 "GEMM extra columns need bf16 operands on the DMA kernel, no second segment, 8-column "
                 "multiples and an aligned Bx with a Cbn output");
    if (gemm_skinny_ok(ctx, d)) {
        KernelScope ks(ctx, prof_name);
        gemm_run_skinny(ctx, d);
        return;
    }
    const int ct_src = bf ? SRC_BF16 : SRC_F32;
    // bf16 A with an f16 or Q8_0 B: the DMA-fed kernel stages B as stored (2 or 1 + 1/16 bytes per
    // element) and decodes it between LDS and the MFMAs
    auto a16 = [](const void* q, int64_t ld_bytes, int align) {
        return (reinterpret_cast<uintptr_t>(q) % (uintptr_t)align) == 0 && ld_bytes % align == 0;
    };
    const bool dq = bf && ctx->gemm_dq && ctx->gemm_dma && d.a_src == SRC_BF16 &&
                    (d.b_src == SRC_F16 || d.b_src == SRC_Q8) && d.Mx == 0 && d.Nx == 0 && !d.b_kn &&
                    d.K % 64 == 0 && d.N % 8 == 0 && a16(d.A, d.lda * 2, 16) &&
                    (d.b_src == SRC_F16 ? a16(d.B, d.ldb * 2, 16)
                                        : a16(d.B, d.ldb, 16) && d.Bs && a16(d.Bs, d.ldbs * 2, 4));
    if (dq) {
        KernelScope ks(ctx, prof_name);
        gemm_run_dma(ctx, d);
        SA3K_LAUNCHED();
        return;
    }
    if (d.a_src == ct_src && d.b_src == ct_src && ctx->gemm_dma) {
        SA3K_REQUIRE((d.ldb * (bf ? 2 : 4)) % 16 == 0 && (d.Mx == 0 || (d.ldax * (bf ? 2 : 4)) % 16 == 0),
                     "GEMM operand rows must be 16-byte aligned");
        KernelScope ks(ctx, prof_name);
        gemm_run_dma(ctx, d);
        SA3K_LAUNCHED();
        return;
    }
    KParams p{d.A, d.lda, d.B, d.ldb, d.Bs, d.ldbs, d.A2, d.lda2, d.B2, d.ldb2, d.K2, d.M, d.N, d.K,
              d.alpha, d.colscale, d.bias, d.C, d.ldc, d.accumulate, d.Cb, d.ldcb, d.U, d.Ub, d.ldu,
              d.Mx, d.Ax, d.ldax, d.A2x, d.lda2x, d.Cx, d.ldcx, d.accumulate_x, d.Cbx, nullptr, 0, d.prescale};
    KernelScope ks(ctx, prof_name);
    if (bf) {
        if (d.a_src == SRC_BF16) launch_b<SRC_BF16, true>(ctx, p, d.b_src);
        else if (d.a_src == SRC_F32) launch_b<SRC_F32, true>(ctx, p, d.b_src);
        else sa3k_throw(SA3K_ERR_UNSUPPORTED, "GEMM A operand type");
    } else {
        SA3K_REQUIRE(d.a_src == SRC_F32, "f32 GEMM needs an f32 A operand");
        launch_b<SRC_F32, false>(ctx, p, d.b_src);
    }
    SA3K_LAUNCHED();
}

}  // namespace sa3k

// ---------------------------------------------------------------------------------- C ABI
namespace sa3k {
namespace {

GemmDesc gemm_nt_desc(int prec, int a_type, const void* A, int64_t lda, int b_type, const void* B, int64_t ldb,
                      const void* B_scales, int64_t ldbs, int64_t M, int64_t N, int64_t K, float alpha,
                      const float* colscale, const float* bias, float* C, int64_t ldc, int accumulate) {
    auto src_of = [](int t, bool transposed_q8) -> int {
        switch (t) {
            case SA3K_TYPE_BF16: return SRC_BF16;
            case SA3K_TYPE_F16: return SRC_F16;
            case SA3K_TYPE_F32: return SRC_F32;
            case SA3K_TYPE_Q8_0: return transposed_q8 ? SRC_Q8T : SRC_Q8;
        }
        sa3k_throw(SA3K_ERR_UNSUPPORTED, "unknown operand type");
        return 0;
    };
    GemmDesc d;
    d.prec = prec;
    d.a_src = src_of(a_type, false);
    d.b_src = src_of(b_type < 0 ? SA3K_TYPE_Q8_0 : b_type, b_type < 0);
    d.A = A; d.lda = lda; d.B = B; d.ldb = ldb; d.Bs = B_scales; d.ldbs = ldbs;
    d.M = M; d.N = N; d.K = K; d.alpha = alpha; d.colscale = colscale; d.bias = bias;
    d.C = C; d.ldc = ldc; d.accumulate = accumulate;
    return d;
}

// For the duration of one call: split-K partials go to the device's scratch array and split sums
// are reduced by the separate launch (the in-kernel reduction's tile counters are not used).
struct FixedScratchScope {
    sa3k_ctx* c;
    int fixup;
    explicit FixedScratchScope(sa3k_ctx* ctx) : c(ctx), fixup(ctx->gemm_fixup) {
        c->ws_fixed = c->noalloc_scratch;
        c->ws_fixed_bytes = kNoAllocScratchFloats * sizeof(float);
        c->gemm_fixup = 0;
    }
    ~FixedScratchScope() {
        c->ws_fixed = nullptr;
        c->ws_fixed_bytes = 0;
        c->gemm_fixup = fixup;
    }
    FixedScratchScope(const FixedScratchScope&) = delete;
    FixedScratchScope& operator=(const FixedScratchScope&) = delete;
};

}  // namespace
}  // namespace sa3k

extern "C" SA3K_API int sa3k_gemm_nt(sa3k_ctx* ctx, int prec, int a_type, const void* A, int64_t lda,
                                     int b_type, const void* B, int64_t ldb, const void* B_scales,
                                     int64_t ldbs, int64_t M, int64_t N, int64_t K, float alpha,
                                     const float* colscale, const float* bias, float* C, int64_t ldc,
                                     int accumulate) {
    using namespace sa3k;
    return sa3k_guard(ctx, "sa3k_gemm_nt", [&] {
        const GemmDesc d = gemm_nt_desc(prec, a_type, A, lda, b_type, B, ldb, B_scales, ldbs, M, N, K, alpha,
                                        colscale, bias, C, ldc, accumulate);
        gemm_run(ctx, d, "gemm_nt");
    });
}

extern "C" SA3K_API int sa3k_gemm_nt_noalloc(sa3k_ctx* ctx, int prec, int a_type, const void* A, int64_t lda,
                                             int b_type, const void* B, int64_t ldb, const void* B_scales,
                                             int64_t ldbs, int64_t M, int64_t N, int64_t K, float alpha,
                                             const float* colscale, const float* bias, float* C, int64_t ldc,
                                             int accumulate) {
    using namespace sa3k;
    return sa3k_guard(ctx, "sa3k_gemm_nt_noalloc", [&] {
        SA3K_REQUIRE(ctx->noalloc_scratch != nullptr, "the device scratch array was not set up");
        SA3K_REQUIRE(ctx->stream == ctx->main_stream, "called while work is routed to the second stream");
        const GemmDesc d = gemm_nt_desc(prec, a_type, A, lda, b_type, B, ldb, B_scales, ldbs, M, N, K, alpha,
                                        colscale, bias, C, ldc, accumulate);
        FixedScratchScope scope(ctx);
        gemm_run(ctx, d, "gemm_nt");
    });
}
