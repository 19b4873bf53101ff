// K1/K2 GEMM kernels and their host dispatch. See gemm.h for the contract.
#include "gemm.h"

#include <algorithm>

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
};

__device__ inline uint4 zero4() { return make_uint4(0u, 0u, 0u, 0u); }

__device__ inline uint4 pack8(const float (&f)[8]) {
    bf16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (bf16)f[e];
    return __builtin_bit_cast(uint4, v);
}

// 16 bytes of the compute type for row `row`, elements k .. k+CE-1 of a K-contiguous source.
template <int SRC, bool BF16>
__device__ inline uint4 load_chunk(const void* base, int64_t ld, const void* sc, int64_t lds,
                                   int64_t row, int64_t k) {
    if constexpr (BF16) {
        if constexpr (SRC == SRC_BF16) {
            return *reinterpret_cast<const uint4*>(static_cast<const bf16*>(base) + row * ld + k);
        } else if constexpr (SRC == SRC_F32) {
            const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + row * ld + k);
            const float4 a = p[0], b = p[1];
            const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            return pack8(f);
        } else if constexpr (SRC == SRC_F16) {
            const f16x8 h = *reinterpret_cast<const f16x8*>(static_cast<const _Float16*>(base) + row * ld + k);
            float f[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = (float)h[e];
            return pack8(f);
        } else if constexpr (SRC == SRC_Q8) {
            // quants [row][k], scales [row][k/32]
            const uint2 q = *reinterpret_cast<const uint2*>(static_cast<const int8_t*>(base) + row * ld + k);
            const float d = (float)static_cast<const _Float16*>(sc)[row * lds + (k >> 5)];
            float f[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                f[e] = d * (float)(int8_t)((q.x >> (8 * e)) & 0xff);
                f[4 + e] = d * (float)(int8_t)((q.y >> (8 * e)) & 0xff);
            }
            return pack8(f);
        } else {  // SRC_Q8T: quants [row][k], scales [row/32][k]
            const uint2 q = *reinterpret_cast<const uint2*>(static_cast<const int8_t*>(base) + row * ld + k);
            const f16x8 d = *reinterpret_cast<const f16x8*>(static_cast<const _Float16*>(sc) + (row >> 5) * lds + k);
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
            return *reinterpret_cast<const uint4*>(static_cast<const float*>(base) + row * ld + k);
        } else {  // SRC_F16
            const f16x4 h = *reinterpret_cast<const f16x4*>(static_cast<const _Float16*>(base) + row * ld + k);
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

template <int BM, int BN, int WMW, int ASRC, int BSRC, bool BF16>
__global__ __launch_bounds__(kThreads) void gemm_kernel(KParams p) {
    constexpr int WNW = 4 / WMW;
    constexpr int WTM = BM / WMW, WTN = BN / WNW;
    constexpr int FM = WTM / 16, FN = WTN / 16;
    constexpr int NA = BM * 8 / kThreads, NB = BN * 8 / kThreads;
    constexpr int BKE = BF16 ? 64 : 32;   // elements per K tile
    constexpr int CE = BF16 ? 8 : 4;      // elements per 16-byte chunk
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

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    uint4 ra[NA], rb[NB];
    const int KT = (int)(p.K / BKE);
    const int T = KT + (p.K2 > 0 ? 1 : 0);

    auto load = [&](int t) {
#pragma unroll
        for (int q = 0; q < NA; ++q) {
            const int c = tid + q * kThreads, row = c >> 3, part = c & 7;
            const int64_t gm = m0 + row;
            constexpr int CTSRC = BF16 ? SRC_BF16 : SRC_F32;
            if (gm < p.M) {
                if (t < KT) ra[q] = load_chunk<ASRC, BF16>(p.A, p.lda, nullptr, 0, gm, (int64_t)t * BKE + part * CE);
                else ra[q] = (part * CE < p.K2) ? load_chunk<CTSRC, BF16>(p.A2, p.lda2, nullptr, 0, gm, part * CE) : zero4();
            } else if (gm < Mt) {
                const int64_t xr = gm - p.M;
                if (t < KT) ra[q] = load_chunk<CTSRC, BF16>(p.Ax, p.ldax, nullptr, 0, xr, (int64_t)t * BKE + part * CE);
                else ra[q] = (part * CE < p.K2) ? load_chunk<CTSRC, BF16>(p.A2x, p.lda2x, nullptr, 0, xr, part * CE) : zero4();
            } else {
                ra[q] = zero4();
            }
        }
#pragma unroll
        for (int q = 0; q < NB; ++q) {
            const int c = tid + q * kThreads, row = c >> 3, part = c & 7;
            const int64_t gn = n0 + row;
            if (gn >= p.N) rb[q] = zero4();
            else if (t < KT) rb[q] = load_chunk<BSRC, BF16>(p.B, p.ldb, p.Bs, p.ldbs, gn, (int64_t)t * BKE + part * CE);
            else rb[q] = (part * CE < p.K2) ? load_chunk<BF16 ? SRC_BF16 : SRC_F32, BF16>(p.B2, p.ldb2, nullptr, 0, gn, part * CE) : zero4();
        }
    };
    auto store = [&](int buf) {
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

    if (T > 0) {
        load(0);
        store(0);
    }
    __syncthreads();
    for (int t = 0; t < T; ++t) {
        if (t + 1 < T) load(t + 1);
        const char* base = lds + (t & 1) * (BM + BN) * kRowBytes;
        mma_tile<FM, FN, BF16>(base, base + BM * kRowBytes, wm0, wn0, lane, acc);
        if (t + 1 < T) store((t + 1) & 1);
        __syncthreads();
    }

    // epilogue: lane holds rows 4*(lane/16)+v, column lane%16 of each 16x16 block
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int64_t n = n0 + wn0 + 16 * j + (lane & 15);
        if (n >= p.N) continue;
        const float cs = p.colscale ? p.colscale[n] : 1.0f;
        const float bi = p.bias ? p.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t m = m0 + wm0 + 16 * i + 4 * (lane >> 4) + v;
                if (m >= p.M) {
                    if (m < Mt) {
                        float* cx = p.Cx + (m - p.M) * p.ldcx + n;
                        const float x = p.alpha * acc[i][j][v];
                        *cx = p.accumulate_x ? *cx + x : x;
                    }
                    continue;
                }
                float x = p.alpha * acc[i][j][v];
                if (p.U) p.U[m * p.ldu + n] = x;
                if (p.Ub) p.Ub[m * p.ldu + n] = (bf16)x;
                if (p.colscale) x = x * cs;
                if (p.bias) x = x + bi;
                if (p.C) {
                    if (p.accumulate) p.C[m * p.ldc + n] += x;
                    else p.C[m * p.ldc + n] = x;
                }
                if (p.Cb) p.Cb[m * p.ldcb + n] = (bf16)x;
            }
        }
    }
}

template <int BM, int BN, int WMW, int ASRC, int BSRC, bool BF16>
void launch(sa3k_ctx* ctx, const KParams& p) {
    const int64_t tiles = ceil_div(p.M + p.Mx, BM) * ceil_div(p.N, BN);
    const int64_t grid = ceil_div(tiles, 8) * 8;
    gemm_kernel<BM, BN, WMW, ASRC, BSRC, BF16><<<(unsigned)grid, kThreads, 0, ctx->stream>>>(p);
}

template <int ASRC, int BSRC, bool BF16>
void launch_tiles(sa3k_ctx* ctx, const KParams& p) {
    if (p.M + p.Mx <= 32) launch<32, 128, 1, ASRC, BSRC, BF16>(ctx, p);
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
    SA3K_REQUIRE(d.Mx == 0 || (d.Ax && d.Cx && al16(d.Ax) && (d.K2 == 0 || (d.A2x && al16(d.A2x)))),
                 "GEMM extra rows need Ax, Cx (and A2x with a second segment)");
    KParams p{d.A, d.lda, d.B, d.ldb, d.Bs, d.ldbs, d.A2, d.lda2, d.B2, d.ldb2, d.K2, d.M, d.N, d.K,
              d.alpha, d.colscale, d.bias, d.C, d.ldc, d.accumulate, d.Cb, d.ldcb, d.U, d.Ub, d.ldu,
              d.Mx, d.Ax, d.ldax, d.A2x, d.lda2x, d.Cx, d.ldcx, d.accumulate_x};
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
extern "C" SA3K_API int sa3k_gemm_nt(sa3k_ctx* ctx, int prec, int a_type, const void* A, int64_t lda,
                                     int b_type, const void* B, int64_t ldb, const void* B_scales,
                                     int64_t ldbs, int64_t M, int64_t N, int64_t K, float alpha,
                                     const float* colscale, const float* bias, float* C, int64_t ldc,
                                     int accumulate) {
    using namespace sa3k;
    return sa3k_guard(ctx, "sa3k_gemm_nt", [&] {
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
        gemm_run(ctx, d, "gemm_nt");
    });
}
