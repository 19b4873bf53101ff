// K1/K2 fast path: C = A . B^T with both operands already in the compute type (bf16 or f32).
//
// Operand tiles go straight from global memory into LDS with global_load_lds_dwordx4 (gfx950),
// so no VGPR staging and no per-element work happens in the K loop: the loop is DMA issue,
// one barrier, and 16-byte LDS fragment reads feeding the MFMAs. A STAGES-deep LDS ring keeps
// STAGES-1 K tiles in flight. LDS rows are 128 bytes (64 bf16 / 32 f32 of K) without padding;
// the eight 16-byte chunks of row r are stored XOR-swizzled (chunk kc at kc ^ swz(r)) so that the
// 16 rows a fragment read touches fall into distinct banks. The DMA writes 64 consecutive 16-byte
// slots per wave instruction, so the swizzle is applied on the global side: the lane that owns
// LDS slot s fetches the chunk that belongs there.
//
// Rows past M+Mx / N are clamped to a valid row (their results are never stored); K chunks past
// K2 in the second segment read a zero page, since they feed valid outputs.
#include "gemm.h"

#include <algorithm>

namespace sa3k {

struct DmaParams {
    const void* A; int64_t lda;
    const void* B; int64_t ldb;
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
    float* ws;
    int kps;
    const void* zero;   // >= 16 zero bytes
    int* counters;      // split-K arrival counters per tile (all zero between launches), or null
};

namespace {

constexpr int kThreads = 256;
constexpr int kRow = 128;   // LDS bytes per tile row

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

template <int N>
struct IC {
    static constexpr int value = N;
};
// f(IC<0>{}), ..., f(IC<N-1>{}) in order
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(IC<I>{});
        static_for<N, I + 1>(f);
    }
}

// s_waitcnt vmcnt(n) leaving the other counters untouched (gfx9 encoding)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ void dma16(const void* g, char* lds_slot_base_wave) {
    // every lane writes 16 bytes at lds_slot_base_wave + lane*16
    __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds_slot_base_wave, 16, 0, 0);
}

__device__ inline void epilogue_elem(const DmaParams& p, int64_t m, int64_t n, float acc) {
    float x = p.alpha * acc;
    if (m >= p.M) {
        float* cx = p.Cx + (m - p.M) * p.ldcx + n;
        *cx = p.accumulate_x ? *cx + x : x;
        return;
    }
    if (p.U) p.U[m * p.ldu + n] = x;
    if (p.Ub) p.Ub[m * p.ldu + n] = (bf16)x;
    if (p.colscale) x = x * p.colscale[n];
    if (p.bias) x = x + p.bias[n];
    if (p.C) {
        if (p.accumulate) p.C[m * p.ldc + n] += x;
        else p.C[m * p.ldc + n] = x;
    }
    if (p.Cb) p.Cb[m * p.ldcb + n] = (bf16)x;
}

template <int BM, int BN, int WMW, int STAGES, bool BF16>
__global__ __launch_bounds__(kThreads) void gemm_dma_kernel(DmaParams p) {
    constexpr int WNW = 4 / WMW;
    constexpr int WTM = BM / WMW, WTN = BN / WNW;
    constexpr int FM = WTM / 16, FN = WTN / 16;
    constexpr int NA = BM * 8 / kThreads, NB = BN * 8 / kThreads;   // 16-byte chunks per thread per tile
    constexpr int LPT = NA + NB;                                     // DMA instructions per thread per tile
    constexpr int CE = BF16 ? 8 : 4;                                 // elements per chunk
    constexpr int EB = BF16 ? 2 : 4;                                 // bytes per element
    constexpr int BKE = 8 * CE;                                      // K elements per tile
    constexpr int STAGE_BYTES = (BM + BN) * kRow;
    static_assert(NA >= 1 && NB >= 1 && FM >= 1 && FN >= 1, "tile too small");
    static_assert(STAGES >= 2 && STAGES <= 4 && (STAGES - 1) * LPT < 64, "pipeline depth");
    // One LDS object per stage, always addressed by a compile-time stage index: the compiler then
    // knows that the DMA filling stage s+STAGES-1 cannot alias the stage the MFMAs read, and keeps
    // it in flight instead of waiting for every outstanding DMA before each LDS read. (Stages a
    // configuration does not use are never referenced and take no LDS.)
    __shared__ __attribute__((aligned(1024))) char lds0[STAGE_BYTES];
    __shared__ __attribute__((aligned(1024))) char lds1[STAGE_BYTES];
    __shared__ __attribute__((aligned(1024))) char lds2[STAGE_BYTES];
    __shared__ __attribute__((aligned(1024))) char lds3[STAGE_BYTES];
    auto stage = [&](auto s) -> char* {
        constexpr int S = decltype(s)::value % STAGES;
        if constexpr (S == 0) return lds0;
        else if constexpr (S == 1) return lds1;
        else if constexpr (S == 2) return lds2;
        else return lds3;
    };

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

    const int KT = (int)(p.K / BKE);
    const int z = blockIdx.y;
    const int kt0 = z * p.kps;
    const int Tm = max(0, min(KT, kt0 + p.kps) - kt0);
    const bool ext = p.K2 > 0 && z == (int)gridDim.y - 1;
    const int T = Tm + (ext ? 1 : 0);
    const int64_t k0 = (int64_t)kt0 * BKE;

    // Source of the chunk this thread DMAs into slot (q*256 + tid) of the A / B region of a stage:
    // row = slot/8, logical chunk kc = (slot%8) ^ swz(row).
    const char* ag[NA];    // main-segment chunk pointer at the split's first tile
    const char* a2g[NA];   // second-segment chunk pointer (zero page when past K2)
#pragma unroll
    for (int q = 0; q < NA; ++q) {
        const int s = q * kThreads + tid, row = s >> 3, kc = (s & 7) ^ swz(row);
        int64_t gm = m0 + row;
        if (gm >= Mt) gm = 0;   // clamped: this output row is never stored
        if (gm < p.M) {
            ag[q] = static_cast<const char*>(p.A) + (gm * p.lda + k0 + kc * CE) * EB;
            a2g[q] = (kc * CE < p.K2) ? static_cast<const char*>(p.A2) + (gm * p.lda2 + kc * CE) * EB
                                      : static_cast<const char*>(p.zero);
        } else {
            const int64_t xr = gm - p.M;
            ag[q] = static_cast<const char*>(p.Ax) + (xr * p.ldax + k0 + kc * CE) * EB;
            a2g[q] = (kc * CE < p.K2) ? static_cast<const char*>(p.A2x) + (xr * p.lda2x + kc * CE) * EB
                                      : static_cast<const char*>(p.zero);
        }
    }
    const char* bg[NB];
    const char* b2g[NB];
#pragma unroll
    for (int q = 0; q < NB; ++q) {
        const int s = q * kThreads + tid, row = s >> 3, kc = (s & 7) ^ swz(row);
        int64_t gn = n0 + row;
        if (gn >= p.N) gn = 0;
        bg[q] = static_cast<const char*>(p.B) + (gn * p.ldb + k0 + kc * CE) * EB;
        b2g[q] = (kc * CE < p.K2) ? static_cast<const char*>(p.B2) + (gn * p.ldb2 + kc * CE) * EB
                                  : static_cast<const char*>(p.zero);
    }

    auto issue = [&](char* st, int t) {
        if (t < Tm) {
#pragma unroll
            for (int q = 0; q < NA; ++q) dma16(ag[q] + (int64_t)t * (BKE * EB), st + (q * kThreads + wave * 64) * 16);
#pragma unroll
            for (int q = 0; q < NB; ++q) dma16(bg[q] + (int64_t)t * (BKE * EB), st + BM * kRow + (q * kThreads + wave * 64) * 16);
        } else {
#pragma unroll
            for (int q = 0; q < NA; ++q) dma16(a2g[q], st + (q * kThreads + wave * 64) * 16);
#pragma unroll
            for (int q = 0; q < NB; ++q) dma16(b2g[q], st + BM * kRow + (q * kThreads + wave * 64) * 16);
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](const char* As) {
        const char* Bs = As + BM * kRow;
        const int r = lane & 15, g = lane >> 4;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int kc = 4 * s + g;
            if constexpr (BF16) {
                bf16x8 af[FM], bfr[FN];
#pragma unroll
                for (int i = 0; i < FM; ++i) {
                    const int row = wm0 + 16 * i + r;
                    af[i] = *reinterpret_cast<const bf16x8*>(As + row * kRow + ((kc ^ swz(row)) << 4));
                }
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const int row = wn0 + 16 * j + r;
                    bfr[j] = *reinterpret_cast<const bf16x8*>(Bs + row * kRow + ((kc ^ swz(row)) << 4));
                }
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
            } else {
                f32x4 af[FM], bfr[FN];
#pragma unroll
                for (int i = 0; i < FM; ++i) {
                    const int row = wm0 + 16 * i + r;
                    af[i] = *reinterpret_cast<const f32x4*>(As + row * kRow + ((kc ^ swz(row)) << 4));
                }
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const int row = wn0 + 16 * j + r;
                    bfr[j] = *reinterpret_cast<const f32x4*>(Bs + row * kRow + ((kc ^ swz(row)) << 4));
                }
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int i = 0; i < FM; ++i)
#pragma unroll
                        for (int j = 0; j < FN; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][e], bfr[j][e], acc[i][j], 0, 0, 0);
            }
        }
    };

    // prologue: STAGES-1 tiles in flight; tile t always lives in stage t % STAGES
    static_for<STAGES - 1>([&](auto s) {
        if (decltype(s)::value < T) issue(stage(s), decltype(s)::value);
    });
    for (int t0 = 0; t0 < T; t0 += STAGES) {
        static_for<STAGES>([&](auto s) {
            const int t = t0 + decltype(s)::value;
            if (t >= T) return;
            // tile t has landed once at most min(STAGES-2, T-1-t) later tiles are outstanding
            const int later = min(STAGES - 2, T - 1 - t);
            if (later >= STAGES - 2) wait_vmcnt<(STAGES - 2) * LPT>();
            else if constexpr (STAGES >= 3) {
                if (later == 1) wait_vmcnt<LPT>();
                else wait_vmcnt<0>();
            } else {
                wait_vmcnt<0>();
            }
            // tile t visible to all waves; every wave is done with tile t-1. A bare s_barrier: the
            // fence __syncthreads adds would wait for every in-flight DMA (vmcnt 0), not just tile t.
            __asm__ volatile("s_barrier" ::: "memory");
            if (t + STAGES - 1 < T) issue(stage(IC<decltype(s)::value + STAGES - 1>{}), t + STAGES - 1);
            compute(stage(s));
        });
    }

    if (p.ws) {  // split-K partial sums
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
                    if (m < Mt) st_coherent(w + m * p.N + n, acc[i][j][v]);
                }
        }
        if (!p.counters) return;   // reduced by gemm_dma_splitk_reduce
        // The last split of this tile to arrive sums the partials in split order (deterministic:
        // independent of the arrival order) and runs the epilogue; nobody waits for anybody.
        __shared__ int s_last;
        if (!arrive_last(&p.counters[bid], (int)gridDim.y, &s_last)) return;
        const int splits = (int)gridDim.y;
        for (int e = tid; e < BM * BN; e += kThreads) {
            const int64_t m = m0 + e / BN, n = n0 + e % BN;
            if (m >= Mt || n >= p.N) continue;
            float sum = 0.f;
            for (int zz = 0; zz < splits; ++zz) sum += ld_coherent(p.ws + (int64_t)zz * Mt * p.N + m * p.N + n);
            epilogue_elem(p, m, n, sum);
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

__global__ __launch_bounds__(kThreads) void gemm_dma_splitk_reduce(DmaParams p, int splits) {
    const int64_t Mt = p.M + p.Mx;
    const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (idx >= Mt * p.N) return;
    float s = 0.f;
    for (int z = 0; z < splits; ++z) s += p.ws[(int64_t)z * Mt * p.N + idx];
    const int64_t m = idx / p.N, n = idx - m * p.N;
    epilogue_elem(p, m, n, s);
}

template <int BM, int BN, int WMW, int STAGES, bool BF16>
void launch_dma(sa3k_ctx* ctx, DmaParams p) {
    const int64_t tiles = ceil_div(p.M + p.Mx, BM) * ceil_div(p.N, BN);
    const int64_t grid = ceil_div(tiles, 8) * 8;
    const int KT = (int)(p.K / (BF16 ? 64 : 32));
    int splits = 1;
    const int64_t slots = (int64_t)256 * ctx->gemm_wg_per_cu;
    if (ctx->gemm_split && tiles < slots && KT >= 8)
        splits = (int)std::min<int64_t>({(int64_t)16, KT / 4, std::max<int64_t>(1, slots / tiles)});
    p.kps = std::max(1, (KT + splits - 1) / splits);
    splits = std::max(1, (KT + p.kps - 1) / p.kps);
    p.ws = nullptr;
    p.counters = nullptr;
    if (splits > 1) {
        p.ws = gemm_workspace_bytes(ctx, (size_t)splits * (size_t)(p.M + p.Mx) * (size_t)p.N * sizeof(float));
        if (ctx->gemm_fixup && tiles <= kMaxFixupTiles) p.counters = ctx->tile_counters;
    }
    dim3 g((unsigned)grid, (unsigned)splits);
    {
        // profiled per kernel instantiation, with its algorithmic flops (padding excluded)
        static const std::string name = std::string("gemm_dma<") + std::to_string(BM) + "," + std::to_string(BN) + "," +
                                        std::to_string(WMW) + "," + std::to_string(STAGES) + (BF16 ? ",bf16>" : ",f32>");
        KernelScope ks(ctx, name.c_str(), 2.0 * (double)(p.M + p.Mx) * (double)p.N * (double)(p.K + p.K2));
        gemm_dma_kernel<BM, BN, WMW, STAGES, BF16><<<g, kThreads, 0, ctx->stream>>>(p);
        SA3K_LAUNCHED();
    }
    if (splits > 1 && !p.counters) {
        KernelScope ks(ctx, "gemm_splitk_reduce");
        gemm_dma_splitk_reduce<<<(unsigned)ceil_div((p.M + p.Mx) * p.N, kThreads), kThreads, 0, ctx->stream>>>(p, splits);
    }
}

template <bool BF16>
void dispatch_dma(sa3k_ctx* ctx, const DmaParams& p) {
    const int64_t Mt = p.M + p.Mx;
    if (Mt <= 32) return launch_dma<32, 128, 1, 4, BF16>(ctx, p);
    if (p.N <= 32) return launch_dma<128, 32, 4, 4, BF16>(ctx, p);
    if (p.N <= 64) return launch_dma<128, 64, 4, 4, BF16>(ctx, p);
    switch (ctx->gemm_cfg) {
        case 1: return launch_dma<128, 128, 2, 4, BF16>(ctx, p);
        case 2: return launch_dma<256, 128, 2, 3, BF16>(ctx, p);
        case 3: return launch_dma<128, 256, 2, 3, BF16>(ctx, p);
        default: return launch_dma<128, 128, 2, 2, BF16>(ctx, p);   // 64 KiB LDS: two workgroups per CU
    }
}

}  // namespace

void gemm_run_dma(sa3k_ctx* ctx, const GemmDesc& d) {
    DmaParams p{d.A, d.lda, d.B, d.ldb, d.A2, d.lda2, d.B2, d.ldb2, d.K2, d.M, d.N, d.K, d.alpha,
                d.colscale, d.bias, d.C, d.ldc, d.accumulate, d.Cb, d.ldcb, d.U, d.Ub, d.ldu,
                d.Mx, d.Ax, d.ldax, d.A2x, d.lda2x, d.Cx, d.ldcx, d.accumulate_x, nullptr, 0, ctx->zero_page};
    if (d.prec == SA3K_PREC_BF16) dispatch_dma<true>(ctx, p);
    else dispatch_dma<false>(ctx, p);
}

}  // namespace sa3k
