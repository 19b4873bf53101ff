// Skinny NT product C[Mt][n] = alpha * A[Mt][K] . B[n][K]^T for n <= 32 output columns, both
// operands bf16: the rank-sized products of the adapted linear, s X A^T (forward, K = in) and
// s dU B (backward, K = out, with the r DoRA rows s (B^T diag(gn) B) appended as extra A rows).
//
// These contract a long K into a few columns: the work is reading A once (2176 x 1536..12288 bf16
// at the DiT's size). The tiled GEMM covers the chip with 128 x 32 tiles split over K plus a
// separate reduction launch. Here no workgroup depends on another:
//  * a workgroup owns 16 rows and 16 output columns (one v_mfma_f32_16x16x32_bf16 block) and the
//    whole K range; its 8 waves take the 64-wide K chunks round-robin and sum their tiles through
//    LDS in wave order at the end (deterministic);
//  * the two 16-column halves of a row tile are launched on the same XCD (block b runs on XCD
//    b % 8), so the second reads the A rows from that XCD's L2;
//  * operands come straight from global memory in the MFMA's own layout: lane l feeds row l % 16
//    with the 8 K elements [32 q + 8 (l / 16), +8) of step q, so the four lanes of a row read one
//    contiguous 64-byte sector per load instruction. Nothing is reused, so nothing is staged in LDS;
//  * each wave keeps two groups of 4 chunks in flight: the loads of group i + 1 are issued before
//    the MFMAs of group i wait for theirs.
#include "gemm.h"

namespace sa3k {

namespace {

constexpr int kSkWaves = 8;
constexpr int kSkThreads = kSkWaves * 64;
constexpr int kSkRows = 16;
constexpr int kSkCols = 16;          // per workgroup; a product has at most 2 column halves
constexpr int kSkGroup = 4;          // 64-wide K chunks per load group
constexpr int64_t kSkMaxK = 3072;    // longer K stays on the tiled kernel

struct SkinnyParams {
    const bf16* A; int64_t lda; int64_t M;
    const bf16* Ax; int64_t ldax; int64_t Mx;
    const bf16* B; int64_t ldb; int n;
    int KC;          // 64-wide K chunks
    int halves;      // column halves (1 or 2)
    int64_t tiles;   // 16-row tiles
    float alpha;
    float* C; bf16* Cb; int64_t ldc;
    float* Cx; bf16* Cbx; int64_t ldcx;
};

struct Group {
    bf16x8 a[kSkGroup][2], b[kSkGroup][2];
};

__global__ __launch_bounds__(kSkThreads) void skinny_nt_kernel(SkinnyParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    // block -> (row tile, column half): both halves of a tile on the XCD of (tile % 8)
    int64_t tile;
    int half;
    if (p.halves == 2) {
        const int64_t b = blockIdx.x;
        tile = (b / 16) * 8 + (b % 8);
        half = (int)((b / 8) % 2);
    } else {
        tile = blockIdx.x;
        half = 0;
    }
    if (tile >= p.tiles) return;
    const int64_t Mt = p.M + p.Mx;
    const int64_t row0 = tile * kSkRows;

    // the A row this lane feeds (clamped rows feed results that are never stored) and the B row
    // of output column half*16 + r (clamped to the last valid column)
    int64_t row = row0 + r;
    if (row >= Mt) row = Mt - 1;
    const bf16* arow = (row < p.M ? p.A + row * p.lda : p.Ax + (row - p.M) * p.ldax) + 8 * g;
    const bf16* brow = p.B + (int64_t)min(half * kSkCols + r, p.n - 1) * p.ldb + 8 * g;

    auto load = [&](Group& G, int c0) {   // chunks c0, c0 + 8, ... of this wave (c0 wave-uniform)
#pragma unroll
        for (int u = 0; u < kSkGroup; ++u) {
            const int c = c0 + u * kSkWaves;
            if (c < p.KC) {
                const int64_t k = (int64_t)c * 64;
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    G.a[u][q] = *reinterpret_cast<const bf16x8*>(arow + k + 32 * q);
                    G.b[u][q] = *reinterpret_cast<const bf16x8*>(brow + k + 32 * q);
                }
            } else {
#pragma unroll
                for (int q = 0; q < 2; ++q)
#pragma unroll
                    for (int e = 0; e < 8; ++e) G.a[u][q][e] = G.b[u][q][e] = (bf16)0.f;
            }
        }
    };
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    auto mma = [&](const Group& G) {
#pragma unroll
        for (int u = 0; u < kSkGroup; ++u)
#pragma unroll
            for (int q = 0; q < 2; ++q) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(G.a[u][q], G.b[u][q], acc, 0, 0, 0);
    };
    constexpr int STEP = kSkWaves * kSkGroup;   // chunks per group over all waves
    Group g0, g1;
    int c = wave;
    load(g0, c);
    while (true) {
        if (c + STEP < p.KC) load(g1, c + STEP);
        mma(g0);
        c += STEP;
        if (c >= p.KC) break;
        if (c + STEP < p.KC) load(g0, c + STEP);
        mma(g1);
        c += STEP;
        if (c >= p.KC) break;
    }

    // wave tiles [wave][16][16]: register v of lane l holds row 4 (l / 16) + v, column l % 16
    __shared__ float red[kSkWaves][kSkRows * kSkCols];
#pragma unroll
    for (int v = 0; v < 4; ++v) red[wave][(4 * g + v) * kSkCols + r] = acc[v];
    __syncthreads();
    const int t = threadIdx.x;
    if (t >= kSkRows * kSkCols) return;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kSkWaves; ++w) s += red[w][t];
    s *= p.alpha;
    const int64_t m = row0 + t / kSkCols;
    const int col = half * kSkCols + t % kSkCols;
    if (m >= Mt || col >= p.n) return;
    if (m < p.M) {
        if (p.Cb) p.Cb[m * p.ldc + col] = (bf16)s;
        else p.C[m * p.ldc + col] = s;
    } else {
        if (p.Cbx) p.Cbx[(m - p.M) * p.ldcx + col] = (bf16)s;
        else p.Cx[(m - p.M) * p.ldcx + col] = s;
    }
}

}  // namespace

bool gemm_skinny_ok(const sa3k_ctx* ctx, const GemmDesc& d) {
    if (d.prescale || d.Nx > 0 || d.b_kn) return false;
    if (!ctx->gemm_skinny) return false;
    if (d.prec != SA3K_PREC_BF16 || d.a_src != SRC_BF16 || d.b_src != SRC_BF16) return false;
    if (d.N > 2 * kSkCols || d.K2 != 0 || d.K % 64 != 0 || d.K == 0) return false;
    // Measured on MI355X (2176 rows): faster than the split-K tiled kernel up to K = 3072 (K 1536:
    // 7.9 vs 9.3 us), slower beyond (each wave's load groups run one memory round trip apart)
    if (d.K > kSkMaxK) return false;
    if (d.colscale || d.bias || d.U || d.Ub || d.accumulate || d.accumulate_x) return false;
    if ((d.C != nullptr) == (d.Cb != nullptr)) return false;   // exactly one main output
    if (d.Mx > 0 && (d.Cx != nullptr) == (d.Cbx != nullptr)) return false;
    // 16-byte operand loads
    auto al16 = [](const void* q, int64_t ld) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0 && (ld * 2) % 16 == 0; };
    return al16(d.A, d.lda) && al16(d.B, d.ldb) && (d.Mx == 0 || al16(d.Ax, d.ldax));
}

void gemm_run_skinny(sa3k_ctx* ctx, const GemmDesc& d) {
    const int64_t Mt = d.M + d.Mx;
    const int64_t tiles = ceil_div(Mt, kSkRows);
    const int halves = d.N > kSkCols ? 2 : 1;
    // with two halves the grid is padded to whole groups of 8 tiles (blocks past the tiles exit)
    const int64_t blocks = halves == 2 ? ceil_div(tiles, 8) * 16 : tiles;
    SkinnyParams p{static_cast<const bf16*>(d.A), d.lda, d.M, static_cast<const bf16*>(d.Ax), d.ldax, d.Mx,
                   static_cast<const bf16*>(d.B), d.ldb, (int)d.N, (int)(d.K / 64), halves, tiles, d.alpha,
                   d.C, d.Cb, d.Cb ? d.ldcb : d.ldc, d.Cx, d.Cbx, d.ldcx};
    KernelScope ks(ctx, "skinny_nt", 2.0 * (double)Mt * (double)d.N * (double)d.K);
    launch_k(ctx, true, skinny_nt_kernel, dim3((unsigned)blocks), dim3(kSkThreads), 0, p);
    SA3K_LAUNCHED();
}

}  // namespace sa3k
