// K1/K2: LDS-tiled MFMA GEMM for gfx950, C[M][N] = alpha * (A[M][K] . B[N][K]^T (+ A2 . B2^T)).
//
// Both operands are K-contiguous ("NT"): the frozen base weight W [out][in] is the B operand of
// the forward product X W^T, and its transposed copy W^T [in][out] (laid out once when the weight
// is loaded) is the B operand of dX = dU W. The B operand is decoded in the global->LDS path from
// its stored type (bf16, f16, f32, or Q8_0 quants + f16 scales) into the compute type, so a Q8_0 or
// f16 base is never expanded in HBM.
//
// Compute types: bf16 (v_mfma_f32_16x16x32_bf16, fp32 accumulation) and f32
// (v_mfma_f32_16x16x4_f32). Tiles: 256 threads = 4 wave64s; BK = 128 bytes of the compute type
// per row (64 bf16 or 32 f32); every LDS row is padded to 144 bytes; double-buffered LDS with one
// barrier per K step; each lane feeds the MFMAs from 16-byte LDS reads.
//
// The optional second segment (A2 [M][K2], B2 [N][K2], K2 <= one K tile, stored in the compute
// type) appends a rank-K2 product to the same accumulators: the LoRA term s.(X A^T) B^T of the
// forward and the (dU B) A term of dX ride on the base GEMM this way.
//
// Extra rows (Mx) let a rank-sized product that contracts the same B operand ride on the same
// GEMM: the DoRA term 2s B^T diag(gn) W of dA shares the W^T tiles of dX.
//
// Epilogue per column n: v = alpha*acc; U = v (optional pre-scale copy); v *= colscale[n] (unless
// prescale: then the main segment's accumulators were scaled before the second segment was added);
// v += bias[n]; C = v (or C += v); Cb = bf16(v).
#pragma once

#include "sa3k_internal.h"

namespace sa3k {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));

enum SrcType { SRC_BF16 = 0, SRC_F16 = 1, SRC_F32 = 2, SRC_Q8 = 3, SRC_Q8T = 4 };

// Per-head q/k preparation in a GEMM epilogue (the DiT's attention inputs, src/dit.h:207-217): the
// N = parts x dim output columns are parts k = 0 .. parts - 1 of dim columns each. Each 64-column
// head slice h of part k, taken as C receives it, is RMS-normed with the gain gamma[k] (null:
// copied as is), rotated by NeoX RoPE over rope_dims dims when rope[k] (table tab [Sx][rope_dims]:
// the half-pair cosines, then the sines), and stored bf16 to out[k] [B][H][Sx][64] (row m = b Sx +
// t); the norm's 1/rms goes to rstd[(m H + h) parts + k].
struct HeadPrep {
    int parts = 0, Sx = 0, H = 0, dim = 0, rope_dims = 0;
    float eps = 0.0f;
    const float* tab = nullptr;
    bf16* out[5] = {};
    const float* gamma[5] = {};
    int rope[5] = {};
    float* rstd = nullptr;
};

// The attention backward's inputs from the product that computes dO = the gradient of the attention
// output (rows b Sq + t, columns h 64 + d): dOh [B][H][Sq][64] = bf16(dO) and the row dots
// dn1/dn2 [B][H][Sq] = sum_d dO . o1/o2 over each head's 64 dims, o1/o2 [B][H][Sq][64] the two
// branch outputs of the forward.
struct AttnDot {
    const bf16* o1 = nullptr;
    const bf16* o2 = nullptr;
    bf16* doh = nullptr;
    float* dn1 = nullptr;
    float* dn2 = nullptr;
    int H = 0, Sq = 0;
};

// The SwiGLU backward of the FFN (src/dit.h:259-264) from the product that computes dG, the gradient
// of g = val * silu(glu) ([M][I]): with F = [val | glu] ([M][2 I] bf16), du [M][2 I] = bf16(dsc (.)
// [d val | d glu]) (dsc null: 1), the up-projection's output gradient as its backward reads it.
struct SwiBwd {
    const bf16* F = nullptr;
    bf16* du = nullptr;
    const float* dsc = nullptr;
    int64_t I = 0;
};

struct GemmDesc {
    int prec = SA3K_PREC_BF16;   // compute type
    int a_src = SRC_BF16;        // SRC_BF16 or SRC_F32
    int b_src = SRC_BF16;        // any SrcType
    const void* A = nullptr;     // [M][lda]
    int64_t lda = 0;
    const void* B = nullptr;     // [N][ldb] (Q8/Q8T: int8 quants)
    int64_t ldb = 0;
    const void* Bs = nullptr;    // Q8: f16 scales [N][ldbs] per 32 K; Q8T: [N/32][ldbs] per 32 N
    int64_t ldbs = 0;
    const void* A2 = nullptr;    // [M][lda2] compute type
    int64_t lda2 = 0;
    const void* B2 = nullptr;    // [N][ldb2] compute type
    int64_t ldb2 = 0;
    int K2 = 0;
    int64_t M = 0, N = 0, K = 0;
    float alpha = 1.0f;
    const float* colscale = nullptr;  // [N]
    const float* bias = nullptr;      // [N]
    float* C = nullptr;               // [M][ldc]
    int64_t ldc = 0;
    int accumulate = 0;               // C += v
    bf16* Cb = nullptr;               // [M][ldcb]
    int64_t ldcb = 0;
    float* U = nullptr;               // [M][ldu] pre-colscale copy (f32)
    bf16* Ub = nullptr;               // [M][ldu] pre-colscale copy (bf16)
    int64_t ldu = 0;
    // Mx extra rows appended below A (compute type, [Mx][ldax]), with their own second-segment rows
    // A2x [Mx][lda2x]; their results go to Cx [Mx][ldcx] (+= when accumulate_x) without the
    // epilogue's colscale/bias. They share every B tile with the main rows.
    int64_t Mx = 0;
    const void* Ax = nullptr;
    int64_t ldax = 0;
    const void* A2x = nullptr;
    int64_t lda2x = 0;
    float* Cx = nullptr;
    int64_t ldcx = 0;
    int accumulate_x = 0;
    bf16* Cbx = nullptr;   // instead of Cx: extra rows stored as bf16 [Mx][ldcx] (no accumulation)
    // Nx extra columns appended after B's N rows (bf16, [Nx][ldbx], K-contiguous; DMA-fed kernels,
    // no second segment): they share every A tile with the main columns, and alpha_x times their
    // sums goes to Cbn [M][ldcn] as bf16, without colscale, bias, U or accumulation. The corner of
    // extra rows and extra columns is not stored.
    // 1: B is stored [K][ldb] (N contiguous: the dX product dU W reads W [out][in] as it lies);
    // bf16 on the DMA-fed kernels, no second segment and no extra columns
    int b_kn = 0;
    int64_t Nx = 0;
    const void* Bx = nullptr;
    int64_t ldbx = 0;
    float alpha_x = 1.0f;
    bf16* Cbn = nullptr;
    int64_t ldcn = 0;
    // 1: colscale multiplies the main segment A . B^T only, before the second segment is added
    // (C = colscale (.) (A B^T) + A2 B2^T); needs colscale, no extra rows and no U / Ub copies
    int prescale = 0;
    // Paired SwiGLU epilogue (the DiT FFN up-projection, src/dit.h:259-264): the N = 2 sw_half
    // output columns are [val | glu]. Where the chosen tiles allow it (bf16 256-column tiles, no
    // split over K, the staged epilogue), a tile holds columns [c, c + 128) of both halves and also
    // writes sw_g [M][sw_ldg] = bf16(val * glu * sigmoid(glu)) from its final values; *sw_done is
    // set then (else the caller applies SwiGLU itself). C, U and every other output are unchanged.
    int64_t sw_half = 0;
    bf16* sw_g = nullptr;
    int64_t sw_ldg = 0;
    int* sw_done = nullptr;
    // Per-head q/k preparation (HeadPrep; parts 0: off) where the chosen tiles allow it (bf16
    // 128 x 256 tiles, no split over K, the staged epilogue, dim a multiple of 256); *hp_done is
    // set then (else the caller prepares the heads itself). C and every other output unchanged.
    HeadPrep hp;
    int* hp_done = nullptr;
    // 1: C is written only where neither the SwiGLU nor the head preparation epilogue applies (the
    // callers that keep a bf16 copy Cb for later passes need the f32 C only for their own
    // separate SwiGLU / head preparation kernels)
    int c_unfused_only = 0;
    // Backward epilogues that write what the consumer of C needs in place of C: the attention dO
    // epilogue (AttnDot; doh null: off; N = H 64, M = B Sq) and the SwiGLU backward (SwiBwd; du
    // null: off; N = I), where the chosen tiles allow it (the bf16 DMA kernels' staged epilogues, no
    // split over K, no accumulation; the attention dots on tiles of 64 or more columns). C is then
    // not written and *bwd_done is set; else C is written and the caller computes them from it.
    AttnDot ad;
    SwiBwd sb;
    int* bwd_done = nullptr;
};

// Enqueue one GEMM on the context stream (validates shapes, picks the kernel and tile
// configuration): operands already in the compute type take the DMA-fed kernel (gemm_dma.hip),
// any other source type the kernel that decodes it on its way into LDS (gemm.hip).
void gemm_run(sa3k_ctx* ctx, const GemmDesc& d, const char* prof_name);
void gemm_run_dma(sa3k_ctx* ctx, const GemmDesc& d);
// whether Nx extra output columns ride on a bf16 Mt x N x K product without another round of
// workgroups
bool gemm_extra_cols_free(const sa3k_ctx* ctx, int64_t Mt, int64_t N, int64_t K, int64_t Nx);
// bf16 products with at most 32 output columns and a plain epilogue (gemm_skinny.hip)
bool gemm_skinny_ok(const sa3k_ctx* ctx, const GemmDesc& d);
void gemm_run_skinny(sa3k_ctx* ctx, const GemmDesc& d);
// split-K partial-sum workspace owned by the context (grows on demand)
float* gemm_workspace_bytes(sa3k_ctx* ctx, size_t bytes);
// The most f32 partial sums a split plan of the dispatch's own choosing writes: it splits only
// while splits x tiles <= the launch's resident workgroup slots, and every tile family keeps slots x
// tile area <= 2^24 (512 x 128 x 128, 256 x 128 x 256, 256 x 256 x 256; checked at compile time
// per instantiation). Forced splits (option gemm_splits) or slot counts (gemm_wg_per_cu) may exceed it.
constexpr int64_t kMaxSplitFloats = (int64_t)1 << 24;
// Look up this device's copy of the allocation-free entry point's scratch array (once per
// device, with the context's device current) and keep its address in the context.
void gemm_noalloc_setup(sa3k_ctx* ctx);

}  // namespace sa3k
