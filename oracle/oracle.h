/* oracle — CPU restatement of sa3.cpp's DiT LoRA/DoRA training-update math.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load this library, and only as the checker (or the timed CPU baseline), never as part of
 * the product path. The product (sa3.cpp_amd/libsa3k.so) never links or calls it.
 *
 * Each function names the reference file:line it restates. The reference's own implementation
 * (header-only C++ over the un-vendored ggml fork betweentwomidnights/ggml tag
 * sa3-training-v1-metal, commit 922875a6) cannot be compiled here, so this is a from-scratch
 * restatement: float loops where the reference is a host float loop (optimizer, clip, quantizer),
 * double accumulation where the reference is a ggml graph (dit_lin, attention, block), so that the
 * oracle is closer to the exact value than any single-precision implementation.
 *
 * Pinning (how each part is checked beyond restating it) is listed per function in the test
 * files; parts without an independent check say "parity unpinned".
 */
#ifndef SA3_ORACLE_H
#define SA3_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- optimizer (src/train_optimizer.h, src/train_loop.h) ---- */
float orc_inverse_lr(float base_lr, int step0, float inv_gamma, float power, float warmup, float final_lr);
/* adamw_update_vector on one tensor; returns 0 ok, 1 size/step error (src/train_optimizer.h:42-66) */
int orc_adamw_update_vector(float* param, const float* grad, float* m, float* v, int64_t n,
                            float lr, float b1, float b2, float eps, float wd, int step);
/* train_average_and_clip over tensors laid end to end in the order the reference visits them
 * (A, B, mxs, mag, mag_r, mag_c per target): grad is modified in place like accum is.
 * (src/train_loop.h:147-171) */
void orc_average_and_clip(float* grad, int64_t n, int count, float grad_clip, double* norm_out,
                          float* scale_out);
/* train_apply_accumulated_adamw on a flat arena (src/train_loop.h:173-211). grad is modified
 * (averaged/clipped) like the reference modifies its accumulator. */
int orc_apply_accumulated_adamw(float* param, float* grad, float* m, float* v, int64_t n,
                                float lr, float b1, float b2, float eps, float wd, float clip,
                                int step, int count, double* norm_out, float* scale_out);

/* ---- Q8_0 / f16 (ggml block_q8_0, quantize_row_q8_0_ref, dequantize_row_q8_0) ---- */
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_f16_row(const float* x, uint16_t* y, int64_t n);
void orc_f16_to_f32_row(const uint16_t* x, float* y, int64_t n);
void orc_q8_0_quantize(const float* x, void* blocks, int64_t n);
void orc_q8_0_dequant(const void* blocks, float* y, int64_t n);

/* ---- adapter state (src/train_lora.h) ---- */
/* W [out][in] f32 (an f16 or Q8_0 base is decoded first). */
void orc_row_norm_sq(const float* W, int64_t in, int64_t out, float eps, float* nsq);  /* :160-174 */
void orc_row_norms(const float* W, int64_t in, int64_t out, float* norms);               /* :141-155 */
/* materialised effective weight (train_lora_effective_weight, :301-329) for lora / dora-rows */
void orc_effective_weight(const float* W, int64_t in, int64_t out, const float* A, const float* B,
                          const float* mag, int rank, float alpha, int dora, float* Weff);

/* ---- dit_lin (src/dit.h:92-149) forward and closed-form backward, double accumulation ----
 * X [N][in], W [out][in], A [r][in], B [out][r], mag/bnsq [out], bias [out] or NULL, s = alpha/r.
 * fwd writes Y [N][out] and (nullable) U [N][out] (pre-row-scale) and dscale [out] (m/sqrt(nsq),
 * or 1 for lora) and nsq [out]. */
void orc_dit_lin_fwd(const float* X, int64_t N, const float* W, int64_t in, int64_t out,
                     const float* A, const float* B, int rank, float s, int dora, const float* mag,
                     const float* bnsq, const float* bias, float* Y, float* U, float* dscale,
                     float* nsq_out);
/* sum (Y - tgt)^2 with Y in double (finite-difference checks) */
double orc_dit_lin_sqloss(const float* X, int64_t N, const float* W, int64_t in, int64_t out,
                          const float* A, const float* B, int rank, float s, int dora, const float* mag,
                          const float* bnsq, const float* bias, const float* tgt);
/* bwd from dY [N][out]: dX [N][in], dA [r][in], dB [out][r], dm [out] (dora; nullable otherwise).
 * Any output pointer may be NULL to skip it. */
void orc_dit_lin_bwd(const float* X, int64_t N, const float* W, int64_t in, int64_t out,
                     const float* A, const float* B, int rank, float s, int dora, const float* mag,
                     const float* bnsq, const float* dY, float* dX, float* dA, float* dB, float* dm);
/* plain double-accumulated products used by tests: C[M][N] = A[M][K] * B[N][K]^T */
void orc_gemm_nt(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K);

/* ---- composed adapter chains over a frozen base (src/lora.h:111-143, 372-622; src/dit.h:108-117) ---- */
typedef struct {
    int dora;            /* 0: lora, 1: dora-rows */
    int rank;
    float alpha, strength;   /* residual scale (alpha / rank) * strength; strength 0 skips the adapter */
    const float* A;      /* [rank][in] */
    const float* B;      /* [out][rank] */
    const float* mag;    /* [out] (dora-rows) */
} orc_chain_adapter;
/* sequential merge of the chain into W_eff [out][in] (apply_loras for lora / dora-rows) */
void orc_chain_merge(const float* W, int64_t in, int64_t out, int n, const orc_chain_adapter* ad, float* Weff);
/* build_functional_lora's constants: base_scale [out]; Bp [out][R] = the active adapters' row-scaled B'
 * side by side in chain order (R = sum of their ranks); scales [n_active] = (alpha/rank)*strength */
void orc_chain_fold(const float* W, int64_t in, int64_t out, int n, const orc_chain_adapter* ad, float* base_scale,
                    float* Bp, float* scales);
/* the composed functional forward Y [N][out] = base_scale * (X W^T) + sum_k s_k (X A_k^T) B'_k^T (+ bias) */
void orc_chain_forward(const float* X, int64_t N, const float* W, int64_t in, int64_t out, int n,
                       const orc_chain_adapter* ad, const float* bias, float* Y);

/* ---- differential attention (src/dit.h:151-158, src/nn.h:135-144), double accumulation ----
 * Q1, Q2 [BH][Sq][D]; K1, K2, V [BH][Sk][D]; window 0 = dense, else |i-j| <= window/2.
 * fwd: O = O1 - O2 [BH][Sq][D] (O1, O2, lse1, lse2 [BH][Sq] nullable; lse natural log of the
 * scaled-score softmax denominator). bwd from dO: dQ1, dK1, dQ2, dK2, dV. */
void orc_diff_attn_fwd(const float* Q1, const float* K1, const float* Q2, const float* K2, const float* V,
                       int BH, int Sq, int Sk, int D, float scale, int window, float* O, float* O1, float* O2,
                       float* lse1, float* lse2);
void orc_diff_attn_bwd(const float* Q1, const float* K1, const float* Q2, const float* K2, const float* V,
                       const float* dO, int BH, int Sq, int Sk, int D, float scale, int window, float* dQ1,
                       float* dK1, float* dQ2, float* dK2, float* dV);

/* ---- one DiT block (src/dit.h:164-266), batch-major tokens [B][S][dim] ---- */
typedef struct orc_block {
    int B, S, Ctx, dim, heads, inner, rope_dims, window;
    float rope_base, norm_eps, qk_eps;
    const float *ssg, *pre_g, *cross_g, *ff_g, *sq_g, *sk_g, *cq_g, *ck_g;
    /* 7 targets: 0 self.qkv, 1 self.out, 2 cross.q, 3 cross.kv, 4 cross.out, 5 ff.proj, 6 ff.out */
    const float* W[7];
    const float* bias[7];
    const float* A[7];
    const float* Bm[7];
    const float* mag[7];
    const float* bnsq[7];
    int rank, dora;
    float scale;
    /* inpaint local add (src/dit.h:244-254), NULL when absent: ladd [B][S][dim] is added to the
     * residual after the cross-attention (memory rows hold zeros); the backward writes the
     * gradient of that sum (the feed-forward input) to dladd [B][S][dim] when non-NULL */
    const float* ladd;
    float* dladd;
} orc_block;
/* the block's NEOX rotary (rope_dims of each 64-wide head vector, positions pos[j]), exported for tests */
void orc_rope_neox(float* v, int n, int rope, const float* pos, float base);
void orc_block_fwd(const orc_block* p, const float* x, const float* ctx, const float* gcond, float* out);
void orc_block_bwd(const orc_block* p, const float* x, const float* ctx, const float* gcond, const float* dout,
                   float* dx, float* dctx, float* dgcond, float* const* dA, float* const* dB, float* const* dm);

/* ---- the whole DiT training loss (dit_head / dit_block x depth / dit_tail, src/dit.h:269-338,
 * loss src/train_dit.h:174-184), batch-major ---- */
typedef struct orc_lin {
    const float *W, *bias, *A, *B, *mag, *bnsq;   /* A/B NULL: no adapter (plain mul_mat) */
    int in, out;
} orc_lin;
/* head/tail linears, in this order */
enum { ORC_PRE_CONV, ORC_PROJ_IN, ORC_TIME0, ORC_TIME2, ORC_GLOBAL0, ORC_GLOBAL2, ORC_GCE0, ORC_GCE2,
       ORC_COND0, ORC_COND2, ORC_PROJ_OUT, ORC_POST_CONV, ORC_NHEAD };
typedef struct orc_dit {
    int B, T, Ctx, io, dim, heads, inner, depth, mem, cond_dim, time_dim, rope_dims, window;
    float rope_base, norm_eps, qk_eps, time_min_freq, time_max_freq;
    const orc_block* blocks;     /* depth blocks: W/bias/vectors/adapters (their B/S/Ctx are ignored) */
    orc_lin head[ORC_NHEAD];
    const float* memory_tokens;  /* [mem][dim] */
    int rank, dora;
    float scale;
    /* inpaint local conditioning (src/dit.h:244-254): local [depth*2] = per block local.0
     * (local_dim -> dim, bias) and local.2 (dim -> dim, bias); local_cond [B][T][local_dim]. Both
     * NULL (or local_dim 0): no local add. The local linears' adapters follow the blocks' rules. */
    int local_dim;
    const orc_lin* local;
    const float* local_cond;
} orc_dit;
/* Forward to the per-sample losses (loss [B]) and, if dA_* is non-NULL, the backward: adapter
 * gradients of sum_b loss_b ADDED to dA/dB/dm (blocks: [depth*7], head: [ORC_NHEAD], local:
 * [depth*2] (NULL arrays allowed when there is no local add), entries of un-adapted linears
 * ignored). x_t, target [B][T][io]; t [B]; cross [B][Ctx][cond_dim]; glob
 * [B][cond_dim]; loss_weight [B][T] or NULL (uniform 1/(io*T)); velocity [B][T][io] nullable. */
void orc_dit_loss(const orc_dit* p, const float* x_t, const float* target, const float* t, const float* cross,
                  const float* glob, const float* loss_weight, float* velocity, double* loss,
                  float* const* dA_blocks, float* const* dB_blocks, float* const* dm_blocks,
                  float* const* dA_head, float* const* dB_head, float* const* dm_head,
                  float* const* dA_local, float* const* dB_local, float* const* dm_local);
/* ExpoFourierFeatures of t into out[dim] (expo_features, src/sa3_pipeline.h:57-67) */
void orc_expo_features(float t, float* out, int dim, float min_f, float max_f);

int orc_num_threads(void);

/* 1: the linears (orc_dit_lin_*, and through them the block and DiT functions) and the attention
 * compute in float, with AVX2/FMA products where orc_f32_fast() says the CPU has them: the CPU
 * baseline's mode. 0 (the default): double, the pinned oracle. Not thread-safe; set it between
 * calls. */
void orc_set_f32(int on);
int orc_f32_fast(void);

#ifdef __cplusplus
}
#endif

#endif
