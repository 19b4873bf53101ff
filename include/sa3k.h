/* sa3k — C ABI of the MI355X (gfx950) kernels behind sa3.cpp's DiT LoRA/DoRA training update.
 *
 * The reference runs this path as ggml graphs (src/train_ckpt.h:143-474 builds them,
 * src/train_loop.h:309-441 executes them, src/train_loop.h:147-211 + src/train_optimizer.h:42-66
 * apply the clip and AdamW on the host). There is no training entry in the reference's own C ABI
 * (src/libsa3.h:163-191 is inference only), so this header is a new thin layer that follows
 * libsa3's conventions:
 *
 *   Lifecycle:  sa3k_create() -> sa3k_* calls -> sa3k_destroy().
 *   Ownership:  device buffers come from sa3k_malloc() and are released with sa3k_free(); opaque
 *               objects (weights, linears) have their own *_destroy().
 *   Threading:  a context owns one HIP device and one stream. It is NOT reentrant: serialise calls
 *               per context (libsa3 contract, src/libsa3.h:8).
 *   Ordering:   every compute call is enqueued on the context stream and returns before the GPU is
 *               done, except calls that hand a host scalar back (documented per call), which
 *               synchronise the stream.
 *   Errors:     no C++ exception crosses this boundary. Every call returns SA3K_OK (0) or a non-zero
 *               code; sa3k_last_error() returns the message of the last failure on that context
 *               (libsa3 copies messages into `err`, src/libsa3.cpp:25-27; sa3k_create() does the same
 *               since there is no context yet).
 *
 * Layout conventions (PyTorch order; ggml `ne` is the reverse):
 *   weight W   [out][in]  row-major (ggml ne=[in,out], src/train_lora.h:149-151)
 *   activation X [N][in] token-major (ggml ne=[in,N])
 *   lora_A     [rank][in] row-major (src/train_lora.h:26)
 *   lora_B     [out][rank] row-major (src/train_lora.h:27)
 *   magnitude  [out]     (dora-rows, src/train_lora.h:31)
 */
#ifndef SA3K_H
#define SA3K_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SA3K_API __attribute__((visibility("default")))

enum {
    SA3K_OK = 0,
    SA3K_ERR_INVALID = 1,     /* bad argument (shape, null pointer, size mismatch, step <= 0 ...) */
    SA3K_ERR_DEVICE = 2,      /* HIP runtime failure */
    SA3K_ERR_NOMEM = 3,       /* device allocation failed */
    SA3K_ERR_UNSUPPORTED = 4  /* shape/type combination the kernels do not implement */
};

/* Element / block types of a frozen base weight (the GGUF tensor types the path reads). */
enum {
    SA3K_TYPE_F32 = 0,
    SA3K_TYPE_F16 = 1,
    SA3K_TYPE_Q8_0 = 8,   /* 32-element blocks {f16 d; int8 qs[32]} = 34 bytes, ggml block_q8_0 */
    SA3K_TYPE_BF16 = 30
};

/* Arithmetic of the contractions. */
enum {
    SA3K_PREC_F32 = 0,    /* fp32 MFMA, fp32 operands (1e-4 gradient tolerance) */
    SA3K_PREC_BF16 = 1    /* bf16 MFMA operands, fp32 accumulation */
};

typedef struct sa3k_ctx sa3k_ctx;

/* ---------------------------------------------------------------- context / memory */

/* Create a context on HIP device `device` with its own stream. Returns NULL on failure and copies
 * the message into err (err_len bytes, NUL-terminated), like sa3_init (src/libsa3.h:163). */
SA3K_API sa3k_ctx* sa3k_create(int device, char* err, int err_len);
SA3K_API void sa3k_destroy(sa3k_ctx* ctx);
SA3K_API const char* sa3k_last_error(const sa3k_ctx* ctx);
SA3K_API const char* sa3k_version(void);

SA3K_API int sa3k_malloc(sa3k_ctx* ctx, size_t bytes, void** out);
SA3K_API int sa3k_free(sa3k_ctx* ctx, void* ptr);
/* Stream-ordered copies; host memory may be pageable. Both return once the copy is enqueued
 * (upload) or complete (download: synchronises the stream). */
SA3K_API int sa3k_upload(sa3k_ctx* ctx, void* dst_dev, const void* src_host, size_t bytes);
SA3K_API int sa3k_download(sa3k_ctx* ctx, void* dst_host, const void* src_dev, size_t bytes);
SA3K_API int sa3k_copy_d2d(sa3k_ctx* ctx, void* dst_dev, const void* src_dev, size_t bytes);
SA3K_API int sa3k_memset(sa3k_ctx* ctx, void* dst_dev, int value, size_t bytes);
SA3K_API int sa3k_sync(sa3k_ctx* ctx);
/* Free and total device memory of the context's GPU (hipMemGetInfo). No reference counterpart:
 * the host mirror's build_train_dit_ckpt uses it to choose the schedule that fits. */
SA3K_API int sa3k_device_memory(sa3k_ctx* ctx, size_t* free_bytes, size_t* total_bytes);
/* dst[i] += src[i] in f32 for n device floats (16-byte aligned): train_accum_add
 * (src/train_loop.h:75-78) on the device, the host mirror's device-resident gradient accumulator. */
SA3K_API int sa3k_vec_add(sa3k_ctx* ctx, float* dst_dev, const float* src_dev, int64_t n);

/* Implementation knobs of a context (no reference counterpart; for tests and measurement):
 *   "gemm_split"  1: split K when a GEMM's output tiles cannot fill the chip (default 1)
 *   "gemm_fixup"  1: split partial sums are reduced by the last split to arrive, in split order,
 *                 inside the producing kernel; 0: by a separate reduction launch; 2: in-kernel for
 *                 outputs of at most 2^18 floats, a separate launch for larger ones (default 0)
 *   "gemm_dma"    1: DMA-fed kernel for compute-type operands (default 1)
 *   "gemm_dq"     1: bf16 products with an f16 or Q8_0 B operand (no extra rows or columns) run on the
 *                 DMA-fed kernel, B staged in LDS as stored and decoded between LDS and the MFMAs
 *                 (2: the same with 2 x 4 waves per tile instead of 1 x 8); 0: the kernel that
 *                 decodes on the way into LDS (default 1; all decode to the same bf16 values, the
 *                 last one's tiles sum in another order)
 *   "gemm_cfg"    DMA kernel tile configuration: 0 (default) 128 x 256 tiles of 16 waves for bf16
 *                 (and 16-wave 256 x 256 tiles where those are taken) and 128 x 128 for f32;
 *                 1: 128 x 128; 4: 128 x 256 and 256 x 256 of 8 waves (3 / 2 stages);
 *                 7: 128 x 256 of 8 waves (2 stages)
 *   "gemm_small"  DMA kernel tile configuration for GEMMs whose 128x128 grid cannot fill the chip
 *                 (default 4: bf16 128x128 tiles of eight waves at any K, f32 and decoded B 64x128
 *                 below K 2048 / 4096; 2: 64x128 tiles below those K; 0: the default tile, split
 *                 over K)
 *   "gemm_nt_store" 1: GEMM outputs are written with non-temporal stores (default 1)
 *   "gemm_skinny" 1: bf16 products with at most 32 output columns and a plain epilogue (the rank
 *                 products s X A^T and s dU B) run on a kernel that splits K across the waves of
 *                 one workgroup instead of over workgroups (default 1)
 *   "gemm_big"    bf16 products on 256 x 256 tiles (8 waves, one workgroup per CU): 0 never,
 *                 1 where they fill the chip about as evenly as 128 x 256 tiles, 2 always (when
 *                 operand extents and output alignment allow), 3 as 1 plus every product with
 *                 K >= 8192, split over K (default 3)
 *   "gemm_splits" > 0: the split-K count of DMA-fed GEMMs that split, in place of the one chosen
 *                 from the grid (clamped to the number of K tiles; default 0: chosen)
 *   "side_stream" 1: independent kernels of a backward pass (column reductions, attention dQ, the
 *                 context K/V projection) run on a second stream of the context beside the main
 *                 one, joined before the call returns (default 1; off while a profiler scope is
 *                 open)
 *   "fork_tail"   1: the second stream waits on the completion event of the kernel that produces
 *                 its inputs (recorded by that kernel's launch) rather than on a separate event
 *                 record on the main stream (default 1)
 *   "late_join"   1: in a DiT backward over resident activations, the second-stream work at the
 *                 end of one block (its last column reduction and dA sums) runs beside the next
 *                 block, which waits for it only before it rewrites the scratch that work reads
 *                 (default 1)
 *   "lin_merge"   1: a bf16-precision adapted linear prepared from now on contracts the merged
 *                 weight W + s B A, rounded once to bf16 and refreshed by every prepare, in its
 *                 forward and dX products (the rank products s X A^T and s dU B then only feed
 *                 the adapter gradients and run beside them); 0: the base and the rank term as two
 *                 segments of one product (default 1). It holds for a linear or linear group from
 *                 its next prepare (a DiT: from its setup).
 *   "rank_cols"   bit 0: a merged linear's rank product s X A^T rides on its forward product as r
 *                 extra output columns where they cost it no extra round of workgroups (default 1);
 *                 bit 1: likewise s dU B on its dX product (default 0: measured slower on MI355X
 *                 than the separate product beside it; with merge_kn 1 it needs in % 64 == 0)
 *   "tn_fuse"     bit mask of split reductions summed by their own last split to arrive instead of
 *                 a separate launch (each stream has its own arrival counters): 1 the block's
 *                 modulation-gradient column sums, 2 an adapted linear's dA sums, 4 an adapted
 *                 linear's dU column reduction with its per-row step (dm, dB, the dA rows operand)
 *                 (default 5)
 *   "kv_stack"    1: a DiT set up from now on computes its blocks' context K/V projections (one
 *                 shared input) as one product over their stacked merged weights, with the rank
 *                 products as its extra columns; each block's backward stays its own (default 1)
 *   "merge_kn"    1: a merged linear's dX product reads W + s B A in its stored [out][in] layout as
 *                 a K-major operand (transposed by the LDS reads), so the refresh writes one bf16
 *                 copy; 0: the refresh also writes the transposed copy [in][out] and dX reads
 *                 that (default 1). It holds from a linear's next prepare (a DiT: its setup).
 *   "attn_fwd32"  1: attention forwards over more than 128 keys run on 32x32x16 MFMA blocks with
 *                 one branch per wave; 0: every forward on the 16x16x32 kernel that carries both
 *                 branches per wave (default 1)
 *   "head_f32"    1: a DiT's twelve head / tail linears (pre_conv, proj_in, the time, global,
 *                 gce and cond embeddings, proj_out, post_conv) compute on f32 MFMA when the base
 *                 is f32 or f16, each refreshed by its own two-segment prepare; 0: bf16 like the
 *                 blocks (default 1). It holds from a DiT's setup.
 *   "prep_side"   1: with f32 head linears, a DiT's bf16 group refresh runs on the second stream
 *                 beside the heads' refresh and forward on the main one (default 1)
 *   "head_quick"  1: a DiT's context MLP and x path (pre_conv, proj_in) run on a third stream of
 *                 the context beside the modulation chain in the forward, and the context MLP's
 *                 backward beside the x path's (default 1; off while a profiler scope is open)
 *   "epi_fuse"    bit 0: a block's FFN SwiGLU val * silu(glu) is written by the up-projection's
 *                 GEMM epilogue (each 256-column output tile holds matching val and glu columns);
 *                 bit 1: the per-head q/k RMS norm, RoPE and head-major bf16 layout of the
 *                 attention inputs come out of the QKV and cross-query projections' epilogues;
 *                 bit 2: the attention backward's head-major bf16 dO and per-head row dots come
 *                 out of the out-projections' dX epilogues (the f32 dO is then not written);
 *                 bit 3: the SwiGLU backward (the up-projection's bf16 dU) comes out of the FFN
 *                 down-projection's dX epilogue, with act_bf16 bit 0 (the f32 dG is then not
 *                 written); each where the chosen tiles allow it (no split over K), else by its
 *                 own kernel (default 3: measured on MI355X, the DiT update with bits 2 / 2 and 3
 *                 takes 32.20 / 32.34 ms against 32.14 ms, the epilogue's extra loads stalling a
 *                 tile's whole workgroup where the separate kernels stream at full occupancy)
 *   "gemm_prio"   1: the DMA GEMMs raise their waves' priority over the MFMA clusters of the K
 *                 loop, so a wave that has its operands keeps issuing while the others read
 *                 (default 1)
 *   "act_bf16"    bit 0: a block's backward reads a bf16 copy of the FFN up-projection's output
 *                 (written by its epilogue) instead of the f32 output, which then is forward
 *                 scratch; bit 1: likewise for the QKV and cross-query outputs (default 1). It
 *                 holds for workspaces built from now on (a DiT: from its setup).
 * Every setting gives results identical to the defaults bit for bit except gemm_split, gemm_cfg,
 * gemm_small, gemm_skinny, gemm_big, gemm_splits, gemm_dq, lin_merge, rank_cols, merge_kn,
 * kv_stack, attn_fwd32, head_f32 and act_bf16, which change the rounding or the f32 summation order
 * (prep_side and head_quick change only the stream work runs on; epi_fuse only which kernel computes
 * SwiGLU and its backward, the head preparation and the attention row dots).
 * Not to
 * be changed while a graph is being captured. */
SA3K_API int sa3k_set_option(sa3k_ctx* ctx, const char* name, int value);

/* The current value of an option (the names of sa3k_set_option). No reference counterpart: the
 * tests use it to run with, and to restore, the shipped defaults. */
SA3K_API int sa3k_get_option(sa3k_ctx* ctx, const char* name, int* value);

/* The name of option `index` (0, 1, ...), NULL past the last one. No reference counterpart. */
SA3K_API const char* sa3k_option_name(int index);

/* Stream timer: sa3k_timer_start records an event on the context stream, sa3k_timer_stop records a
 * second one, synchronises and returns the elapsed milliseconds between them. */
SA3K_API int sa3k_timer_start(sa3k_ctx* ctx);
SA3K_API int sa3k_timer_stop(sa3k_ctx* ctx, float* ms);

/* Per-kernel timing with HIP events on the context stream (off by default; the reference's
 * SA3_TRAIN_PROFILE wall-clock phases, src/train_loop.h:314-437, have no per-kernel counterpart).
 * While enabled every kernel launch is bracketed by an event pair; sa3k_profile_report writes one
 * line per scope name, "name launches total_ms work\n", into buf (synchronises the stream); work is
 * the algorithmic flop count of the launches where the library counts it (the GEMMs: 2 (M + extra
 * rows) N (K + rank extension) per launch), else 0. */
SA3K_API int sa3k_profile_enable(sa3k_ctx* ctx, int on);
SA3K_API int sa3k_profile_reset(sa3k_ctx* ctx);
SA3K_API int sa3k_profile_report(sa3k_ctx* ctx, char* buf, int buf_len);

/* ---------------------------------------------------------------- K6: AdamW + global clip */

/* Mirrors TrainAdamWParams (src/train_optimizer.h:28-35). */
typedef struct {
    float learning_rate;
    float beta1;
    float beta2;
    float eps;
    float weight_decay;
    float grad_clip;      /* global L2 clip; <= 0 disables (reference default 1.0 in training) */
} sa3k_adamw_params;

/* One fused update of a flat arena of n f32 adapter parameters (every A, B and magnitude of every
 * target laid end to end). Replaces, on device, the host pair
 *   train_average_and_clip   (src/train_loop.h:147-171)  and
 *   adamw_update_vector      (src/train_optimizer.h:42-66) over every tensor
 * as called by train_apply_accumulated_adamw (src/train_loop.h:173-211):
 *   g := g * (1/count)                 if count > 1            (float)
 *   norm := sqrt(sum (double)g^2)      over the whole arena    (double)
 *   g := g * (float)(clip/(norm+1e-6)) if clip > 0 && norm > clip
 *   m := b1*m + (1-b1)*g ; v := b2*v + (1-b2)*g*g
 *   p := p - lr*((m/b1c)/(sqrt(v/b2c)+eps) + wd*p), b1c = 1-powf(b1,step), b2c = 1-powf(b2,step)
 * evaluated with the same float operation order (no contraction), so param/m/v are bit-identical
 * to the reference whenever the float clip scale is (the double sum is reduced in a different
 * order; see sa3k_adamw_clip_scale). `grad` is not modified. step must be >= 1 (the reference
 * rejects step <= 0, src/train_optimizer.h:49-52) and count >= 1 (src/train_loop.h:176-179).
 * grad_norm_out (nullable) receives the pre-clip global norm; passing it synchronises the stream. */
SA3K_API int sa3k_adamw_clip(sa3k_ctx* ctx, float* param, const float* grad, float* m, float* v,
                             int64_t n, const sa3k_adamw_params* hp, int step, int count,
                             double* grad_norm_out);

/* train_average_and_clip (src/train_loop.h:147-171) in place on a device arena of n gradients:
 * g := g * (1/count) if count > 1, then g := g * (float)(clip/(norm+1e-6)) if clip > 0 and the
 * double global norm exceeds clip. grad_norm_out (nullable, synchronises) gets the pre-clip norm. */
SA3K_API int sa3k_average_and_clip(sa3k_ctx* ctx, float* grad, int64_t n, int count, float grad_clip,
                                   double* grad_norm_out);

/* The float clip scale and pre-clip norm the last sa3k_adamw_clip on this context used
 * (scale = 1 when no clipping happened). Synchronises the stream. */
SA3K_API int sa3k_adamw_clip_scale(sa3k_ctx* ctx, double* norm_out, float* scale_out);

/* ---------------------------------------------------------------- a5: Q8_0 weight blocks */

/* Decode n_elems (multiple of 32) Q8_0 elements from raw GGUF blocks (34 bytes each, 2-byte
 * aligned) into f32: y = f32(d) * qs[i] — exact, so bit-identical to ggml's dequantize_row_q8_0
 * (called at tools/sa3-quant-check.cpp:43, used by mul_mat over a Q8_0 base in src/lora.h:239-251). */
SA3K_API int sa3k_q8_0_dequant(sa3k_ctx* ctx, const void* blocks, float* out, int64_t n_elems);

/* Encode n_elems (multiple of 32) f32 values into Q8_0 blocks with ggml's reference quantizer
 * (per block: d = amax/127, q = roundf(x * (1/d)), d stored as f16), the re-encode the reference's
 * quantizer tool applies to 2D weights (tools/sa3-quantize.cpp:43-56, 79-85). */
SA3K_API int sa3k_q8_0_quantize(sa3k_ctx* ctx, const float* x, void* blocks, int64_t n_elems);

/* ---------------------------------------------------------------- K1/K2: the MFMA GEMM */

/* C[M][N] = alpha * A[M][K] . B[N][K]^T, then *colscale[n] (nullable), +bias[n] (nullable),
 * written (accumulate = 0) or added (accumulate = 1) to f32 C [M][ldc]. Both operands are
 * K-contiguous. prec: SA3K_PREC_BF16 (A: f32 or bf16; B: f32, f16, bf16 or Q8_0 decoded in the
 * kernel) or SA3K_PREC_F32 (A f32; B f32 or f16). For b_type SA3K_TYPE_Q8_0, B holds int8 quants
 * [N][ldb] and B_scales the f16 block scales [N][ldbs] (one per 32 K); b_type -8 selects the
 * transposed Q8_0 layout (quants [N][K], scales [N/32][ldbs] per 32 rows). This is the kernel under
 * the reference's ggml_mul_mat(W, x) (src/dit.h:107) and its autodiff out_prod, exposed for tests
 * and measurement; dit_lin itself is sa3k_lin_*. K must be a multiple of 64 (bf16) / 32 (f32). */
SA3K_API int sa3k_gemm_nt(sa3k_ctx* ctx, int prec, int a_type, const void* A, int64_t lda,
                          int b_type, const void* B, int64_t ldb, const void* B_scales, int64_t ldbs,
                          int64_t M, int64_t N, int64_t K, float alpha, const float* colscale,
                          const float* bias, float* C, int64_t ldc, int accumulate);

/* sa3k_gemm_nt for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). No reference counterpart: ggml allocates
 * its graphs up front (src/train_ckpt.h), and this entry point serves those callers instead.
 * Same arguments, kernels and results (bit for bit) as sa3k_gemm_nt, but the split-K partial sums
 * go to a fixed 64 MiB scratch array in device memory that the library's code object carries (one
 * copy per GPU, held until the process ends), and the call never allocates. Every split plan the
 * dispatch chooses by itself fits; a plan that would need more (only possible when the
 * "gemm_splits" option forces a split count) fails with SA3K_ERR_INVALID before anything is
 * launched. All calls on one GPU share that array, from every context: calls that overlap on one
 * GPU (two streams, two contexts, two threads) race and must be serialised by the caller. */
SA3K_API int sa3k_gemm_nt_noalloc(sa3k_ctx* ctx, int prec, int a_type, const void* A, int64_t lda,
                                  int b_type, const void* B, int64_t ldb, const void* B_scales, int64_t ldbs,
                                  int64_t M, int64_t N, int64_t K, float alpha, const float* colscale,
                                  const float* bias, float* C, int64_t ldc, int accumulate);

/* ---------------------------------------------------------------- frozen base weights */

typedef struct sa3k_weight sa3k_weight;

/* Load a frozen base weight W [out][in] of GGUF type `type` (f32 / f16 / bf16 elements, or raw
 * Q8_0 blocks) from host memory (data_on_device = 0) or device memory. The library keeps the
 * forward layout and a transposed copy for the backward; Q8_0 blocks are split into int8 quants
 * and f16 scales (the same bytes, not re-encoded) in both layouts, so every contraction decodes
 * the stored blocks exactly. in must be a multiple of 64; out a multiple of 8 (32 for Q8_0).
 * The reference reads weights through GgufModel::get (src/gguf_model.h:200-276). */
SA3K_API int sa3k_weight_create(sa3k_ctx* ctx, int type, int64_t in, int64_t out, const void* data,
                                int data_on_device, sa3k_weight** out_w);
SA3K_API int sa3k_weight_destroy(sa3k_ctx* ctx, sa3k_weight* w);
/* Free the bf16 working copies (forward and transposed) that sa3k_weight_create decodes from an
 * f16 / f32 / Q8_0 base for the bf16-precision contractions; afterwards those contractions decode
 * the stored elements or Q8_0 blocks inside the GEMM on their way into LDS (same results, less
 * memory, slower). No reference counterpart (ggml decodes inside mul_mat, src/dit.h:100-107). */
SA3K_API int sa3k_weight_drop_working_copy(sa3k_ctx* ctx, sa3k_weight* w);
/* nsq[o] = (float)(sum_i (double)W[o][i]^2 + in*eps)   (train_row_norm_sq, src/train_lora.h:160-174)
 * norms[o] = (float)sqrt(sum_i (double)W[o][i]^2)       (train_row_norms,   src/train_lora.h:141-155)
 * over the decoded weight; outputs are device [out] f32. */
SA3K_API int sa3k_weight_row_norm_sq(sa3k_ctx* ctx, const sa3k_weight* w, float eps, float* nsq);
SA3K_API int sa3k_weight_row_norms(sa3k_ctx* ctx, const sa3k_weight* w, float* norms);
/* The same two reductions over a dense device matrix W [out][in] of element type f32 / f16 / bf16
 * with no shape constraint: mode 0 norms, mode 1 norm_sq (+ in*eps); result device f32 [out]. */
SA3K_API int sa3k_row_norms(sa3k_ctx* ctx, int type, int64_t in, int64_t out, const void* W, int mode, float eps,
                            float* result);

/* ---------------------------------------------------------------- K1-K4: dit_lin (lora / dora-rows) */

/* One adapted linear: the functional dit_lin of src/dit.h:92-149 over a frozen sa3k_weight, with
 * its own device scratch for up to max_tokens rows (saved activations and backward workspace).
 * rank: 0 (plain mul_mat) or 8/16/24/32; prec: SA3K_PREC_F32 (f32/f16 weights) or SA3K_PREC_BF16. */
typedef struct sa3k_lin sa3k_lin;
SA3K_API int sa3k_lin_create(sa3k_ctx* ctx, const sa3k_weight* W, int rank, int prec, int64_t max_tokens,
                             sa3k_lin** out_l);
SA3K_API int sa3k_lin_destroy(sa3k_ctx* ctx, sa3k_lin* l);

/* Refresh the adapter-derived terms after A/B/magnitude change (once per optimizer step):
 * A [rank][in], B [out][rank], scale = alpha/rank (src/train_dit.h:151); dora = 1 adds the
 * dora-rows row scale d = m / sqrt(bnsq + 2s.t2 + s^2.t3) with t2 = rowsum((W A^T) * B) and
 * t3 = rowsum(B * (B A A^T)) (src/dit.h:123-145), base_norm_sq from sa3k_weight_row_norm_sq with
 * eps 1e-12 (src/train_dit.h:159). All pointers are device memory and must stay valid and
 * unchanged until the next prepare (the backward reads B and magnitude). */
SA3K_API int sa3k_lin_prepare(sa3k_ctx* ctx, sa3k_lin* l, const float* A, const float* B, float scale,
                              int dora, const float* magnitude, const float* base_norm_sq);

/* Y [N][out] f32 = (X W^T + s (X A^T) B^T) * d + bias  (bias nullable; d = 1 for lora).
 * X [N][in] is f32 (x_type SA3K_TYPE_F32) or, with bf16 precision, bf16. Saves what the
 * backward needs (s X A^T and, for dora, the pre-scale output) in the linear's scratch. */
SA3K_API int sa3k_lin_forward(sa3k_ctx* ctx, sa3k_lin* l, int x_type, const void* X, int64_t N,
                              const float* bias, float* Y);

/* Backward of the last forward (same X and N), the closed form of ggml's autodiff of dit_lin:
 *   dX  = dU W + s (dU B) A                 (dU = dY * d)      -> written, or added if dx_accumulate
 *   dA += s (dU B)^T X + 2s B^T diag(gn) W + 2s^2 (B^T diag(gn) B) A
 *   dB += s dU^T (X A^T) + 2s diag(gn) W A^T + 2s^2 diag(gn) B A A^T
 *   dm += gd / sqrt(nsq)                    (gd = sum_n dY * U, gn = -gd m nsq^-3/2 / 2; dora only)
 * dA [rank][in], dB [out][rank], dm [out] are f32 accumulators (the micro-batch sum of
 * train_accum_add, src/train_loop.h:75-78). dX may be NULL (no input gradient). With rank 0 the
 * linear is a plain mul_mat and only dX = dY W is computed (dA/dB/dm may be NULL). */
SA3K_API int sa3k_lin_backward(sa3k_ctx* ctx, sa3k_lin* l, int x_type, const void* X, int64_t N,
                               const float* dY, float* dX, int dx_accumulate, float* dA, float* dB,
                               float* dm);

/* ---------------------------------------------------------------- inference: adapter chains */

/* One adapter of a chain over a frozen base weight (LoraAdapter, src/lora.h:28-34, with its tensors
 * for one target on the device): the residual scale is (alpha / rank) * strength, and an adapter of
 * strength 0 is the identity (skipped, as apply_loras skips it). */
typedef struct {
    int dora;                  /* 0: lora, 1: dora-rows */
    int rank;                  /* > 0 */
    float alpha;
    float strength;
    const float* A;            /* [rank][in] device f32 (GGUF lora_A ne = [in, rank]) */
    const float* B;            /* [out][rank] device f32 (GGUF lora_B ne = [rank, out]) */
    const float* magnitude;    /* [out] device f32 (dora-rows), else NULL */
} sa3k_chain_adapter;

typedef struct sa3k_lora_chain sa3k_lora_chain;

/* build_functional_lora (src/lora.h:372-622) for one target: up to 32 adapters applied in order over
 * the frozen base W (f32 / f16 / bf16 / Q8_0, which is never dequantised into HBM), whose active
 * ranks add up to at most 512 (up to 64 the rank term rides on the base product as its second
 * segment, above that it is a GEMM of its own accumulating into Y). Folds every dora-rows row scale into constants once, in double
 * precision: base_scale c0 [out] and the row-scaled B'_k, so that the chain's output equals merging
 * the adapters into W one after another (apply_loras, src/lora.h:111-143). Scratch for up to
 * max_tokens rows. The adapter pointers are read during this call only. */
SA3K_API int sa3k_lora_chain_create(sa3k_ctx* ctx, const sa3k_weight* W, int n_adapters,
                                    const sa3k_chain_adapter* adapters, int64_t max_tokens, sa3k_lora_chain** out);
SA3K_API int sa3k_lora_chain_destroy(sa3k_ctx* ctx, sa3k_lora_chain* chain);
/* dit_lin over the chain (src/dit.h:108-117): Y [N][out] f32 = c0 (.) (X W^T) + sum_k s_k (X A_k^T) B'_k^T
 * + bias (nullable); X [N][in] f32 or bf16 (x_type). bf16 MFMA with f32 accumulation; a Q8_0 / f16
 * base without a bf16 working copy is decoded on its way into LDS. */
SA3K_API int sa3k_lora_chain_forward(sa3k_ctx* ctx, sa3k_lora_chain* chain, int x_type, const void* X, int64_t N,
                                     const float* bias, float* Y);
/* The folded constants (device f32, nullable outputs): base_scale [out] and B' [out][R], the active
 * adapters' B'_k side by side in chain order; total_rank receives R. */
SA3K_API int sa3k_lora_chain_constants(sa3k_ctx* ctx, const sa3k_lora_chain* chain, float* base_scale, float* Bp,
                                       int* total_rank);

/* ---------------------------------------------------------------- K5: differential attention */

/* Flash-style differential attention (dit_diff_attn, src/dit.h:151-158, over nn::sdpa,
 * src/nn.h:135-144): per (batch, head) O = softmax(Q1 K1^T scale) V - softmax(Q2 K2^T scale) V,
 * without materialising the scores. q1, q2 [B*H][Sq][64] and k1, k2, v [B*H][Sk][64] are bf16
 * (head-major); window 0 is dense (the reference), window > 0 keeps |q - k| <= window/2 and needs
 * Sq == Sk. Attention weights below 2^-126 (keys more than ~87 nats under the row maximum) are
 * flushed to zero. Outputs: o bf16 [B][Sq][H*64] (token-major, the out-projection input), o1, o2 bf16
 * [B*H][Sq][64] (the normalised branch outputs) and lse1, lse2 f32 [B*H][Sq] (base-2 log-sum-exp
 * of scale*log2(e)*scores), which the backward consumes. */
SA3K_API int sa3k_diff_attn_fwd(sa3k_ctx* ctx, const void* q1, const void* k1, const void* q2, const void* k2,
                                const void* v, int B, int H, int Sq, int Sk, int head_dim, int window, float scale,
                                void* o, void* o1, void* o2, float* lse1, float* lse2);

/* Backward of sa3k_diff_attn_fwd from dO f32 [B][Sq][H*64] (token-major): writes dq1, dq2
 * [B*H][Sq][64], dk1, dk2, dv [B*H][Sk][64] (f32). The scores are recomputed from lse (ggml's
 * soft_max_back over stored scores in the reference). Scratch: dOh bf16 [B*H][Sq][64] and dn
 * f32 [2][B*H][Sq], caller-provided. */
SA3K_API int sa3k_diff_attn_bwd(sa3k_ctx* ctx, const void* q1, const void* k1, const void* q2, const void* k2,
                                const void* v, const void* o1, const void* o2, const float* lse1, const float* lse2,
                                const float* dO, int B, int H, int Sq, int Sk, int head_dim, int window, float scale,
                                void* scratch_dOh, float* scratch_dn, float* dq1, float* dk1, float* dq2, float* dk2,
                                float* dv);

/* ---------------------------------------------------------------- C3: one DiT block */

/* Shape of a (differential) DiT block, the DitConfig fields dit_block reads (src/dit.h:20-46). */
typedef struct {
    int dim;          /* model width = heads * head_dim */
    int heads;
    int head_dim;     /* 64 */
    int inner;        /* feed-forward inner width (ff.proj has 2*inner outputs: value | gate) */
    int rope_dims;    /* DitConfig::rot, rotary dims per head (NEOX pairs i, i + rope_dims/2) */
    int window;       /* self-attention window (0 dense, the reference); see sa3k_diff_attn_fwd */
    float rope_base;
    float norm_eps;
    float qk_eps;
} sa3k_block_config;

/* Frozen block tensors in host memory. Targets: 0 self.qkv [5*dim][dim], 1 self.out [dim][dim],
 * 2 cross.q [2*dim][dim], 3 cross.kv [3*dim][dim], 4 cross.out [dim][dim], 5 ff.proj
 * [2*inner][dim], 6 ff.out [dim][inner]; W[t] of GGUF type weight_type, bias[t] f32 or NULL.
 * ssg [6][dim] = the scale/shift/gate table (sc_a, sh_a, g_a, sc_f, sh_f, g_f); *_g are the
 * norm gammas (pre/cross/ff [dim], self q/k and cross q/k per-head [64]). */
typedef struct {
    int weight_type;
    const void* W[7];
    const float* bias[7];
    const float *ssg, *pre_g, *cross_g, *ff_g, *sq_g, *sk_g, *cq_g, *ck_g;
} sa3k_block_weights;

typedef struct sa3k_block sa3k_block;        /* frozen weights + 7 adapted linears */
typedef struct sa3k_block_ws sa3k_block_ws;  /* activations of one forward, backward scratch */

/* Upload a block's frozen tensors, build its 7 bf16-precision adapted linears (rank 0 = plain
 * mul_mat) with scratch for max_tokens latent rows (max_ctx_tokens rows for cross.kv), and compute
 * every target's base_norm_sq (eps 1e-12) for dora. */
SA3K_API int sa3k_block_create(sa3k_ctx* ctx, const sa3k_block_config* cfg, const sa3k_block_weights* w,
                               int rank, int64_t max_tokens, int64_t max_ctx_tokens, sa3k_block** out);
SA3K_API int sa3k_block_destroy(sa3k_ctx* ctx, sa3k_block* b);
/* Device pointer to target t's base_norm_sq [out] (owned by the block). */
SA3K_API int sa3k_block_base_norm_sq(sa3k_ctx* ctx, const sa3k_block* b, int target, const float** nsq);
/* Workspace for a batch of B samples of S latent tokens (memory tokens included) and Ctx context
 * tokens; one workspace can serve every block of a stack (it holds one block's activations). */
SA3K_API int sa3k_block_ws_create(sa3k_ctx* ctx, const sa3k_block_config* cfg, int B, int S, int Ctx,
                                  sa3k_block_ws** out);
SA3K_API int sa3k_block_ws_destroy(sa3k_ctx* ctx, sa3k_block_ws* ws);
/* Bind the adapters: A[t] [rank][in], B[t] [out][rank], mag[t] [out] (dora) device f32, same
 * contract as sa3k_lin_prepare. */
SA3K_API int sa3k_block_prepare(sa3k_ctx* ctx, sa3k_block* b, const float* const* A, const float* const* B,
                                const float* const* mag, float scale, int dora);
/* dit_block (src/dit.h:164-266) forward: x, out [B][S][dim], context [B][Ctx][dim], gcond
 * [B][6*dim], all f32 device. x and context must stay unchanged until the matching backward. */
SA3K_API int sa3k_block_forward(sa3k_ctx* ctx, sa3k_block* b, sa3k_block_ws* ws, const float* x,
                                const float* context, const float* gcond, float* out);
/* Backward of the last sa3k_block_forward on ws: dx [B][S][dim] is written; dcontext
 * [B][Ctx][dim] and dgcond [B][6*dim] are ADDED to (they are shared by every block of a stack);
 * dA/dB/dm[t] accumulate as in sa3k_lin_backward (dm may be NULL for lora). */
SA3K_API int sa3k_block_backward(sa3k_ctx* ctx, sa3k_block* b, sa3k_block_ws* ws, const float* dout, float* dx,
                                 float* dcontext, float* dgcond, float* const* dA, float* const* dB,
                                 float* const* dm);

/* ---------------------------------------------------------------- C4: the DiT training step */

/* DitConfig (src/dit.h:20-46) of a differential DiT, plus the feed-forward inner width and the
 * self-attention window of this build (0 = dense, the reference). local_dim > 0 (dit.local_dim,
 * src/dit.h:29-30; 257 in the inpaint model) adds each block's inpaint local-conditioning linears
 * dit.<l>.local.0 [dim][local_dim] and dit.<l>.local.2 [dim][dim], with biases (src/dit.h:244-254). */
typedef struct {
    int io, dim, depth, heads, head_dim, cond_dim, mem_tokens, rope_dims, time_dim, inner, window;
    float rope_base, norm_eps, qk_eps, time_min_freq, time_max_freq;
    int local_dim;
} sa3k_dit_config;

/* The training setup: adapter family and scope (TrainLoraScope, src/train_lora.h:53-97), the
 * micro-batch shape, and the activation schedule. */
typedef struct {
    int rank;          /* 8 / 16 / 24 / 32 */
    float alpha;       /* scale = alpha / rank (src/train_dit.h:151) */
    int dora;          /* 1: dora-rows, 0: lora */
    int scope;         /* SA3K_SCOPE_CORE (the 7 block projections) or SA3K_SCOPE_FULL (+ 12 head/tail) */
    int batch;         /* samples per accumulate call */
    int frames;        /* latent frames T per sample (tokens = mem_tokens + T) */
    int ctx_tokens;    /* cross-attention conditioning tokens per sample */
    int recompute;     /* 1: gradient-checkpointed schedule of src/train_ckpt.h (one block of
                          activations, every block but the last recomputed before its backward);
                          0: every block keeps its forward activations (no recompute) */
} sa3k_dit_train;
#define SA3K_SCOPE_CORE 0
#define SA3K_SCOPE_FULL 1

typedef struct sa3k_dit sa3k_dit;

/* A DiT whose 2-D weights are stored as weight_type (f32 / f16 / bf16) and every other tensor
 * (biases, norm gammas, ssg tables, memory tokens) as f32. Tensors are named as in the DiT GGUF
 * (dit.memory_tokens, dit.pre_conv.weight, dit.<l>.self.qkv.weight, dit.<l>.ssg, ...,
 * GgufModel::get, src/gguf_model.h:200-276) and are filled by sa3k_dit_set_tensor or
 * sa3k_dit_init_random before sa3k_dit_setup. */
SA3K_API int sa3k_dit_create(sa3k_ctx* ctx, const sa3k_dit_config* cfg, int weight_type, sa3k_dit** out);
SA3K_API int sa3k_dit_destroy(sa3k_ctx* ctx, sa3k_dit* dit);
/* Number of named tensors and the name / element count / stored type of tensor i. */
SA3K_API int sa3k_dit_tensor_count(sa3k_ctx* ctx, const sa3k_dit* dit, int* count);
SA3K_API int sa3k_dit_tensor_info(sa3k_ctx* ctx, const sa3k_dit* dit, int i, char* name, int name_len,
                                  int64_t* rows, int64_t* cols, int* type);
/* Copy a tensor's elements (host, in its stored type) into the model. */
SA3K_API int sa3k_dit_set_tensor(sa3k_ctx* ctx, sa3k_dit* dit, const char* name, const void* data, int64_t bytes);
/* Synthetic model on the device (counter-based Philox4x32-10 + Box-Muller): 2-D weights
 * N(0, w_sd), biases N(0, 0.02), ssg tables N(0, 0.1), gammas 1 + N(0, 0.1), memory tokens N(0, 1). */
SA3K_API int sa3k_dit_init_random(sa3k_ctx* ctx, sa3k_dit* dit, uint64_t seed, float w_sd);
/* Row norms of the named 2-D weight (decoded): mode 0 writes norms[o] = sqrt(sum_i W[o][i]^2)
 * (train_row_norms, src/train_lora.h:141-155), mode 1 writes sum_i W[o][i]^2 + in*eps
 * (train_row_norm_sq, :160-174); double accumulation, out device f32 [rows]. Valid before and
 * after sa3k_dit_setup. */
SA3K_API int sa3k_dit_weight_row_norms(sa3k_ctx* ctx, sa3k_dit* dit, const char* name, int mode, float eps,
                                       float* out);
/* Build the frozen weights (decoded bf16 working copies, base_norm_sq), the adapted linears, the
 * flat adapter arena and the activation workspaces for one micro-batch shape. */
SA3K_API int sa3k_dit_setup(sa3k_ctx* ctx, sa3k_dit* dit, const sa3k_dit_train* train);

/* The adapter arena: every selected target, in the reference's order (weight names sorted,
 * src/train_lora.h:99-121), holds A [rank][in], B [out][rank] and (dora) magnitude [out], laid
 * end to end (the order train_apply_accumulated_adamw visits them, src/train_loop.h:181-207).
 * which: 0 parameters, 1 accumulated gradients, 2 AdamW first moments, 3 second moments. */
SA3K_API int sa3k_dit_arena(sa3k_ctx* ctx, sa3k_dit* dit, int which, float** ptr, int64_t* n);
/* The device memory the resident schedule (recompute = 0) takes beyond the checkpointed one
 * (recompute = 1) for this model and micro-batch shape: depth - 1 more block workspaces. Valid
 * before sa3k_dit_setup. No reference counterpart: build_train_dit_ckpt (src/train_ckpt.h:143-474)
 * of the host mirror picks the resident schedule when it fits (both give the same results bit for
 * bit). */
SA3K_API int sa3k_dit_resident_bytes(sa3k_ctx* ctx, const sa3k_dit* dit, const sa3k_dit_train* train, size_t* bytes);
SA3K_API int sa3k_dit_target_count(sa3k_ctx* ctx, const sa3k_dit* dit, int* count);
SA3K_API int sa3k_dit_target_info(sa3k_ctx* ctx, const sa3k_dit* dit, int i, char* name, int name_len,
                                  int64_t* in, int64_t* out, int64_t* off_a, int64_t* off_b, int64_t* off_m);
/* Initialise the adapters on the device: A Kaiming-uniform U(+-1/sqrt(in)), B ~ N(0, b_sd) (0 =
 * zeros, the reference's init), magnitude = row norms of the decoded base (train_row_norms,
 * src/train_lora.h:141-155, init_train_lora_state :205-273). Moments and gradients are zeroed. */
SA3K_API int sa3k_dit_adapters_init(sa3k_ctx* ctx, sa3k_dit* dit, uint64_t seed, float b_sd);
/* Mark the adapter arena as changed outside the library (e.g. uploaded): the derived terms are
 * refreshed before the next forward. */
SA3K_API int sa3k_dit_adapters_changed(sa3k_ctx* ctx, sa3k_dit* dit);

/* One micro-batch of the rectified-flow step (run_train_dit_accumulate[_ckpt], src/train_loop.h:
 * 212-441, over build_train_dit_forward_graph, src/train_dit.h:30-218): forward, velocity MSE, and
 * the gradients of sum_b loss_b ADDED to the gradient arena (the accumulator adds one sample per
 * graph run in the reference; here the batch runs at once and counts batch samples). Device
 * inputs: x_t, target [B][T][io]; t [B]; cross [B][Ctx][cond_dim]; glob [B][cond_dim]; loss_weight
 * [B][T] (per-frame weights of the inpaint loss, src/train_dit.h:175-182) or NULL for the uniform
 * mean 1/(io*T). loss_out (host, nullable) receives the B per-sample losses and synchronises. */
SA3K_API int sa3k_dit_accumulate(sa3k_ctx* ctx, sa3k_dit* dit, const float* x_t, const float* target,
                                 const float* t, const float* cross, const float* glob,
                                 const float* loss_weight, double* loss_out);
/* train_apply_accumulated_adamw (src/train_loop.h:173-211) over the arena: average over the
 * accumulated sample count, global clip, AdamW (sa3k_adamw_clip), then clear the accumulator. */
SA3K_API int sa3k_dit_apply_adamw(sa3k_ctx* ctx, sa3k_dit* dit, const sa3k_adamw_params* hp, int step,
                                  double* grad_norm_out);
/* Replay the accumulate step as a captured HIP graph (default off; environment SA3K_DIT_GRAPH=1
 * turns it on): the first call runs eagerly, the next captures the step for its input pointers
 * (with and without the adapter refresh), later calls with the same pointers replay it. Results
 * are identical to the eager path. While profiling is on the step always runs eagerly. The eager
 * step is faster on MI355X (launches hide behind the kernels, and the second stream's kernels,
 * option "side_stream", run beside the main stream's, which a replay of the graph overlaps less):
 * 34.2 against 38.5 ms per update at the DiT's benchmark size. */
SA3K_API int sa3k_dit_set_graphs(sa3k_ctx* ctx, sa3k_dit* dit, int on);
/* Whether the accumulate step replays captured graphs: 1 after sa3k_dit_set_graphs(on = 1) until a
 * capture fails (the step then runs eagerly from that call on). No reference counterpart: the
 * tests use it to check that the graph path ran. */
SA3K_API int sa3k_dit_get_graphs(sa3k_ctx* ctx, sa3k_dit* dit, int* on);
/* run_eval_dit_loss (src/train_loop.h:455-476): the forward and the per-sample velocity MSE of
 * sa3k_dit_accumulate (same kernels, so the same losses bit for bit) without the backward; the
 * gradient arena and the accumulated sample count are untouched. loss_out (host, required) receives
 * the B per-sample losses; synchronises the stream. */
SA3K_API int sa3k_dit_eval_loss(sa3k_ctx* ctx, sa3k_dit* dit, const float* x_t, const float* target, const float* t,
                                const float* cross, const float* glob, const float* loss_weight, double* loss_out);
/* Bind the inpaint local conditioning [B][T][local_dim] f32 (device; TrainInpaint::local,
 * src/train_inpaint.h:145-194, set as TrainDitGraph::local by run_train_dit_accumulate,
 * src/train_loop.h:239-242) for the following sa3k_dit_accumulate / sa3k_dit_eval_loss /
 * sa3k_dit_forward calls: each block then adds local.2(silu(local.0(local))) to its T latent rows
 * after the cross-attention (src/dit.h:244-254), and in the full scope the local linears' adapters
 * receive gradients. NULL (the default) runs the model without the local add, as the reference's
 * non-inpaint graph does (their adapters then get no gradient). The memory must stay valid and
 * unchanged until the calls that use it have finished. */
SA3K_API int sa3k_dit_set_local(sa3k_ctx* ctx, sa3k_dit* dit, const float* local);
/* Forward only: velocity [B][T][io] (dit_forward, src/dit.h:327-338). */
SA3K_API int sa3k_dit_forward(sa3k_ctx* ctx, sa3k_dit* dit, const float* x_t, const float* t, const float* cross,
                              const float* glob, float* velocity);

#ifdef __cplusplus
}
#endif

#endif /* SA3K_H */
