// Internal API of lora.hip beyond the C ABI: a group of bf16-precision adapted linears whose
// adapter-derived terms are refreshed together (one launch per stage for the whole group).
#pragma once

#include "gemm.h"

// A frozen base weight W [out][in] of the C ABI (opaque to callers).
struct sa3k_weight {
    int type = SA3K_TYPE_F32;
    int64_t in = 0, out = 0;
    void* w = nullptr;      // forward layout [out][in] (Q8_0: int8 quants)
    void* ws = nullptr;     // Q8_0: f16 scales [out][in/32]
    void* wt = nullptr;     // transposed [in][out] (Q8_0: int8 quants)
    void* wts = nullptr;    // Q8_0: f16 scales [in/32][out]
    // bf16 working copies of the decoded weight, [out][in] and [in][out], built at load for every
    // non-bf16 type: the frozen base is contracted three times per training step (forward,
    // checkpoint recompute, dX), and the bf16-MFMA kernels round every decoded element to bf16
    // anyway, so decoding once keeps bit-identical results and takes the per-element decode off
    // the GEMM's inner loop. sa3k_weight_drop_working_copy frees them; the GEMMs then decode the
    // stored blocks in the global->LDS path instead.
    void* wb = nullptr;
    void* wbt = nullptr;
};

namespace sa3k {

struct LinGroup;

// lins: bf16-precision linears with bf16 working copies, all of rank `rank` (> 0); A/B/mag/bnsq
// are the device adapter pointers of each (mag/bnsq for dora), fixed for the group's lifetime.
LinGroup* lin_group_create(sa3k_ctx* ctx, sa3k_lin* const* lins, int n, const float* const* A, const float* const* B,
                           const float* const* mag, const float* const* bnsq, float scale, int dora);
// the grouped equivalent of sa3k_lin_prepare on every member
void lin_group_prepare(sa3k_ctx* ctx, LinGroup* g);
void lin_group_free(LinGroup* g);
// A short role name ("qkv", "ff.out", ...) appended to the linear's profiler scope names, so a
// per-kernel profile separates the projections (no effect while profiling is off).
void lin_set_tag(sa3k_lin* l, const char* tag);
// The output-gradient hand-off of a bf16-precision linear: a kernel producing the gradient dY of
// the linear's output may write dU = bf16(scale (.) dY) into lin_du(L) ([tokens][out]), with scale
// = lin_du_scale(L) per output column (the DoRA row scale d; null: 1), and then call
// lin_backward_du, which is sa3k_lin_backward on that dU (the f32 dY is never materialised).
bf16* lin_du(sa3k_lin* L);
const float* lin_du_scale(const sa3k_lin* L);
// Backward epilogues of the dX product that write what consumes dX in place of dX (GemmDesc::ad,
// GemmDesc::sb): *done is set where the chosen kernel ran them (dX is then not written).
struct DxEpi {
    AttnDot ad;
    SwiBwd sb;
    int* done = nullptr;
};
void lin_backward_du(sa3k_ctx* ctx, sa3k_lin* L, int x_type, const void* X, int64_t N, float* dX, int dx_accumulate,
                     float* dA, float* dB, float* dm, const DxEpi* epi = nullptr);
// A stacked product: n bf16 merged adapted linears of one shape and rank that read the same input
// (the DiT's per-block context K/V projections). Created before the linears are prepared, it moves
// their W_eff, row scales d, A copies and the saved U / s X A^T into contiguous slabs, so that one
// GEMM (lin_stack_forward) computes every member's forward: Y [N][n out] f32 (owned by the stack,
// member i in columns i out .. (i+1) out - 1). Each member's backward then runs as usual on that
// member (reading its slices of U and s X A^T); its own forward is refused. Null when the linears
// are not eligible (or the merged refresh is off).
struct LinStack;
LinStack* lin_stack_create(sa3k_ctx* ctx, sa3k_lin* const* lins, int n);
const float* lin_stack_forward(sa3k_ctx* ctx, LinStack* st, const float* X, int64_t N);
int64_t lin_stack_ld(const LinStack* st);   // row stride of Y (n out)
const float* lin_stack_y(const LinStack* st);   // Y (fixed for the stack's lifetime)
void lin_stack_free(LinStack* st);
// sa3k_lin_forward of a bf16 FFN up-projection (Y = [val | glu], bf16 X) that also writes the
// SwiGLU g = bf16(val * silu(glu)) [N][out / 2] from its GEMM epilogue when the option epi_fuse has
// bit 0 set and the chosen kernel allows it, and returns whether it did (if not, the caller computes
// g from Y). Yb (optional): a bf16 copy of Y, with Y then written only where g is not fused.
bool lin_forward_swiglu(sa3k_ctx* ctx, sa3k_lin* L, const bf16* X, int64_t N, const float* bias, float* Y, bf16* Yb,
                        bf16* g);
// sa3k_lin_forward of an attention projection (no bias, bf16 X) that also prepares its heads (the
// per-head q/k RMS norm, RoPE and head-major bf16 outputs of HeadPrep) from its GEMM epilogue when
// bit 1 of the option epi_fuse is set and the chosen kernel allows it, and returns whether it did
// (if not, the caller prepares them from Y). Yb (optional): a bf16 copy of Y, with Y then written
// only where the heads are not prepared in the epilogue.
bool lin_forward_headprep(sa3k_ctx* ctx, sa3k_lin* L, const bf16* X, int64_t N, float* Y, bf16* Yb,
                          const HeadPrep& hp);
// The B operand of X W^T (forward orientation) in g's precision: the bf16 working copy when the
// weight has one and the precision is bf16, else the stored elements or Q8_0 planes, which the
// GEMM decodes on their way into LDS.
void weight_fwd_operand(const sa3k_weight* W, GemmDesc& g);

}  // namespace sa3k
