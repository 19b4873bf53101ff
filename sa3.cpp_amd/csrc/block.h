// One DiT block (block.hip): frozen weights + 7 adapted linears, and the workspace holding one
// forward's activations. Shared by the C ABI in block.hip and the stack runner in dit.hip.
#pragma once

#include "gemm.h"

#include <vector>

struct sa3k_block {
    static constexpr int NT = 7;   // 0 self.qkv, 1 self.out, 2 cross.q, 3 cross.kv, 4 cross.out, 5 ff.proj, 6 ff.out
    sa3k_block_config cfg{};
    int rank = 0;
    int64_t max_tokens = 0, max_ctx = 0;
    sa3k_weight* W[NT] = {};
    sa3k_lin* L[NT] = {};
    float* bias[NT] = {};
    float* bnsq[NT] = {};
    float *ssg = nullptr, *pre_g = nullptr, *cross_g = nullptr, *ff_g = nullptr;
    float *sq_g = nullptr, *sk_g = nullptr, *cq_g = nullptr, *ck_g = nullptr;
};

struct sa3k_block_ws {
    int B = 0, S = 0, Ctx = 0, dim = 0, H = 0, inner = 0;
    // forward activations (read again by the backward). With act_bf16 bit 0 (bit 1) the f32
    // output F of the FFN up-projection (qkv and qf of the QKV and cross-query projections) is
    // forward scratch, written only where the separate SwiGLU (head-preparation) kernel needs it,
    // and the backward reads its bf16 copy Fb (qkvb, qfb), which the projection's epilogue always
    // writes; otherwise the copy is null and the backward reads the f32 output.
    int act_bf16 = 0;
    float* modv; const float* x; float* rs_a; sa3k::bf16* h; float* qkv; sa3k::bf16* qkvb;
    sa3k::bf16 *q1, *k1, *q2, *k2, *v; float* rq;
    sa3k::bf16* o; sa3k::bf16 *o1, *o2; float *l1, *l2; float* y; float* x1; float* rs_c; sa3k::bf16* hc;
    float* qf; sa3k::bf16* qfb; float* kv; const float* ctxf; sa3k::bf16 *cq1, *ck1, *cq2, *ck2, *cv; float *rcq, *rck;
    // when set, the block's context K/V projection was computed by a stacked product: its rows of
    // kv_ld floats hold this block's 3 dim outputs (the block skips its own cross.kv forward)
    const float* kv_ext = nullptr; int64_t kv_ld = 0;
    sa3k::bf16* oc; sa3k::bf16 *co1, *co2; float *cl1, *cl2; float* x2; float* rs_f; sa3k::bf16* fin; float* F;
    sa3k::bf16* Fb; sa3k::bf16* g; float* yf;
    // inpaint local conditioning (src/dit.h:244-254), set by the caller per block or null: the
    // forward adds ladd [B][ladd_T][dim] to the latent rows (the last ladd_T of each sample's S)
    // after the cross-attention; the backward writes the gradient of that sum to dladd (same shape)
    const float* ladd = nullptr; float* dladd = nullptr; int ladd_T = 0;
    // scratch of the forward (yc) and the backward: may be shared by several workspaces that are
    // used one at a time on the same stream
    float* yc;
    float *dg, *dfin, *dx2, *doc, *dhc, *dx1, *dob, *dh;
    sa3k::bf16* dOh; float* dn; float *dq1, *dk1, *dq2, *dk2, *dv;
    float* dssg; float* part; int part_chunks;
    // RoPE cos/sin table of positions 0..S-1 for (rope_tab_dims, rope_tab_base); 0: not built yet
    float* rope_tab; int rope_tab_dims = 0; float rope_tab_base = 0.f;
    std::vector<void*> allocs;
};

namespace sa3k {

// W[t] (type weight_type), bias[t] (f32 or null) and vecs = {ssg, pre_g, cross_g, ff_g, sq_g, sk_g,
// cq_g, ck_g} in host (on_device = 0) or device memory.
sa3k_block* block_build(sa3k_ctx* ctx, const sa3k_block_config& cfg, int weight_type, const void* const* W,
                        const float* const* bias, const float* const* vecs, int on_device, int rank,
                        int64_t max_tokens, int64_t max_ctx);
void block_free(sa3k_ctx* ctx, sa3k_block* b);
// share_scratch: take the forward/backward scratch of another workspace of the same shape
// act_bf16 (the option of that name): bit 0 keeps a bf16 copy of the FFN up-projection's output for
// the backward (the f32 output becomes forward scratch), bit 1 likewise for the QKV and
// cross-query outputs
// count_bytes (optional): allocate nothing, add the bytes the workspace would take and return null
sa3k_block_ws* block_ws_build(const sa3k_block_config& cfg, int B, int S, int Ctx, const sa3k_block_ws* share_scratch,
                              int act_bf16, size_t* count_bytes = nullptr);
void block_ws_free(sa3k_block_ws* w);
void block_prepare(sa3k_ctx* ctx, sa3k_block* b, const float* const* A, const float* const* Bm,
                   const float* const* mag, float scale, int dora);
void block_forward(sa3k_ctx* ctx, sa3k_block* b, sa3k_block_ws* w, const float* x, const float* context,
                   const float* gcond, float* out);
// late_join: leave the second stream's last work of the block running past the return (its
// completion is recorded in ctx->block_tail_ev and waited for before this workspace's scratch is
// written again, by the next block_backward on a workspace that shares it); the caller joins the
// second stream after its last block. Only for workspaces whose activations are not rewritten in
// between (no recompute).
void block_backward(sa3k_ctx* ctx, sa3k_block* b, sa3k_block_ws* w, const float* dout, float* dx, float* dcontext,
                    float* dgcond, float* const* dA, float* const* dB, float* const* dm, bool late_join = false);

}  // namespace sa3k
