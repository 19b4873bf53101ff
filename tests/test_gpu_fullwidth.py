"""Full-width parity against the oracle: the shapes the benchmark runs, at sequence lengths the
double-precision oracle finishes in seconds.

* one DiT block at dim 1536, 24 heads, FFN inner 6144, DoRA rank 32 on all 7 projections, f16
  base, batch 2 x (64 memory + 72 latent) tokens, 128 context tokens, windows 256 and 0 (dense);
* a depth-1 DiT at full width (io 64, cond 768, time 256, 64 memory tokens, T 72, Ctx 128, window
  256, full scope with the 12 head/tail targets, DoRA rank 32, f16 base);
every output and every adapter gradient to the bf16 bar (normwise relative error <= 2e-2, cosine
>= 0.9999; losses to 1e-3). At these widths the GEMMs take the tile shapes, split-K counts,
skinny-product and column-reduction splits, and the attention kernels their grids and query
splits, that the 1536-wide model uses; the small-width tests elsewhere do not reach them.
"""
import os
import sys

import numpy as np
import pytest

from conftest import ROOT, assert_shipped_options, cosine, rel_err, rng, sa3k
from test_gpu_block import GpuBlock, run_gpu, to_f16_grid
from test_gpu_dit import grads_by_target, make_gpu, upload_inputs

sys.path.insert(0, os.path.join(ROOT, "oracle"))
import block_binding as bb  # noqa: E402
import dit_binding as db  # noqa: E402

pytestmark = pytest.mark.gpu

TOL_REL, TOL_COS = 2e-2, 0.9999


def check(got, ref, what, worst):
    e, c = rel_err(got, ref), cosine(got, ref)
    worst.append((e, c, what))
    assert e <= TOL_REL and c >= TOL_COS, f"{what}: rel {e:.3e} cos {c:.6f}"


@pytest.mark.parametrize("window", [256, 0])
def test_block_full_width_vs_oracle(ctx, window):
    assert_shipped_options(ctx)   # the shipped configuration: every option at its default
    B, S, Ctx = 2, 64 + 72, 128
    print(f"full-width block vs oracle: window {window}, B {B}, S {S}, Ctx {Ctx}", flush=True)
    cfg, w, x, cx, gc = bb.random_block(51 + window, B=B, S=S, Ctx=Ctx, dim=1536, heads=24, inner=6144, rank=32,
                                        alpha=32.0, dora=True, window=window, w_sd=0.02, b_sd=0.01)
    w["W"] = [to_f16_grid(W) for W in w["W"]]   # the oracle sees the f16 values the GPU decodes
    w["bnsq"] = [((W.astype(np.float64) ** 2).sum(1) + W.shape[1] * 1e-12).astype(np.float32) for W in w["W"]]
    dout = rng(52 + window).normal(0, 1e-2, x.shape).astype(np.float32)
    gb = GpuBlock(ctx, cfg, w, sa3k.TYPE_F16, B * S, B * Ctx)
    try:
        got = run_gpu(ctx, gb, x, cx, gc, dout)
    finally:
        gb.destroy()
    ref_out = bb.block_fwd(cfg, w, x, cx, gc)
    ref = bb.block_bwd(cfg, w, x, cx, gc, dout)
    worst = []
    check(got["out"] - x, ref_out - x, "out - x", worst)
    check(got["dx"] - dout, ref["dx"] - dout, "dx - dout", worst)
    check(got["dctx"], ref["dctx"], "dcontext", worst)
    check(got["dgcond"], ref["dgcond"], "dgcond", worst)
    for t in range(7):
        check(got["dA"][t], ref["dA"][t], f"dA[{t}]", worst)
        check(got["dB"][t], ref["dB"][t], f"dB[{t}]", worst)
        check(got["dm"][t], ref["dm"][t], f"dm[{t}]", worst)
    e, c, what = max(worst)
    print(f"worst normwise error {e:.3e} ({what}), lowest cosine {min(x[1] for x in worst):.7f}")


@pytest.mark.parametrize("local_dim", [0, 257])
def test_dit_depth1_full_width_vs_oracle(ctx, local_dim):
    # local_dim 257: the reference's inpaint model ([mask | z * mask] over its 256 latent channels),
    # local.0's input padded to 320 columns on the device, the local linears adapted (full scope)
    assert_shipped_options(ctx)   # the shipped configuration: every option at its default
    cfg = dict(B=2, T=72, Ctx=128, io=64, dim=1536, heads=24, inner=6144, depth=1, mem=64, cond_dim=768,
               time_dim=256, rope_dims=32, window=256, rank=32, alpha=32.0, dora=True, local_dim=local_dim)
    print(f"full-width depth-1 DiT vs oracle: T 72, Ctx 128, window 256, DoRA r32 full scope, local_dim {local_dim}",
          flush=True)
    tensors, adapters, inputs = db.random_dit(53, cfg, "full", w_sd=0.02, b_sd=0.01)
    tensors = {k: (v.astype(np.float16).astype(np.float32) if k.endswith(".weight") else v)
               for k, v in tensors.items()}
    d = make_gpu(ctx, cfg, tensors, adapters, "full", sa3k.TYPE_F16)
    try:
        up, _ = upload_inputs(ctx, inputs)
        if local_dim:
            d.set_local(up["local"])
        loss = d.accumulate(up["x_t"], up["target"], up["t"], up["cross"], up["glob"])
        vel = ctx.empty((cfg["B"], cfg["T"], cfg["io"]))
        d.forward(up["x_t"], up["t"], up["cross"], up["glob"], vel)
        got = grads_by_target(d, d.arena(1).numpy())
        ref_loss, ref_vel, ref = db.dit_loss(cfg, tensors, adapters, inputs)
        assert np.allclose(loss, ref_loss, rtol=1e-3), (loss, ref_loss)
        worst = []
        check(vel.numpy(), ref_vel, "velocity", worst)
        assert len(ref) == (21 if local_dim else 19)
        for n, (dA, dB, dm) in ref.items():
            check(got[n][0], dA, f"dA {n}", worst)
            check(got[n][1], dB, f"dB {n}", worst)
            check(got[n][2], dm, f"dm {n}", worst)
        e, c, what = max(worst)
        print(f"worst normwise error {e:.3e} ({what}), lowest cosine {min(x[1] for x in worst):.7f}")
    finally:
        d.destroy()


@pytest.mark.parametrize("S", [64 + 960, 64 + 1024])
def test_block_epilogue_fusions_bitwise(ctx, S):
    """The GEMM-epilogue fusions (option epi_fuse) against their separate kernels at the benchmark's
    width: the FFN SwiGLU from the up-projection's epilogue (bit 0), the per-head q/k RMS norm,
    RoPE and head-major bf16 outputs from the QKV and cross-query projections' epilogues (bit 1),
    the attention backward's head-major bf16 dO and row dots from the two out-projections' dX
    epilogues (bit 2) and the SwiGLU backward (the up-projection's dU) from the down-projection's dX
    epilogue (bit 3). 2 x 1024 tokens take the 128 x 256 DMA tiles without a split over K for the
    forward products, 2 x 1088 (the benchmark's 2176 tokens) the 256 x 256 tiles for the
    up-projection; the out-projections' dX products take the small-grid 128 x 128 tiles, the
    down-projection's the 256 x 256 ones. Each fused path evaluates the same expressions per
    element, so every output and gradient agrees bit for bit; the profile shows which separate
    kernels ran (SwiGLU: one forward and one backward launch, each unless fused; head prep: self +
    cross query + context K/V unfused, context K/V only fused; attention dots: self + cross unfused,
    none fused)."""
    assert_shipped_options(ctx)
    B, Ctx = 2, 128
    print(f"epilogue fusions: B {B}, S {S}, Ctx {Ctx}", flush=True)
    cfg, w, x, cx, gc = bb.random_block(61, B=B, S=S, Ctx=Ctx, dim=1536, heads=24, inner=6144, rank=32,
                                        alpha=32.0, dora=True, window=256, w_sd=0.02, b_sd=0.01)
    dout = rng(62).normal(0, 1e-2, x.shape).astype(np.float32)
    gb = GpuBlock(ctx, cfg, w, sa3k.TYPE_F16, B * S, B * Ctx)
    res, launches = {}, {}
    try:
        for fuse in (15, 0, 1, 2, 3, 4, 8):
            ctx.set_option("epi_fuse", fuse)
            ctx.profile(True)
            ctx.profile_reset()
            res[fuse] = run_gpu(ctx, gb, x, cx, gc, dout)
            rep = ctx.profile_report()
            ctx.profile(False)
            launches[fuse] = tuple(sum(v[0] for k, v in rep.items() if k.startswith(n))
                                   for n in ("blk_swiglu", "blk_prep_fwd", "attn_bwd_dot"))
    finally:
        ctx.profile(False)
        ctx.set_options(ctx.defaults)
        gb.destroy()
    want = {f: ((0 if f & 1 else 1) + (0 if f & 8 else 1), 1 if f & 2 else 3, 0 if f & 4 else 2) for f in launches}
    assert launches == want, launches
    for fuse in (0, 1, 2, 3, 4, 8):
        for k in ("out", "dx", "dctx", "dgcond"):
            assert np.array_equal(res[15][k], res[fuse][k]), (fuse, k)
        for k in ("dA", "dB", "dm"):
            for t in range(7):
                assert np.array_equal(res[15][k][t], res[fuse][k][t]), (fuse, f"{k}[{t}]")


@pytest.mark.parametrize("act_bf16", [1, 3])
def test_block_fused_epilogues_vs_oracle(ctx, act_bf16):
    """The fused epilogues against the oracle directly: the full-width block at 2 x 136 tokens with
    every epilogue fusion on (epi_fuse 15) and the split over K and the small-grid tile switched
    off, so that the up-projection, QKV and cross-query products and the out- and down-projections'
    dX products take unsplit 128 x 256 tiles and the fusions apply (shipped, these small grids take
    split or 64 x 128 tiles and the separate kernels, which the other full-width tests cover); the
    backward reading the bf16 copy of the FFN up-projection's output (act_bf16 1, the default) and
    also those of the QKV and cross-query outputs (3)."""
    B, S, Ctx = 2, 64 + 72, 128
    cfg, w, x, cx, gc = bb.random_block(71, B=B, S=S, Ctx=Ctx, dim=1536, heads=24, inner=6144, rank=32,
                                        alpha=32.0, dora=True, window=256, w_sd=0.02, b_sd=0.01)
    w["W"] = [to_f16_grid(W) for W in w["W"]]
    w["bnsq"] = [((W.astype(np.float64) ** 2).sum(1) + W.shape[1] * 1e-12).astype(np.float32) for W in w["W"]]
    dout = rng(72).normal(0, 1e-2, x.shape).astype(np.float32)
    gb = GpuBlock(ctx, cfg, w, sa3k.TYPE_F16, B * S, B * Ctx)
    try:
        ctx.set_option("gemm_split", 0)
        ctx.set_option("gemm_small", 0)
        ctx.set_option("act_bf16", act_bf16)
        ctx.set_option("epi_fuse", 15)   # every epilogue fusion, the backward ones included
        ctx.profile(True)
        ctx.profile_reset()
        got = run_gpu(ctx, gb, x, cx, gc, dout)
        rep = ctx.profile_report()
    finally:
        ctx.profile(False)
        ctx.set_options(ctx.defaults)
        gb.destroy()
    n = tuple(sum(v[0] for k, v in rep.items() if k.startswith(p))
              for p in ("blk_swiglu", "blk_prep_fwd", "attn_bwd_dot"))
    assert n == (0, 1, 0), n   # the context K/V prep only: no SwiGLU or attention dot kernel
    ref_out = bb.block_fwd(cfg, w, x, cx, gc)
    ref = bb.block_bwd(cfg, w, x, cx, gc, dout)
    worst = []
    check(got["out"] - x, ref_out - x, "out - x", worst)
    check(got["dx"] - dout, ref["dx"] - dout, "dx - dout", worst)
    check(got["dctx"], ref["dctx"], "dcontext", worst)
    check(got["dgcond"], ref["dgcond"], "dgcond", worst)
    for t in range(7):
        check(got["dA"][t], ref["dA"][t], f"dA[{t}]", worst)
        check(got["dB"][t], ref["dB"][t], f"dB[{t}]", worst)
        check(got["dm"][t], ref["dm"][t], f"dm[{t}]", worst)
    e, c, what = max(worst)
    print(f"worst normwise error {e:.3e} ({what}), lowest cosine {min(x[1] for x in worst):.7f}")
