"""C4: the DiT training step (run_train_dit_accumulate_ckpt + train_apply_accumulated_adamw,
src/train_loop.h:173-441) on the GPU vs the whole-DiT oracle (oracle/dit.cpp, pinned against
torch float64 autograd in tests/test_oracle_dit.py).

* depth-2 model, full scope (12 head/tail targets + blocks, DoRA, dense attention) and core scope
  (blocks only, LoRA, banded attention, per-frame loss weights), f32 and f16 bases, adapted
  products over the merged weight W + s B A and with the rank term as a second segment: per-sample
  losses, the velocity and every adapter gradient to the bf16 bar (normwise relative error
  <= 2e-2 and cosine >= 0.9999; the loss to 1e-3);
* the arena layout is the reference's: targets in sorted weight-name order, [A | B | m] each;
* the checkpointed (recompute) and resident schedules give bitwise-identical losses and gradients;
* two accumulate calls give exactly twice the gradients; apply_adamw equals the oracle's
  train_apply_accumulated_adamw on the same arena (bit-exact parameters and moments);
* the full-size step (24 blocks, batch 2 x (64 + 1024) tokens, io 64, window 256, DoRA r32):
  finite, deterministic, and the loss falls over a few updates on a fixed batch;
* the inpaint local conditioning (dit.<l>.local.{0,2}, src/dit.h:244-254) with local_dim 65 and
  257 (local.0's input padded to 128 / 320 columns on the device): losses, velocity and every
  adapter gradient (the local linears' included in the full scope) against the oracle, resident ==
  recompute bitwise, and a step without bound conditioning equals the model without the local add
  with zero local gradients.
"""
import os
import sys

import numpy as np
import pytest

from conftest import ROOT, assert_shipped_options, cosine, oracle, rel_err, sa3k

sys.path.insert(0, os.path.join(ROOT, "oracle"))
import dit_binding as db  # noqa: E402

pytestmark = pytest.mark.gpu

CFG = dict(B=2, T=12, Ctx=5, io=64, dim=128, heads=2, inner=128, depth=2, mem=4, cond_dim=64, time_dim=64,
           rope_dims=32, window=0, rank=8, alpha=16.0, dora=True)
HP = (1e-3, 0.9, 0.999, 1e-8, 0.01, 1.0)


def make_gpu(ctx, cfg, tensors, adapters, scope, wtype, recompute=False):
    c = sa3k.dit_config(cfg["io"], cfg["dim"], cfg["depth"], cfg["heads"], cfg["cond_dim"], cfg["mem"],
                        cfg["time_dim"], cfg["inner"], cfg["window"], local_dim=cfg.get("local_dim", 0))
    d = sa3k.Dit(ctx, c, wtype)
    for name, rows, cols, typ in d.tensors():
        a = tensors[name]
        if typ == sa3k.TYPE_F16:
            a = a.astype(np.float16)
        d.set_tensor(name, a)
    d.setup(cfg["rank"], cfg["alpha"], cfg["dora"], sa3k.SCOPE_FULL if scope == "full" else sa3k.SCOPE_CORE,
            cfg["B"], cfg["T"], cfg["Ctx"], recompute)
    p = np.zeros(d.arena(0).shape, np.float32)
    for name, i, o, oa, ob, om in d.targets():
        A, Bm, mag = adapters[name]
        p[oa:oa + A.size] = A.ravel()
        p[ob:ob + Bm.size] = Bm.ravel()
        if om >= 0:
            p[om:om + o] = mag
    ctx.copy_into(d.arena(0), p)
    d.adapters_changed()
    return d


def upload_inputs(ctx, inputs, lw=None):
    up = {k: ctx.upload(np.ascontiguousarray(v, np.float32)) for k, v in inputs.items()}
    return up, (ctx.upload(lw) if lw is not None else None)


def grads_by_target(d, g):
    out = {}
    for name, i, o, oa, ob, om in d.targets():
        r = (ob - oa) // i
        out[name] = (g[oa:oa + r * i].reshape(r, i), g[ob:ob + o * r].reshape(o, r),
                     g[om:om + o] if om >= 0 else None)
    return out


def check(got, ref, what):
    e, c = rel_err(got, ref), cosine(got, ref)
    assert e <= 2e-2 and c >= 0.9999, f"{what}: rel {e:.3e} cos {c:.6f}"


# Every oracle comparison runs these seeds: each seed draws a new model, adapters and inputs.
SEEDS = (41, 42, 43, 44)
CASES = {"full_dora_dense_f32": ("full", True, 0, False, sa3k.TYPE_F32, 1),
         "full_dora_dense_f16": ("full", True, 0, False, sa3k.TYPE_F16, 1),
         "full_dora_dense_f16_segments": ("full", True, 0, False, sa3k.TYPE_F16, 0),
         "core_lora_band_weighted_f16": ("core", False, 6, True, sa3k.TYPE_F16, 1),
         "core_lora_band_weighted_f16_segments": ("core", False, 6, True, sa3k.TYPE_F16, 0)}


@pytest.mark.parametrize("seed", SEEDS)
@pytest.mark.parametrize("name", sorted(CASES))
def test_dit_step_vs_oracle(ctx, name, seed):
    # lin_merge 1 (default): the adapted products contract W + s B A; 0: the rank term as a second
    # segment of each product. Every other option at its shipped default.
    scope, dora, window, weighted, wtype, merge = CASES[name]
    cfg = dict(CFG, dora=dora, window=window)
    tensors, adapters, inputs = db.random_dit(seed, cfg, scope)
    if wtype == sa3k.TYPE_F16:   # the oracle sees the f16 values the GPU decodes
        tensors = {k: (v.astype(np.float16).astype(np.float32) if (k.endswith(".weight")) else v)
                   for k, v in tensors.items()}
    lw = None
    if weighted:
        lw = np.random.Generator(np.random.Philox(seed + 7)).uniform(
            0, 2.0 / (cfg["io"] * cfg["T"]), (cfg["B"], cfg["T"])).astype(np.float32)
    assert_shipped_options(ctx)
    ctx.set_option("lin_merge", merge)
    try:
        d = make_gpu(ctx, cfg, tensors, adapters, scope, wtype)
    finally:
        ctx.set_options(ctx.defaults)
    try:
        assert [t[0] for t in d.targets()] == db.target_names(cfg, scope)
        up, lw_d = upload_inputs(ctx, inputs, lw)
        loss = d.accumulate(up["x_t"], up["target"], up["t"], up["cross"], up["glob"], lw_d)
        vel = ctx.empty((cfg["B"], cfg["T"], cfg["io"]))
        d.forward(up["x_t"], up["t"], up["cross"], up["glob"], vel)
        g_arena = d.arena(1).numpy()
        # run_eval_dit_loss: the same losses bit for bit, gradients untouched
        ev = d.eval_loss(up["x_t"], up["target"], up["t"], up["cross"], up["glob"], lw_d)
        assert np.array_equal(ev, loss)
        assert np.array_equal(d.arena(1).numpy(), g_arena)
        got = grads_by_target(d, g_arena)
        ref_loss, ref_vel, ref = db.dit_loss(cfg, tensors, adapters, inputs, loss_weight=lw)
        assert np.allclose(loss, ref_loss, rtol=1e-3), (loss, ref_loss)
        check(vel.numpy(), ref_vel, "velocity")
        for n, (dA, dB, dm) in ref.items():
            check(got[n][0], dA, f"dA {n}")
            check(got[n][1], dB, f"dB {n}")
            if dora:
                check(got[n][2], dm, f"dm {n}")
    finally:
        d.destroy()


LOCAL_CASES = {"full_dora_local65_f16": ("full", True, 0, False, 65),
               "full_dora_local257_band_f16": ("full", True, 6, False, 257),
               "core_lora_local65_band_weighted_f16": ("core", False, 6, True, 65)}


@pytest.mark.parametrize("seed", SEEDS)
@pytest.mark.parametrize("name", sorted(LOCAL_CASES))
def test_dit_local_conditioning_vs_oracle(ctx, name, seed):
    scope, dora, window, weighted, local_dim = LOCAL_CASES[name]
    assert_shipped_options(ctx)
    cfg = dict(CFG, dora=dora, window=window, local_dim=local_dim)
    wtype = sa3k.TYPE_F32 if name.endswith("f32") else sa3k.TYPE_F16
    tensors, adapters, inputs = db.random_dit(seed, cfg, scope)
    if wtype == sa3k.TYPE_F16:
        tensors = {k: (v.astype(np.float16).astype(np.float32) if k.endswith(".weight") else v)
                   for k, v in tensors.items()}
    lw = None
    if weighted:
        lw = np.random.Generator(np.random.Philox(seed + 7)).uniform(
            0, 2.0 / (cfg["io"] * cfg["T"]), (cfg["B"], cfg["T"])).astype(np.float32)
    print(f"[local] {name}", flush=True)
    d = make_gpu(ctx, cfg, tensors, adapters, scope, wtype)
    try:
        assert [t[0] for t in d.targets()] == db.target_names(cfg, scope)
        up, lw_d = upload_inputs(ctx, inputs, lw)
        d.set_local(up["local"])
        loss = d.accumulate(up["x_t"], up["target"], up["t"], up["cross"], up["glob"], lw_d)
        vel = ctx.empty((cfg["B"], cfg["T"], cfg["io"]))
        d.forward(up["x_t"], up["t"], up["cross"], up["glob"], vel)
        ev = d.eval_loss(up["x_t"], up["target"], up["t"], up["cross"], up["glob"], lw_d)
        assert np.array_equal(ev, loss)
        got = grads_by_target(d, d.arena(1).numpy())
        ref_loss, ref_vel, ref = db.dit_loss(cfg, tensors, adapters, inputs, loss_weight=lw)
        assert np.allclose(loss, ref_loss, rtol=1e-3), (loss, ref_loss)
        check(vel.numpy(), ref_vel, "velocity")
        assert any(".local." in n for n in ref) == (scope == "full")
        for n, (dA, dB, dm) in ref.items():   # every target, head and tail included
            check(got[n][0], dA, f"dA {n}")
            check(got[n][1], dB, f"dB {n}")
            if dora:
                check(got[n][2], dm, f"dm {n}")
    finally:
        d.destroy()


def test_dit_local_conditioning_schedules_and_unbound(ctx):
    cfg = dict(CFG, window=4, local_dim=65)
    tensors, adapters, inputs = db.random_dit(46, cfg, "full")
    up, _ = upload_inputs(ctx, inputs)
    runs = []
    for recompute in (False, True):
        d = make_gpu(ctx, cfg, tensors, adapters, "full", sa3k.TYPE_F16, recompute)
        d.set_local(up["local"])
        l1 = d.accumulate(up["x_t"], up["target"], up["t"], up["cross"], up["glob"])
        runs.append((l1, d.arena(1).numpy()))
        d.destroy()
    assert np.array_equal(runs[0][0], runs[1][0]) and np.array_equal(runs[0][1], runs[1][1]), \
        "resident and recompute schedules must agree bitwise with the local add"
    # no conditioning bound: the model without the local add, no gradient for the local adapters
    d = make_gpu(ctx, cfg, tensors, adapters, "full", sa3k.TYPE_F16)
    base_cfg = dict(cfg, local_dim=0)
    base = {n: a for n, a in adapters.items() if ".local." not in n}
    d0 = make_gpu(ctx, base_cfg, {k: v for k, v in tensors.items() if ".local." not in k}, base, "full",
                  sa3k.TYPE_F16)
    try:
        l_un = d.accumulate(up["x_t"], up["target"], up["t"], up["cross"], up["glob"])
        l_0 = d0.accumulate(up["x_t"], up["target"], up["t"], up["cross"], up["glob"])
        assert np.array_equal(l_un, l_0)
        g_un, g_0 = grads_by_target(d, d.arena(1).numpy()), grads_by_target(d0, d0.arena(1).numpy())
        for n, gr in g_un.items():
            if ".local." in n:
                assert not any(np.any(a) for a in gr if a is not None), n
            else:
                assert all(np.array_equal(a, b) for a, b in zip(gr, g_0[n]) if a is not None), n
        assert not np.array_equal(l_un, runs[0][0]), "the local add changes the loss"
    finally:
        d.destroy()
        d0.destroy()


def test_dit_schedules_accumulation_and_adamw(ctx):
    cfg = dict(CFG, window=4)
    tensors, adapters, inputs = db.random_dit(43, cfg, "full")
    runs = []
    for recompute in (False, True):
        d = make_gpu(ctx, cfg, tensors, adapters, "full", sa3k.TYPE_F16, recompute)
        up, _ = upload_inputs(ctx, inputs)
        l1 = d.accumulate(up["x_t"], up["target"], up["t"], up["cross"], up["glob"])
        g1 = d.arena(1).numpy()
        l2 = d.accumulate(up["x_t"], up["target"], up["t"], up["cross"], up["glob"])
        g2 = d.arena(1).numpy()
        assert np.array_equal(l1, l2)
        # each target's gradient is added in several terms, so the sum is 2 g1 up to f32 rounding
        assert rel_err(g2, 2 * g1) < 1e-6, "two identical micro-batches must add"
        p0, m0, v0 = d.arena(0).numpy(), d.arena(2).numpy(), d.arena(3).numpy()
        nrm = d.apply_adamw(HP, 1, want_norm=True)
        _, gscale = ctx.adamw_clip_scale()
        # oracle: train_apply_accumulated_adamw on the same arena, count = 2 micro-batches x 2 samples
        pr, _, mr, vr, onorm, oscale = oracle.apply_accumulated_adamw(p0, g2, m0, v0, *HP, 1, 4)
        assert abs(nrm - onorm) <= 1e-12 * max(1.0, onorm)
        assert np.float32(gscale) == np.float32(oscale)
        assert np.array_equal(d.arena(0).numpy(), pr)
        assert np.array_equal(d.arena(2).numpy(), mr) and np.array_equal(d.arena(3).numpy(), vr)
        assert not np.any(d.arena(1).numpy()), "the accumulator is cleared"
        runs.append((l1, g1))
        d.destroy()
    assert np.array_equal(runs[0][0], runs[1][0]) and np.array_equal(runs[0][1], runs[1][1]), \
        "resident and recompute schedules must agree bitwise"


@pytest.mark.parametrize("local_dim", [0, 65])
def test_dit_graph_replays_match_eager(ctx, local_dim):
    # the captured step (with and without the adapter refresh) replayed over several updates, with
    # eager work and host round trips in between, gives the eager path's results bit for bit; with
    # the inpaint local conditioning, the captured graph also holds the per-block events of the
    # local MLPs on the second stream and their shared backward scratch
    cfg = dict(CFG, window=6, local_dim=local_dim)
    tensors, adapters, inputs = db.random_dit(44, cfg, "full")
    models = []
    up, _ = upload_inputs(ctx, inputs)
    for graphs in (False, True):
        d = make_gpu(ctx, cfg, tensors, adapters, "full", sa3k.TYPE_F16)
        d.set_graphs(graphs)
        if local_dim:
            d.set_local(up["local"])
        models.append(d)
    try:
        for step in range(1, 6):
            res = []
            for d in models:
                l1 = d.accumulate(up["x_t"], up["target"], up["t"], up["cross"], up["glob"])
                l2 = d.accumulate(up["x_t"], up["target"], up["t"], up["cross"], up["glob"])   # no refresh
                g = d.arena(1).numpy()
                d.apply_adamw(HP, step)
                res.append((l1, l2, g, d.arena(0).numpy(), d.arena(3).numpy()))
            for a, b in zip(res[0], res[1]):
                assert np.array_equal(a, b), f"graph replay differs from eager at step {step}"
        # a failed capture falls back to the eager step: the graph path must have run throughout
        assert models[1].graphs() == 1, "the step was not captured (eager fallback)"
    finally:
        for d in models:
            d.destroy()


@pytest.mark.parametrize("local_dim", [0, 65])
def test_dit_side_stream_matches_one_stream(ctx, local_dim):
    # the backward kernels forked to the context's second stream give the one-stream results bit for
    # bit, over two updates (adapter refresh and AdamW in between): with forks recorded by the
    # producer kernels or by separate event records, and with each block's last second-stream work
    # joined at the block's end or overlapping the next block (two blocks); with the head's context
    # MLP and x path on the third stream or not; with the inpaint local conditioning, the local
    # MLPs' forwards and backwards on the second stream too
    cfg = dict(CFG, window=5, local_dim=local_dim)
    tensors, adapters, inputs = db.random_dit(46, cfg, "full")
    schedules = [dict(side_stream=0), dict(side_stream=1, fork_tail=0, late_join=0, head_quick=0),
                 dict(side_stream=1, fork_tail=1, late_join=0, head_quick=1),
                 dict(side_stream=1, fork_tail=1, late_join=1, head_quick=1)]
    res = []
    try:
        for sched in schedules:
            for k, v in sched.items():
                ctx.set_option(k, v)
            d = make_gpu(ctx, cfg, tensors, adapters, "full", sa3k.TYPE_F16)
            up, _ = upload_inputs(ctx, inputs)
            if local_dim:
                d.set_local(up["local"])
            out = []
            for step in (1, 2):
                loss = d.accumulate(up["x_t"], up["target"], up["t"], up["cross"], up["glob"])
                out += [loss, d.arena(1).numpy()]
                d.apply_adamw(HP, step)
            out.append(d.arena(0).numpy())
            res.append(out)
            d.destroy()
    finally:
        ctx.set_options(ctx.defaults)
    for sched, r in zip(schedules[1:], res[1:]):
        for a, b in zip(res[0], r):
            assert np.array_equal(a, b), f"stream schedule {sched} changes the results"


@pytest.mark.parametrize("recompute", [0, 1])
def test_dit_stacked_context_kv_matches_per_block(ctx, recompute):
    # the blocks' context K/V projections computed as one product over their stacked merged weights
    # (option kv_stack) give the per-block products' loss and gradients within f32 summation-order
    # rounding, over two updates (refresh and AdamW between), resident and recomputed
    cfg = dict(CFG, window=4)
    tensors, adapters, inputs = db.random_dit(47, cfg, "full")
    res = []
    try:
        for kv in (0, 1):
            ctx.set_option("kv_stack", kv)
            d = make_gpu(ctx, cfg, tensors, adapters, "full", sa3k.TYPE_F16, recompute=recompute)
            up, _ = upload_inputs(ctx, inputs)
            out = []
            for step in (1, 2):
                loss = d.accumulate(up["x_t"], up["target"], up["t"], up["cross"], up["glob"])
                out += [np.float64(loss), d.arena(1).numpy()]
                d.apply_adamw(HP, step)
            res.append(out)
            d.destroy()
    finally:
        ctx.set_options(ctx.defaults)
    for a, b in zip(res[0], res[1]):
        assert rel_err(np.atleast_1d(b), np.atleast_1d(a)) < 1e-4


@pytest.mark.parametrize("side", [0, 1])
def test_dit_in_kernel_reductions_match_separate_launches(ctx, side):
    # every split reduction done by the last arriving workgroup (GEMM split-K under gemm_fixup; the
    # modulation gradients, the adapted linears' dA sums and their dU column reductions with the
    # rows step under tn_fuse bits 1, 2, 4) gives the separate-launch results bit for bit, on one
    # stream and on two (each stream with its own arrival counters)
    cfg = dict(CFG, window=4)
    tensors, adapters, inputs = db.random_dit(45, cfg, "full")
    res = []
    try:
        ctx.set_option("side_stream", side)
        for tn_fuse, fixup in ((0, 0), (1, 0), (7, 0), (0, 1), (7, 1), (0, 2)):
            ctx.set_option("tn_fuse", tn_fuse)
            ctx.set_option("gemm_fixup", fixup)
            d = make_gpu(ctx, cfg, tensors, adapters, "full", sa3k.TYPE_F16)
            up, _ = upload_inputs(ctx, inputs)
            loss = d.accumulate(up["x_t"], up["target"], up["t"], up["cross"], up["glob"])
            res.append((loss, d.arena(1).numpy()))
            d.destroy()
    finally:
        ctx.set_options(ctx.defaults)
    for other in res[1:]:
        assert np.array_equal(res[0][0], other[0]) and np.array_equal(res[0][1], other[1])


def test_dit_full_size_step(ctx):
    # 24 blocks, dim 1536, 24 heads, FFN 6144, io 64, batch 2 x (64 + 1024), 128 context tokens of 768,
    # in the shipped configuration
    assert_shipped_options(ctx)
    c = sa3k.dit_config(64, 1536, 24, 24, 768, 64, 256, 6144, window=256)
    d = sa3k.Dit(ctx, c, sa3k.TYPE_F16)
    try:
        d.init_random(1234, 0.02)
        d.setup(32, 32.0, True, sa3k.SCOPE_FULL, 2, 1024, 128, recompute=False)
        d.adapters_init(99, 0.01)
        g = np.random.Generator(np.random.Philox(5))
        x = ctx.upload(g.normal(0, 1, (2, 1024, 64)).astype(np.float32))
        tg = ctx.upload(g.normal(0, 1, (2, 1024, 64)).astype(np.float32))
        t = ctx.upload(g.uniform(0, 1, 2).astype(np.float32))
        cr = ctx.upload(g.normal(0, 1, (2, 128, 768)).astype(np.float32))
        gl = ctx.upload(g.normal(0, 1, (2, 768)).astype(np.float32))
        l0 = d.accumulate(x, tg, t, cr, gl)
        g0 = d.arena(1).numpy()
        assert np.all(np.isfinite(l0)) and np.all(np.isfinite(g0)) and np.any(g0)
        # the same micro-batch again, on a cleared accumulator, gives the same loss and gradients
        ctx.check(ctx.lib.sa3k_memset(ctx.h, d.arena(1).ptr, 0, d.arena(1).nbytes))
        assert np.array_equal(d.accumulate(x, tg, t, cr, gl), l0)
        assert np.array_equal(d.arena(1).numpy(), g0)
        losses = [float(np.mean(l0))]
        hp = (1e-3, 0.9, 0.999, 1e-8, 0.01, 1.0)
        for step in range(1, 4):
            d.apply_adamw(hp, step)
            losses.append(float(np.mean(d.accumulate(x, tg, t, cr, gl))))
        assert losses[-1] < losses[0], losses
    finally:
        d.destroy()
