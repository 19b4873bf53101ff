"""Benchmark of the DiT LoRA/DoRA training update on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints ONE JSON line. A step is one pass of the hot path over one batch of synthetic input that is
already resident in HBM. Inputs are drawn from a seeded Philox generator (numpy), so the oracle
and the GPU see identical tensors.
"""
import argparse
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "ms per DoRA update (DiT fwd+bwd+AdamW, 1 GPU); MFMA TFLOP/s; HBM GB/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_MFMA_PEAK_TFLOPS = 157.3


def _load(name, path):
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def rng(seed):
    return np.random.Generator(np.random.Philox(seed))


# ------------------------------------------------------------------------------------ workloads
class AdamWWorkload:
    """Fused AdamW + global L2 clip over the 48M-parameter f32 adapter arena (beta 0.9/0.999,
    eps 1e-8, wd 0.01, lr 1e-4, clip 1.0, grads ~ N(0, 1e-3), moments zero)."""
    name = "adamw_clip_48M"
    dtype = "f32"

    def __init__(self, ctx, n=48_000_000):
        self.ctx, self.n = ctx, n
        r = rng(5)
        self.p_host = r.normal(0, 0.05, n).astype(np.float32)
        self.g_host = r.normal(0, 1e-3, n).astype(np.float32)
        self.p = ctx.upload(self.p_host)
        self.g = ctx.upload(self.g_host)
        self.m = ctx.zeros(n)
        self.v = ctx.zeros(n)
        self.hp = (1e-4, 0.9, 0.999, 1e-8, 0.01, 1.0)
        self.k = 0

    def step(self):
        self.k += 1
        self.ctx.adamw_clip(self.p, self.g, self.m, self.v, self.hp, self.k, 1)

    def config(self):
        return {"workload": self.name, "params": self.n, "grad_clip": 1.0, "lr": 1e-4,
                "betas": [0.9, 0.999], "weight_decay": 0.01}

    def roofline(self, prof, steps):
        # dominant kernel: adamw_update reads p, g, m, v and writes p, m, v = 28 B/param
        cnt, ms = prof["adamw_update"][:2]
        avg_ms = ms / cnt
        achieved = 28.0 * self.n / (avg_ms * 1e-3) / 1e9
        return {"kernel": "adamw_update", "bound": "hbm", "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": None, "avg_launch_ms": round(avg_ms, 5),
                "algorithmic_bytes_per_launch": 28 * self.n}

    def extra(self, ms_per_step):
        return {"hbm_GBs_whole_update": round(32.0 * self.n / (ms_per_step * 1e-3) / 1e9, 1)}

    def cpu_baseline(self):
        oracle = _load("sa3_oracle", os.path.join(ROOT, "oracle", "oracle.py"))
        n = 8_000_000   # bounded sample of the same arena
        p, g = self.p_host[:n], self.g_host[:n]
        z = np.zeros(n, np.float32)
        times = []
        t_end = time.time() + 12.0
        while time.time() < t_end or len(times) < 2:
            t0 = time.perf_counter()
            oracle.apply_accumulated_adamw(p, g, z, z, *self.hp, 1, 1)
            times.append(time.perf_counter() - t0)
        per_param = float(np.median(times)) / n
        return {"value": round(per_param * self.n * 1e3, 2), "unit": "ms/update (48M params)", "cores": 1,
                "kind": "port", "sample": f"{len(times)} updates of an {n}-param slice of the arena, scaled to 48M"}


class LinearWorkload:
    """One full adapter update of a single functional LoRA/DoRA linear (dit_lin, src/dit.h:92-149):
    prepare (DoRA norms) + forward + backward + fused clip/AdamW over its adapter arena [A | B | m].

    dora_q8: DoRA rank 32 (alpha 32), 1536 -> 6144, Q8_0 base quantised from N(0, 0.02),
             X [2048 x 1536] ~ N(0,1), dY ~ N(0, 1e-2), bf16 MFMA.
    lora_f32: LoRA rank 16 (alpha 16), 1536 -> 1536, f32 base N(0, 0.02), fp32 MFMA."""

    def __init__(self, ctx, kind):
        sa3k = sys.modules["sa3k"]
        self.ctx, self.kind = ctx, kind
        if kind == "dora_q8":
            self.N, self.in_, self.out_, self.r, alpha = 2048, 1536, 6144, 32, 32.0
            self.dora, self.prec, self.dtype = True, sa3k.PREC_BF16, "bf16"
            self.name = "dora_linear_q8_0_2048x1536x6144_r32"
            self.peak = BF16_PEAK_TFLOPS
        else:
            self.N, self.in_, self.out_, self.r, alpha = 2048, 1536, 1536, 16, 16.0
            self.dora, self.prec, self.dtype = False, sa3k.PREC_F32, "f32"
            self.name = "lora_linear_f32_2048x1536x1536_r16"
            self.peak = FP32_MFMA_PEAK_TFLOPS
        self.s = alpha / self.r
        N, in_, out_, r = self.N, self.in_, self.out_, self.r
        g = rng(1 if kind == "dora_q8" else 0)
        self.X_host = g.normal(0, 1, (N, in_)).astype(np.float32)
        self.dY_host = g.normal(0, 1e-2, (N, out_)).astype(np.float32)
        self.W_host = g.normal(0, 0.02, (out_, in_)).astype(np.float32)
        bound = 1.0 / np.sqrt(in_)
        self.A_host = g.uniform(-bound, bound, (r, in_)).astype(np.float32)
        self.B_host = g.normal(0, 0.01, (out_, r)).astype(np.float32)
        if kind == "dora_q8":
            wf = ctx.upload(self.W_host)
            blocks = ctx.zeros(out_ * in_ // 32 * 34, np.uint8)
            ctx.q8_0_quantize(wf, blocks, out_ * in_)
            self.blocks_host = blocks.numpy()
            self.w = ctx.weight((self.blocks_host, in_, out_), sa3k.TYPE_Q8_0)
        else:
            self.w = ctx.weight(self.W_host, sa3k.TYPE_F32)
        self.lin = ctx.lin(self.w, r, self.prec, N)
        # adapter arena [A | B | m] (the reference's visit order A, B, magnitude per target)
        nA, nB, nm = r * in_, out_ * r, out_ if self.dora else 0
        self.n = nA + nB + nm
        self.p = ctx.zeros(self.n)
        ctx.copy_into(self.p.view(0, (nA,)), self.A_host.ravel())
        ctx.copy_into(self.p.view(nA, (nB,)), self.B_host.ravel())
        self.A, self.B = self.p.view(0, (r, in_)), self.p.view(nA, (out_, r))
        self.grad = ctx.zeros(self.n)
        self.gA, self.gB = self.grad.view(0, (r, in_)), self.grad.view(nA, (out_, r))
        self.m, self.v = ctx.zeros(self.n), ctx.zeros(self.n)
        if self.dora:
            self.bnsq = self.w.row_norm_sq(1e-12)
            norms = self.w.row_norms()
            ctx.check(ctx.lib.sa3k_copy_d2d(ctx.h, self.p.ptr + 4 * (nA + nB), norms.ptr, 4 * nm))
            self.mag, self.gm = self.p.view(nA + nB, (nm,)), self.grad.view(nA + nB, (nm,))
        else:
            self.bnsq = self.mag = self.gm = None
        self.X, self.dY = ctx.upload(self.X_host), ctx.upload(self.dY_host)
        self.Y, self.dX = ctx.empty((N, out_)), ctx.empty((N, in_))
        self.hp = (1e-4, 0.9, 0.999, 1e-8, 0.01, 1.0)
        self.k = 0

    def step(self):
        self.k += 1
        c = self.ctx
        self.lin.prepare(self.A, self.B, self.s, self.dora, self.mag, self.bnsq)
        c.check(c.lib.sa3k_memset(c.h, self.grad.ptr, 0, self.grad.nbytes))
        self.lin.forward(self.X, self.N, self.Y)
        self.lin.backward(self.X, self.N, self.dY, self.dX, self.gA, self.gB, self.gm)
        c.adamw_clip(self.p, self.grad, self.m, self.v, self.hp, self.k, 1)

    def flops(self):
        N, i, o, r = self.N, self.in_, self.out_, self.r
        main = 2.0 * N * i * o
        fwd = main + 2.0 * N * i * r + 2.0 * N * r * o + (2.0 * r * i * o if self.dora else 0.0)
        bwd = main + 2.0 * N * o * r + 2.0 * N * r * i + 2.0 * N * o * r + 2.0 * N * r * i + \
            (2.0 * r * i * o if self.dora else 0.0)
        return fwd, bwd

    def config(self):
        return {"workload": self.name, "tokens": self.N, "in": self.in_, "out": self.out_, "rank": self.r,
                "adapter": "dora-rows" if self.dora else "lora",
                "base": "q8_0" if self.kind == "dora_q8" else "f32"}

    def roofline(self, prof, steps):
        return gemm_roofline(prof, steps)

    def extra(self, ms_per_step):
        fwd, bwd = self.flops()
        return {"algorithmic_gflop_per_update": round((fwd + bwd) / 1e9, 2),
                "tflops_whole_update": round((fwd + bwd) / (ms_per_step * 1e-3) / 1e12, 1)}

    def cpu_baseline(self):
        oracle = _load("sa3_oracle", os.path.join(ROOT, "oracle", "oracle.py"))
        Wd = oracle.q8_0_dequant(self.blocks_host, self.out_ * self.in_).reshape(self.out_, self.in_) \
            if self.kind == "dora_q8" else self.W_host
        mag = oracle.row_norms(Wd) if self.dora else None
        bnsq = oracle.row_norm_sq(Wd) if self.dora else None
        def once():
            oracle.dit_lin_fwd(self.X_host, Wd, self.A_host, self.B_host, self.s, self.dora, mag, bnsq)
            oracle.dit_lin_bwd(self.X_host, Wd, self.dY_host, self.A_host, self.B_host, self.s, self.dora, mag, bnsq)
        with oracle.f32_mode():
            t, times = _median_time(once, runs=5)
        return {"value": round(t * 1e3, 1), "unit": "ms/update (fwd+bwd, same shapes)",
                "cores": oracle.lib().orc_num_threads(), "kind": "port",
                "sample": f"median of {len(times)} full-size fwd+bwd after a warm-up: the oracle restatement in its "
                          f"f32 mode (float accumulation, AVX2/FMA products, OpenMP)"}


class ChainWorkload:
    """Inference reuse: one forward of a composed adapter chain (build_functional_lora,
    src/lora.h:372-622, and the chain branch of dit_lin, src/dit.h:108-117) over a frozen Q8_0 base
    1536 -> 6144 at 2176 tokens: dora-rows r32 (strength 1), lora r16 (0.7), dora-rows r16 (0.5),
    folded at create; a step is the chain's forward (X f32 -> bf16, the rank GEMM, the base GEMM with
    the folded row scale and the stacked rank term). kind "q8": the base decoded from its Q8_0 blocks
    between LDS and the MFMAs (no bf16 copy); "q8_copy": the same chain over the bf16 working copy."""

    def __init__(self, ctx, kind):
        sa3k = sys.modules["sa3k"]
        oracle = _load("sa3_oracle", os.path.join(ROOT, "oracle", "oracle.py"))
        self.ctx, self.kind = ctx, kind
        self.N, self.in_, self.out_ = 2176, 1536, 6144
        self.dtype = "bf16"
        self.specs = [(1, 32, 32.0, 1.0), (0, 16, 16.0, 0.7), (1, 16, 32.0, 0.5)]
        g = rng(7)
        W = g.normal(0, 0.02, (self.out_, self.in_)).astype(np.float32)
        self.blocks = oracle.q8_0_quantize(W)
        self.Wdec = oracle.q8_0_dequant(self.blocks, self.out_ * self.in_).reshape(self.out_, self.in_)
        self.w = ctx.weight((self.blocks, self.in_, self.out_), sa3k.TYPE_Q8_0)
        if kind == "q8":
            self.w.drop_working_copy()
        norms = np.sqrt((self.Wdec.astype(np.float64) ** 2).sum(1))
        self.ads = []
        for dora, r, alpha, strength in self.specs:
            A = g.uniform(-1 / np.sqrt(self.in_), 1 / np.sqrt(self.in_), (r, self.in_)).astype(np.float32)
            B = g.normal(0, 0.02, (self.out_, r)).astype(np.float32)
            mag = (norms * (1.0 + 0.1 * g.standard_normal(self.out_))).astype(np.float32) if dora else None
            self.ads.append((dora, r, alpha, strength, A, B, mag))
        dev = [(d, r, a, st, ctx.upload(A), ctx.upload(B), ctx.upload(m) if m is not None else None)
               for d, r, a, st, A, B, m in self.ads]
        self.chain = ctx.lora_chain(self.w, dev, self.N)
        self.X_host = g.normal(0, 1, (self.N, self.in_)).astype(np.float32)
        self.X = ctx.upload(self.X_host)
        self.Y = ctx.empty((self.N, self.out_))

    def step(self):
        self.chain.forward(self.X, self.N, self.Y)

    def flops(self):
        R = sum(r for _, r, _, _ in self.specs)
        return 2.0 * self.N * self.in_ * self.out_ + 2.0 * self.N * self.in_ * R + 2.0 * self.N * R * self.out_

    def config(self):
        return {"workload": "lora_chain_q8_0_2176x1536x6144_3adapters" + ("" if self.kind == "q8" else "_bf16_copy"),
                "tokens": self.N, "in": self.in_, "out": self.out_, "adapters": "dora r32, lora r16, dora r16",
                "base": "q8_0 decoded in the GEMM" if self.kind == "q8" else "q8_0 via its bf16 working copy"}

    def roofline(self, prof, steps):
        return gemm_roofline(prof, steps)

    def extra(self, ms_per_step):
        return {"algorithmic_gflop_per_forward": round(self.flops() / 1e9, 2),
                "tflops_whole_forward": round(self.flops() / (ms_per_step * 1e-3) / 1e12, 1)}

    def cpu_baseline(self):
        oracle = _load("sa3_oracle", os.path.join(ROOT, "oracle", "oracle.py"))
        n = 128
        Xs = self.X_host[:n]
        t, times = _median_time(lambda: oracle.chain_forward(Xs, self.Wdec, self.ads), runs=3)
        return {"value": round(t * 1e3 * self.N / n, 1), "unit": "ms/forward", "cores": 1, "kind": "port",
                "sample": f"the oracle's chain forward (double accumulation) on {n} of the {self.N} tokens, median of "
                          f"{len(times)} after a warm-up ({t * 1e3:.1f} ms), scaled by {self.N}/{n}"}


def _median_time(fn, runs=3):
    """one untimed warm-up call (it also maps the memory the later calls reuse), then the median of
    `runs` timed calls: (median seconds, [seconds])"""
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), times


def block_flops(B, S, Ctx, dim, inner, r, window, dora=True, heads=None):
    """Algorithmic flops of one DiT block forward and backward (dit_block, src/dit.h:164-266).

    Linears: forward X W^T + the rank terms; backward dX only for the frozen base (no dW) + the
    rank terms (dU B, (dU B) A, dU^T H, (s dU B)^T X); dora adds W A^T (forward) and B^T gn W
    (backward). Attention: QK^T and PV per branch per kept (query, key) pair, 2 x 2 x 2 x 64
    flops; its backward counted as twice the forward. Recompute is not counted."""
    heads = heads or dim // 64
    N, NC = B * S, B * Ctx
    tg = [(dim, 5 * dim, N), (dim, dim, N), (dim, 2 * dim, N), (dim, 3 * dim, NC), (dim, dim, N),
          (dim, 2 * inner, N), (inner, dim, N)]
    fwd = bwd = 0.0
    for i, o, n in tg:
        fwd += 2.0 * n * i * o + 2.0 * n * i * r + 2.0 * n * r * o + (2.0 * r * i * o if dora else 0.0)
        bwd += 2.0 * n * o * i + 2.0 * n * r * i + 2.0 * n * o * r * 2 + 2.0 * n * r * i + \
            (2.0 * r * i * o if dora else 0.0)
    q = np.arange(S)
    if window > 0:
        h = window // 2
        pairs = float(np.sum(np.minimum(q + h, S - 1) - np.maximum(q - h, 0) + 1))
    else:
        pairs = float(S) * S
    attn = B * heads * (pairs + S * Ctx) * 2 * 2 * 2 * 64
    return fwd + attn, bwd + 2 * attn


class BlockWorkload:
    """One DiT block fwd+bwd + clip/AdamW over its adapter arena: dim 1536, 24 heads x 64, FFN
    1536 -> 2x6144 -> 1536 (SwiGLU), batch 2 x (64 memory + 1024 latent) tokens, self-attention
    window 256, cross-attention to 128 context tokens (already projected to 1536, N(0,1)), DoRA rank
    32 (alpha 32) on all 7 projections, f16 base ~ N(0, 0.02); gcond ~ N(0, 0.1), dout ~ N(0, 1e-2)."""
    name = "dit_block_1536_s1088_b2_w256_dora_r32"
    dtype = "bf16"

    def __init__(self, ctx, B=2, S=1088, Ctx=128, dim=1536, heads=24, inner=6144, r=32, window=256, seed=7):
        sa3k = sys.modules["sa3k"]
        self.ctx = ctx
        self.B, self.S, self.Ctx, self.dim, self.heads, self.inner, self.r, self.window = \
            B, S, Ctx, dim, heads, inner, r, window
        g = rng(seed)
        nd = lambda shape, sd: g.normal(0, sd, shape).astype(np.float32)
        dims = sa3k.block_target_dims(dim, inner)
        self.W_host = [nd((o, i), 0.02).astype(np.float16) for i, o in dims]
        self.bias_host = [None] * 5 + [nd(dims[5][1], 0.02), nd(dims[6][1], 0.02)]
        self.vecs = dict(ssg=nd(6 * dim, 0.1), pre_g=1 + nd(dim, 0.1), cross_g=1 + nd(dim, 0.1),
                         ff_g=1 + nd(dim, 0.1), sq_g=1 + nd(64, 0.1), sk_g=1 + nd(64, 0.1), cq_g=1 + nd(64, 0.1),
                         ck_g=1 + nd(64, 0.1))
        self.cfg = sa3k.BlockConfig(dim, heads, 64, inner, 32, window, 1e4, 1e-5, 1e-6)
        self.blk = sa3k.Block(ctx, self.cfg, self.W_host, self.bias_host, self.vecs, r, B * S, B * Ctx,
                              sa3k.TYPE_F16)
        # adapter arena: per target [A | B | m] (A Kaiming-uniform, B ~ N(0, 0.01), m = row norms)
        sizes = [(r * i, o * r, o) for i, o in dims]
        self.n = sum(a + b + m for a, b, m in sizes)
        self.p, self.grad = ctx.zeros(self.n), ctx.zeros(self.n)
        self.m, self.v = ctx.zeros(self.n), ctx.zeros(self.n)
        self.A, self.Bm, self.mag, self.gA, self.gB, self.gm = [], [], [], [], [], []
        self.A_host, self.B_host, self.mag_host = [], [], []
        off = 0
        for (i, o), (na, nb, nm), W in zip(dims, sizes, self.W_host):
            a = g.uniform(-1 / np.sqrt(i), 1 / np.sqrt(i), (r, i)).astype(np.float32)
            b = nd((o, r), 0.01)
            mg = np.sqrt((W.astype(np.float64) ** 2).sum(1)).astype(np.float32)
            for host, lst, glst, n_, shape in ((a, self.A, self.gA, na, (r, i)), (b, self.Bm, self.gB, nb, (o, r)),
                                                (mg, self.mag, self.gm, nm, (o,))):
                ctx.copy_into(self.p.view(off, (n_,)), host.ravel())
                lst.append(self.p.view(off, shape))
                glst.append(self.grad.view(off, shape))
                off += n_
            self.A_host.append(a)
            self.B_host.append(b)
            self.mag_host.append(mg)
        self.x_host = nd((B, S, dim), 1.0)
        self.ctx_host = nd((B, Ctx, dim), 1.0)
        self.gc_host = nd((B, 6 * dim), 0.1)
        self.dout_host = nd((B, S, dim), 1e-2)
        self.x, self.cx, self.gc = ctx.upload(self.x_host), ctx.upload(self.ctx_host), ctx.upload(self.gc_host)
        self.dout = ctx.upload(self.dout_host)
        self.out, self.dx = ctx.empty((B, S, dim)), ctx.empty((B, S, dim))
        self.dctx, self.dgc = ctx.zeros((B, Ctx, dim)), ctx.zeros((B, 6 * dim))
        self.ws = sa3k.BlockWorkspace(ctx, self.cfg, B, S, Ctx)
        self.hp = (1e-4, 0.9, 0.999, 1e-8, 0.01, 1.0)
        self.k = 0

    def step(self):
        self.k += 1
        c = self.ctx
        self.blk.prepare(self.A, self.Bm, 1.0, True, self.mag)
        c.check(c.lib.sa3k_memset(c.h, self.grad.ptr, 0, self.grad.nbytes))
        self.blk.forward(self.ws, self.x, self.cx, self.gc, self.out)
        self.blk.backward(self.ws, self.dout, self.dx, self.dctx, self.dgc, self.gA, self.gB, self.gm)
        c.adamw_clip(self.p, self.grad, self.m, self.v, self.hp, self.k, 1)

    def flops(self):
        return block_flops(self.B, self.S, self.Ctx, self.dim, self.inner, self.r, self.window)

    def config(self):
        return {"workload": self.name, "batch": self.B, "tokens_per_sample": self.S, "memory_tokens": 64,
                "context_tokens": self.Ctx, "dim": self.dim, "heads": self.heads, "ffn_inner": self.inner,
                "window": self.window, "rank": self.r, "adapter": "dora-rows", "base": "f16"}

    def roofline(self, prof, steps):
        return gemm_roofline(prof, steps)

    def extra(self, ms_per_step):
        fwd, bwd = self.flops()
        return {"algorithmic_gflop_per_update": round((fwd + bwd) / 1e9, 2),
                "tflops_whole_update": round((fwd + bwd) / (ms_per_step * 1e-3) / 1e12, 1)}

    def oracle_block(self):
        """the oracle's view of this block (full size): (block_binding, cfg, weights, x, ctx, gcond, dout)"""
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        _load("oracle", os.path.join(ROOT, "oracle", "oracle.py"))
        bb = _load("block_binding", os.path.join(ROOT, "oracle", "block_binding.py"))
        cfg = dict(B=self.B, S=self.S, Ctx=self.Ctx, dim=self.dim, heads=self.heads, inner=self.inner,
                   window=self.window, rank=self.r, alpha=32.0, dora=True)
        W = [w.astype(np.float32) for w in self.W_host]
        w = dict(self.vecs, W=W, bias=self.bias_host, A=self.A_host, B=self.B_host, mag=self.mag_host,
                 bnsq=[((x.astype(np.float64) ** 2).sum(1) + x.shape[1] * 1e-12).astype(np.float32) for x in W])
        return bb, cfg, w, self.x_host, self.ctx_host, self.gc_host, self.dout_host

    def cpu_baseline(self):
        bb, cfg, w, x, ctx, gc, dout = self.oracle_block()
        with sys.modules["oracle"].f32_mode():
            t, times = _median_time(lambda: bb.block_bwd(cfg, w, x, ctx, gc, dout), runs=3)
        return {"value": round(t * 1e3, 1), "unit": "ms/update (block fwd+bwd at full size)",
                "cores": bb.lib().orc_num_threads(), "kind": "port",
                "sample": f"median of {len(times)} runs after a warm-up ({', '.join(f'{v:.2f}' for v in times)} s) "
                          f"of the oracle block forward + backward at B={self.B}, S={self.S} in its f32 mode "
                          f"(float accumulation, AVX2/FMA products, OpenMP); the adapter update itself not included"}


def dit_head_flops(B, T, Ctx, io, dim, cond_dim, time_dim, r, dora=True, adapted=True):
    """(forward, backward) algorithmic flops of the 12 head/tail linears (same conventions)"""
    tg = [(io, io, B * T), (io, dim, B * T), (time_dim, dim, B), (dim, dim, B), (cond_dim, dim, B), (dim, dim, B),
          (dim, dim, B), (dim, 6 * dim, B), (cond_dim, dim, B * Ctx), (dim, dim, B * Ctx), (dim, io, B * T),
          (io, io, B * T)]
    fwd = bwd = 0.0
    for i, o, n in tg:
        fwd += 2.0 * n * i * o
        bwd += 2.0 * n * o * i
        if adapted:
            fwd += 2.0 * n * i * r + 2.0 * n * r * o + (2.0 * r * i * o if dora else 0.0)
            bwd += 2.0 * n * r * i + 2.0 * n * o * r * 2 + 2.0 * n * r * i + (2.0 * r * i * o if dora else 0.0)
    return fwd, bwd


class DitWorkload:
    """One full DoRA update of the 24-block DiT: forward + velocity MSE + backward through every
    adapter (all 168 block projections + the 12 head/tail linears, rank 32, alpha 32) and the fused
    clip + AdamW over the 43.4M-parameter arena. dim 1536, 24 heads x 64, FFN 6144, io 64, batch 2 x
    (64 memory + 1024 latent) tokens, self-attention window 256, 128 context tokens of 768, f16 base
    ~ N(0, 0.02) (random init on the device); x_t, target ~ N(0,1), t ~ U(0,1). Every block keeps
    its activations (no recompute; the checkpointed schedule is --recompute). local_dim > 0 adds each
    block's inpaint local-conditioning MLP (local.0 local_dim -> 1536, SiLU, local.2 1536 -> 1536, both
    adapted: 228 targets) with a bound [B][T][local_dim] conditioning ~ N(0,1)."""
    dtype = "bf16"

    def __init__(self, ctx, recompute=False, B=2, T=1024, Ctx=128, depth=24, window=256, r=32, local_dim=0, micro=1):
        sa3k = sys.modules["sa3k"]
        self.ctx, self.B, self.T, self.Ctx, self.depth, self.window, self.r = ctx, B, T, Ctx, depth, window, r
        self.micro = micro   # accumulate calls (micro-batches of B samples) per optimizer update
        self.dim, self.heads, self.inner, self.io, self.cond_dim, self.time_dim, self.mem = 1536, 24, 6144, 64, 768, 256, 64
        self.recompute, self.local_dim = recompute, local_dim
        self.name = f"dit_update_{depth}x1536_b{B}_t{T}_w{window}_dora_r{r}" + ("_recompute" if recompute else "") + \
            (f"_inpaint_local{local_dim}" if local_dim else "") + (f"_x{micro}" if micro > 1 else "")
        cfg = sa3k.dit_config(self.io, self.dim, depth, self.heads, self.cond_dim, self.mem, self.time_dim,
                              self.inner, window, local_dim=local_dim)
        self.d = sa3k.Dit(ctx, cfg, sa3k.TYPE_F16)
        self.d.init_random(1234, 0.02)
        self.d.setup(r, 32.0, True, sa3k.SCOPE_FULL, B, T, Ctx, recompute)
        self.d.adapters_init(99, 0.01)
        self.n = self.d.arena(0).size
        g = rng(4)
        self.host = dict(x=g.normal(0, 1, (B, T, self.io)).astype(np.float32),
                         tg=g.normal(0, 1, (B, T, self.io)).astype(np.float32),
                         t=g.uniform(0, 1, B).astype(np.float32),
                         cr=g.normal(0, 1, (B, Ctx, self.cond_dim)).astype(np.float32),
                         gl=g.normal(0, 1, (B, self.cond_dim)).astype(np.float32))
        if local_dim:
            self.host["lc"] = g.normal(0, 1, (B, T, local_dim)).astype(np.float32)
        self.dev = {k: ctx.upload(v) for k, v in self.host.items()}
        if local_dim:
            self.d.set_local(self.dev["lc"])
        self.hp = (1e-4, 0.9, 0.999, 1e-8, 0.01, 1.0)
        self.k = 0

    def step(self):
        self.k += 1
        v = self.dev
        for _ in range(self.micro):
            self.d.accumulate(v["x"], v["tg"], v["t"], v["cr"], v["gl"], want_loss=False)
        self.d.apply_adamw(self.hp, self.k)

    def flops(self):
        S = self.mem + self.T
        f, b = block_flops(self.B, S, self.Ctx, self.dim, self.inner, self.r, self.window)
        hf, hb = dit_head_flops(self.B, self.T, self.Ctx, self.io, self.dim, self.cond_dim, self.time_dim, self.r)
        if self.local_dim:   # the local MLP's base products: forward both, backward local.2's dX
            n = self.B * self.T
            hf += self.depth * 2 * n * self.dim * (self.local_dim + self.dim)
            hb += self.depth * 2 * n * self.dim * self.dim
        return self.micro * (self.depth * f + hf), self.micro * (self.depth * b + hb)

    def config(self):
        return {"workload": self.name, "blocks": self.depth, "batch": self.B, "frames": self.T,
                "memory_tokens": self.mem, "context_tokens": self.Ctx, "io": self.io, "dim": self.dim,
                "heads": self.heads, "ffn_inner": self.inner, "window": self.window, "rank": self.r,
                "adapter": "dora-rows", "base": "f16",
                "scope": f"full ({(9 if self.local_dim else 7) * self.depth + 12} targets)",
                **({"local_dim": self.local_dim} if self.local_dim else {}),
                "adapter_params": self.n, "schedule": "checkpointed recompute" if self.recompute else "resident",
                **({"micro_batches_per_update": self.micro} if self.micro > 1 else {})}

    def roofline(self, prof, steps):
        return gemm_roofline(prof, steps)

    def extra(self, ms_per_step):
        fwd, bwd = self.flops()
        return {"algorithmic_gflop_per_update": round((fwd + bwd) / 1e9, 1),
                "tflops_whole_update": round((fwd + bwd) / (ms_per_step * 1e-3) / 1e12, 1)}

    def cpu_baseline(self):
        """The oracle in its f32 mode on the host cores, timed, not extrapolated: one block of this model
        at full size (B 2, S 64 + 1024, window 256, DoRA r 32 on all 7 projections), forward + backward,
        median of 3 runs after a warm-up; the head and tail (a depth-0 DiT loss + gradient at T 1024,
        median of 3); the update = head/tail + 24 x block. The AdamW step is not included."""
        blk = BlockWorkload.__new__(BlockWorkload)
        g = rng(7)
        nd = lambda shape, sd: g.normal(0, sd, shape).astype(np.float32)
        S = self.mem + self.T
        dims = sys.modules["sa3k"].block_target_dims(self.dim, self.inner)
        blk.B, blk.S, blk.Ctx, blk.dim, blk.heads, blk.inner, blk.r, blk.window = \
            self.B, S, self.Ctx, self.dim, self.heads, self.inner, self.r, self.window
        blk.W_host = [nd((o, i), 0.02) for i, o in dims]
        blk.bias_host = [None] * 5 + [nd(dims[5][1], 0.02), nd(dims[6][1], 0.02)]
        blk.vecs = dict(ssg=nd(6 * self.dim, 0.1), pre_g=1 + nd(self.dim, 0.1), cross_g=1 + nd(self.dim, 0.1),
                        ff_g=1 + nd(self.dim, 0.1), sq_g=1 + nd(64, 0.1), sk_g=1 + nd(64, 0.1),
                        cq_g=1 + nd(64, 0.1), ck_g=1 + nd(64, 0.1))
        blk.A_host = [g.uniform(-1 / np.sqrt(i), 1 / np.sqrt(i), (self.r, i)).astype(np.float32) for i, o in dims]
        blk.B_host = [nd((o, self.r), 0.01) for i, o in dims]
        blk.mag_host = [np.sqrt((W.astype(np.float64) ** 2).sum(1)).astype(np.float32) for W in blk.W_host]
        blk.x_host, blk.ctx_host = nd((self.B, S, self.dim), 1.0), nd((self.B, self.Ctx, self.dim), 1.0)
        blk.gc_host, blk.dout_host = nd((self.B, 6 * self.dim), 0.1), nd((self.B, S, self.dim), 1e-2)
        bb, cfg, w, x, ctx, gc, dout = blk.oracle_block()
        db = _load("dit_binding", os.path.join(ROOT, "oracle", "dit_binding.py"))
        hcfg = dict(B=self.B, T=self.T, Ctx=self.Ctx, io=self.io, dim=self.dim, heads=self.heads,
                    inner=self.inner, depth=0, mem=self.mem, cond_dim=self.cond_dim, time_dim=self.time_dim,
                    rope_dims=32, window=self.window, rank=self.r, alpha=32.0, dora=True)
        tensors, adapters, inputs = db.random_dit(3, hcfg, "full", w_sd=0.02, b_sd=0.01)
        with sys.modules["oracle"].f32_mode():
            t_b, tb = _median_time(lambda: bb.block_bwd(cfg, w, x, ctx, gc, dout), runs=3)
            t_h, th = _median_time(lambda: db.dit_loss(hcfg, tensors, adapters, inputs), runs=3)
        # the clip + AdamW of the reference's loop (the oracle's literal transcription, one core) over
        # an 8M-parameter slice of the arena, scaled to its size
        oracle = sys.modules["sa3_oracle"] if "sa3_oracle" in sys.modules else \
            _load("sa3_oracle", os.path.join(ROOT, "oracle", "oracle.py"))
        ns = 8_000_000
        pa, ga = g.normal(0, 0.05, ns).astype(np.float32), g.normal(0, 1e-3, ns).astype(np.float32)
        z = np.zeros(ns, np.float32)
        t_a, ta = _median_time(lambda: oracle.apply_accumulated_adamw(pa, ga, z, z, *self.hp, 1, 1), runs=3)
        t_adamw = t_a / ns * self.n
        value = t_h + self.depth * t_b + t_adamw
        return {"value": round(value * 1e3, 1), "unit": "ms/update (forward + backward + clip/AdamW)",
                "cores": bb.lib().orc_num_threads(), "kind": "port",
                "sample": f"the oracle in its f32 mode (float accumulation, AVX2/FMA products, OpenMP): one "
                          f"full-size block fwd+bwd (B {self.B}, S {S}), median of {len(tb)} after a warm-up "
                          f"= {t_b:.2f} s ({', '.join(f'{v:.2f}' for v in tb)}); head + tail (depth-0 DiT "
                          f"loss+grad, T {self.T}) median {t_h:.2f} s; clip + AdamW (one core) over an "
                          f"{ns}-param slice, median {t_a:.3f} s, scaled to the {self.n}-param arena "
                          f"= {t_adamw:.3f} s; update = head/tail + {self.depth} x block + AdamW"}


class MirrorWorkload:
    """The reference trainer's default update (tools/sa3-train.cpp:574-714) through the C++ host
    mirror of its interface (sa3.cpp_amd/host/sa3/*.h, driven by host/mirror_bench.cpp in
    libsa3mirror.so): the same 24-block model and full-scope dora-rows r32 adapters as `dit`
    (adapters from init_train_lora_state), build_train_dit_ckpt (which keeps every block's
    activations when they fit), then per update two samples of 1024 frames, one per
    run_train_dit_accumulate_ckpt call as the reference runs them, and train_apply_accumulated_adamw.
    device_resident: the adapters, the gradient window and the moments stay on the device (this
    build's mode); otherwise the reference's per-sample upload / gradient read-back and the host
    AdamW vectors (round trips through PCIe). Timed by the wall clock: every call synchronises."""
    dtype = "bf16"
    wall_timed = True

    def __init__(self, ctx, device_resident=True, micro=2, frames=1024):
        import ctypes as C
        self.C = C
        self.lib = C.CDLL(os.path.join(ROOT, "sa3.cpp_amd", "libsa3mirror.so"))
        self.lib.sa3m_create.restype = C.c_void_p
        self.lib.sa3m_create.argtypes = [C.c_int, C.c_int, C.c_int, C.c_char_p, C.c_int]
        self.lib.sa3m_update.argtypes = [C.c_void_p, C.c_char_p, C.c_int]
        self.lib.sa3m_info.argtypes = [C.c_void_p, C.POINTER(C.c_int), C.POINTER(C.c_longlong),
                                       C.POINTER(C.c_double), C.POINTER(C.c_double)]
        self.lib.sa3m_destroy.argtypes = [C.c_void_p]
        self.err = C.create_string_buffer(1024)
        self.h = self.lib.sa3m_create(int(device_resident), micro, frames, self.err, 1024)
        if not self.h:
            raise RuntimeError("mirror setup: " + self.err.value.decode())
        self.device_resident, self.micro, self.frames = device_resident, micro, frames
        self.name = f"dit_update_mirror_24x1536_{micro}x1_t{frames}_w256_dora_r32" + \
            ("" if device_resident else "_roundtrip")

    def step(self):
        if self.lib.sa3m_update(self.h, self.err, 1024) != 0:
            raise RuntimeError("mirror update: " + self.err.value.decode())

    def info(self):
        C = self.C
        rc, n, loss, norm = C.c_int(), C.c_longlong(), C.c_double(), C.c_double()
        self.lib.sa3m_info(self.h, C.byref(rc), C.byref(n), C.byref(loss), C.byref(norm))
        return rc.value, n.value, loss.value, norm.value

    def config(self):
        rc, n, _, _ = self.info()
        return {"workload": self.name, "blocks": 24, "samples_per_update": self.micro, "batch_per_call": 1,
                "frames": self.frames, "memory_tokens": 64, "context_tokens": 128, "io": 64, "dim": 1536,
                "heads": 24, "ffn_inner": 6144, "window": 256, "rank": 32, "adapter": "dora-rows", "base": "f16",
                "scope": "full (180 targets)", "adapter_params": n,
                "path": "host mirror (train_loop.h) " + ("device-resident" if self.device_resident else
                                                         "per-sample round trips"),
                "schedule": "checkpointed recompute" if rc else "resident"}

    def roofline(self, prof, steps):
        return None

    def extra(self, ms_per_step):
        _, _, loss, norm = self.info()
        return {"last_mean_loss": round(loss, 6), "last_grad_norm": round(norm, 6)}

    def cpu_baseline(self):
        return None


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed PMC summaries under profiles/ (a line
    'traffic: kernel=<name> bytes_per_launch=<B>', written from rocprofv3 FETCH_SIZE + WRITE_SIZE
    runs scaled by the counters' reading for a copy of known size), or None."""
    pdir = os.path.join(ROOT, "profiles")
    if not os.path.isdir(pdir):
        return None
    for f in sorted(os.listdir(pdir)):
        if not f.endswith(".md"):
            continue
        for line in open(os.path.join(pdir, f)):
            if line.startswith("traffic:") and f"kernel={kernel} " in line + " ":
                return float(line.split("bytes_per_launch=")[1].split()[0])
    return None


def gemm_roofline(prof, steps):
    """Roofline of the GEMM kernel instantiation with the largest total time. The library counts
    each launch's algorithmic flops, 2 (M + extra rows) N (K + rank extension), at launch time, so
    achieved = counted flops / measured time = flops per launch / average launch duration."""
    cands = {k: v for k, v in prof.items() if k.startswith(("gemm_dma<", "gemm_big<", "gemm_decode<")) and v[2] > 0}
    k = max(cands, key=lambda n: cands[n][1])
    cnt, ms, work = cands[k]
    peak = BF16_PEAK_TFLOPS if k.endswith("bf16>") else FP32_MFMA_PEAK_TFLOPS
    ach = work / (ms * 1e-3) / 1e12
    return {"kernel": k, "bound": "mfma", "achieved": round(ach, 1), "peak": peak, "unit": "TFLOP/s",
            "frac": round(ach / peak, 4), "traffic": measured_traffic(k), "avg_launch_ms": round(ms / cnt, 5),
            "launches_per_step": round(cnt / steps, 1), "algorithmic_flops_per_launch": work / cnt}


WORKLOADS = {"adamw": AdamWWorkload,
             "dora_linear": lambda ctx: LinearWorkload(ctx, "dora_q8"),
             "lora_linear": lambda ctx: LinearWorkload(ctx, "lora_f32"),
             "block": BlockWorkload,
             "dit": DitWorkload,
             "dit_recompute": lambda ctx: DitWorkload(ctx, recompute=True),
             "dit_inpaint": lambda ctx: DitWorkload(ctx, local_dim=257),
             "dit_inpaint_recompute": lambda ctx: DitWorkload(ctx, recompute=True, local_dim=257),
             "dit_b1x2": lambda ctx: DitWorkload(ctx, B=1, micro=2),
             "dit_mirror": lambda ctx: MirrorWorkload(ctx, device_resident=True),
             "dit_mirror_roundtrip": lambda ctx: MirrorWorkload(ctx, device_resident=False),
             "chain_q8": lambda ctx: ChainWorkload(ctx, "q8"),
             "chain_q8_copy": lambda ctx: ChainWorkload(ctx, "q8_copy")}
DEFAULT = "dit"
WALL_TIMED = {"dit_mirror", "dit_mirror_roundtrip"}


class _WallClock:
    """Stands in for the library context in main() for a workload that runs on a context of its own
    (timed by the wall clock)."""

    def sync(self):
        pass

    def timer_start(self):
        pass

    def timer_stop(self):
        return 0.0

    def close(self):
        pass


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default=DEFAULT, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="only run 5 device-to-device copies of this many bytes (the reference kernel of "
                         "known traffic that scales the FETCH_SIZE / WRITE_SIZE counters) and exit")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the library has no multi-GPU path "
              "(data-parallel sharding of the update over ranks is not implemented).", file=sys.stderr)
        sys.exit(2)

    sa3k = _load("sa3k", os.path.join(ROOT, "sa3.cpp_amd", "sa3k.py"))
    # the mirror workloads run on the host mirror's own context; a second context here would share
    # the process's hardware queues with its streams
    ctx = _WallClock() if a.workload in WALL_TIMED else sa3k.Context(0)
    if a.copy_bytes > 0:
        src, dst = ctx.empty(a.copy_bytes // 4, np.float32), ctx.empty(a.copy_bytes // 4, np.float32)
        for _ in range(5):
            ctx.copy_d2d(dst, src, a.copy_bytes // 4 * 4)
        ctx.sync()
        print(json.dumps({"copy_bytes": a.copy_bytes // 4 * 4, "copies": 5}), flush=True)
        ctx.close()
        return
    log(f"workload {a.workload}: setting up")
    wl = WORKLOADS[a.workload](ctx)
    ctx.sync()
    log(f"warmup {a.warmup}")
    for _ in range(a.warmup):
        wl.step()
    ctx.sync()
    # timed region: K steps bracketed by stream events (single process: the barrier is a no-op);
    # per-kernel event timing is off here, so the DiT step runs eagerly on the library's two
    # streams (HIP-graph replay is an option of the library, off by default)
    log(f"timing {a.steps} steps")
    ctx.sync()
    t0 = time.perf_counter()
    ctx.timer_start()
    for _ in range(a.steps):
        wl.step()
    ms_total = ctx.timer_stop()
    wall = time.perf_counter() - t0
    ms_per_step = ms_total / a.steps
    if getattr(wl, "wall_timed", False):   # work on another context's streams: the wall clock
        ms_per_step = wall * 1e3 / a.steps
    log(f"{ms_per_step:.4f} ms/step (wall {wall * 1e3 / a.steps:.4f} ms/step)")
    prof, ms_prof = {}, None
    if not getattr(wl, "wall_timed", False):
        # profiled pass: the same K steps again with a HIP event pair around every kernel launch on
        # the library's stream (launched eagerly), for the per-kernel averages and the roofline
        ctx.profile(True)
        ctx.profile_reset()
        ctx.timer_start()
        for _ in range(a.steps):
            wl.step()
        ms_prof = ctx.timer_stop() / a.steps
        prof = ctx.profile_report(with_work=True)
        ctx.profile(False)
        log(f"profiled pass {ms_prof:.4f} ms/step; kernels: {prof}")

    cpu = None
    if not a.no_cpu_baseline:
        log("cpu baseline")
        cpu = wl.cpu_baseline()
    out = {
        "metric": METRIC, "value": round(ms_per_step, 5), "unit": "ms/update", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": wl.dtype,
        "data": "synthetic (seeded Philox normals; random-init weights)", "config": wl.config(),
        "roofline": wl.roofline(prof, a.steps), "cpu_baseline": cpu,
        "kernels_ms": {k: round(v[1] / max(v[0], 1), 5) for k, v in prof.items()},
        "profiled_pass_ms_per_step": round(ms_prof, 5) if ms_prof is not None else None,
    }
    out.update(wl.extra(ms_per_step))
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
