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
        cnt, ms = prof["adamw_update"]
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
        # dominant kernel: the largest of the two base GEMMs (forward X W^T and backward dU W)
        N, i, o = self.N, self.in_, self.out_
        cands = {"lin_fwd_main": 2.0 * N * i * o + 2.0 * N * self.r * o,
                 "lin_bwd_dx": 2.0 * N * i * o + 2.0 * N * self.r * i + (2.0 * self.r * i * o if self.dora else 0)}
        k = max(cands, key=lambda n: prof.get(n, (1, 0.0))[1])
        cnt, ms = prof[k]
        avg = ms / cnt
        ach = cands[k] / (avg * 1e-3) / 1e12
        return {"kernel": k, "bound": "mfma", "achieved": round(ach, 1), "peak": self.peak, "unit": "TFLOP/s",
                "frac": round(ach / self.peak, 4), "traffic": None, "avg_launch_ms": round(avg, 5),
                "algorithmic_flops_per_launch": cands[k]}

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
        times = []
        t_end = time.time() + 10.0
        while time.time() < t_end or not times:
            t0 = time.perf_counter()
            oracle.dit_lin_fwd(self.X_host, Wd, self.A_host, self.B_host, self.s, self.dora, mag, bnsq)
            oracle.dit_lin_bwd(self.X_host, Wd, self.dY_host, self.A_host, self.B_host, self.s, self.dora, mag, bnsq)
            times.append(time.perf_counter() - t0)
        return {"value": round(float(np.median(times)) * 1e3, 1), "unit": "ms/update (fwd+bwd, same shapes)",
                "cores": oracle.lib().orc_num_threads(), "kind": "port",
                "sample": f"{len(times)} full-size fwd+bwd of the oracle restatement (double accumulation, OpenMP)"}


WORKLOADS = {"adamw": AdamWWorkload,
             "dora_linear": lambda ctx: LinearWorkload(ctx, "dora_q8"),
             "lora_linear": lambda ctx: LinearWorkload(ctx, "lora_f32")}
DEFAULT = "dora_linear"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default=DEFAULT, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the data-parallel design is described in DESIGN.md).", file=sys.stderr)
        sys.exit(2)

    sa3k = _load("sa3k", os.path.join(ROOT, "sa3.cpp_amd", "sa3k.py"))
    ctx = sa3k.Context(0)
    log(f"workload {a.workload}: setting up")
    wl = WORKLOADS[a.workload](ctx)
    ctx.sync()
    log(f"warmup {a.warmup}")
    for _ in range(a.warmup):
        wl.step()
    ctx.sync()
    # timed region: K steps bracketed by stream events (single process: the barrier is a no-op)
    log(f"timing {a.steps} steps")
    ctx.profile(True)
    ctx.profile_reset()
    ctx.sync()
    t0 = time.perf_counter()
    ctx.timer_start()
    for _ in range(a.steps):
        wl.step()
    ms_total = ctx.timer_stop()
    wall = time.perf_counter() - t0
    prof = ctx.profile_report()
    ctx.profile(False)
    ms_per_step = ms_total / a.steps
    log(f"{ms_per_step:.4f} ms/step (wall {wall * 1e3 / a.steps:.4f} ms/step); kernels: {prof}")

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
    }
    out.update(wl.extra(ms_per_step))
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
