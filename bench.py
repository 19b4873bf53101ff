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


WORKLOADS = {"adamw": AdamWWorkload}
DEFAULT = "adamw"


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
