"""Write tests/golden/dit_autograd.npz: the whole DiT training loss (dit_head, dit_block x depth,
dit_tail, src/dit.h:269-338; MSE src/train_dit.h:174-184) of a depth-2 model and every adapter
gradient, from torch float64 autograd of a torch restatement that shares nothing with the
oracle's hand-derived backward; and tests/golden/dit_local_autograd.npz: the same for a model
with the inpaint local conditioning (dit.<l>.local.{0,2}, src/dit.h:244-254) and its per-block
MLP adapted in the full scope. Build-container only; the GPU tests never import torch.

python tests/golden/make_dit_fixtures.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
sys.path.insert(0, HERE)
from dit_binding import BLOCK_TARGETS, BLOCK_VECTORS, HEAD_TARGETS, HEAD_BIAS, random_dit, bnsq_of  # noqa: E402
from make_block_fixtures import T, block, lin  # noqa: E402

CFG = dict(B=2, T=12, Ctx=5, io=64, dim=128, heads=2, inner=128, depth=2, mem=4, cond_dim=64, time_dim=64,
           rope_dims=32, window=0, rank=8, alpha=16.0, dora=True)
CASES = {"full_dora_dense": (41, "full", True, 0, False), "core_lora_band_weighted": (42, "core", False, 6, True)}
# local_dim 65 = [mask | z * mask] over io 64 channels (src/train_inpaint.h:165-194)
LOCAL_CASES = {"full_dora_local": (43, "full", True, 0, False, 65),
               "core_lora_band_local_weighted": (44, "core", False, 6, True, 65)}


def expo(t, dim, lo=0.5, hi=1e4):
    # The float32 time features are an input of the model, taken from the oracle's
    # expo_features (itself checked against the closed form in tests/test_oracle_dit.py): the
    # float32 argument of the highest frequencies reaches 2 pi * 1e4, where one ulp of a
    # different exp/cos implementation would change the feature by ~4e-3.
    from dit_binding import expo_features
    return expo_features(float(t), dim, lo, hi)


def model_loss(cfg, tensors, ad, inputs, lw):
    s = cfg["alpha"] / cfg["rank"]
    dora = cfg["dora"]

    def L(name, X, bias=None):
        W = T(tensors[name])
        if name in ad:
            A, Bm, mag = ad[name]
            return lin(X, W, A, Bm, s, dora, mag, T(bnsq_of(tensors[name])) if dora else None, bias)
        y = X @ W.T
        return y + bias if bias is not None else y

    def mlp(stem, x, bias):
        b0 = T(tensors[f"dit.{stem}.0.bias"]) if bias else None
        b2 = T(tensors[f"dit.{stem}.2.bias"]) if bias else None
        h = torch.nn.functional.silu(L(f"dit.{stem}.0.weight", x, b0))
        return L(f"dit.{stem}.2.weight", h, b2)

    B, Tn, io, mem, dim = cfg["B"], cfg["T"], cfg["io"], cfg["mem"], cfg["dim"]
    total = 0
    losses = []
    for b in range(B):
        tf = T(expo(inputs["t"][b], cfg["time_dim"]))[None]
        te = mlp("time_embed", tf, True)
        g = mlp("global_embed", T(inputs["glob"][b])[None], False) + te
        gc = mlp("gce", g, True)                                      # [1, 6dim]
        ctx = mlp("cond_embed", T(inputs["cross"][b]), False)[None]   # [1, Ctx, dim]
        xin = T(inputs["x_t"][b])
        lc = T(inputs["local"][b]) if cfg.get("local_dim", 0) > 0 else None
        x = L("dit.pre_conv.weight", xin) + xin
        x = L("dit.proj_in.weight", x)
        x = torch.cat([T(tensors["dit.memory_tokens"]), x], 0)[None]
        for l in range(cfg["depth"]):
            p = f"dit.{l}."
            w = {k: tensors[p + n] for k, n in BLOCK_VECTORS.items()}
            w["W"] = [tensors[p + t + ".weight"] for t in BLOCK_TARGETS]
            w["bias"] = [tensors.get(p + t + ".bias") for t in BLOCK_TARGETS]
            w["bnsq"] = [bnsq_of(W) for W in w["W"]]
            A = [ad[p + t + ".weight"][0] for t in BLOCK_TARGETS]
            Bm = [ad[p + t + ".weight"][1] for t in BLOCK_TARGETS]
            mg = [ad[p + t + ".weight"][2] for t in BLOCK_TARGETS]
            bc = dict(cfg, B=1, S=mem + Tn)
            ladd = None
            if lc is not None:   # le = local.2(silu(local.0(lc))), added to the latent rows only
                le = mlp(f"{l}.local", lc, True)
                ladd = torch.cat([torch.zeros(mem, dim, dtype=torch.float64), le], 0)[None]
            x = block(bc, w, A, Bm, mg, x, ctx, gc, ladd)
        v = L("dit.proj_out.weight", x[0, mem:])
        v = L("dit.post_conv.weight", v) + v
        d2 = (v - T(inputs["target"][b])) ** 2
        lb = (d2 * T(lw[b])[:, None]).sum() if lw is not None else d2.sum() / (io * Tn)
        losses.append(lb.item())
        total = total + lb
    return total, np.array(losses)


def case(seed, scope, dora, window, weighted, local_dim=0):
    cfg = dict(CFG, dora=dora, window=window, local_dim=local_dim)
    tensors, adapters, inputs = random_dit(seed, cfg, scope)
    ad = {n: (T(a).requires_grad_(), T(b).requires_grad_(), T(m).requires_grad_() if m is not None else None)
          for n, (a, b, m) in adapters.items()}
    lw = None
    if weighted:
        lw = np.random.Generator(np.random.Philox(seed + 7)).uniform(0, 2.0 / (cfg["io"] * cfg["T"]),
                                                                      (cfg["B"], cfg["T"])).astype(np.float32)
    total, losses = model_loss(cfg, tensors, ad, inputs, lw)
    total.backward()
    res = {"loss": losses}
    if lw is not None:
        res["loss_weight"] = lw
    for n, (a, b, m) in ad.items():
        res[f"dA:{n}"] = a.grad.numpy().astype(np.float32)
        res[f"dB:{n}"] = b.grad.numpy().astype(np.float32)
        if m is not None:
            res[f"dm:{n}"] = m.grad.numpy().astype(np.float32)
    return res


def main():
    flat = {}
    for name, args in CASES.items():
        for k, v in case(*args).items():
            flat[f"{name}/{k}"] = v
    np.savez_compressed(os.path.join(HERE, "dit_autograd.npz"), **flat)
    print("wrote", len(flat), "arrays")
    flat = {}
    for name, args in LOCAL_CASES.items():
        for k, v in case(*args).items():
            flat[f"{name}/{k}"] = v
    np.savez_compressed(os.path.join(HERE, "dit_local_autograd.npz"), **flat)
    print("wrote", len(flat), "arrays")


if __name__ == "__main__":
    main()
