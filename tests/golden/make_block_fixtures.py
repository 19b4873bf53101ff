"""Write tests/golden/dit_block_autograd.npz: one DiT block (src/dit.h:164-266) forward and its
input/adapter gradients from torch float64 autograd, an implementation independent of the oracle's
hand-derived backward. Build-container only; the GPU tests never import torch.

python tests/golden/make_block_fixtures.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
from block_binding import random_block  # noqa: E402  (seeded inputs only)

T = lambda a: torch.tensor(a, dtype=torch.float64)


def rms(x, g, eps):
    return x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps) * g


def rope(x, pos, n, base):
    half = n // 2
    i = torch.arange(half, dtype=torch.float64)
    th = pos[:, None] * base ** (-2.0 * i / n)            # [S, half]
    c, s = torch.cos(th), torch.sin(th)
    a, b = x[..., :half], x[..., half:n]
    return torch.cat([a * c - b * s, a * s + b * c, x[..., n:]], -1)


def lin(X, W, A, Bm, s, dora, mag, bnsq, bias):
    y = X @ W.T + s * (X @ A.T) @ Bm.T
    if dora:
        t2 = ((W @ A.T) * Bm).sum(1)
        t3 = (Bm * (Bm @ (A @ A.T))).sum(1)
        y = y * (mag / torch.sqrt(bnsq + 2 * s * t2 + s * s * t3))
    return y + bias if bias is not None else y


def attn(q, k, v, qd, kd, window):
    Sq, Sk = q.shape[2], k.shape[2]
    i, j = torch.arange(Sq)[:, None], torch.arange(Sk)[None, :]
    mask = (2 * (i - j).abs() <= window) if window > 0 else torch.ones(Sq, Sk, dtype=torch.bool)
    def br(a, b):
        s = (a @ b.transpose(-1, -2)) / 8.0
        return torch.softmax(s.masked_fill(~mask, float("-inf")), -1) @ v
    return br(q, k) - br(qd, kd)


def block(cfg, w, A, Bm, mag, x, ctx, gc, ladd=None):
    B, S, Ctx, dim, H, I = cfg["B"], cfg["S"], cfg["Ctx"], cfg["dim"], cfg["heads"], cfg["inner"]
    s = cfg["alpha"] / cfg["rank"]
    dora = cfg["dora"]
    L = lambda t, X: lin(X, T(w["W"][t]), A[t], Bm[t], s, dora, mag[t] if dora else None,
                         T(w["bnsq"][t]) if dora else None, T(w["bias"][t]) if w["bias"][t] is not None else None)
    ssg = T(w["ssg"])[None] + gc                            # [B, 6dim]
    m = [ssg[:, i * dim:(i + 1) * dim][:, None, :] for i in range(6)]
    pos = torch.arange(S, dtype=torch.float64)
    hd = lambda t, n: t.reshape(B, n, H, 64).transpose(1, 2)       # [B, H, n, 64]
    h = rms(x, T(w["pre_g"]), 1e-5) * (1 + m[0]) + m[1]
    qkv = L(0, h)
    parts = [hd(qkv[..., i * dim:(i + 1) * dim], S) for i in range(5)]
    qn = lambda t, g, r: (rope(rms(t, T(g), 1e-6), pos, 32, 1e4) if r else rms(t, T(g), 1e-6))
    q, k, v, qd, kd = qn(parts[0], w["sq_g"], 1), qn(parts[1], w["sk_g"], 1), parts[2], qn(parts[3], w["sq_g"], 1), qn(parts[4], w["sk_g"], 1)
    o = attn(q, k, v, qd, kd, cfg["window"]).transpose(1, 2).reshape(B, S, dim)
    x1 = x + L(1, o) * torch.sigmoid(1 - m[2])
    hc = rms(x1, T(w["cross_g"]), 1e-5)
    qf, kv = L(2, hc), L(3, ctx)
    cq, cqd = qn(hd(qf[..., :dim], S), w["cq_g"], 0), qn(hd(qf[..., dim:], S), w["cq_g"], 0)
    ck, ckd = qn(hd(kv[..., :dim], Ctx), w["ck_g"], 0), qn(hd(kv[..., dim:2 * dim], Ctx), w["ck_g"], 0)
    cv = hd(kv[..., 2 * dim:], Ctx)
    x2 = x1 + L(4, attn(cq, ck, cv, cqd, ckd, 0).transpose(1, 2).reshape(B, S, dim))
    if ladd is not None:   # inpaint local add after the cross-attention (src/dit.h:244-254)
        x2 = x2 + ladd
    f = rms(x2, T(w["ff_g"]), 1e-5) * (1 + m[3]) + m[4]
    F = L(5, f)
    g = F[..., :I] * torch.nn.functional.silu(F[..., I:])
    return x2 + L(6, g) * torch.sigmoid(1 - m[5])


def case(seed, window, dora):
    cfg, w, x, ctx, gc = random_block(seed, B=2, S=20, Ctx=6, dim=128, heads=2, inner=96, rank=8, alpha=16.0,
                                      dora=dora, window=window, w_sd=0.05, b_sd=0.05)
    A = [T(a).requires_grad_() for a in w["A"]]
    Bm = [T(b).requires_grad_() for b in w["B"]]
    mag = [T(m).requires_grad_() if m is not None else None for m in w["mag"]]
    xt, ct, gt = T(x).requires_grad_(), T(ctx).requires_grad_(), T(gc).requires_grad_()
    out = block(cfg, w, A, Bm, mag, xt, ct, gt)
    dout = np.random.Generator(np.random.Philox(seed + 1)).normal(0, 1, out.shape).astype(np.float32)
    out.backward(T(dout))
    res = dict(out=out.detach().numpy(), dout=dout, dx=xt.grad.numpy(), dctx=ct.grad.numpy(), dgcond=gt.grad.numpy())
    for t in range(7):
        res[f"dA{t}"] = A[t].grad.numpy()
        res[f"dB{t}"] = Bm[t].grad.numpy()
        if dora:
            res[f"dm{t}"] = mag[t].grad.numpy()
    return res


def main():
    flat = {}
    for name, (seed, window, dora) in {"dora_dense": (11, 0, True), "lora_band": (12, 8, False)}.items():
        for k, v in case(seed, window, dora).items():
            flat[f"{name}/{k}"] = v
    np.savez_compressed(os.path.join(HERE, "dit_block_autograd.npz"), **flat)
    print("wrote", len(flat), "arrays")


if __name__ == "__main__":
    main()
