"""Write tests/golden/diff_attn_autograd.npz: differential attention forward/backward vectors from
torch float64 autograd (dense and banded), an independent differentiation of
O = softmax(Q1 K1^T s) V - softmax(Q2 K2^T s) V (src/dit.h:151-158, src/nn.h:135-144) that pins
the oracle's backward. Build-container only; the GPU tests never import torch.

python tests/golden/make_attn_fixtures.py
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def attn(Q1, K1, Q2, K2, V, scale, window):
    Sq, Sk = Q1.shape[1], K1.shape[1]
    i = torch.arange(Sq)[:, None]
    j = torch.arange(Sk)[None, :]
    mask = (2 * (i - j).abs() <= window) if window > 0 else torch.ones(Sq, Sk, dtype=torch.bool)

    def branch(Q, K):
        s = (Q @ K.transpose(1, 2)) * scale
        s = s.masked_fill(~mask, float("-inf"))
        return torch.softmax(s, dim=-1) @ V

    return branch(Q1, K1) - branch(Q2, K2)


def case(seed, BH, Sq, Sk, D, window):
    g = np.random.Generator(np.random.Philox(seed))
    arrs = {k: g.normal(0, 1, (BH, Sq if k in ("Q1", "Q2") else Sk, D)).astype(np.float32)
            for k in ("Q1", "K1", "Q2", "K2", "V")}
    dO = g.normal(0, 1, (BH, Sq, D)).astype(np.float32)
    t = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True) for k, v in arrs.items()}
    O = attn(t["Q1"], t["K1"], t["Q2"], t["K2"], t["V"], 1.0 / np.sqrt(D), window)
    O.backward(torch.tensor(dO, dtype=torch.float64))
    out = dict(arrs, dO=dO, window=np.int32(window), O=O.detach().numpy())
    for k in arrs:
        out["d" + k] = t[k].grad.numpy()
    return out


def main():
    cases = {"dense": case(1, 2, 12, 12, 8, 0), "cross": case(2, 3, 10, 7, 8, 0),
             "band": case(3, 2, 16, 16, 8, 6)}
    flat = {f"{n}/{k}": v for n, c in cases.items() for k, v in c.items()}
    np.savez_compressed(os.path.join(HERE, "diff_attn_autograd.npz"), **flat)
    print("wrote", len(flat), "arrays")


if __name__ == "__main__":
    main()
