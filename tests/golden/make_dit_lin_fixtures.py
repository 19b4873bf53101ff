"""Write tests/golden/dit_lin_autograd.npz: small dit_lin forward/backward vectors from torch float64
autograd, an independent differentiation of the dit_lin forward (src/dit.h:92-149) used to pin the
oracle's closed-form backward. Torch is only used here, in the build container, to write the
fixture; the GPU tests never import it.

python tests/golden/make_dit_lin_fixtures.py
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def dit_lin_torch(X, W, A, B, s, dora, mag, bnsq, bias):
    # y = mul_mat(W, x); y += s * B(Ax); dora: y *= m / sqrt(bnsq + 2s t2 + s^2 t3); + bias
    y = X @ W.T + s * ((X @ A.T) @ B.T)
    if dora:
        P = W @ A.T                       # [out, r]
        t2 = (P * B).sum(1)
        G = A @ A.T
        t3 = (B * (B @ G)).sum(1)
        nsq = bnsq + 2 * s * t2 + s * s * t3
        y = y * (mag / torch.sqrt(nsq))
    if bias is not None:
        y = y + bias
    return y


def case(seed, N, in_, out_, r, alpha, dora, with_bias):
    g = np.random.Generator(np.random.Philox(seed))
    f = lambda *shape, sd=1.0: g.normal(0, sd, shape).astype(np.float32)
    X, W = f(N, in_), f(out_, in_, sd=0.5)
    A, B = f(r, in_, sd=0.3), f(out_, r, sd=0.3)
    mag = (np.sqrt((W.astype(np.float64) ** 2).sum(1)) * 1.1 + 0.05).astype(np.float32)
    bnsq = ((W.astype(np.float64) ** 2).sum(1) + in_ * 1e-12).astype(np.float32)
    bias = f(out_) if with_bias else None
    dY = f(N, out_, sd=0.1)
    t = {k: torch.tensor(v, dtype=torch.float64, requires_grad=k in ("X", "A", "B", "mag"))
         for k, v in dict(X=X, W=W, A=A, B=B, mag=mag, bnsq=bnsq).items()}
    tb = torch.tensor(bias, dtype=torch.float64) if bias is not None else None
    y = dit_lin_torch(t["X"], t["W"], t["A"], t["B"], alpha / r, dora, t["mag"], t["bnsq"], tb)
    y.backward(torch.tensor(dY, dtype=torch.float64))
    out = dict(X=X, W=W, A=A, B=B, mag=mag, bnsq=bnsq, dY=dY, s=np.float32(alpha / r), dora=np.int32(dora),
               Y=y.detach().numpy(), dX=t["X"].grad.numpy(), dA=t["A"].grad.numpy(), dB=t["B"].grad.numpy(),
               dm=t["mag"].grad.numpy() if dora else np.zeros(out_))
    if bias is not None:
        out["bias"] = bias
    return out


def main():
    cases = {
        "lora": case(1, 5, 64, 24, 4, 8.0, False, False),
        "dora": case(2, 7, 64, 40, 8, 8.0, True, False),
        "dora_bias": case(3, 4, 128, 32, 8, 16.0, True, True),
    }
    flat = {f"{name}/{k}": v for name, c in cases.items() for k, v in c.items()}
    np.savez_compressed(os.path.join(HERE, "dit_lin_autograd.npz"), **flat)
    print("wrote", len(flat), "arrays")


if __name__ == "__main__":
    main()
