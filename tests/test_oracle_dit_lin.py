"""Oracle pinning for dit_lin (src/dit.h:92-149) and the adapter state helpers (no GPU).

Pins, beyond restating the forward:
  * tests/dit_lin_functional_test.cpp re-expressed (IN 8, OUT 6, RK 2, SEQ 4, alpha 4,
    N(0, 0.5) inputs, magnitude = 1.1 ||W_o|| + 0.05): functional lora / dora-rows == materialised
    W_eff (train_lora_effective_weight) within 1e-4, f16 base within 5e-3 of the f32 reference,
    rank 0 == plain mul_mat bit for bit, and A/B/m/x gradients == central finite differences;
  * torch float64 autograd vectors (tests/golden/dit_lin_autograd.npz) for the closed-form backward;
  * train_row_norms on W = 1..32 (4 x 8): magnitude[0] in (5.47, 5.48) (tests/train_lora_test.cpp:72).
"""
import os

import numpy as np
import pytest

from conftest import oracle, rel_err

HERE = os.path.dirname(os.path.abspath(__file__))


def small_case(seed=1234, IN=8, OUT=6, RK=2, SEQ=4):
    g = np.random.Generator(np.random.Philox(seed))
    nd = lambda *s: g.normal(0, 0.5, s).astype(np.float32)
    W, A, B, X = nd(OUT, IN), nd(RK, IN), nd(OUT, RK), nd(SEQ, IN)
    mag = (np.sqrt((W.astype(np.float64) ** 2).sum(1)) * 1.1 + 0.05).astype(np.float32)
    return W, A, B, X, mag


def maxrel(a, b, floor=1e-4):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b) / (np.abs(b) + floor)))


@pytest.mark.parametrize("dora", [False, True])
def test_functional_matches_materialised(dora):
    W, A, B, X, mag = small_case()
    alpha, RK = 4.0, 2
    bnsq = oracle.row_norm_sq(W)
    y = oracle.dit_lin_fwd(X, W, A, B, alpha / RK, dora, mag, bnsq)["Y"]
    Weff = oracle.effective_weight(W, A, B, mag, alpha, dora)
    ref = oracle.gemm_nt(X, Weff)
    assert maxrel(y, ref) < 1e-4


def test_f16_base_matches_f32():
    W, A, B, X, mag = small_case()
    W16 = W.astype(np.float16).astype(np.float32)
    y16 = oracle.dit_lin_fwd(X, W16, A, B, 2.0, True, mag, oracle.row_norm_sq(W16))["Y"]
    ref = oracle.gemm_nt(X, oracle.effective_weight(W, A, B, mag, 4.0, True))
    assert maxrel(y16, ref) < 5e-3


def test_rank0_is_plain_mul_mat():
    W, _, _, X, _ = small_case()
    y = oracle.dit_lin_fwd(X, W)["Y"]
    assert np.array_equal(y, oracle.gemm_nt(X, W))


def test_row_norms_known_value():
    W = np.arange(1, 33, dtype=np.float32).reshape(8, 4)   # ne=[4,8]: in=4, out=8
    m = oracle.row_norms(W)
    assert 5.47 < m[0] < 5.48
    nsq = oracle.row_norm_sq(W, 1e-12)
    assert abs(nsq[0] - (1 + 4 + 9 + 16)) < 1e-5


def loss_and_grads(X, W, A, B, s, dora, mag, bnsq, tgt):
    f = oracle.dit_lin_fwd(X, W, A, B, s, dora, mag, bnsq)
    dY = 2.0 * (f["Y"].astype(np.float64) - tgt)
    g = oracle.dit_lin_bwd(X, W, dY.astype(np.float32), A, B, s, dora, mag, bnsq)
    return oracle.dit_lin_sqloss(X, W, tgt, A, B, s, dora, mag, bnsq), g


@pytest.mark.parametrize("dora", [False, True])
def test_gradients_match_finite_differences(dora):
    # tests/dit_lin_functional_test.cpp:131-259: loss = sum((y - tgt)^2)
    g = np.random.Generator(np.random.Philox(99))
    IN, OUT, RK, SEQ = 8, 6, 2, 4
    nd = lambda *s: g.normal(0, 0.5, s).astype(np.float32)
    W, A, B, X, tgt = nd(OUT, IN), nd(RK, IN) * 0.3, nd(OUT, RK) * 0.3, nd(SEQ, IN), nd(SEQ, OUT)
    mag = (np.sqrt((W.astype(np.float64) ** 2).sum(1)) + 0.1).astype(np.float32)
    bnsq = oracle.row_norm_sq(W)
    s = 2.0
    _, grads = loss_and_grads(X, W, A, B, s, dora, mag, bnsq, tgt)
    params = {"A": A, "B": B, "X": X}
    if dora:
        params["mag"] = mag
    names = {"A": "dA", "B": "dB", "X": "dX", "mag": "dm"}
    for name, p in params.items():
        ana = grads[names[name]]
        h = 1e-2 if name == "X" else 1e-3
        num = np.zeros_like(p, dtype=np.float64)
        for k in range(p.size):
            orig = p.flat[k]
            p.flat[k] = orig + h
            lp, _ = loss_and_grads(X, W, A, B, s, dora, mag, bnsq, tgt)
            p.flat[k] = orig - h
            lm, _ = loss_and_grads(X, W, A, B, s, dora, mag, bnsq, tgt)
            p.flat[k] = orig
            num.flat[k] = (lp - lm) / (2 * h)
        err = np.max(np.abs(num - ana) / (np.abs(num) + 1e-2))
        assert err < 1e-4, f"{name}: {err}"


@pytest.mark.parametrize("name", ["lora", "dora", "dora_bias"])
def test_matches_torch_autograd(name):
    z = np.load(os.path.join(HERE, "golden", "dit_lin_autograd.npz"))
    c = {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(name + "/")}
    dora = bool(c["dora"])
    f = oracle.dit_lin_fwd(c["X"], c["W"], c["A"], c["B"], float(c["s"]), dora, c["mag"], c["bnsq"],
                           c.get("bias"))
    assert rel_err(f["Y"], c["Y"]) < 1e-6
    g = oracle.dit_lin_bwd(c["X"], c["W"], c["dY"], c["A"], c["B"], float(c["s"]), dora, c["mag"], c["bnsq"])
    for k in ("dX", "dA", "dB") + (("dm",) if dora else ()):
        assert rel_err(g[k], c[k]) < 1e-6, k
