"""Oracle pinning for differential attention (src/dit.h:151-158, src/nn.h:135-144), no GPU.

Pins: torch float64 autograd vectors (dense self, cross with Sk != Sq, banded); central finite
differences of a scalar loss <O, G>; window >= 2*S equals dense; a single visible key makes the
branch output that key's value row (closed form)."""
import os

import numpy as np
import pytest

from conftest import oracle, rel_err, rng

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.parametrize("name", ["dense", "cross", "band"])
def test_matches_torch_autograd(name):
    z = np.load(os.path.join(HERE, "golden", "diff_attn_autograd.npz"))
    c = {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(name + "/")}
    D = c["Q1"].shape[2]
    w = int(c["window"])
    f = oracle.diff_attn_fwd(c["Q1"], c["K1"], c["Q2"], c["K2"], c["V"], 1.0 / np.sqrt(D), w)
    assert rel_err(f["O"], c["O"]) < 1e-6
    g = oracle.diff_attn_bwd(c["Q1"], c["K1"], c["Q2"], c["K2"], c["V"], c["dO"], 1.0 / np.sqrt(D), w)
    for k in ("Q1", "K1", "Q2", "K2", "V"):
        assert rel_err(g["d" + k], c["d" + k]) < 1e-6, k


def test_finite_differences():
    r = rng(21)
    BH, S, D = 1, 6, 4
    X = {k: r.normal(0, 1, (BH, S, D)).astype(np.float32) for k in ("Q1", "K1", "Q2", "K2", "V")}
    G = r.normal(0, 1, (BH, S, D)).astype(np.float32)
    loss = lambda: float((oracle.diff_attn_fwd(X["Q1"], X["K1"], X["Q2"], X["K2"], X["V"], 0.5)["O"].astype(np.float64) * G).sum())
    g = oracle.diff_attn_bwd(X["Q1"], X["K1"], X["Q2"], X["K2"], X["V"], G, 0.5)
    h = 1e-2
    for k in X:
        num = np.zeros(X[k].size)
        for i in range(X[k].size):
            o = X[k].flat[i]
            X[k].flat[i] = o + h
            lp = loss()
            X[k].flat[i] = o - h
            lm = loss()
            X[k].flat[i] = o
            num[i] = (lp - lm) / (2 * h)
        assert np.max(np.abs(num - g["d" + k].ravel())) < 2e-3 * max(1.0, np.max(np.abs(num))), k


def test_wide_window_equals_dense_and_single_key():
    r = rng(22)
    X = [r.normal(0, 1, (2, 9, 8)).astype(np.float32) for _ in range(5)]
    a = oracle.diff_attn_fwd(*X, scale=0.3, window=0)
    b = oracle.diff_attn_fwd(*X, scale=0.3, window=100)
    assert np.array_equal(a["O"], b["O"])
    # window 0 < w < 2: only j == i is visible -> each branch returns V[i], O = 0, lse = scaled q.k
    c = oracle.diff_attn_fwd(*X, scale=0.3, window=1)
    assert np.max(np.abs(c["O1"] - X[4])) < 1e-6 and np.max(np.abs(c["O"])) < 1e-6
    qk = (X[0].astype(np.float64) * X[1]).sum(-1) * 0.3
    assert np.max(np.abs(c["lse1"] - qk)) < 1e-5
