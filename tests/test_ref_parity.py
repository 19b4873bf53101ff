"""The oracle against the reference's own code where that code builds here: src/train_optimizer.h
(AdamW, InverseLR) compiled from the reference tree into oracle/_ref/libsa3ref.so (oracle/Makefile,
target `ref`). Bit-exact. Skipped where the reference tree was not present at build time (the GPU
boxes); the oracle is pinned there by the tests in test_oracle_optim.py."""
import os
import sys

import numpy as np
import pytest

from conftest import ROOT, oracle, rng

sys.path.insert(0, os.path.join(ROOT, "oracle"))
import ref  # noqa: E402

pytestmark = pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built (no reference tree)")


@pytest.mark.parametrize("hp", [(1e-4, 0.9, 0.999, 1e-8, 0.01), (3e-4, 0.9, 0.95, 1e-8, 0.0),
                                (1e-3, 0.8, 0.99, 1e-6, 0.1)])
def test_adamw_update_vector_matches_reference(hp):
    # src/train_optimizer.h:42-66 (the reference) vs oracle/optim.cpp over 20 steps of one tensor
    lr, b1, b2, eps, wd = hp
    r = rng(11)
    n = 10_007
    p = r.normal(0, 0.05, n).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    rp, rm, rv = p.copy(), m.copy(), v.copy()
    for step in range(1, 21):
        g = r.normal(0, 1e-3 * step, n).astype(np.float32)
        g[:7] = [0.0, -0.0, 1e-30, -1e-30, 1e3, -1e3, 3e-8]   # zeros, denormal-scale, large, tiny
        p, m, v = oracle.adamw_update_vector(p, g, m, v, lr, b1, b2, eps, wd, step)
        rp, rm, rv = ref.adamw_update_vector(rp, g, rm, rv, lr, b1, b2, eps, wd, step)
        for a, b in ((p, rp), (m, rm), (v, rv)):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step {step}"


def test_inverse_lr_matches_reference():
    # src/train_optimizer.h:20-27 over the step range and the configurations the trainer uses
    for base, inv_gamma, power, warmup, final in [(1e-4, 1e6, 0.5, 0.995, 0.0), (3e-4, 1e4, 1.0, 0.0, 1e-6),
                                                  (1e-3, 100.0, 0.75, 0.9, 5e-4)]:
        for step0 in list(range(0, 50)) + [99, 1000, 12345, 10 ** 6, 2 ** 30]:
            a = oracle.inverse_lr(base, step0, inv_gamma, power, warmup, final)
            b = ref.inverse_lr(base, step0, inv_gamma, power, warmup, final)
            assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), (base, step0)
