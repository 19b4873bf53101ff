"""Oracle pinning for the optimizer path (no GPU).

Pins: the InverseLR golden table of the reference (tests/train_optimizer_test.cpp:35-45), the
reference's directional AdamW checks (:25-30), the closed-form first AdamW step, and the clip
invariants (post-clip norm == clip, scale only when norm > clip, src/train_loop.h:161-170).
"""
import numpy as np
import pytest

from conftest import oracle, rng

# tests/train_optimizer_test.cpp:35-45 — values from the Python reference's closed form
INVERSE_LR_TABLE = [
    (0, 5.0000000000e-07), (1, 9.9749950125e-07), (10, 5.3645151961e-06),
    (100, 3.9723855426e-05), (500, 9.1860637497e-05), (1000, 9.9288298382e-05),
    (2499, 9.9874922989e-05),
]


@pytest.mark.parametrize("step0,lr", INVERSE_LR_TABLE)
def test_inverse_lr_golden(step0, lr):
    got = oracle.inverse_lr(1.0e-4, step0, 1.0e6, 0.5, 0.995, 0.0)
    assert abs(got - lr) / lr < 1e-5


def test_inverse_lr_no_warmup():
    # tests/train_optimizer_test.cpp:46-47
    assert abs(oracle.inverse_lr(1.0e-4, 0, 1.0e6, 0.5, 0.0, 0.0) - 1.0e-4) < 1e-10


def test_adamw_directional():
    # tests/train_optimizer_test.cpp:18-30: lr 0.1, wd 0.01, p = {1,-1}, g = {0.5,-0.25}
    p, m, v = oracle.adamw_update_vector([1.0, -1.0], [0.5, -0.25], [0, 0], [0, 0],
                                         0.1, 0.9, 0.999, 1e-8, 0.01, 1)
    assert p[0] < 1.0 and p[1] > -1.0
    with pytest.raises(ValueError):
        oracle.adamw_update_vector([1.0], [1.0], [0], [0], 0.1, 0.9, 0.999, 1e-8, 0.0, 0)


def test_adamw_first_step_closed_form():
    # step 1, m = v = 0: m = (1-b1) g, v = (1-b2) g^2, so m/b1c = g and v/b2c = g^2 up to float
    # rounding; p1 = p - lr (g/(|g|+eps) + wd p). A dropped or mis-signed term moves p1 by >> 1e-6.
    r = rng(1)
    p = r.normal(0, 1, 4096).astype(np.float32)
    g = r.normal(0, 1e-3, 4096).astype(np.float32)
    lr, b1, b2, eps, wd = 1e-4, 0.9, 0.999, 1e-8, 0.01
    p1, m1, v1 = oracle.adamw_update_vector(p, g, np.zeros_like(p), np.zeros_like(p), lr, b1, b2, eps, wd, 1)
    pd, gd = p.astype(np.float64), g.astype(np.float64)
    expect = pd - lr * (gd / (np.abs(gd) + eps) + wd * pd)
    # one float32 rounding of p (<= 2^-24 |p|) plus 1e-6 of the step; the wd term alone is lr*wd*|p|
    tol = 2.0 ** -23 * np.abs(pd) + 1e-6 * lr
    assert np.all(np.abs(p1 - expect) <= tol)
    assert np.max(lr * wd * np.abs(pd) / tol) > 5  # the check can see a dropped decay term
    omb1 = float(np.float32(1) - np.float32(b1))
    omb2 = float(np.float32(1) - np.float32(b2))
    np.testing.assert_allclose(m1, omb1 * gd, rtol=1e-6)
    np.testing.assert_allclose(v1, omb2 * gd * gd, rtol=1e-6)


def test_average_and_clip_invariants():
    r = rng(2)
    g = r.normal(0, 1e-1, 100_000).astype(np.float32)
    # count 2: averaged norm is half the raw norm; clip 1.0 triggers (raw norm ~ 31.6)
    p = np.zeros_like(g)
    _, g_out, _, _, norm, scale = oracle.apply_accumulated_adamw(p, g, p, p, 1e-4, 0.9, 0.999, 1e-8, 0.0,
                                                                  1.0, 1, 2)
    raw = np.linalg.norm(g.astype(np.float64) * np.float32(0.5))
    assert abs(norm - raw) / raw < 1e-12
    assert abs(scale - 1.0 / (raw + 1e-6)) / scale < 1e-6
    assert abs(np.linalg.norm(g_out.astype(np.float64)) - 1.0) < 1e-5
    # below the threshold nothing is scaled
    small = (g * np.float32(1e-3)).astype(np.float32)
    _, g2, _, _, norm2, scale2 = oracle.apply_accumulated_adamw(p, small, p, p, 1e-4, 0.9, 0.999, 1e-8, 0.0,
                                                                 1.0, 1, 1)
    assert scale2 == 1.0 and np.array_equal(g2, small) and norm2 < 1.0


def test_adamw_continuation_deterministic():
    # tests/train_checkpoint_test.cpp:55-77 synthetic grads; 6 uninterrupted steps == 3 + 3
    n = 64
    p0 = np.linspace(-1, 1, n).astype(np.float32)

    def grad(update):
        j = np.arange(n, dtype=np.float32)
        return (np.float32(0.01) * np.float32(update + 1) + np.float32(0.001) * j).astype(np.float32)

    def run(p, m, v, steps):
        for step, update in steps:
            p, _, m, v, _, _ = oracle.apply_accumulated_adamw(p, grad(update), m, v, 1e-3, 0.9, 0.95, 1e-8,
                                                              0.01, 0.0, step, 1)
        return p, m, v

    z = np.zeros(n, np.float32)
    pa, ma, va = run(p0, z, z, [(i + 1, i) for i in range(6)])
    pb, mb, vb = run(p0, z, z, [(i + 1, i) for i in range(3)])
    pb, mb, vb = run(pb.copy(), mb.copy(), vb.copy(), [(i + 1, i) for i in range(3, 6)])
    assert np.array_equal(pa, pb) and np.array_equal(ma, mb) and np.array_equal(va, vb)
