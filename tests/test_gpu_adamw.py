"""K6 (fused mean + global clip + AdamW) on the GPU vs the oracle: bit-exact params and moments.

The oracle is the literal float transcription of train_average_and_clip + adamw_update_vector
(src/train_loop.h:147-211, src/train_optimizer.h:42-66). The GPU reduces the double sum of squares
in a different order, so bit-exactness of the float clip scale is asserted too; the parameter,
m and v comparisons are on raw bits.
"""
import numpy as np
import pytest

from conftest import oracle, rng, sa3k

pytestmark = pytest.mark.gpu

HP = (1e-4, 0.9, 0.999, 1e-8, 0.01, 1.0)   # lr, b1, b2, eps, wd, clip (the 48M-param config)


def run_gpu(ctx, p, g, m, v, hp, step, count, offset=0):
    """offset > 0 places the arena at an unaligned element offset (exercises the scalar path)"""
    n = p.size
    bufs = []
    for a in (p, g, m, v):
        d = ctx.zeros(n + offset, np.float32)
        ctx.copy_into(d.view(offset, (n,)), a) if n else None
        bufs.append((d, d.view(offset, (n,))))
    norm = ctx.adamw_clip(bufs[0][1], bufs[1][1], bufs[2][1], bufs[3][1], hp, step, count, want_norm=True)
    _, scale = ctx.adamw_clip_scale()
    out = [b[1].numpy() for b in bufs]
    return out[0], out[1], out[2], out[3], norm, scale


def run_oracle(p, g, m, v, hp, step, count):
    lr, b1, b2, eps, wd, clip = hp
    return oracle.apply_accumulated_adamw(p, g, m, v, lr, b1, b2, eps, wd, clip, step, count)


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("n,count,clip,offset", [
    (1, 1, 1.0, 0), (3, 1, 1.0, 0), (4, 1, 0.0, 0), (1000, 2, 1.0, 0), (4097, 3, 1.0, 1),
    (65536, 1, 1.0, 0), (1 << 20, 4, 0.5, 0), (999_999, 1, 1.0, 3), (300_001, 1, 1e9, 0),
])
def test_adamw_bit_exact(ctx, n, count, clip, offset):
    r = rng(100 + n)
    p = r.normal(0, 0.05, n).astype(np.float32)
    g = r.normal(0, 1e-2, n).astype(np.float32) * np.float32(count)
    m = r.normal(0, 1e-3, n).astype(np.float32)
    v = np.abs(r.normal(0, 1e-5, n)).astype(np.float32)
    hp = HP[:5] + (clip,)
    gp, gg, gm, gv, gnorm, gscale = run_gpu(ctx, p, g, m, v, hp, 7, count, offset)
    op, og, om, ov, onorm, oscale = run_oracle(p, g, m, v, hp, 7, count)
    assert abs(gnorm - onorm) <= 1e-12 * onorm
    assert np.float32(gscale) == np.float32(oscale)
    assert bits_equal(gg, g), "the gradient arena is read-only"
    assert bits_equal(gp, op) and bits_equal(gm, om) and bits_equal(gv, ov)


def test_adamw_empty_and_errors(ctx):
    z = ctx.zeros(4, np.float32)
    e = z.view(0, (0,))
    ctx.adamw_clip(e, e, e, e, HP, 1, 1)
    with pytest.raises(sa3k.Sa3kError):
        ctx.adamw_clip(z, z, z, z, HP, 0, 1)       # step must be positive
    with pytest.raises(sa3k.Sa3kError):
        ctx.adamw_clip(z, z, z, z, HP, 1, 0)       # empty gradient batch


def test_adamw_continuation_six_steps(ctx):
    # tests/train_checkpoint_test.cpp:55-190 inputs; 6 GPU steps == 6 oracle steps, bit for bit,
    # and 3 + 3 split across a host round-trip of the state equals 6 uninterrupted
    n = 5000
    j = np.arange(n, dtype=np.float32)
    p0 = np.sin(j).astype(np.float32) * np.float32(0.1)
    hp = (1e-3, 0.9, 0.95, 1e-8, 0.01, 0.0)

    def grad(update):
        return (np.float32(0.01) * np.float32(update + 1) + np.float32(0.001) * j).astype(np.float32)

    dp, dg, dm, dv = ctx.upload(p0), ctx.zeros(n), ctx.zeros(n), ctx.zeros(n)
    op, om, ov = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    for u in range(6):
        ctx.copy_into(dg, grad(u))
        ctx.adamw_clip(dp, dg, dm, dv, hp, u + 1, 1)
        if u == 2:  # round-trip the state through the host (checkpoint + reload)
            saved = [x.numpy() for x in (dp, dm, dv)]
            dp, dm, dv = (ctx.upload(s) for s in saved)
        op, _, om, ov, _, _ = run_oracle(op, grad(u), om, ov, hp, u + 1, 1)
    assert bits_equal(dp.numpy(), op) and bits_equal(dm.numpy(), om) and bits_equal(dv.numpy(), ov)


@pytest.mark.parametrize("n", [42_265_088, 48_000_000])
def test_adamw_full_size(ctx, n):
    # the full-scope rank-32 DoRA arena (42,265,088) and the 48M-parameter configuration
    r = rng(5)
    p = r.normal(0, 0.05, n).astype(np.float32)
    g = r.normal(0, 1e-3, n).astype(np.float32)
    z = np.zeros(n, np.float32)
    gp, _, gm, gv, gnorm, gscale = run_gpu(ctx, p, g, z, z, HP, 1, 1)
    op, _, om, ov, onorm, oscale = run_oracle(p, g, z, z, HP, 1, 1)
    assert onorm > 1.0, "the clip is active at this size"
    assert np.float32(gscale) == np.float32(oscale)
    assert bits_equal(gp, op) and bits_equal(gm, om) and bits_equal(gv, ov)
