"""Invariants of one DiT block (src/dit.h:164-266) that the oracle must satisfy, each fixed by the
reference's formulas rather than by a restatement of them, and each chosen so that a plausible
misreading of the reference fails it:

* gate h * sigmoid(1 - g) (src/dit.h:186-193, 223, 265): g = +40 switches the self-attention and
  feed-forward branches off (their weights no longer matter), g = -40 switches them fully on, and
  g = 1 passes exactly half of the fully-on branch; a gate read as sigmoid(g), sigmoid(g - 1) or
  sigmoid(-g) fails one of these;
* adaLN modulation h * (1 + sc) + sh (src/dit.h:177-185): sc = -1, sh = 0 zeroes the self branch's
  input, so with no bias on self.qkv / self.out the branch vanishes; h * sc + sh would not;
* slice order of the fused projections: self.qkv is q | k | v | qd | kd (src/dit.h:208-217) and
  cross.kv is k | kd | v (src/dit.h:228-236): zeroing exactly the v rows (and their adapter rows)
  makes the attention output, and so the branch, exactly zero whatever the other rows hold;
* the block's NEOX rotary (src/nn.h:53-59, ggml GGML_ROPE_TYPE_NEOX over rot = 32 of 64 dims):
  position 0 is the identity, only the pairs (i, i + 16) for i < 16 rotate, the rotation is a
  group in the position (scores depend on the relative position only), and pair i turns by
  base^(-2i/32) radians per position.
No GPU. Small shapes (dim 128, 2 heads) keep each oracle call well under a second."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

from conftest import ROOT, rel_err, rng

sys.path.insert(0, os.path.join(ROOT, "oracle"))
import block_binding as bb  # noqa: E402
import oracle as orc_mod  # noqa: E402

DIM = 128


def small_block(seed, window=0, dora=True):
    cfg, w, x, cx, gc = bb.random_block(seed, B=2, S=20, Ctx=6, dim=DIM, heads=2, inner=96, rank=8, alpha=16.0,
                                        dora=dora, window=window, w_sd=0.05, b_sd=0.05)
    return cfg, w, x, cx, np.zeros_like(gc)   # gcond 0: the modulation vectors are the ssg table's


def with_ssg(w, slot, value):
    w = dict(w)
    ssg = w["ssg"].copy()
    ssg[slot * DIM:(slot + 1) * DIM] = value
    w["ssg"] = ssg
    return w


def perturbed(w, targets, seed):
    """the same block with new base weights and adapters on the given targets"""
    g = rng(seed)
    w = dict(w, W=list(w["W"]), A=list(w["A"]), B=list(w["B"]), bnsq=list(w["bnsq"]))
    for t in targets:
        w["W"][t] = g.normal(0, 0.05, w["W"][t].shape).astype(np.float32)
        w["A"][t] = g.normal(0, 0.05, w["A"][t].shape).astype(np.float32)
        w["B"][t] = g.normal(0, 0.05, w["B"][t].shape).astype(np.float32)
        if w["bnsq"][t] is not None:
            W = w["W"][t].astype(np.float64)
            w["bnsq"][t] = ((W ** 2).sum(1) + W.shape[1] * 1e-12).astype(np.float32)
    return w


def fwd(cfg, w, x, cx, gc):
    return bb.block_fwd(cfg, w, x, cx, gc).astype(np.float64)


SELF, FF = (0, 1), (5, 6)


@pytest.mark.parametrize("seed", [1, 2])
def test_gate_off_on_and_half(seed):
    cfg, w, x, cx, gc = small_block(seed)
    off = with_ssg(with_ssg(w, 2, 40.0), 5, 40.0)     # g_a = g_f = +40
    on = with_ssg(with_ssg(w, 2, -40.0), 5, -40.0)    # g_a = g_f = -40
    base_off = fwd(cfg, off, x, cx, gc)
    # branches off: new self-attention and feed-forward weights change nothing
    alt_off = fwd(cfg, perturbed(off, SELF + FF, seed + 10), x, cx, gc)
    assert np.max(np.abs(alt_off - base_off)) <= 1e-6 * np.max(np.abs(base_off))
    # branches on: they do
    base_on = fwd(cfg, on, x, cx, gc)
    alt_on = fwd(cfg, perturbed(on, SELF + FF, seed + 10), x, cx, gc)
    assert rel_err(alt_on - x, base_on - x) > 1e-2
    # g_f = 1 (self branch off): the feed-forward branch enters with weight sigmoid(0) = 1/2
    ff_off = base_off
    ff_on = fwd(cfg, with_ssg(off, 5, -40.0), x, cx, gc)
    ff_half = fwd(cfg, with_ssg(off, 5, 1.0), x, cx, gc)
    assert rel_err(ff_half - ff_off, 0.5 * (ff_on - ff_off)) < 1e-5


@pytest.mark.parametrize("seed", [3, 4])
def test_modulation_scale_minus_one_zeroes_the_self_branch(seed):
    cfg, w, x, cx, gc = small_block(seed)
    w = with_ssg(w, 2, -40.0)                           # self branch fully on
    zeroed = with_ssg(with_ssg(w, 0, -1.0), 1, 0.0)     # sc_a = -1, sh_a = 0
    a = fwd(cfg, zeroed, x, cx, gc)
    b = fwd(cfg, perturbed(zeroed, SELF, seed + 20), x, cx, gc)
    assert np.array_equal(a, b)
    # any other scale keeps the branch alive (a constant shift alone would not: identical tokens
    # give both differential branches the same output, which cancels exactly)
    halved = with_ssg(zeroed, 0, -0.5)
    c = fwd(cfg, halved, x, cx, gc)
    d = fwd(cfg, perturbed(halved, SELF, seed + 20), x, cx, gc)
    assert rel_err(d - x, c - x) > 1e-3


def zero_rows(w, t, lo, hi):
    w = dict(w, W=list(w["W"]), B=list(w["B"]))
    W, B = w["W"][t].copy(), w["B"][t].copy()
    W[lo:hi] = 0.0
    B[lo:hi] = 0.0
    w["W"][t], w["B"][t] = W, B
    if w["bnsq"][t] is not None:
        w["bnsq"] = list(w["bnsq"])
        w["bnsq"][t] = ((W.astype(np.float64) ** 2).sum(1) + W.shape[1] * 1e-12).astype(np.float32)
    return w


def rows_replaced(w, t, ranges, seed):
    g = rng(seed)
    w = dict(w, W=list(w["W"]), B=list(w["B"]))
    W, B = w["W"][t].copy(), w["B"][t].copy()
    for lo, hi in ranges:
        W[lo:hi] = g.normal(0, 0.05, W[lo:hi].shape)
        B[lo:hi] = g.normal(0, 0.05, B[lo:hi].shape)
    w["W"][t], w["B"][t] = W, B
    if w["bnsq"][t] is not None:
        w["bnsq"] = list(w["bnsq"])
        w["bnsq"][t] = ((W.astype(np.float64) ** 2).sum(1) + W.shape[1] * 1e-12).astype(np.float32)
    return w


@pytest.mark.parametrize("dora", [True, False])
def test_self_qkv_slice_order(dora):
    cfg, w, x, cx, gc = small_block(5, dora=dora)
    w = with_ssg(w, 2, -40.0)
    w = zero_rows(w, 0, 2 * DIM, 3 * DIM)              # v of q | k | v | qd | kd
    a = fwd(cfg, w, x, cx, gc)
    others = [(0, DIM), (DIM, 2 * DIM), (3 * DIM, 4 * DIM), (4 * DIM, 5 * DIM)]
    b = fwd(cfg, rows_replaced(w, 0, others, 30), x, cx, gc)
    assert np.array_equal(a, b)
    # the same rows hold a live input under any other reading: zeroing qd instead leaves v alive
    w2 = zero_rows(small_block(5, dora=dora)[1], 0, 3 * DIM, 4 * DIM)
    w2 = with_ssg(w2, 2, -40.0)
    c = fwd(cfg, w2, x, cx, gc)
    d = fwd(cfg, rows_replaced(w2, 0, [(0, DIM)], 31), x, cx, gc)
    assert not np.array_equal(c, d)


@pytest.mark.parametrize("dora", [True, False])
def test_cross_kv_slice_order(dora):
    cfg, w, x, cx, gc = small_block(6, dora=dora)
    w = zero_rows(w, 3, 2 * DIM, 3 * DIM)              # v of k | kd | v
    a = fwd(cfg, w, x, cx, gc)
    b = fwd(cfg, rows_replaced(rows_replaced(w, 3, [(0, 2 * DIM)], 40), 2, [(0, 2 * DIM)], 41), x, cx, gc)
    assert np.array_equal(a, b)
    w2 = zero_rows(small_block(6, dora=dora)[1], 3, DIM, 2 * DIM)   # kd only: v stays live
    c = fwd(cfg, w2, x, cx, gc)
    d = fwd(cfg, rows_replaced(w2, 3, [(0, DIM)], 42), x, cx, gc)
    assert not np.array_equal(c, d)


def rope(v, pos, rot=32, base=1e4):
    v = np.ascontiguousarray(v, np.float32).copy()
    p = np.ascontiguousarray(pos, np.float32)
    L = orc_mod.lib()
    L.orc_rope_neox.restype = None
    L.orc_rope_neox.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_float]
    L.orc_rope_neox(v.ctypes.data, v.shape[0], rot, p.ctypes.data, base)
    return v.astype(np.float64)


def test_rope_identity_at_zero_and_pairs():
    g = rng(7)
    v = g.normal(0, 1, (8, 64)).astype(np.float32)
    assert np.array_equal(rope(v, np.zeros(8)), v.astype(np.float64))
    # a basis vector e_i (i < 16) stays in the plane of dims (i, i + 16) with its length; e_i for
    # i >= 32 is untouched
    for i in (0, 5, 15, 16, 31, 32, 50, 63):
        e = np.zeros((1, 64), np.float32)
        e[0, i] = 1.0
        r = rope(e, [7.0])[0]
        plane = {i, i + 16} if i < 16 else ({i - 16, i} if i < 32 else {i})
        assert np.all(r[[k for k in range(64) if k not in plane]] == 0.0), i
        assert abs(np.linalg.norm(r) - 1.0) < 1e-6, i


def test_rope_relative_positions_and_frequencies():
    g = rng(8)
    q, k = g.normal(0, 1, (1, 64)).astype(np.float32), g.normal(0, 1, (1, 64)).astype(np.float32)
    # <R_m q, R_n k> = <R_(m-n) q, k>: scores depend on the offset only
    for m, n in ((9, 4), (300, 295), (1087, 1082), (40, 100)):
        lhs = float(rope(q, [m])[0] @ rope(k, [n])[0])
        rhs = float(rope(q, [m - n])[0] @ k[0].astype(np.float64))
        assert abs(lhs - rhs) < 1e-4 * (1 + abs(rhs)), (m, n)
    # pair i turns by base^(-2i/32) per position (positive sense: e_i -> cos e_i + sin e_(i+16))
    for i in (0, 1, 7, 15):
        e = np.zeros((1, 64), np.float32)
        e[0, i] = 1.0
        r = rope(e, [1.0])[0]
        theta = np.arctan2(r[i + 16], r[i])
        assert abs(theta - 1e4 ** (-2.0 * i / 32)) < 1e-6, i
