"""The oracle's f32 mode (orc_set_f32), which bench.py times as the CPU baseline, against the
double oracle: the AVX2/FMA sgemm on ragged shapes, the windowed and dense attention, and a whole
DiT block forward + backward, each within float rounding. The double results are unchanged by a
round trip through the f32 mode (the mode is a switch, not state). No GPU."""
import os
import sys

import numpy as np
import pytest

from conftest import ROOT, oracle, rel_err, rng

sys.path.insert(0, os.path.join(ROOT, "oracle"))
import block_binding as bb  # noqa: E402


def test_f32_kernels_available():
    # the hosts this runs on (x86-64-v3 or later) take the AVX2/FMA path, not the generic loops
    assert oracle.lib().orc_f32_fast() == 1


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (7, 17, 33), (97, 50, 64), (200, 31, 1536), (6, 16, 0)])
def test_sgemm_matches_double(M, N, K):
    g = rng(900 + M + N + K)
    A = g.normal(0, 1, (M, K)).astype(np.float32)
    B = g.normal(0, 1, (N, K)).astype(np.float32)
    ref = oracle.dit_lin_fwd(A, B)["Y"]
    with oracle.f32_mode():
        got = oracle.dit_lin_fwd(A, B)["Y"]
    if K == 0:
        assert np.all(got == 0)
        return
    # float accumulation over K terms: |err| <= K eps sum|a b| (loose bound, per element)
    bound = K * np.finfo(np.float32).eps * (np.abs(A) @ np.abs(B).T) + 1e-30
    assert np.all(np.abs(got - ref) <= bound)
    assert rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("window", [0, 8])
def test_attention_matches_double(window):
    g = rng(910 + window)
    BH, S, D = 3, 40, 64
    q1, k1, q2, k2, v, do = (g.normal(0, 1, (BH, S, D)).astype(np.float32) for _ in range(6))
    ref_o = oracle.diff_attn_fwd(q1, k1, q2, k2, v, window=window)
    ref_g = oracle.diff_attn_bwd(q1, k1, q2, k2, v, do, window=window)
    with oracle.f32_mode():
        o = oracle.diff_attn_fwd(q1, k1, q2, k2, v, window=window)
        gr = oracle.diff_attn_bwd(q1, k1, q2, k2, v, do, window=window)
    for k in ("O", "O1", "O2", "lse1", "lse2"):
        assert rel_err(o[k], ref_o[k]) < 1e-5, k
    for k in ref_g:
        assert rel_err(gr[k], ref_g[k]) < 1e-4, k


def test_block_matches_double_and_mode_is_a_switch():
    cfg, w, x, ctx, gc = bb.random_block(5, B=2, S=20, Ctx=6, dim=128, heads=2, inner=96, rank=8, alpha=16.0,
                                         dora=True, window=8, w_sd=0.05, b_sd=0.05)
    dout = rng(920).normal(0, 1, x.shape).astype(np.float32)
    out_d = bb.block_fwd(cfg, w, x, ctx, gc)
    g_d = bb.block_bwd(cfg, w, x, ctx, gc, dout)
    with oracle.f32_mode():
        out_f = bb.block_fwd(cfg, w, x, ctx, gc)
        g_f = bb.block_bwd(cfg, w, x, ctx, gc, dout)
    assert rel_err(out_f, out_d) < 1e-5
    for k in ("dx", "dctx", "dgcond"):
        assert rel_err(g_f[k], g_d[k]) < 1e-4, k
    for t in range(7):
        for k in ("dA", "dB", "dm"):
            assert rel_err(g_f[k][t], g_d[k][t]) < 1e-3, (k, t)
    # back in double mode: bit-identical to the first double run
    assert np.array_equal(bb.block_fwd(cfg, w, x, ctx, gc), out_d)
