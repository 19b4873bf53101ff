"""K5: flash differential attention on the GPU vs the oracle (bf16 operands, fp32 accumulation).

Inputs are rounded to bf16 before the oracle sees them, so the comparison measures the kernel's
arithmetic (bf16 P in the PV / dS products, fp32 accumulation) against a double-precision
restatement: outputs within 2e-2 normwise relative error and cosine >= 0.9999. Shapes cover the
DiT block's self-attention (64 memory + T tokens), its cross-attention to the conditioning tokens,
ragged lengths, the banded window at full size (batch 2, 24 heads, 1088 tokens, windows 0 and 256,
forward and backward) a single-key window (closed form: O = 0) and both forward kernels on self-attention shapes."""
import numpy as np
import pytest

from conftest import bf16_bits, bf16_round, cosine, oracle, rel_err, rng, sa3k

pytestmark = pytest.mark.gpu


def run(ctx, B, H, Sq, Sk, window, seed=0, check_bwd=True):
    r = rng(seed)
    X = {k: bf16_round(r.normal(0, 1, (B * H, Sq if k in ("q1", "q2") else Sk, 64)).astype(np.float32))
         for k in ("q1", "k1", "q2", "k2", "v")}
    dO = r.normal(0, 1, (B, Sq, H * 64)).astype(np.float32)
    dev = {k: ctx.upload(bf16_bits(v)) for k, v in X.items()}
    o, o1, o2, l1, l2 = sa3k.attn_fwd(ctx, dev["q1"], dev["k1"], dev["q2"], dev["k2"], dev["v"], B, H, Sq, Sk, window)
    ref = oracle.diff_attn_fwd(X["q1"], X["k1"], X["q2"], X["k2"], X["v"], 0.125, window)
    got_o = (o.numpy().astype(np.uint32) << 16).view(np.float32).reshape(B, Sq, H, 64).transpose(0, 2, 1, 3)
    ref_o = ref["O"].reshape(B, H, Sq, 64)
    assert rel_err(got_o, ref_o) < 2e-2 and cosine(got_o, ref_o) >= 0.9999
    np.testing.assert_allclose(l1.numpy() / np.log2(np.e), ref["lse1"], rtol=0, atol=2e-2)
    if not check_bwd:
        return
    dOd = ctx.upload(dO)
    g = sa3k.attn_bwd(ctx, dev["q1"], dev["k1"], dev["q2"], dev["k2"], dev["v"], o1, o2, l1, l2, dOd, B, H, Sq, Sk,
                      window)
    dOh = dO.reshape(B, Sq, H, 64).transpose(0, 2, 1, 3).reshape(B * H, Sq, 64)
    rb = oracle.diff_attn_bwd(X["q1"], X["k1"], X["q2"], X["k2"], X["v"], bf16_round(dOh), 0.125, window)
    names = {"dq1": "dQ1", "dk1": "dK1", "dq2": "dQ2", "dk2": "dK2", "dv": "dV"}
    for k in ("dq1", "dk1", "dq2", "dk2", "dv"):
        got, want = g[k].numpy(), rb[names[k]]
        assert rel_err(got, want) < 2e-2 and cosine(got, want) >= 0.9999, (k, rel_err(got, want), cosine(got, want))


@pytest.mark.parametrize("B,H,Sq,Sk,window", [
    (1, 2, 64, 64, 0), (1, 3, 100, 100, 0), (2, 2, 200, 37, 0), (1, 2, 256, 256, 64), (1, 1, 130, 130, 16),
    (2, 24, 1088, 128, 0), (1, 4, 1088, 1088, 256),
    # the block's self-attention at full size (batch 2 x (64 memory + 1024 latent) tokens, 24 heads),
    # dense and windowed, forward and backward
    (2, 24, 1088, 1088, 0), (2, 24, 1088, 1088, 256),
])
def test_attention_matches_oracle(ctx, B, H, Sq, Sk, window):
    run(ctx, B, H, Sq, Sk, window, seed=Sq + Sk + window)


def test_attention_single_key_window(ctx):
    # window 1: every query sees only its own key, so both branches return V and O = 0. Both forward
    # kernels are exact here: the lone weight rounds to bf16 1.0 and l sums it as rounded (the
    # 32x32 kernel) or is the fp32 weight 2^0 = 1 (the 16x16 kernel). 200 keys: past the length
    # from which the 32x32 kernel serves self-attention.
    B, H, S = 1, 2, 200
    r = rng(5)
    X = [ctx.upload(bf16_bits(r.normal(0, 1, (B * H, S, 64)).astype(np.float32))) for _ in range(5)]
    try:
        for fwd32 in (0, 1):
            ctx.set_option("attn_fwd32", fwd32)
            o, o1, o2, l1, l2 = sa3k.attn_fwd(ctx, *X, B, H, S, S, window=1)
            assert np.max(np.abs((o.numpy().astype(np.uint32) << 16).view(np.float32))) == 0.0, fwd32
            assert np.array_equal(o1.numpy(), X[4].numpy()), fwd32
            assert np.array_equal(o2.numpy(), X[4].numpy()), fwd32
    finally:
        ctx.set_options(ctx.defaults)


@pytest.mark.parametrize("fwd32", [0, 1])
@pytest.mark.parametrize("B,H,Sq,Sk,window", [
    (1, 2, 256, 256, 64), (1, 1, 130, 130, 16), (1, 3, 200, 200, 0), (1, 2, 300, 300, 7), (2, 24, 1088, 1088, 256),
])
def test_attention_forward_kernels(ctx, fwd32, B, H, Sq, Sk, window):
    # the 16x16 forward (both branches per wave) and the 32x32 one (one branch per wave) on the
    # self-attention shapes the 32x32 kernel serves, each against the oracle
    ctx.set_option("attn_fwd32", fwd32)
    try:
        run(ctx, B, H, Sq, Sk, window, seed=7 * Sq + window, check_bwd=False)
    finally:
        ctx.set_options(ctx.defaults)
