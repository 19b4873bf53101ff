"""Composed adapter chains over a frozen base on the GPU (sa3k_lora_chain_*: build_functional_lora,
src/lora.h:372-622, and the chain branch of dit_lin, src/dit.h:108-117) against the oracle
(oracle/chain.cpp, pinned against the sequential merge with the reference's own compose cases in
tests/test_oracle_chain.py).

* the folded constants (base_scale c0 and the row-scaled B'_k), computed on the device in double,
  equal the oracle's to 1e-5 relative;
* the chain's forward over a Q8_0 base (1536 -> 6144, the linear of the C2 configuration) and an f16
  base, with the bf16 working copy and with the base decoded on its way into LDS, within the bf16
  bar of the oracle run on the exactly decoded base (normwise relative error <= 2e-2, cosine >=
  0.9999), and the two base paths within 1e-5 of each other;
* lora-only, dora-only and mixed chains, ranks that are not multiples of 8, a zero-strength adapter
  (the identity), an empty chain (a plain mul_mat), a bias; order matters for two dora adapters;
* long chains past the rank segment of the base product (10 adapters, total rank 128; 32 adapters,
  total rank 512: the rank term as a GEMM of its own), against the oracle on both base paths;
* chains beyond the limits (33 adapters, total rank over 512) are rejected.
"""
import numpy as np
import pytest

from conftest import cosine, oracle, q8_0_split, rel_err, rng, sa3k

pytestmark = pytest.mark.gpu


def adapters_for(g, W, specs):
    """specs: [(dora, rank, alpha, strength)] -> host adapters with A, B ~ N(0, 0.02..), mag near the row norms"""
    out_, in_ = W.shape
    norms = np.sqrt((W.astype(np.float64) ** 2).sum(1))
    ads = []
    for dora, r, alpha, strength in specs:
        A = g.uniform(-1 / np.sqrt(in_), 1 / np.sqrt(in_), (r, in_)).astype(np.float32)
        B = g.normal(0, 0.02, (out_, r)).astype(np.float32)
        mag = (norms * (1.0 + 0.1 * g.standard_normal(out_))).astype(np.float32) if dora else None
        ads.append((dora, r, alpha, strength, A, B, mag))
    return ads


def to_device(ctx, ads):
    dev = []
    for dora, r, alpha, strength, A, B, mag in ads:
        dev.append((dora, r, alpha, strength, ctx.upload(A), ctx.upload(B), ctx.upload(mag) if mag is not None else None))
    return dev


def make_weight(ctx, g, out_, in_, wtype):
    W = g.normal(0, 0.02, (out_, in_)).astype(np.float32)
    if wtype == sa3k.TYPE_Q8_0:
        blocks = oracle.q8_0_quantize(W)
        _, _, dec = q8_0_split(blocks, out_, in_)
        return ctx.weight((blocks, in_, out_), sa3k.TYPE_Q8_0), dec
    Wh = W.astype(np.float16)
    return ctx.weight(Wh, sa3k.TYPE_F16), Wh.astype(np.float32)


def run_chain(ctx, w, dev, X, bias=None, decode=False):
    N = X.shape[0]
    ch = ctx.lora_chain(w, dev, N)
    try:
        Y = ctx.empty((N, w.out_))
        ch.forward(ctx.upload(X), N, Y, bias=ctx.upload(bias) if bias is not None else None)
        return Y.numpy(), ch.constants()
    finally:
        ch.destroy()


CHAINS = {
    "dora_lora_dora": [(1, 32, 32.0, 1.0), (0, 16, 16.0, 1.7), (1, 16, 32.0, 0.6)],
    # 10 adapters, total rank 128 (past one K tile: the rank term is its own GEMM)
    "ten_mixed_r128": [(k % 3 == 0, 16 if k < 6 else 8, 16.0, 0.5 + 0.1 * k) for k in range(10)] +
                      [(0, 8, 8.0, 0.0)],
    "lora_r2_r3": [(0, 2, 4.0, 1.0), (0, 3, 6.0, 1.7)],
    "dora_zero_strength": [(1, 8, 16.0, 1.0), (1, 24, 8.0, 0.0), (0, 8, 8.0, 1.0)],
    "empty": [(1, 16, 16.0, 0.0)],
}


@pytest.mark.parametrize("wname", ["q8_0", "f16"])
@pytest.mark.parametrize("chain", sorted(CHAINS))
def test_chain_matches_oracle(ctx, wname, chain):
    wtype = sa3k.TYPE_Q8_0 if wname == "q8_0" else sa3k.TYPE_F16
    g = rng(300 + len(chain) + (7 if wname == "f16" else 0))
    in_, out_, N = 1536, 6144, 256
    w, Wdec = make_weight(ctx, g, out_, in_, wtype)
    ads = adapters_for(g, Wdec, CHAINS[chain])
    X = g.normal(0, 1, (N, in_)).astype(np.float32)
    bias = g.normal(0, 0.02, out_).astype(np.float32) if chain == "lora_r2_r3" else None
    print(f"chain {chain} over {wname} base {out_}x{in_}, N {N}", flush=True)
    try:
        dev = to_device(ctx, ads)
        y_copy, (c0, Bp) = run_chain(ctx, w, dev, X, bias)
        w.drop_working_copy()   # the base decoded on its way into LDS from here on
        y_dec, _ = run_chain(ctx, w, dev, X, bias)
    finally:
        w.destroy()
    ref = oracle.chain_forward(X, Wdec, ads, bias)
    for y, what in ((y_copy, "bf16 working copy"), (y_dec, "decoded in the loader")):
        e, c = rel_err(y, ref), cosine(y, ref)
        assert e <= 2e-2 and c >= 0.9999, f"{what}: rel {e:.3e} cos {c:.6f}"
    assert rel_err(y_dec, y_copy) < 1e-5
    if chain == "empty":
        assert c0 is None
        plain = oracle.gemm_nt(X, Wdec)
        assert rel_err(y_copy, plain) < 2e-2
        return
    rc0, rBp, _ = oracle.chain_fold(Wdec, ads)
    assert np.max(np.abs(c0 - rc0) / np.abs(rc0)) < 1e-5
    assert rel_err(Bp, rBp) < 1e-5 and Bp.shape == rBp.shape


def test_chain_order_matters(ctx):
    g = rng(311)
    in_, out_, N = 512, 768, 128
    w, Wdec = make_weight(ctx, g, out_, in_, sa3k.TYPE_Q8_0)
    a, b = adapters_for(g, Wdec, [(1, 16, 32.0, 1.0), (1, 32, 16.0, 1.0)])
    a[5][:] *= 10.0   # strong dora adapters, so that their order shows
    b[5][:] *= 10.0
    X = g.normal(0, 1, (N, in_)).astype(np.float32)
    try:
        ab, _ = run_chain(ctx, w, to_device(ctx, [a, b]), X)
        ba, _ = run_chain(ctx, w, to_device(ctx, [b, a]), X)
    finally:
        w.destroy()
    ref_ab, ref_ba = oracle.chain_forward(X, Wdec, [a, b]), oracle.chain_forward(X, Wdec, [b, a])
    assert rel_err(ab, ref_ab) < 2e-2 and rel_err(ba, ref_ba) < 2e-2
    assert rel_err(ab, ba) > 5 * max(rel_err(ab, ref_ab), rel_err(ba, ref_ba))


def test_chain_32_adapters_rank_512(ctx):
    # the longest chain: 32 adapters (every fourth dora-rows) of rank 16, total rank 512
    g = rng(313)
    in_, out_, N = 512, 1024, 128
    w, Wdec = make_weight(ctx, g, out_, in_, sa3k.TYPE_Q8_0)
    ads = adapters_for(g, Wdec, [(k % 4 == 1, 16, 16.0, 0.3) for k in range(32)])
    X = g.normal(0, 1, (N, in_)).astype(np.float32)
    try:
        y, (c0, Bp) = run_chain(ctx, w, to_device(ctx, ads), X)
    finally:
        w.destroy()
    ref = oracle.chain_forward(X, Wdec, ads)
    e, c = rel_err(y, ref), cosine(y, ref)
    assert e <= 2e-2 and c >= 0.9999, f"rel {e:.3e} cos {c:.6f}"
    rc0, rBp, _ = oracle.chain_fold(Wdec, ads)
    assert np.max(np.abs(c0 - rc0) / np.abs(rc0)) < 1e-5
    assert rel_err(Bp, rBp) < 1e-5 and Bp.shape == (out_, 512)


def test_chain_limits(ctx):
    g = rng(312)
    w, Wdec = make_weight(ctx, g, 256, 128, sa3k.TYPE_F16)
    try:
        many = to_device(ctx, adapters_for(g, Wdec, [(0, 8, 8.0, 1.0)] * 33))
        with pytest.raises(sa3k.Sa3kError):
            ctx.lora_chain(w, many, 64)
        wide = to_device(ctx, adapters_for(g, Wdec, [(0, 256, 8.0, 1.0), (1, 264, 8.0, 1.0)]))
        with pytest.raises(sa3k.Sa3kError):
            ctx.lora_chain(w, wide, 64)
        ok = ctx.lora_chain(w, wide[:1], 64)   # 256 alone fits
        ok.destroy()
        ok = ctx.lora_chain(w, many[:32], 64)   # 32 adapters of rank 8 fit
        ok.destroy()
    finally:
        w.destroy()
