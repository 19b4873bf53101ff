"""K1-K4: the functional LoRA/DoRA linear (dit_lin, src/dit.h:92-149) on the GPU vs the oracle.

Configurations:
  * f32 LoRA linear 2048x1536 -> 1536, rank 16, alpha 16: fp32 MFMA, every output within 1e-4
    max relative error of the oracle, read both in the infinity norm (conftest.max_rel_err) and
    element by element with a floor of a tenth of the output's RMS (conftest.elem_rel_err);
  * DoRA linear 1536 -> 6144 over a Q8_0 base, rank 32: bf16 MFMA, outputs within 2e-2 normwise
    relative error and cosine >= 0.9999 of the oracle run on the exactly decoded Q8_0 weight;
  * smaller and ragged shapes, f16 and f32 bases, lora and dora, both precisions;
  * bf16 linears both merged (the products contract W + s B A, rounded once to bf16 by the
    refresh) and with the rank term as the second segment of each product (option lin_merge 0),
    and with the frozen base decoded on its way into LDS (no working copy, unmerged).
The oracle is the double-precision restatement in oracle/dit_lin.cpp (pinned in
tests/test_oracle_dit_lin.py).
"""
import numpy as np
import pytest

from conftest import cosine, elem_rel_err, max_rel_err, oracle, q8_0_split, rel_err, rng, sa3k

pytestmark = pytest.mark.gpu


def make_inputs(seed, N, in_, out_, r, w_sd=0.02, b_sd=0.01):
    g = rng(seed)
    X = g.normal(0, 1, (N, in_)).astype(np.float32)
    dY = g.normal(0, 1e-2, (N, out_)).astype(np.float32)
    W = g.normal(0, w_sd, (out_, in_)).astype(np.float32)
    bound = 1.0 / np.sqrt(in_)
    A = g.uniform(-bound, bound, (r, in_)).astype(np.float32)    # Kaiming-uniform (src/train_lora.h:252-260)
    B = g.normal(0, b_sd, (out_, r)).astype(np.float32)
    return X, dY, W, A, B


def run_gpu(ctx, X, dY, Wop, wtype, A, B, s, dora, mag, prec, bias=None, reps=1, decode_in_gemm=False, merge=True):
    N, in_ = X.shape
    out_ = dY.shape[1]
    r = A.shape[0]
    w = ctx.weight(Wop, wtype)
    if decode_in_gemm:
        assert not merge, "the merged products read the refreshed W + s B A, not the stored base"
        w.drop_working_copy()
    lin = ctx.lin(w, r, prec, N)
    dA_, dB_ = ctx.upload(A), ctx.upload(B)
    dmag = ctx.upload(mag) if dora else None
    bnsq = w.row_norm_sq(1e-12) if dora else None
    prev = ctx.options()   # the caller's settings hold for the products below
    ctx.set_option("lin_merge", 1 if merge else 0)
    try:
        lin.prepare(dA_, dB_, s, dora, dmag, bnsq)
    finally:
        ctx.set_options(prev)
    dX_, dY_ = ctx.upload(X), ctx.upload(dY)
    Y = ctx.empty((N, out_))
    gX, gA, gB, gm = ctx.empty((N, in_)), ctx.zeros((r, in_)), ctx.zeros((out_, r)), ctx.zeros(out_)
    for _ in range(reps):
        lin.forward(dX_, N, Y, bias=ctx.upload(bias) if bias is not None else None)
        lin.backward(dX_, N, dY_, gX, gA, gB, gm if dora else None)
    out = dict(Y=Y.numpy(), dX=gX.numpy(), dA=gA.numpy() / reps, dB=gB.numpy() / reps, dm=gm.numpy() / reps,
               bnsq=bnsq.numpy() if dora else None)
    lin.destroy()
    w.destroy()
    return out


def run_oracle(X, dY, Wdec, A, B, s, dora, mag, bias=None):
    bnsq = oracle.row_norm_sq(Wdec, 1e-12) if dora else None
    f = oracle.dit_lin_fwd(X, Wdec, A, B, s, dora, mag, bnsq, bias)
    g = oracle.dit_lin_bwd(X, Wdec, dY, A, B, s, dora, mag, bnsq)
    return dict(Y=f["Y"], dX=g["dX"], dA=g["dA"], dB=g["dB"], dm=g["dm"], bnsq=bnsq)


@pytest.mark.parametrize("N", [256, 2048])
def test_lora_f32_linear(ctx, N):
    # single LoRA linear 2048x1536 -> 1536, rank 16, alpha 16 (s = 1), seed 0, f32
    X, dY, W, A, B = make_inputs(0, N, 1536, 1536, 16)
    got = run_gpu(ctx, X, dY, W, sa3k.TYPE_F32, A, B, 1.0, False, None, sa3k.PREC_F32)
    ref = run_oracle(X, dY, W, A, B, 1.0, False, None)
    for k in ("Y", "dX", "dA", "dB"):
        assert max_rel_err(got[k], ref[k]) < 1e-4, k
        # element-wise: every element within 1e-4 of itself, or of a tenth of the output's RMS
        e = elem_rel_err(got[k], ref[k], 0.1)
        print(f"{k}: element-wise relative error {e:.3e} (floor 0.1 rms)")
        assert e < 1e-4, (k, e)


@pytest.mark.parametrize("N,decode,merge", [(256, False, True), (2048, False, True), (2048, False, False),
                                            (2048, True, False)])
def test_dora_q8_0_linear(ctx, N, decode, merge):
    # DoRA linear 1536 -> 6144, Q8_0 base quantised from N(0, 0.02), rank 32, alpha 32, m = row norms
    in_, out_, r = 1536, 6144, 32
    X, dY, W, A, B = make_inputs(1, N, in_, out_, r)
    blocks = oracle.q8_0_quantize(W)
    _, _, Wdec = q8_0_split(blocks, out_, in_)
    mag = oracle.row_norms(Wdec)
    got = run_gpu(ctx, X, dY, (blocks, in_, out_), sa3k.TYPE_Q8_0, A, B, 1.0, True, mag, sa3k.PREC_BF16,
                  decode_in_gemm=decode, merge=merge)
    ref = run_oracle(X, dY, Wdec, A, B, 1.0, True, mag)
    np.testing.assert_allclose(got["bnsq"], ref["bnsq"], rtol=1e-6)
    for k in ("Y", "dX", "dA", "dB", "dm"):
        assert rel_err(got[k], ref[k]) < 2e-2, k
        assert cosine(got[k], ref[k]) >= 0.9999, k


@pytest.mark.parametrize("prec,mode", [(sa3k.PREC_F32, "stored"), (sa3k.PREC_F32, "decode"),
                                       (sa3k.PREC_BF16, "merged"), (sa3k.PREC_BF16, "stored"),
                                       (sa3k.PREC_BF16, "decode")])
@pytest.mark.parametrize("wt", ["f32", "f16"])
@pytest.mark.parametrize("dora", [False, True])
def test_linear_small_shapes(ctx, prec, mode, wt, dora):
    # ragged token count, non-square, bias on the output
    N, in_, out_, r = 77, 192, 320, 8
    X, dY, W, A, B = make_inputs(2, N, in_, out_, r, w_sd=0.1, b_sd=0.05)
    if wt == "f16":
        Wop, wtype = W.astype(np.float16), sa3k.TYPE_F16
        Wdec = Wop.astype(np.float32)
    else:
        Wop, wtype, Wdec = W, sa3k.TYPE_F32, W
    mag = (oracle.row_norms(Wdec) * 1.1 + 0.05).astype(np.float32)
    bias = rng(3).normal(0, 1, out_).astype(np.float32)
    got = run_gpu(ctx, X, dY, Wop, wtype, A, B, 2.0, dora, mag, prec, bias=bias, decode_in_gemm=mode == "decode",
                  merge=mode == "merged")
    ref = run_oracle(X, dY, Wdec, A, B, 2.0, dora, mag, bias)
    keys = ("Y", "dX", "dA", "dB") + (("dm",) if dora else ())
    for k in keys:
        if prec == sa3k.PREC_F32:
            assert max_rel_err(got[k], ref[k]) < 1e-4, k
        else:
            assert rel_err(got[k], ref[k]) < 2e-2 and cosine(got[k], ref[k]) >= 0.9999, k


@pytest.mark.parametrize("N,in_,out_,r", [(2048, 1536, 6144, 32), (264, 192, 320, 8)])
@pytest.mark.parametrize("merge", [True, False])
def test_dora_linear_big_tiles(ctx, N, in_, out_, r, merge):
    # bf16 DoRA linear with every eligible GEMM on 256 x 256 tiles (gemm_big = 2): the rank segment
    # (K2 = r, unmerged) and the r extra dA rows of the dX GEMM go through the big kernel's descriptors
    X, dY, W, A, B = make_inputs(4, N, in_, out_, r)
    Wh = W.astype(np.float16)
    Wdec = Wh.astype(np.float32)
    mag = (oracle.row_norms(Wdec) * 1.05).astype(np.float32)
    try:
        ctx.set_option("gemm_big", 2)
        got = run_gpu(ctx, X, dY, Wh, sa3k.TYPE_F16, A, B, 1.5, True, mag, sa3k.PREC_BF16, merge=merge)
        ctx.set_option("gemm_big", 0)
        small = run_gpu(ctx, X, dY, Wh, sa3k.TYPE_F16, A, B, 1.5, True, mag, sa3k.PREC_BF16, merge=merge)
    finally:
        ctx.set_options(ctx.defaults)
    ref = run_oracle(X, dY, Wdec, A, B, 1.5, True, mag)
    for k in ("Y", "dX", "dA", "dB", "dm"):
        assert rel_err(got[k], ref[k]) < 2e-2 and cosine(got[k], ref[k]) >= 0.9999, k
        # the tile families differ in f32 summation order only; merged, the rank products ride on
        # the tiled products as extra columns and are rounded to bf16 after that order, so an
        # element of s dU B or s X A^T may round the other way
        assert rel_err(got[k], small[k]) < (1e-4 if merge else 1e-5), k


def test_gradients_accumulate(ctx):
    # dA/dB/dm are accumulators: two identical micro-batches give twice the gradient
    N, in_, out_, r = 64, 128, 256, 16
    X, dY, W, A, B = make_inputs(4, N, in_, out_, r, w_sd=0.1, b_sd=0.05)
    mag = oracle.row_norms(W)
    one = run_gpu(ctx, X, dY, W, sa3k.TYPE_F32, A, B, 1.0, True, mag, sa3k.PREC_F32, reps=1)
    two = run_gpu(ctx, X, dY, W, sa3k.TYPE_F32, A, B, 1.0, True, mag, sa3k.PREC_F32, reps=2)
    for k in ("dA", "dB", "dm"):
        assert max_rel_err(two[k], one[k]) < 1e-5, k


def test_row_norms_match_oracle(ctx):
    g = rng(7)
    W = g.normal(0, 0.02, (384, 1536)).astype(np.float32)
    for Wop, wt, Wdec in ((W, sa3k.TYPE_F32, W),
                          (W.astype(np.float16), sa3k.TYPE_F16, W.astype(np.float16).astype(np.float32))):
        w = ctx.weight(Wop, wt)
        np.testing.assert_allclose(w.row_norm_sq(1e-12).numpy(), oracle.row_norm_sq(Wdec, 1e-12), rtol=1e-6)
        np.testing.assert_allclose(w.row_norms().numpy(), oracle.row_norms(Wdec), rtol=1e-6)
        w.destroy()


def test_lin_rejects_bad_calls(ctx):
    W = np.zeros((64, 128), np.float32)
    w = ctx.weight(W, sa3k.TYPE_F32)
    with pytest.raises(sa3k.Sa3kError):
        ctx.lin(w, 12, sa3k.PREC_BF16, 16)          # rank must be a multiple of 8
    lin = ctx.lin(w, 8, sa3k.PREC_BF16, 16)
    X = ctx.zeros((32, 128))
    with pytest.raises(sa3k.Sa3kError):
        lin.forward(X, 32, ctx.empty((32, 64)))     # more tokens than max_tokens
    lin.destroy()
    w.destroy()


@pytest.mark.parametrize("wt", ["f32", "f16", "bf16", "q8_0"])
@pytest.mark.parametrize("r", [8, 24, 32])
def test_merged_refresh_terms(ctx, wt, r):
    """The merged refresh against the oracle's definitions: d = m / sqrt(|W + s B A|^2 + in eps) per
    row, and the products it feeds. Ragged rank counts (8, 24) exercise the zero-padded MFMA operands;
    every stored element type goes through its own decode (Q8_0: the exact d * q)."""
    N, in_, out_ = 96, 256, 192
    X, dY, W, A, B = make_inputs(11, N, in_, out_, r, w_sd=0.05, b_sd=0.05)
    if wt == "f16":
        Wop, wtype = W.astype(np.float16), sa3k.TYPE_F16
        Wdec = Wop.astype(np.float32)
    elif wt == "bf16":
        bits = (W.view(np.uint32) >> 16).astype(np.uint16)    # truncated to bf16: exact values
        Wdec = (bits.astype(np.uint32) << 16).view(np.float32)
        Wop, wtype = bits, sa3k.TYPE_BF16
    elif wt == "q8_0":
        blocks = oracle.q8_0_quantize(W)
        _, _, Wdec = q8_0_split(blocks, out_, in_)
        Wop, wtype = (blocks, in_, out_), sa3k.TYPE_Q8_0
    else:
        Wop, wtype, Wdec = W, sa3k.TYPE_F32, W
    mag = (oracle.row_norms(Wdec) * 0.9 + 0.01).astype(np.float32)
    got = run_gpu(ctx, X, dY, Wop, wtype, A, B, 0.75, True, mag, sa3k.PREC_BF16, merge=True)
    seg = run_gpu(ctx, X, dY, Wop, wtype, A, B, 0.75, True, mag, sa3k.PREC_BF16, merge=False)
    ref = run_oracle(X, dY, Wdec, A, B, 0.75, True, mag)
    for k in ("Y", "dX", "dA", "dB", "dm"):
        assert rel_err(got[k], ref[k]) < 2e-2 and cosine(got[k], ref[k]) >= 0.9999, k
        # the two formulations differ only by bf16 roundings of the operands
        assert rel_err(got[k], seg[k]) < 1e-2, k


@pytest.mark.parametrize("kn", [0, 1])
@pytest.mark.parametrize("cols", [0, 1, 2, 3])
def test_rank_products_as_extra_columns(ctx, cols, kn):
    """Merged DoRA linear with s X A^T (bit 0) and s dU B (bit 1) as extra output columns of the
    forward / dX products (option rank_cols), at the DiT's 2176-token shape (the 256 x 256, 128 x 256,
    128 x 128 and split-K tilings all carry them) and a ragged one: within the bf16 bar of the
    oracle, and within bf16 rounding of the separate products. The dX product reads the transposed
    merged copy (merge_kn 0, s dU B from B^T [r][out]) or W + s B A itself as a [K][N] operand
    (merge_kn 1, s dU B from B [out][r] as [K][Nx] extra columns)."""
    for N, in_, out_, r in ((2176, 1536, 6144, 32), (2176, 6144, 1536, 32), (120, 192, 320, 16)):
        X, dY, W, A, B = make_inputs(21, N, in_, out_, r)
        Wh = W.astype(np.float16)
        Wdec = Wh.astype(np.float32)
        mag = (oracle.row_norms(Wdec) * 1.02).astype(np.float32)
        try:
            ctx.set_option("merge_kn", kn)
            ctx.set_option("rank_cols", cols)
            got = run_gpu(ctx, X, dY, Wh, sa3k.TYPE_F16, A, B, 1.0, True, mag, sa3k.PREC_BF16)
            ctx.set_option("rank_cols", 0)
            sep = run_gpu(ctx, X, dY, Wh, sa3k.TYPE_F16, A, B, 1.0, True, mag, sa3k.PREC_BF16)
        finally:
            ctx.set_options(ctx.defaults)
        ref = run_oracle(X, dY, Wdec, A, B, 1.0, True, mag)
        for k in ("Y", "dX", "dA", "dB", "dm"):
            assert rel_err(got[k], ref[k]) < 2e-2 and cosine(got[k], ref[k]) >= 0.9999, (N, k)
            assert rel_err(got[k], sep[k]) < 1e-4, (N, k)


@pytest.mark.parametrize("opts", [dict(gemm_cfg=4), dict(gemm_cfg=1), dict(gemm_small=2), dict(gemm_small=0)])
def test_tile_configurations(ctx, opts):
    """The tile families the options select (gemm_cfg 4: 128 x 256 and 256 x 256 workgroups of 8
    waves instead of 16; gemm_cfg 1: 128 x 128 tiles; gemm_small 2 / 0: 64 x 128 tiles or the default
    tile split over K for the small grids instead of 8-wave 128 x 128) give the default's results up
    to the summation order, on a merged DoRA linear's forward ([N][K] B operand) and dX ([K][N])
    products at the DiT's shapes, and stay within the oracle's bar. The bound between the two runs
    is 1e-3: the rank product s X A^T and the DoRA rows reach dA / dB through bf16 roundings, where
    an f32 difference in the last place flips a bf16 value now and then (5.7e-5 seen on dB)."""
    for N, in_, out_, r in ((2176, 1536, 1536, 32), (2176, 1536, 6144, 32), (2176, 6144, 1536, 32)):
        X, dY, W, A, B = make_inputs(37, N, in_, out_, r)
        Wh = W.astype(np.float16)
        Wdec = Wh.astype(np.float32)
        mag = (oracle.row_norms(Wdec) * 0.97).astype(np.float32)
        base = run_gpu(ctx, X, dY, Wh, sa3k.TYPE_F16, A, B, 1.25, True, mag, sa3k.PREC_BF16)
        try:
            for k, v in opts.items():
                ctx.set_option(k, v)
            got = run_gpu(ctx, X, dY, Wh, sa3k.TYPE_F16, A, B, 1.25, True, mag, sa3k.PREC_BF16)
        finally:
            ctx.set_options(ctx.defaults)
        ref = run_oracle(X, dY, Wdec, A, B, 1.25, True, mag)
        for k in ("Y", "dX", "dA", "dB", "dm"):
            assert rel_err(got[k], base[k]) < 1e-3, (N, in_, out_, k)
            assert rel_err(got[k], ref[k]) < 2e-2 and cosine(got[k], ref[k]) >= 0.9999, (N, in_, out_, k)


@pytest.mark.parametrize("big", [0, 1, 2])
def test_dx_k_major_operand(ctx, big):
    """Merged linears' dX product reads W + s B A in its stored [out][in] layout as a K-major B
    operand (option merge_kn 1, transposed through the LDS reads) instead of a transposed copy
    (merge_kn 0): the same f32 sums over the same K tiles, on every tile family (gemm_big 0/1/2:
    never, by shape, always 256 x 256), at the DiT's shapes and small ones whose tiles reach past
    the last column (those sub-tiles read a clamped valid column and are never stored)."""
    for N, in_, out_, r in ((2176, 1536, 6144, 32), (2176, 6144, 1536, 32), (120, 192, 320, 16),
                            (264, 192, 320, 8)):
        X, dY, W, A, B = make_inputs(31, N, in_, out_, r)
        Wh = W.astype(np.float16)
        Wdec = Wh.astype(np.float32)
        mag = (oracle.row_norms(Wdec) * 0.97).astype(np.float32)
        try:
            ctx.set_option("gemm_big", big)
            ctx.set_option("merge_kn", 1)
            kn = run_gpu(ctx, X, dY, Wh, sa3k.TYPE_F16, A, B, 1.25, True, mag, sa3k.PREC_BF16)
            ctx.set_option("merge_kn", 0)
            nk = run_gpu(ctx, X, dY, Wh, sa3k.TYPE_F16, A, B, 1.25, True, mag, sa3k.PREC_BF16)
        finally:
            ctx.set_options(ctx.defaults)
        ref = run_oracle(X, dY, Wdec, A, B, 1.25, True, mag)
        for k in ("Y", "dX", "dA", "dB", "dm"):
            assert rel_err(kn[k], ref[k]) < 2e-2 and cosine(kn[k], ref[k]) >= 0.9999, (N, k)
            assert rel_err(kn[k], nk[k]) < 1e-5, (N, k)


@pytest.mark.parametrize("merge", [True, False])
@pytest.mark.parametrize("dora", [True, False])
def test_fused_reductions_bit_identical(ctx, merge, dora):
    """The column reduction of dU with the per-row step (dm, dB, the dA rows operand) and the dA
    column reduction each summed by their own last split to arrive (option tn_fuse bits 4 and 2)
    give the separate reduce / rows launches' results bit for bit (the same split order and
    formulas), at the DiT's QKV shape and a ragged one."""
    for N, in_, out_, r in ((2176, 1536, 4608, 32), (200, 192, 320, 8)):
        X, dY, W, A, B = make_inputs(41, N, in_, out_, r)
        Wh = W.astype(np.float16)
        mag = (oracle.row_norms(Wh.astype(np.float32)) * 1.01).astype(np.float32) if dora else None
        res = []
        try:
            for fuse in (0, 2, 4, 6):
                ctx.set_option("tn_fuse", fuse)
                res.append(run_gpu(ctx, X, dY, Wh, sa3k.TYPE_F16, A, B, 0.5, dora, mag, sa3k.PREC_BF16, reps=2,
                                   merge=merge))
        finally:
            ctx.set_options(ctx.defaults)
        for other in res[1:]:
            for k in ("Y", "dX", "dA", "dB") + (("dm",) if dora else ()):
                assert np.array_equal(res[0][k], other[k]), (N, k)
