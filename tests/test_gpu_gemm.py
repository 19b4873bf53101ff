"""K1/K2 MFMA GEMM on the GPU vs float64 products of the same (rounded) operands.

bf16 compute: operands are rounded to bf16 by the kernel's loader, so the reference multiplies the
bf16-rounded values in float64; what remains is fp32 accumulation error (<= 1e-5 normwise).
f32 compute (v_mfma_f32_16x16x4_f32): reference is the float64 product of the f32 operands.
"""
import numpy as np
import pytest

from conftest import bf16_bits, bf16_round, max_rel_err, oracle, q8_0_split, rel_err, rng, sa3k

pytestmark = pytest.mark.gpu


def run(ctx, A, Bop, M, N, K, prec, a_type, b_type, B_scales=None, ldbs=0, **kw):
    dA = ctx.upload(A)
    dB = ctx.upload(Bop)
    dS = ctx.upload(B_scales) if B_scales is not None else None
    colscale = kw.pop("colscale", None)
    bias = kw.pop("bias", None)
    c0 = kw.pop("c0", None)
    dC = ctx.upload(c0) if c0 is not None else ctx.zeros((M, N))
    ctx.gemm_nt(dA, dB, M, N, K, prec=prec, a_type=a_type, b_type=b_type, B_scales=dS, ldbs=ldbs,
                colscale=ctx.upload(colscale) if colscale is not None else None,
                bias=ctx.upload(bias) if bias is not None else None, C=dC, **kw)
    return dC.numpy()


@pytest.mark.parametrize("M,N,K", [(128, 128, 64), (200, 96, 192), (2048, 1536, 1536), (37, 20, 128),
                                   (16, 640, 256), (300, 64, 1024), (2176, 7680, 1536), (2176, 1536, 6144),
                                   (2048, 32, 6144)])
@pytest.mark.parametrize("btype", ["f32", "f16", "bf16", "bf16-dma"])
def test_gemm_bf16(ctx, M, N, K, btype):
    # "bf16-dma": both operands bf16, the DMA-fed kernel; the others decode on the way into LDS
    r = rng(M * 7 + N)
    A = r.normal(0, 1, (M, K)).astype(np.float32)
    W = r.normal(0, 0.02, (N, K)).astype(np.float32)
    a_op, a_type = A, sa3k.TYPE_F32
    if btype == "f32":
        Bop, bt, Wd = W, sa3k.TYPE_F32, W
    elif btype == "f16":
        Bop = W.astype(np.float16)
        bt, Wd = sa3k.TYPE_F16, Bop.astype(np.float32)
    else:
        Bop, bt, Wd = bf16_bits(W), sa3k.TYPE_BF16, bf16_round(W)
        if btype == "bf16-dma":
            a_op, a_type = bf16_bits(A), sa3k.TYPE_BF16
    got = run(ctx, a_op, Bop, M, N, K, sa3k.PREC_BF16, a_type, bt)
    ref = bf16_round(A).astype(np.float64) @ bf16_round(Wd).astype(np.float64).T
    assert rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("M,N,K", [(256, 384, 1536), (100, 6144, 1536), (2048, 1536, 6144)])
def test_gemm_q8_0(ctx, M, N, K):
    r = rng(N)
    W = r.normal(0, 0.02, (N, K)).astype(np.float32)
    q, sc, dec = q8_0_split(oracle.q8_0_quantize(W), N, K)
    A = r.normal(0, 1, (M, K)).astype(np.float32)
    got = run(ctx, A, q, M, N, K, sa3k.PREC_BF16, sa3k.TYPE_F32, sa3k.TYPE_Q8_0, B_scales=sc, ldbs=K // 32)
    ref = bf16_round(A).astype(np.float64) @ bf16_round(dec).astype(np.float64).T
    assert rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("M,out_,in_", [(128, 256, 128), (2048, 6144, 1536), (77, 1536, 512)])
def test_gemm_q8_0_transposed(ctx, M, out_, in_):
    # dX = dU . W with W Q8_0 [out][in]: B operand rows are the `in` index, K is `out`
    r = rng(in_)
    W = r.normal(0, 0.02, (out_, in_)).astype(np.float32)
    q, sc, dec = q8_0_split(oracle.q8_0_quantize(W), out_, in_)
    qT = np.ascontiguousarray(q.T)                      # [in][out]
    scT = np.ascontiguousarray(sc.T)                    # [in/32][out]
    dU = r.normal(0, 1e-2, (M, out_)).astype(np.float32)
    got = run(ctx, dU, qT, M, in_, out_, sa3k.PREC_BF16, sa3k.TYPE_F32, -8, B_scales=scT, ldbs=out_)
    ref = bf16_round(dU).astype(np.float64) @ bf16_round(dec).astype(np.float64)
    assert rel_err(got, ref) < 1e-5


def test_gemm_epilogue(ctx):
    r = rng(11)
    M, N, K = 300, 200, 256
    A = r.normal(0, 1, (M, K)).astype(np.float32)
    W = r.normal(0, 0.05, (N, K)).astype(np.float32)
    cs = r.uniform(0.5, 2, N).astype(np.float32)
    b = r.normal(0, 1, N).astype(np.float32)
    c0 = r.normal(0, 1, (M, N)).astype(np.float32)
    got = run(ctx, A, W, M, N, K, sa3k.PREC_BF16, sa3k.TYPE_F32, sa3k.TYPE_F32, alpha=0.5, colscale=cs,
              bias=b, c0=c0, accumulate=True)
    ref = c0 + (0.5 * (bf16_round(A).astype(np.float64) @ bf16_round(W).astype(np.float64).T)) * cs + b
    assert rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("M,N,K", [(2048, 1536, 1536), (130, 40, 96), (64, 16, 1536)])
@pytest.mark.parametrize("btype", ["f32", "f16"])
def test_gemm_f32(ctx, M, N, K, btype):
    r = rng(M + N + K)
    A = r.normal(0, 1, (M, K)).astype(np.float32)
    W = r.normal(0, 0.02, (N, K)).astype(np.float32)
    if btype == "f16":
        Bop, bt, Wd = W.astype(np.float16), sa3k.TYPE_F16, W.astype(np.float16).astype(np.float32)
    else:
        Bop, bt, Wd = W, sa3k.TYPE_F32, W
    got = run(ctx, A, Bop, M, N, K, sa3k.PREC_F32, sa3k.TYPE_F32, bt)
    ref = A.astype(np.float64) @ Wd.astype(np.float64).T
    assert rel_err(got, ref) < 2e-6


def test_gemm_rejects_bad_shapes(ctx):
    a = ctx.zeros((64, 100))
    with pytest.raises(sa3k.Sa3kError):
        ctx.gemm_nt(a, a, 64, 64, 100, C=ctx.zeros((64, 64)))   # K not a multiple of 64


@pytest.mark.parametrize("M,N,K", [(2176, 1536, 1536), (2048, 32, 6144), (32, 1536, 6144), (2208, 1536, 6144)])
def test_split_k_fixup_matches_separate_reduction(ctx, M, N, K):
    # split-K partial sums reduced inside the kernel by the last split to arrive give exactly the
    # separate reduction launch's result (same split order), for several launches in a row
    r = rng(M + N + K)
    A = bf16_bits(r.normal(0, 1, (M, K)).astype(np.float32))
    B = bf16_bits(r.normal(0, 0.02, (N, K)).astype(np.float32))
    bias = r.normal(0, 1, N).astype(np.float32)
    out = {}
    try:
        for fixup in (0, 1, 2, 0, 1, 2):
            ctx.set_option("gemm_fixup", fixup)
            res = run(ctx, A, B, M, N, K, sa3k.PREC_BF16, sa3k.TYPE_BF16, sa3k.TYPE_BF16, bias=bias)
            if fixup in out:
                assert np.array_equal(res, out[fixup]), "not deterministic"
            out[fixup] = res
    finally:
        ctx.set_options(ctx.defaults)
    assert np.array_equal(out[0], out[1]) and np.array_equal(out[0], out[2])


@pytest.mark.parametrize("M,N,K", [(2176, 32, 1536), (2176, 32, 12288), (2208, 32, 7680), (37, 20, 128),
                                   (1, 1, 64), (130, 17, 192), (16, 32, 64), (300, 31, 6144)])
def test_skinny_gemm(ctx, M, N, K):
    # products with <= 32 output columns (the rank products s X A^T, s dU B) run on the skinny
    # kernel: f32 accumulation error only, bit-identical on a repeat, and within rounding of the
    # tiled kernel (gemm_skinny = 0), which sums K in another order
    r = rng(M * 31 + N * 7 + K)
    A = r.normal(0, 1, (M, K)).astype(np.float32)
    W = r.normal(0, 0.02, (N, K)).astype(np.float32)
    ref = bf16_round(A).astype(np.float64) @ bf16_round(W).astype(np.float64).T
    args = (bf16_bits(A), bf16_bits(W), M, N, K, sa3k.PREC_BF16, sa3k.TYPE_BF16, sa3k.TYPE_BF16)
    got = run(ctx, *args)
    again = run(ctx, *args)
    try:
        ctx.set_option("gemm_skinny", 0)
        tiled = run(ctx, *args)
    finally:
        ctx.set_options(ctx.defaults)
    assert np.array_equal(got, again), "not deterministic"
    assert rel_err(got, ref) < 1e-5
    assert rel_err(tiled, ref) < 1e-5
    assert max_rel_err(got, tiled) < 1e-5


@pytest.mark.parametrize("M,N,K", [(2176, 12288, 1536), (2176, 6144, 1536), (300, 640, 256), (520, 1000, 192),
                                   (2176, 1536, 6144)])
def test_big_tile_gemm(ctx, M, N, K):
    # 256 x 256 tiles forced (gemm_big = 2): f32 accumulation error only, within rounding of the
    # 128 x 128 kernel, and bit-identical on a repeat; ragged M and N clamp their loads
    r = rng(M + 3 * N + K)
    A = r.normal(0, 1, (M, K)).astype(np.float32)
    W = r.normal(0, 0.02, (N, K)).astype(np.float32)
    bias = r.normal(0, 1, N).astype(np.float32)
    cs = r.uniform(0.5, 1.5, N).astype(np.float32)
    args = (bf16_bits(A), bf16_bits(W), M, N, K, sa3k.PREC_BF16, sa3k.TYPE_BF16, sa3k.TYPE_BF16)
    ref = (bf16_round(A).astype(np.float64) @ bf16_round(W).astype(np.float64).T) * cs + bias
    try:
        ctx.set_option("gemm_big", 2)
        got = run(ctx, *args, bias=bias, colscale=cs)
        again = run(ctx, *args, bias=bias, colscale=cs)
        ctx.set_option("gemm_big", 0)
        small = run(ctx, *args, bias=bias, colscale=cs)
    finally:
        ctx.set_options(ctx.defaults)
    assert np.array_equal(got, again), "not deterministic"
    assert rel_err(got, ref) < 1e-5
    assert max_rel_err(got, small) < 1e-5


@pytest.mark.parametrize("M,N,K", [(2176, 7680, 1536), (2176, 1536, 1536), (256, 6144, 1536), (96, 384, 256)])
@pytest.mark.parametrize("btype", ["f16", "q8_0"])
def test_gemm_decoded_b_on_dma_kernel(ctx, M, N, K, btype):
    """bf16 A with an f16 or Q8_0 B on the DMA-fed kernel (option gemm_dq 1: B staged in LDS as
    stored and decoded between LDS and the MFMAs) gives the same bits as the same kernel over the
    decoded bf16 copy (the decode is the same RNE of the exact value), and the loader-decode kernel
    (gemm_dq 0) within fp32 accumulation order; both within 1e-5 of the float64 product."""
    r = rng(M + 3 * N + K)
    A = bf16_bits(r.normal(0, 1, (M, K)).astype(np.float32))
    W = r.normal(0, 0.02, (N, K)).astype(np.float32)
    if btype == "f16":
        Bop, sc, ldbs, bt = W.astype(np.float16), None, 0, sa3k.TYPE_F16
        dec = Bop.astype(np.float32)
    else:
        q, sc, dec = q8_0_split(oracle.q8_0_quantize(W), N, K)
        Bop, ldbs, bt = q, K // 32, sa3k.TYPE_Q8_0
    try:
        ctx.set_option("gemm_big", 0)
        got = run(ctx, A, Bop, M, N, K, sa3k.PREC_BF16, sa3k.TYPE_BF16, bt, B_scales=sc, ldbs=ldbs)
        copy = run(ctx, A, bf16_bits(dec), M, N, K, sa3k.PREC_BF16, sa3k.TYPE_BF16, sa3k.TYPE_BF16)
        ctx.set_option("gemm_dq", 0)
        loader = run(ctx, A, Bop, M, N, K, sa3k.PREC_BF16, sa3k.TYPE_BF16, bt, B_scales=sc, ldbs=ldbs)
    finally:
        ctx.set_options(ctx.defaults)
    Af = (A.astype(np.uint32) << 16).view(np.float32)
    ref = Af.astype(np.float64) @ bf16_round(dec).astype(np.float64).T
    assert np.array_equal(got, copy)
    assert rel_err(got, ref) < 1e-5 and rel_err(loader, ref) < 1e-5
