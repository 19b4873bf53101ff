"""sa3k_gemm_nt_noalloc (split-K partials in the library's fixed device scratch array, no
allocation) against sa3k_gemm_nt (the same kernels with the context's growing workspace), bit for
bit, through the C ABI.

Shapes are chosen so that the dispatch splits K (few output tiles, long K), which is when the
scratch is used; two calls run in a row with the second smaller than the first, so stale partials
of a larger earlier call would show. Runs on the GPU only.
"""
import numpy as np
import pytest

from conftest import bf16_bits, oracle, q8_0_split, rng, sa3k

pytestmark = pytest.mark.gpu


def _inputs(r, M, N, K, kind):
    A = r.normal(0, 1, (M, K)).astype(np.float32)
    W = r.normal(0, 0.02, (N, K)).astype(np.float32)
    if kind == "bf16-dma":     # both operands bf16: the DMA-fed kernel
        return bf16_bits(A), sa3k.TYPE_BF16, bf16_bits(W), sa3k.TYPE_BF16, None, 0, sa3k.PREC_BF16
    if kind == "f16-decode":   # f32 A, f16 B decoded on its way into LDS
        return A, sa3k.TYPE_F32, W.astype(np.float16), sa3k.TYPE_F16, None, 0, sa3k.PREC_BF16
    if kind == "q8_0":         # Q8_0 quants + f16 scales decoded in the loader
        q, sc, _ = q8_0_split(oracle.q8_0_quantize(W), N, K)
        return A, sa3k.TYPE_F32, q, sa3k.TYPE_Q8_0, sc, K // 32, sa3k.PREC_BF16
    assert kind == "f32"       # fp32 MFMA
    return A, sa3k.TYPE_F32, W, sa3k.TYPE_F32, None, 0, sa3k.PREC_F32


def _pair(ctx, r, M, N, K, kind, epilogue):
    """(existing entry point's C, no-alloc entry point's C) for one set of inputs"""
    A, at, B, bt, S, ldbs, prec = _inputs(r, M, N, K, kind)
    dA, dB = ctx.upload(A), ctx.upload(B)
    dS = ctx.upload(S) if S is not None else None
    kw = {}
    c0 = None
    if epilogue:
        kw["colscale"] = ctx.upload(r.uniform(0.5, 1.5, N).astype(np.float32))
        kw["bias"] = ctx.upload(r.normal(0, 1, N).astype(np.float32))
        kw["accumulate"] = True
        kw["alpha"] = 0.75
        c0 = r.normal(0, 1, (M, N)).astype(np.float32)
    out = []
    for noalloc in (False, True):
        dC = ctx.upload(c0) if c0 is not None else ctx.zeros((M, N))
        print(f"gemm_nt{'_noalloc' if noalloc else ''} {kind} M={M} N={N} K={K} epilogue={epilogue}", flush=True)
        ctx.gemm_nt(dA, dB, M, N, K, prec=prec, a_type=at, b_type=bt, B_scales=dS, ldbs=ldbs, C=dC,
                    noalloc=noalloc, **kw)
        out.append(dC.numpy())
    return out


# (first call, second smaller call); each splits K over workgroups
CASES = {
    "bf16-dma": ((256, 256, 4096), (130, 72, 1024)),
    "f16-decode": ((200, 96, 3072), (64, 40, 2048)),
    "q8_0": ((128, 256, 4096), (96, 64, 1536)),
    "f32": ((64, 128, 2048), (40, 64, 1024)),
}


@pytest.mark.parametrize("kind", sorted(CASES))
@pytest.mark.parametrize("epilogue", [False, True])
def test_noalloc_matches_gemm_nt(ctx, kind, epilogue):
    r = rng(17 + len(kind) + (5 if epilogue else 0))
    for (M, N, K) in CASES[kind]:
        ref, got = _pair(ctx, r, M, N, K, kind, epilogue)
        assert np.isfinite(ref).all()
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), (kind, M, N, K)


def test_noalloc_without_split(ctx):
    # a grid that fills the chip takes no split: the entry point works without touching the scratch
    r = rng(3)
    ref, got = _pair(ctx, r, 2176, 1536, 1536, "bf16-dma", False)
    assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))


def test_noalloc_rejects_plan_beyond_scratch(ctx):
    # a forced split count whose partials exceed the 64 MiB array: a clear error before any launch,
    # after which the entry point and the context keep working
    r = rng(5)
    M = N = 1024
    K = 4096
    A, at, B, bt, _, _, prec = _inputs(r, M, N, K, "bf16-dma")
    dA, dB = ctx.upload(A), ctx.upload(B)
    dC = ctx.zeros((M, N))
    ctx.set_option("gemm_splits", 32)   # 32 x 1024 x 1024 floats = 128 MiB of partials
    try:
        print("gemm_nt_noalloc forced split beyond the scratch (host-side rejection)", flush=True)
        with pytest.raises(sa3k.Sa3kError) as e:
            ctx.gemm_nt(dA, dB, M, N, K, prec=prec, a_type=at, b_type=bt, C=dC, noalloc=True)
        assert e.value.code == 1 and "scratch" in str(e.value)
    finally:
        ctx.set_options(ctx.defaults)
    ref, got = _pair(ctx, r, 256, 256, 4096, "bf16-dma", False)
    assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))
