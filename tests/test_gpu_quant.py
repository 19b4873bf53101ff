"""a5: Q8_0 decode/encode on the GPU vs the oracle, bit-exact."""
import numpy as np
import pytest

from conftest import oracle, rng

pytestmark = pytest.mark.gpu


def test_q8_0_dequant_exhaustive(ctx):
    scales = np.arange(65536, dtype=np.uint16)
    keep = np.isfinite(scales.view(np.float16))
    scales = scales[keep]
    q = (np.arange(256) - 128).astype(np.int8)
    blocks = np.zeros((scales.size, 8, 34), np.uint8)
    blocks[:, :, 0:2] = scales.view(np.uint8).reshape(-1, 1, 2)
    blocks[:, :, 2:] = q.view(np.uint8).reshape(1, 8, 32)
    n = scales.size * 8 * 32
    db = ctx.upload(blocks.ravel())
    out = ctx.empty(n, np.float32)
    ctx.q8_0_dequant(db, out, n)
    got = out.numpy()
    ref = oracle.q8_0_dequant(blocks.ravel(), n)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("n", [32, 32 * 1000, 6144 * 1536])
def test_q8_0_quantize_matches_oracle(ctx, n):
    r = rng(6)
    x = r.normal(0, 0.02, n).astype(np.float32)
    # ties: blocks whose elements land exactly on k + 0.5 quantisation steps
    t = min(n // 32, 64)
    xb = x.reshape(-1, 32)
    xb[:t, 0] = 127.0
    xb[:t, 1:] = (np.arange(31) - 15 + 0.5).astype(np.float32)
    dx = ctx.upload(x)
    blocks = ctx.zeros(n // 32 * 34, np.uint8)
    ctx.q8_0_quantize(dx, blocks, n)
    assert np.array_equal(blocks.numpy(), oracle.q8_0_quantize(x))
