"""Oracle pinning for f16 conversion and Q8_0 blocks (no GPU).

Pins: f16 <-> f32 against numpy's IEEE float16 (round-to-nearest-even) over every f16 value and
over random and tie-breaking f32 inputs; Q8_0 decode against the closed form f32(d)*q over all
2^16 scales x 256 quants; Q8_0 encode by its invariants (|x - deq| <= d/2 up to f16 rounding of d,
max |q| = 127 on the element holding amax, zero blocks encode to d = 0, q = 0).
"""
import numpy as np

from conftest import oracle, rng


def test_f16_roundtrip_all_values():
    h = np.arange(65536, dtype=np.uint16)
    f = oracle.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(f[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(f[np.isnan(ref)]))
    back = oracle.f32_to_f16_bits(f[finite])
    assert np.array_equal(back, h[finite])


def test_f32_to_f16_matches_numpy_rne():
    r = rng(3)
    x = np.concatenate([
        r.normal(0, 1, 200_000), r.normal(0, 1e-5, 50_000), r.normal(0, 3e4, 50_000),
        np.array([65504.0, 65519.0, 65520.0, 70000.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 0.0, -0.0]),
    ]).astype(np.float32)
    # exact halfway points between adjacent f16 values
    h = r.integers(0, 0x7bff, 10_000).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    x = np.concatenate([x, ((lo + hi) / 2).astype(np.float32)])
    got = oracle.f32_to_f16_bits(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_q8_0_dequant_closed_form_exhaustive():
    # every (scale, quant) pair: 65536 blocks whose quants sweep all 256 int8 values
    scales = np.arange(65536, dtype=np.uint16)
    sf = scales.view(np.float16).astype(np.float32)
    keep = np.isfinite(sf)
    scales, sf = scales[keep], sf[keep]
    q = (np.arange(256) - 128).astype(np.int8)
    for part in range(8):  # 32 quants per block, 8 blocks per scale cover all 256 quants
        qs = q[part * 32:(part + 1) * 32]
        blocks = np.zeros((scales.size, 34), np.uint8)
        blocks[:, 0:2] = scales.view(np.uint8).reshape(-1, 2)
        blocks[:, 2:] = qs.view(np.uint8)[None, :]
        y = oracle.q8_0_dequant(blocks.ravel(), scales.size * 32).reshape(-1, 32)
        ref = sf[:, None] * qs.astype(np.float32)[None, :]
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_q8_0_quantize_invariants():
    r = rng(4)
    x = r.normal(0, 0.02, 32 * 4096).astype(np.float32)
    x[:32] = 0.0                                        # an all-zero block
    x[32:64] = np.linspace(-1, 1, 32).astype(np.float32)
    b = oracle.q8_0_quantize(x).reshape(-1, 34)
    d = b[:, 0:2].copy().view(np.uint16).ravel().view(np.float16).astype(np.float64)
    qs = b[:, 2:].view(np.int8).astype(np.int64)
    xb = x.reshape(-1, 32).astype(np.float64)
    amax = np.abs(xb).max(axis=1)
    assert d[0] == 0.0 and np.all(qs[0] == 0)
    nz = amax > 0
    # the f16 scale is amax/127 rounded to f16
    assert np.all(np.abs(d[nz] - amax[nz] / 127) <= np.abs(amax[nz] / 127) * 2.0 ** -11 * 1.0001)
    assert np.all(np.abs(qs[nz]).max(axis=1) == 127)
    deq = oracle.q8_0_dequant(b.ravel(), x.size).reshape(-1, 32).astype(np.float64)
    # |x - d q| <= d_f32/2 + 127 |d_f32 - d_f16|
    dd = amax / 127
    bound = dd / 2 + 127 * np.abs(dd - d) + 1e-12
    assert np.all(np.abs(deq - xb) <= bound[:, None])
    # round half away from zero on exact ties: x = 2.5 d
    t = np.zeros(32, np.float32)
    t[0] = 127.0
    t[1] = 2.5
    t[2] = -2.5
    bt = oracle.q8_0_quantize(t)
    assert bt[2 + 1].view(np.int8) == 3 and bt[2 + 2:2 + 3].view(np.int8)[0] == -3
