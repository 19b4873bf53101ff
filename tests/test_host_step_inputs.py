"""The host mirror's step-input producers (sa3.cpp_amd/host/sa3/train_diffusion.h, train_inpaint.h,
dist_shift.h) against the reference.

* TrainDiffusionSampler, generate_inpaint_mask, build_train_inpaint: bit-identical to the
  reference's own src/train_diffusion.h / src/train_inpaint.h, compiled from the reference tree
  into oracle/_ref (committed outputs in tests/golden/step_inputs_ref.npz, written by
  tests/golden/make_step_input_fixtures.py; compared live, on more seeds, where oracle/_ref is
  built). Plus the reference tests' own properties (tests/train_diffusion_test.cpp,
  tests/train_inpaint_test.cpp): rectified-flow identity, draw_t + sample_at == sample, exact
  continuation after a state save/restore, mask shapes per type, the type frequencies, the loss
  weights summing to one over the generated positions.
* dist_shift_warp / expo_features (src/sa3_pipeline.h, not buildable here: it includes the ggml
  pipeline): pinned by their closed forms in float64 and by their special cases.
The host headers are compiled with g++ into a test-only shim (tests/host/step_inputs_shim.cpp).
"""
import ctypes as C
import os
import subprocess
import sys
import time

import numpy as np
import pytest

from conftest import PKG, ROOT, oracle
from step_input_cases import BUILD, DIFFUSION, INPAINT, latent

sys.path.insert(0, os.path.join(ROOT, "oracle"))
import ref  # noqa: E402

GOLD = os.path.join(ROOT, "tests", "golden", "step_inputs_ref.npz")
f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


@pytest.fixture(scope="module")
def host(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("step_inputs") / "libstep_inputs.so")
    cmd = ["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", "-Werror", "-ffp-contract=off",
           "-I", os.path.join(PKG, "host"), os.path.join(ROOT, "tests", "host", "step_inputs_shim.cpp"), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    L = C.CDLL(out)
    F, I, I64, U64, D = C.c_float, C.c_int, C.c_int64, C.c_uint64, C.c_double
    L.host_diffusion_samples.restype = I
    L.host_diffusion_samples.argtypes = [U64, C.c_char_p, f32p, I64, I, f32p, f32p, f32p, f32p, C.c_char_p, I]
    L.host_diffusion_continuation.restype = I
    L.host_diffusion_continuation.argtypes = [U64, C.c_char_p, f32p, I64]
    L.host_norm_icdf.restype, L.host_norm_icdf.argtypes = D, [D]
    L.host_norm_cdf.restype, L.host_norm_cdf.argtypes = D, [D]
    L.host_inpaint_masks.restype = None
    L.host_inpaint_masks.argtypes = [U64, I, I, f64p, I, I, I, I, I, D, D, f64p, I, f32p, i32p]
    L.host_build_train_inpaint.restype = None
    L.host_build_train_inpaint.argtypes = [f32p, f32p, I, I, I, F, I, f32p, f32p, i32p]
    L.host_dist_shift_warp.restype = F
    L.host_dist_shift_warp.argtypes = [C.c_char_p, F, I, F, F, F, F]
    L.host_dist_shift_defaults.restype = None
    L.host_dist_shift_defaults.argtypes = [C.c_char_p, f32p]
    L.host_expo_features.restype = None
    L.host_expo_features.argtypes = [F, f32p, I, F, F]
    return L


def diffusion(L, seed, mode, z, count):
    n = z.size
    t = np.zeros(count, np.float32)
    noise, x_t, v = (np.zeros((count, n), np.float32) for _ in range(3))
    st = C.create_string_buffer(1 << 16)
    assert L.host_diffusion_samples(seed, mode.encode(), z, n, count, t, noise, x_t, v, st, 1 << 16) == 0
    return t, noise, x_t, v, st.value.decode()


def masks(L, seed, frames, real_len, probs, count, mask_padding=True, max_mask_segments=10, max_spans=4,
          ratio_lo=0.2, ratio_hi=1.0, span_w=()):
    probs = np.ascontiguousarray(probs, np.float64)
    sw = np.ascontiguousarray(span_w if len(span_w) else [0.0], np.float64)
    m = np.zeros((count, frames), np.float32)
    ty = np.zeros(count, np.int32)
    L.host_inpaint_masks(seed, frames, real_len, probs, probs.size, count, int(mask_padding), max_mask_segments,
                         max_spans, ratio_lo, ratio_hi, sw, len(span_w), m, ty)
    return m, ty


def build(L, z, mask, io, frames, w, mpa):
    local = np.zeros((io + 1) * frames, np.float32)
    weight = np.zeros(io * frames, np.float32)
    counts = np.zeros(2, np.int32)
    L.host_build_train_inpaint(z, mask, io, frames, io + 1, w, int(mpa), local, weight, counts)
    return local, weight, counts


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                                                 b.view(np.uint32) if b.dtype == np.float32 else b)


# ---------------------------------------------------------------- against the reference's outputs
def test_diffusion_sampler_matches_reference_fixtures(host):
    g = np.load(GOLD)
    for k, (seed, mode, n, count) in enumerate(DIFFUSION):
        t, noise, x_t, v, st = diffusion(host, seed, mode, latent(seed, n), count)
        assert same(t, g[f"diff{k}_t"]) and same(noise, g[f"diff{k}_noise"]), (seed, mode)
        assert same(x_t, g[f"diff{k}_x_t"]) and same(v, g[f"diff{k}_v"]), (seed, mode)
        assert st == bytes(g[f"diff{k}_state"]).decode(), (seed, mode)


def test_inpaint_masks_match_reference_fixtures(host):
    g = np.load(GOLD)
    for k, c in enumerate(INPAINT):
        m, ty = masks(host, **c)
        assert same(m, g[f"mask{k}"]) and np.array_equal(ty, g[f"mask{k}_types"]), c


def test_build_train_inpaint_matches_reference_fixtures(host):
    g = np.load(GOLD)
    for k, (io, frames, seed, w, mpa) in enumerate(BUILD):
        z = latent(seed, io * frames)
        mask = (np.random.default_rng(seed).random(frames) < 0.4).astype(np.float32)
        local, weight, counts = build(host, z, mask, io, frames, w, mpa)
        assert same(local, g[f"build{k}_local"]) and same(weight, g[f"build{k}_weight"]), (io, frames)
        assert np.array_equal(counts, g[f"build{k}_counts"])


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built (no reference tree)")
def test_step_inputs_match_reference_live(host):
    # more seeds and shapes than the fixtures, straight against the reference's compiled code
    for seed in range(40):
        mode = ("uniform", "trunc_logit_normal")[seed % 2]
        z = latent(seed, 64 * (1 + seed % 5))
        a = diffusion(host, seed, mode, z, 3)
        b = ref.diffusion_samples(seed, mode, z, 3)
        assert all(same(x, y) for x, y in zip(a[:4], b[:4])) and a[4] == b[4], (seed, mode)
        probs = ([0.2, 0.3, 0.1, 0.4], [0.1, 0.8, 0.1], [0.5, 0.0, 0.5])[seed % 3]
        frames = 16 + 7 * seed
        real = frames - seed % 9
        c = dict(seed=1000 + seed, frames=frames, real_len=real, probs=probs, count=25, max_spans=1 + seed % 5,
                 ratio_lo=0.05, ratio_hi=0.9, span_w=(1.0,) * (seed % 3))
        mh, th = masks(host, **c)
        mr, tr = ref.inpaint_masks(**c)
        assert same(mh, mr) and np.array_equal(th, tr), c


# ---------------------------------------------------------------- the reference tests' properties
def test_rectified_flow_identity_and_continuation(host):
    # tests/train_diffusion_test.cpp: x_t - t v recovers z; draw_t + sample_at == sample; a restored
    # sampler continues the sequence; an empty latent is rejected
    z = np.array([1.0, -2.0, 0.5, 0.0], np.float32)
    for mode in ("uniform", "trunc_logit_normal"):
        t, noise, x_t, v, _ = diffusion(host, 123, mode, z, 20)
        assert np.all((t >= 0.0) & (t <= 1.0))
        assert np.max(np.abs(x_t - t[:, None] * v - z[None, :])) < 1e-6
        assert host.host_diffusion_continuation(123, mode.encode(), z, z.size) == 0


def test_trunc_logit_normal_distribution(host):
    # t = 1 - rescaled sigmoid(Phi^-1(U[Phi(logit .075), 1])): its CDF is closed-form,
    # P(t <= x) = 1 - (Phi(logit(l + (1 - l)(1 - x))) - Phi(logit l)) / (1 - Phi(logit l)), l = .075
    t = diffusion(host, 9, "trunc_logit_normal", np.zeros(1, np.float32), 20000)[0].astype(np.float64)
    from math import erf, log, sqrt
    Phi = lambda x: 0.5 * (1 + erf(x / sqrt(2)))
    l = 0.075
    lo = Phi(log(l / (1 - l)))
    for x in (0.1, 0.3, 0.5, 0.7, 0.9):
        y = l + (1 - l) * (1 - x)
        cdf = 1 - (Phi(log(y / (1 - y))) - lo) / (1 - lo)
        assert abs(np.mean(t <= x) - cdf) < 0.015, x


def test_norm_icdf_and_cdf(host):
    # Acklam's approximation is within 1.15e-9 relative error of the exact quantile (scipy's ndtri)
    # on both tails and the centre; the CDF is the exact one (scipy's ndtr)
    from scipy.special import ndtr, ndtri
    ps = np.concatenate([np.logspace(-12, -1.7, 23), np.linspace(0.02, 0.98, 49), 1 - np.logspace(-12, -1.7, 23)])
    for p in ps:
        x, want = host.host_norm_icdf(float(p)), float(ndtri(p))
        assert abs(x - want) <= 1.2e-9 * abs(want) + 1e-15, p
    for x in np.linspace(-8, 8, 33):
        assert abs(host.host_norm_cdf(float(x)) - float(ndtr(x))) <= 1e-15 + 1e-13 * float(ndtr(x)), x
    assert host.host_norm_icdf(0.0) == -1e9 and host.host_norm_icdf(1.0) == 1e9


def test_inpaint_mask_types(host):
    # tests/train_inpaint_test.cpp: FULL is all zeros; CAUSAL keeps a prefix; SEGMENTS has the
    # requested length; [0.2, 0.6, 0.2] gives all-zero masks about 60% of the time
    m, ty = masks(host, 1, 64, 64, [0.0, 1.0, 0.0], 20)
    assert np.all(ty == 1) and np.all(m == 0)
    m, ty = masks(host, 2, 64, 64, [0.0, 0.0, 1.0], 200)
    assert np.all(ty == 2) and np.all(np.diff(m, axis=1) <= 0)
    m, ty = masks(host, 3, 64, 64, [1.0, 0.0, 0.0], 5)
    assert np.all(ty == 0) and m.shape == (5, 64)
    m, _ = masks(host, 1234, 64, 64, [0.2, 0.6, 0.2], 20000)
    assert 0.57 < np.mean(np.all(m == 0, axis=1)) < 0.66
    m, ty = masks(host, 5, 64, 40, [0.0, 0.0, 0.0, 1.0], 200)   # spans: padding masked, real part partly kept
    assert np.all(ty == 3) and np.all(m[:, 40:] == 0) and np.all(m[:, :40].sum(axis=1) < 40)


def test_build_train_inpaint_weights(host):
    # tests/train_inpaint_test.cpp: layout [mask | z * mask]; with padding attention the generated
    # positions' weights sum to 1 and context weighs 0; without it, gen + w ctx sum to 1
    io, frames = 4, 6
    z = np.arange(1, io * frames + 1, dtype=np.float32)
    mask = np.array([1, 1, 0, 0, 0, 0], np.float32)
    local, weight, counts = build(host, z, mask, io, frames, 1.0, True)
    assert list(counts) == [4, 2]
    loc = local.reshape(frames, io + 1)
    assert np.array_equal(loc[:, 0], mask) and np.array_equal(loc[:, 1:], z.reshape(frames, io) * mask[:, None])
    w = weight.reshape(frames, io)
    assert abs(w[2:].sum() - 1.0) < 1e-6 and np.all(w[:2] == 0)
    _, weight, _ = build(host, z, mask, io, frames, 0.5, False)
    w = weight.reshape(frames, io)
    assert abs(w[2:].sum() + w[:2].sum() - 1.0) < 1e-6 and abs(w[0, 0] / w[2, 0] - 0.5) < 1e-6


# ---------------------------------------------------------------- closed forms (no buildable reference)
def test_dist_shift_warp_closed_forms(host):
    def warp(ty, t, L, p):
        return host.host_dist_shift_warp(ty.encode(), t, L, *p)
    ts = np.linspace(0.01, 0.99, 25)
    for ty in ("LogSNR", "Flux", "Full", "None"):
        p = np.zeros(4, np.float32)
        host.host_dist_shift_defaults(ty.encode(), p)
        for L in (64, 256, 1024, 2000, 5000):
            for t in ts:
                got = warp(ty, float(t), L, p)
                if ty == "LogSNR":
                    start = p[1] - p[2] * np.log2(L / p[0])
                    want = 1 / (1 + np.exp(p[3] - t * (p[3] - start)))
                elif ty == "Flux":
                    x = (np.log(np.clip(L, p[0], p[1])) - np.log(p[0])) / (np.log(p[1]) - np.log(p[0]))
                    a = np.exp(np.log(p[2]) + x * (np.log(p[3]) - np.log(p[2])))
                    want = a * t / (1 + (a - 1) * t)
                elif ty == "Full":
                    x = (np.clip(L, p[2], p[3]) - p[2]) / (p[3] - p[2])
                    mu = -(p[0] + (p[1] - p[0]) * x)
                    want = 1 - np.exp(mu) / (np.exp(mu) + t / (1 - t))
                else:
                    want = t
                assert abs(got - want) <= 2e-6, (ty, L, t)
    # defaults as shipped; identity cases; stale parameters fall back to t
    for ty, want in (("LogSNR", [2000, -6.2, 0, 2]), ("Flux", [256, 4096, 6.93, 6.93]),
                     ("Full", [0.5, 1.15, 256, 4096]), ("None", [0, 0, 0, 0])):
        p = np.zeros(4, np.float32)
        host.host_dist_shift_defaults(ty.encode(), p)
        assert np.allclose(p, want)
    assert warp("Flux", 0.3, 512, (256, 4096, 1.0, 1.0)) == np.float32(0.3)         # alpha 1
    assert warp("Flux", 0.3, 512, (2000, -6.2, 0.0, 2.0)) == np.float32(0.3)        # LogSNR params
    assert warp("Full", 0.3, 512, (0.5, 1.15, 4096, 256)) == np.float32(0.3)        # empty range
    assert warp("Weird", 0.3, 512, (1, 2, 3, 4)) == np.float32(0.3)
    # LogSNR at the anchor length with rate 0 is sigmoid(-(end - t (end - anchor_logsnr)))
    assert abs(warp("LogSNR", 0.5, 2000, (2000, -6.2, 0.0, 2.0)) - 1 / (1 + np.exp(2.0 - 0.5 * 8.2))) < 1e-7


def test_expo_features_match_oracle(host):
    for t in (0.0, 0.013, 0.5, 0.999):
        for dim, lo, hi in ((256, 1.0, 1000.0), (64, 0.5, 64.0), (2, 1.0, 1.0)):
            got = np.zeros(dim, np.float32)
            host.host_expo_features(t, got, dim, lo, hi)
            want = np.zeros(dim, np.float32)
            fn = oracle.lib().orc_expo_features
            fn.restype = None
            fn(C.c_float(t), want.ctypes.data_as(C.c_void_p), C.c_int(dim), C.c_float(lo), C.c_float(hi))
            assert same(got, want), (t, dim)


def test_step_input_time(host):
    # host cost of one update's step inputs at the bench configuration: batch 2 samples of
    # 64 x 1024 latents (noise draw + noising) and one inpaint mask each
    z = latent(0, 64 * 1024)
    t0 = time.perf_counter()
    for s in range(10):
        diffusion(host, s, "trunc_logit_normal", z, 2)
        masks(host, s, 1024, 1024, [0.1, 0.8, 0.1], 2)
    ms = (time.perf_counter() - t0) / 10 * 1e3
    print(f"step inputs for one update (2 samples of 64 x 1024): {ms:.2f} ms on one host core")
    assert ms < 1000
