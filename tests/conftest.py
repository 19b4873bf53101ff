import importlib.util
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "sa3.cpp_amd")


def _load(name, path):
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


sa3k = _load("sa3k", os.path.join(PKG, "sa3k.py"))
oracle = _load("sa3_oracle", os.path.join(ROOT, "oracle", "oracle.py"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libsa3k.so")


@pytest.fixture(scope="session")
def ctx():
    c = sa3k.Context(0)
    c.defaults = c.options()   # the shipped option values, as a fresh context has them
    yield c
    c.close()


@pytest.fixture(autouse=True)
def _restore_options(request):
    """After every test that used the GPU context, put every option back to its shipped default,
    so that no test runs with a value another test left behind."""
    yield
    if "ctx" in request.fixturenames:
        c = request.getfixturevalue("ctx")
        c.set_options(c.defaults)


def assert_shipped_options(c):
    """the context runs the shipped configuration: every option at its default"""
    now = c.options()
    diff = {k: (now[k], v) for k, v in c.defaults.items() if now[k] != v}
    assert not diff, f"options differ from the defaults (now, default): {diff}"


def rng(seed):
    """Counter-based generator shared by tests and the bench (Philox4x32-10, numpy)."""
    return np.random.Generator(np.random.Philox(seed))


def rel_err(a, b):
    """normwise relative error ||a-b|| / ||b||"""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    nb = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (nb if nb > 0 else 1.0))


def max_rel_err(a, b):
    """max relative error in the infinity norm: max_i |a_i-b_i| / max_i |b_i|.

    This is the reading of "max relative error" used for the f32 tolerance: a per-element ratio is
    undefined where the reference crosses zero, and fp32 accumulation over K terms leaves an
    absolute error of order sqrt(K) * 2^-24 * |terms| on every element, near-zero ones included."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    if not b.size:
        return 0.0
    return float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))), 1e-300))


def elem_rel_err(a, b, floor_frac=0.1):
    """element-wise relative error with a floor: max_i |a_i - b_i| / max(|b_i|, floor), floor =
    floor_frac * rms(b). Elements at least as large as the floor are held to their own relative
    error; smaller ones (near the reference's zero crossings, where a ratio is meaningless) to the
    absolute error floor * bound."""
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    if not b.size:
        return 0.0
    floor = floor_frac * max(float(np.sqrt(np.mean(b * b))), 1e-300)
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), floor)))


def bf16_round(x):
    """float32 -> nearest-even bfloat16, returned as float32 (finite inputs)"""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u >> 16) & 1) + 0x7FFF
    return ((u + r) & 0xFFFF0000).astype(np.uint32).view(np.float32)


def bf16_bits(x):
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def q8_0_split(blocks, out_, in_):
    """raw Q8_0 blocks of W [out][in] -> (quants int8 [out][in], f16 scale bits [out][in/32], decoded f32)"""
    b = np.asarray(blocks, np.uint8).reshape(out_, in_ // 32, 34)
    sc = b[:, :, 0:2].copy().view(np.uint16).reshape(out_, in_ // 32)
    q = b[:, :, 2:].copy().view(np.int8).reshape(out_, in_)
    dec = (sc.view(np.float16).astype(np.float32).repeat(32, axis=1) * q.astype(np.float32)).astype(np.float32)
    return q, sc, dec


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))
