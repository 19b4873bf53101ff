"""Oracle pinning for the whole DiT training loss (dit_head / dit_block x depth / dit_tail,
src/dit.h:269-338, MSE src/train_dit.h:174-184), no GPU: orc_dit_loss against torch float64
autograd of an independent torch restatement (tests/golden/dit_autograd.npz) on a depth-2 model,
per-sample losses and every adapter gradient: the full scope (all 12 head/tail targets + the
blocks, DoRA, dense attention) and the core scope (blocks only, LoRA, banded attention, per-frame
loss weights); the same with the inpaint local conditioning (dit.<l>.local.{0,2}, src/dit.h:
244-254; tests/golden/dit_local_autograd.npz), whose local linears are adapted in the full scope
only (src/train_lora.h:85-89)."""
import os
import sys

import numpy as np
import pytest

from conftest import ROOT, rel_err

sys.path.insert(0, os.path.join(ROOT, "oracle"))
import dit_binding as db  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
CFG = dict(B=2, T=12, Ctx=5, io=64, dim=128, heads=2, inner=128, depth=2, mem=4, cond_dim=64, time_dim=64,
           rope_dims=32, window=0, rank=8, alpha=16.0, dora=True)
CASES = {"full_dora_dense": (41, "full", True, 0), "core_lora_band_weighted": (42, "core", False, 6)}
LOCAL_CASES = {"full_dora_local": (43, "full", True, 0, False, 65),
               "core_lora_band_local_weighted": (44, "core", False, 6, True, 65)}


def expo_np(t, dim, lo=0.5, hi=1e4):
    half = dim // 2
    i = np.arange(half, dtype=np.float64)
    f = np.exp(i / (half - 1) * (np.log(hi) - np.log(lo)) + np.log(lo))
    return np.concatenate([np.cos(t * f * 2 * np.pi), np.sin(t * f * 2 * np.pi)])


@pytest.mark.parametrize("name", sorted(CASES))
def test_dit_loss_matches_torch_autograd(name):
    seed, scope, dora, window = CASES[name]
    cfg = dict(CFG, dora=dora, window=window)
    tensors, adapters, inputs = db.random_dit(seed, cfg, scope)
    z = np.load(os.path.join(HERE, "golden", "dit_autograd.npz"))
    ref = {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(name + "/")}
    lw = ref.get("loss_weight")
    loss, vel, grads = db.dit_loss(cfg, tensors, adapters, inputs, loss_weight=lw)
    assert np.allclose(loss, ref["loss"], rtol=1e-6, atol=0), (loss, ref["loss"])
    assert set(grads) == {k.split(":", 1)[1] for k in ref if k.startswith("dA:")}
    for n, (dA, dB, dm) in grads.items():
        assert rel_err(dA, ref[f"dA:{n}"]) < 1e-5, ("dA", n, rel_err(dA, ref[f"dA:{n}"]))
        assert rel_err(dB, ref[f"dB:{n}"]) < 1e-5, ("dB", n)
        if dora:
            assert rel_err(dm, ref[f"dm:{n}"]) < 1e-5, ("dm", n)


@pytest.mark.parametrize("name", sorted(LOCAL_CASES))
def test_dit_local_loss_matches_torch_autograd(name):
    seed, scope, dora, window, weighted, local_dim = LOCAL_CASES[name]
    cfg = dict(CFG, dora=dora, window=window, local_dim=local_dim)
    tensors, adapters, inputs = db.random_dit(seed, cfg, scope)
    z = np.load(os.path.join(HERE, "golden", "dit_local_autograd.npz"))
    ref = {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(name + "/")}
    lw = ref.get("loss_weight")
    assert (lw is not None) == weighted
    loss, vel, grads = db.dit_loss(cfg, tensors, adapters, inputs, loss_weight=lw)
    assert np.allclose(loss, ref["loss"], rtol=1e-6, atol=0), (loss, ref["loss"])
    assert set(grads) == {k.split(":", 1)[1] for k in ref if k.startswith("dA:")}
    assert any(".local." in n for n in grads) == (scope == "full")
    for n, (dA, dB, dm) in grads.items():
        assert rel_err(dA, ref[f"dA:{n}"]) < 1e-5, ("dA", n, rel_err(dA, ref[f"dA:{n}"]))
        assert rel_err(dB, ref[f"dB:{n}"]) < 1e-5, ("dB", n)
        if dora:
            assert rel_err(dm, ref[f"dm:{n}"]) < 1e-5, ("dm", n)


def test_dit_local_add_invariants():
    # (1) a local MLP whose output layer is zero (weight and bias; core scope, so unadapted) adds
    # nothing: the loss and every gradient equal the model without local conditioning, bit for bit.
    # (2) without local_cond (a plain step on an inpaint model) the local adapters get no gradient
    # and the rest equals the model without the local linears.
    cfg = dict(CFG, dora=False, window=6, local_dim=65)
    tensors, adapters, inputs = db.random_dit(44, cfg, "core")
    for l in range(cfg["depth"]):
        tensors[f"dit.{l}.local.2.weight"] = np.zeros_like(tensors[f"dit.{l}.local.2.weight"])
        tensors[f"dit.{l}.local.2.bias"] = np.zeros_like(tensors[f"dit.{l}.local.2.bias"])
    plain = dict(cfg, local_dim=0)
    loss0, vel0, g0 = db.dit_loss(plain, tensors, adapters, inputs)
    loss1, vel1, g1 = db.dit_loss(cfg, tensors, adapters, inputs)
    assert np.array_equal(loss0, loss1) and np.array_equal(vel0, vel1)
    for n in g0:
        assert all(np.array_equal(a, b) for a, b in zip(g0[n][:2], g1[n][:2])), n
    cfg = dict(CFG, local_dim=65)
    tensors, adapters, inputs = db.random_dit(43, cfg, "full")
    no_lc = {k: v for k, v in inputs.items() if k != "local"}
    loss2, vel2, g2 = db.dit_loss(cfg, tensors, adapters, no_lc)
    base = {n: a for n, a in adapters.items() if ".local." not in n}
    loss3, vel3, g3 = db.dit_loss(dict(cfg, local_dim=0), tensors, base, inputs)
    assert np.array_equal(loss2, loss3) and np.array_equal(vel2, vel3)
    for n, gr in g2.items():
        if ".local." in n:
            assert not any(np.any(a) for a in gr if a is not None), n
        else:
            assert all(np.array_equal(a, b) for a, b in zip(gr, g3[n]) if a is not None), n
    # a non-zero local MLP changes the loss (the add is not silently dropped)
    loss4, _, _ = db.dit_loss(cfg, tensors, adapters, inputs, grad=False)
    assert not np.allclose(loss4, loss2)


def test_expo_features_closed_form():
    # cos/sin(2 pi t f_i), f_i log-spaced from 0.5 to 1e4 (src/sa3_pipeline.h:57-67); the float32
    # argument carries a relative rounding error of a few ulp, so the bound grows with |arg|
    for t in (0.0, 0.137, 0.5, 1.0):
        got = db.expo_features(t, 256, 0.5, 1e4)
        i = np.arange(128)
        arg = 2 * np.pi * t * np.exp(i / 127 * (np.log(1e4) - np.log(0.5)) + np.log(0.5))
        bound = 1e-6 + 2e-6 * np.concatenate([arg, arg])   # exp argument ~9.2: f carries ~1e-6 relative
        assert np.all(np.abs(got - expo_np(t, 256)) <= bound)
    assert np.array_equal(db.expo_features(0.0, 8, 0.5, 1e4), np.array([1, 1, 1, 1, 0, 0, 0, 0], np.float32))


def test_target_order_is_sorted_weight_names():
    names = db.target_names(dict(CFG, depth=11), "full")
    assert names == sorted(names)
    assert len(names) == 11 * 7 + 12
    assert names.index("dit.10.cross.kv.weight") < names.index("dit.2.cross.kv.weight")   # string order
    assert len(db.target_names(dict(CFG, depth=24), "core")) == 168   # src/train_lora.h:57-58
    # with the inpaint local linears: full 228 = 24 x 9 + 12, core still 168 (src/train_lora.h:56-58)
    assert len(db.target_names(dict(CFG, depth=24, local_dim=257), "full")) == 228
    assert len(db.target_names(dict(CFG, depth=24, local_dim=257), "core")) == 168
