"""Oracle pinning for one DiT block (src/dit.h:164-266), no GPU: the oracle's forward and its
hand-derived backward against torch float64 autograd of an independent torch restatement
(tests/golden/dit_block_autograd.npz): DoRA dense and LoRA banded cases, every input gradient
(x, context, gcond) and every adapter gradient of the 7 targets."""
import os
import sys

import numpy as np
import pytest

from conftest import ROOT, rel_err

sys.path.insert(0, os.path.join(ROOT, "oracle"))
import block_binding as bb  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = {"dora_dense": (11, 0, True), "lora_band": (12, 8, False)}


@pytest.mark.parametrize("name", sorted(CASES))
def test_block_matches_torch_autograd(name):
    seed, window, dora = CASES[name]
    cfg, w, x, ctx, gc = bb.random_block(seed, B=2, S=20, Ctx=6, dim=128, heads=2, inner=96, rank=8, alpha=16.0,
                                         dora=dora, window=window, w_sd=0.05, b_sd=0.05)
    z = np.load(os.path.join(HERE, "golden", "dit_block_autograd.npz"))
    ref = {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(name + "/")}
    out = bb.block_fwd(cfg, w, x, ctx, gc)
    assert rel_err(out, ref["out"]) < 1e-6
    g = bb.block_bwd(cfg, w, x, ctx, gc, ref["dout"])
    for k in ("dx", "dctx", "dgcond"):
        assert rel_err(g[k], ref[k]) < 1e-5, k
    for t in range(7):
        assert rel_err(g["dA"][t], ref[f"dA{t}"]) < 1e-5, ("dA", t)
        assert rel_err(g["dB"][t], ref[f"dB{t}"]) < 1e-5, ("dB", t)
        if dora:
            assert rel_err(g["dm"][t], ref[f"dm{t}"]) < 1e-5, ("dm", t)
