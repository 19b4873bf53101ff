"""Writes tests/golden/step_inputs_ref.npz: outputs of the reference's own step-input producers
(src/train_diffusion.h TrainDiffusionSampler, src/train_inpaint.h generate_inpaint_mask and
build_train_inpaint), compiled from the reference tree into oracle/_ref/libsa3ref.so
(`make -C oracle ref`). Run from the repository root where that library is built:

    python3 tests/golden/make_step_input_fixtures.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))
import ref  # noqa: E402
from step_input_cases import BUILD, DIFFUSION, INPAINT, latent  # noqa: E402


def main():
    assert ref.available(), "build oracle/_ref first (make -C oracle ref)"
    out = {}
    for k, (seed, mode, n, count) in enumerate(DIFFUSION):
        t, noise, x_t, v, st = ref.diffusion_samples(seed, mode, latent(seed, n), count)
        out[f"diff{k}_t"], out[f"diff{k}_noise"], out[f"diff{k}_x_t"], out[f"diff{k}_v"] = t, noise, x_t, v
        out[f"diff{k}_state"] = np.frombuffer(st.encode(), np.uint8)
    for k, c in enumerate(INPAINT):
        masks, types = ref.inpaint_masks(**c)
        out[f"mask{k}"], out[f"mask{k}_types"] = masks, types
    for k, (io, frames, seed, w, mpa) in enumerate(BUILD):
        z = latent(seed, io * frames)
        mask = (np.random.default_rng(seed).random(frames) < 0.4).astype(np.float32)
        local, weight, n_gen, n_ctx = ref.build_train_inpaint(z, mask, io, frames, io + 1, w, mpa)
        out[f"build{k}_local"], out[f"build{k}_weight"] = local, weight
        out[f"build{k}_counts"] = np.array([n_gen, n_ctx], np.int32)
    np.savez_compressed(os.path.join(ROOT, "tests", "golden", "step_inputs_ref.npz"), **out)
    print("wrote", len(out), "arrays")


if __name__ == "__main__":
    main()
