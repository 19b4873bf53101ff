"""The cases of tests/golden/step_inputs_ref.npz (shared by tests/golden/make_step_input_fixtures.py and
tests/test_host_step_inputs.py)."""
import numpy as np

# (seed, mode, latent elements, samples drawn in a row)
DIFFUSION = [(123, "uniform", 4, 3), (7, "uniform", 64 * 33, 4), (2024, "trunc_logit_normal", 64 * 17, 5),
             (0, "trunc_logit_normal", 3, 50)]

# generate_inpaint_mask runs from one std::mt19937_64(seed), `count` masks in a row
INPAINT = [dict(seed=1, frames=64, real_len=64, probs=[0.1, 0.8, 0.1], count=40),
           dict(seed=2, frames=96, real_len=80, probs=[0.2, 0.6, 0.2], count=60),
           dict(seed=3, frames=64, real_len=64, probs=[1.0, 0.0, 0.0], count=30, max_mask_segments=6),
           dict(seed=4, frames=128, real_len=100, probs=[0.0, 0.0, 1.0], count=30, mask_padding=False),
           dict(seed=5, frames=64, real_len=50, probs=[0.25, 0.25, 0.25, 0.25], count=80, max_spans=4,
                ratio_lo=0.2, ratio_hi=1.0),
           dict(seed=6, frames=256, real_len=256, probs=[0.0, 0.0, 0.0, 1.0], count=60, max_spans=6,
                ratio_lo=0.1, ratio_hi=0.5, span_w=(3.0, 1.0, 1.0)),
           dict(seed=7, frames=32, real_len=0, probs=[0.3, 0.3, 0.4], count=10),
           dict(seed=8, frames=16, real_len=16, probs=[0.0, 0.0, 0.0], count=10)]

# build_train_inpaint: (io, frames, seed, mask_loss_weight, mask_padding_attention)
BUILD = [(4, 6, 1, 1.0, True), (64, 257, 2, 0.5, False), (64, 100, 3, 2.0, True), (8, 40, 4, 0.0, False)]


def latent(seed, n):
    return np.random.default_rng(seed).normal(0, 1, n).astype(np.float32)
