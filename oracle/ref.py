"""ctypes binding of oracle/_ref/libsa3ref.so: the reference's own std-only headers
(src/train_optimizer.h, src/train_diffusion.h, src/train_inpaint.h) compiled where they lie behind
oracle/ref_shim.cpp by `make -C oracle ref`.

TEST INFRASTRUCTURE ONLY: loaded by tests/ and tests/golden/ scripts as the checker of the oracle
and of the host mirror. The library exists only where the reference tree was present when it was
built; callers skip when it is absent.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_ref", "libsa3ref.so")
_lib = None

f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


def available():
    return os.path.exists(LIB_PATH)


def lib():
    global _lib
    if _lib is None:
        L = C.CDLL(LIB_PATH)
        F, I, I64, U64 = C.c_float, C.c_int, C.c_int64, C.c_uint64
        L.ref_inverse_lr.restype, L.ref_inverse_lr.argtypes = F, [F, I, F, F, F, F]
        L.ref_adamw_update_vector.restype = I
        L.ref_adamw_update_vector.argtypes = [f32p, f32p, f32p, f32p, I64, F, F, F, F, F, I]
        L.ref_diffusion_samples.restype = I
        L.ref_diffusion_samples.argtypes = [U64, C.c_char_p, f32p, I64, I, f32p, f32p, f32p, f32p, C.c_char_p, I]
        L.ref_inpaint_masks.restype = None
        L.ref_inpaint_masks.argtypes = [U64, I, I, f64p, I, I, I, I, I, C.c_double, C.c_double, f64p, I, f32p, i32p]
        L.ref_build_train_inpaint.restype = None
        L.ref_build_train_inpaint.argtypes = [f32p, f32p, I, I, I, F, I, f32p, f32p, i32p]
        _lib = L
    return _lib


def inverse_lr(base_lr, step0, inv_gamma, power, warmup, final_lr):
    return lib().ref_inverse_lr(base_lr, step0, inv_gamma, power, warmup, final_lr)


def adamw_update_vector(p, g, m, v, lr, b1, b2, eps, wd, step):
    p, g, m, v = (np.array(a, np.float32, copy=True) for a in (p, g, m, v))
    assert lib().ref_adamw_update_vector(p, g, m, v, p.size, lr, b1, b2, eps, wd, step) == 0
    return p, m, v


def diffusion_samples(seed, mode, z, count):
    z = np.ascontiguousarray(z, np.float32)
    n = z.size
    t = np.zeros(count, np.float32)
    noise, x_t, v = (np.zeros((count, n), np.float32) for _ in range(3))
    st = C.create_string_buffer(1 << 16)
    assert lib().ref_diffusion_samples(seed, mode.encode(), z, n, count, t, noise, x_t, v, st, 1 << 16) == 0
    return t, noise, x_t, v, st.value.decode()


def inpaint_masks(seed, frames, real_len, probs, count, mask_padding=True, max_mask_segments=10, max_spans=4,
                  ratio_lo=0.2, ratio_hi=1.0, span_w=()):
    probs = np.ascontiguousarray(probs, np.float64)
    sw = np.ascontiguousarray(span_w if len(span_w) else [0.0], np.float64)
    masks = np.zeros((count, frames), np.float32)
    types = np.zeros(count, np.int32)
    lib().ref_inpaint_masks(seed, frames, real_len, probs, probs.size, count, int(mask_padding), max_mask_segments,
                            max_spans, ratio_lo, ratio_hi, sw, len(span_w), masks, types)
    return masks, types


def build_train_inpaint(z, mask, io, frames, local_dim, mask_loss_weight, mask_padding_attention=True):
    z = np.ascontiguousarray(z, np.float32)
    mask = np.ascontiguousarray(mask, np.float32)
    local = np.zeros(local_dim * frames, np.float32)
    weight = np.zeros(io * frames, np.float32)
    counts = np.zeros(2, np.int32)
    lib().ref_build_train_inpaint(z, mask, io, frames, local_dim, mask_loss_weight, int(mask_padding_attention),
                                  local, weight, counts)
    return local, weight, int(counts[0]), int(counts[1])
