"""ctypes binding of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker or the timed CPU baseline. Never part of the product path.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")
_lib = None

f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")


def build():
    subprocess.run(["make", "-s", "-C", HERE, "-j8"], check=True)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = C.CDLL(LIB_PATH)
    I64, I, F, D = C.c_int64, C.c_int, C.c_float, C.c_double
    optf = C.c_void_p  # nullable float*
    sigs = {
        "orc_inverse_lr": (F, [F, I, F, F, F, F]),
        "orc_adamw_update_vector": (I, [f32p, f32p, f32p, f32p, I64, F, F, F, F, F, I]),
        "orc_average_and_clip": (None, [f32p, I64, I, F, C.POINTER(D), C.POINTER(F)]),
        "orc_apply_accumulated_adamw": (I, [f32p, f32p, f32p, f32p, I64, F, F, F, F, F, F, I, I,
                                            C.POINTER(D), C.POINTER(F)]),
        "orc_f32_to_f16": (C.c_uint16, [F]),
        "orc_f16_to_f32": (F, [C.c_uint16]),
        "orc_f32_to_f16_row": (None, [f32p, u16p, I64]),
        "orc_f16_to_f32_row": (None, [u16p, f32p, I64]),
        "orc_q8_0_quantize": (None, [f32p, u8p, I64]),
        "orc_q8_0_dequant": (None, [u8p, f32p, I64]),
        "orc_row_norm_sq": (None, [f32p, I64, I64, F, f32p]),
        "orc_row_norms": (None, [f32p, I64, I64, f32p]),
        "orc_effective_weight": (None, [f32p, I64, I64, f32p, f32p, optf, I, F, I, f32p]),
        "orc_dit_lin_fwd": (None, [f32p, I64, f32p, I64, I64, optf, optf, I, F, I, optf, optf, optf,
                                   f32p, optf, optf, optf]),
        "orc_dit_lin_sqloss": (D, [f32p, I64, f32p, I64, I64, optf, optf, I, F, I, optf, optf, optf, f32p]),
        "orc_dit_lin_bwd": (None, [f32p, I64, f32p, I64, I64, optf, optf, I, F, I, optf, optf, f32p,
                                   optf, optf, optf, optf]),
        "orc_gemm_nt": (None, [f32p, f32p, f32p, I64, I64, I64]),
        "orc_num_threads": (I, []),
        "orc_set_f32": (None, [I]),
        "orc_f32_fast": (I, []),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args
    _lib = L
    return L


class f32_mode:
    """with f32_mode(): the linears and the attention (and the block / DiT functions over them)
    compute in float with the AVX2/FMA products: the CPU baseline's mode. The double oracle is
    restored on exit."""

    def __enter__(self):
        lib().orc_set_f32(1)
        return self

    def __exit__(self, *exc):
        lib().orc_set_f32(0)
        return False


def _p(a):
    """nullable pointer of a contiguous float32 array"""
    return None if a is None else a.ctypes.data


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- optimizer
def inverse_lr(base_lr, step0, inv_gamma, power, warmup, final_lr):
    return lib().orc_inverse_lr(base_lr, step0, inv_gamma, power, warmup, final_lr)


def apply_accumulated_adamw(p, g, m, v, lr, b1, b2, eps, wd, clip, step, count):
    """in-place on copies; returns (p, g, m, v, norm, scale)"""
    p, g, m, v = (np.array(x, dtype=np.float32, copy=True) for x in (p, g, m, v))
    norm, scale = C.c_double(), C.c_float()
    rc = lib().orc_apply_accumulated_adamw(p, g, m, v, p.size, lr, b1, b2, eps, wd, clip, step, count,
                                           C.byref(norm), C.byref(scale))
    if rc != 0:
        raise ValueError("oracle AdamW rejected the arguments")
    return p, g, m, v, norm.value, scale.value


def adamw_update_vector(p, g, m, v, lr, b1, b2, eps, wd, step):
    p, g, m, v = (np.array(x, dtype=np.float32, copy=True) for x in (p, g, m, v))
    if lib().orc_adamw_update_vector(p, g, m, v, p.size, lr, b1, b2, eps, wd, step) != 0:
        raise ValueError("oracle AdamW rejected the arguments")
    return p, m, v


# ---------------------------------------------------------------- quant
def f32_to_f16_bits(x):
    x = f32(x).ravel()
    y = np.empty(x.size, np.uint16)
    lib().orc_f32_to_f16_row(x, y, x.size)
    return y


def f16_bits_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    y = np.empty(h.size, np.float32)
    lib().orc_f16_to_f32_row(h, y, h.size)
    return y


def q8_0_quantize(x):
    x = f32(x).ravel()
    assert x.size % 32 == 0
    out = np.empty(x.size // 32 * 34, np.uint8)
    lib().orc_q8_0_quantize(x, out, x.size)
    return out


def q8_0_dequant(blocks, n):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    y = np.empty(n, np.float32)
    lib().orc_q8_0_dequant(blocks, y, n)
    return y


# ---------------------------------------------------------------- adapter state / dit_lin
def row_norm_sq(W, eps=1e-12):
    W = f32(W)
    out_, in_ = W.shape
    y = np.empty(out_, np.float32)
    lib().orc_row_norm_sq(W, in_, out_, eps, y)
    return y


def row_norms(W):
    W = f32(W)
    out_, in_ = W.shape
    y = np.empty(out_, np.float32)
    lib().orc_row_norms(W, in_, out_, y)
    return y


def effective_weight(W, A, B, mag, alpha, dora):
    W, A, B = f32(W), f32(A), f32(B)
    out_, in_ = W.shape
    r = A.shape[0]
    mag = None if mag is None else f32(mag)
    y = np.empty_like(W)
    lib().orc_effective_weight(W, in_, out_, A, B, _p(mag), r, alpha, int(dora), y)
    return y


def dit_lin_fwd(X, W, A=None, B=None, s=1.0, dora=False, mag=None, bnsq=None, bias=None):
    X, W = f32(X), f32(W)
    N, in_ = X.shape
    out_ = W.shape[0]
    r = 0 if A is None else A.shape[0]
    A = None if A is None else f32(A)
    B = None if B is None else f32(B)
    mag = None if mag is None else f32(mag)
    bnsq = None if bnsq is None else f32(bnsq)
    bias = None if bias is None else f32(bias)
    Y = np.empty((N, out_), np.float32)
    U = np.empty((N, out_), np.float32)
    d = np.empty(out_, np.float32)
    nsq = np.empty(out_, np.float32)
    lib().orc_dit_lin_fwd(X, N, W, in_, out_, _p(A), _p(B), r, s, int(dora), _p(mag), _p(bnsq), _p(bias),
                          Y, _p(U), _p(d), _p(nsq))
    return dict(Y=Y, U=U, d=d, nsq=nsq)


def dit_lin_sqloss(X, W, tgt, A=None, B=None, s=1.0, dora=False, mag=None, bnsq=None, bias=None):
    X, W, tgt = f32(X), f32(W), f32(tgt)
    N, in_ = X.shape
    out_ = W.shape[0]
    r = 0 if A is None else A.shape[0]
    A = None if A is None else f32(A)
    B = None if B is None else f32(B)
    mag = None if mag is None else f32(mag)
    bnsq = None if bnsq is None else f32(bnsq)
    bias = None if bias is None else f32(bias)
    return lib().orc_dit_lin_sqloss(X, N, W, in_, out_, _p(A), _p(B), r, s, int(dora), _p(mag), _p(bnsq),
                                    _p(bias), tgt)


def dit_lin_bwd(X, W, dY, A=None, B=None, s=1.0, dora=False, mag=None, bnsq=None):
    X, W, dY = f32(X), f32(W), f32(dY)
    N, in_ = X.shape
    out_ = W.shape[0]
    r = 0 if A is None else A.shape[0]
    A = None if A is None else f32(A)
    B = None if B is None else f32(B)
    mag = None if mag is None else f32(mag)
    bnsq = None if bnsq is None else f32(bnsq)
    dX = np.empty((N, in_), np.float32)
    dA = np.empty((max(r, 1), in_), np.float32)
    dB = np.empty((out_, max(r, 1)), np.float32)
    dm = np.empty(out_, np.float32)
    lib().orc_dit_lin_bwd(X, N, W, in_, out_, _p(A), _p(B), r, s, int(dora), _p(mag), _p(bnsq), dY,
                          dX.ctypes.data, dA.ctypes.data if r else None, dB.ctypes.data if r else None,
                          dm.ctypes.data)
    return dict(dX=dX, dA=dA if r else None, dB=dB if r else None, dm=dm)


def gemm_nt(A, B):
    A, B = f32(A), f32(B)
    M, K = A.shape
    N = B.shape[0]
    Cm = np.empty((M, N), np.float32)
    lib().orc_gemm_nt(A, B, Cm, M, N, K)
    return Cm


# ---------------------------------------------------------------- differential attention
def _attn_sig():
    L = lib()
    if getattr(L, "_attn_declared", False):
        return L
    I, F = C.c_int, C.c_float
    optf = C.c_void_p
    L.orc_diff_attn_fwd.restype = None
    L.orc_diff_attn_fwd.argtypes = [f32p, f32p, f32p, f32p, f32p, I, I, I, I, F, I, f32p, optf, optf, optf, optf]
    L.orc_diff_attn_bwd.restype = None
    L.orc_diff_attn_bwd.argtypes = [f32p, f32p, f32p, f32p, f32p, f32p, I, I, I, I, F, I, f32p, f32p, f32p, f32p, f32p]
    L._attn_declared = True
    return L


def diff_attn_fwd(Q1, K1, Q2, K2, V, scale=0.125, window=0):
    """arrays [BH][S][D]; returns dict O, O1, O2, lse1, lse2"""
    Q1, K1, Q2, K2, V = (f32(x) for x in (Q1, K1, Q2, K2, V))
    BH, Sq, D = Q1.shape
    Sk = K1.shape[1]
    O, O1, O2 = (np.empty((BH, Sq, D), np.float32) for _ in range(3))
    l1, l2 = np.empty((BH, Sq), np.float32), np.empty((BH, Sq), np.float32)
    _attn_sig().orc_diff_attn_fwd(Q1, K1, Q2, K2, V, BH, Sq, Sk, D, scale, window, O, O1.ctypes.data,
                                  O2.ctypes.data, l1.ctypes.data, l2.ctypes.data)
    return dict(O=O, O1=O1, O2=O2, lse1=l1, lse2=l2)


def diff_attn_bwd(Q1, K1, Q2, K2, V, dO, scale=0.125, window=0):
    Q1, K1, Q2, K2, V, dO = (f32(x) for x in (Q1, K1, Q2, K2, V, dO))
    BH, Sq, D = Q1.shape
    Sk = K1.shape[1]
    dQ1, dQ2 = np.empty_like(Q1), np.empty_like(Q2)
    dK1, dK2, dV = np.empty_like(K1), np.empty_like(K2), np.empty_like(V)
    _attn_sig().orc_diff_attn_bwd(Q1, K1, Q2, K2, V, dO, BH, Sq, Sk, D, scale, window, dQ1, dK1, dQ2, dK2, dV)
    return dict(dQ1=dQ1, dK1=dK1, dQ2=dQ2, dK2=dK2, dV=dV)


class _ChainAd(C.Structure):
    _fields_ = [("dora", C.c_int), ("rank", C.c_int), ("alpha", C.c_float), ("strength", C.c_float),
                ("A", C.c_void_p), ("B", C.c_void_p), ("mag", C.c_void_p)]


def _chain(adapters):
    """adapters: [(dora, rank, alpha, strength, A [r][in], B [out][r], mag [out] | None)] -> ctypes array, keep"""
    keep = []
    arr = (_ChainAd * max(1, len(adapters)))()
    for i, (dora, rank, alpha, strength, A, B, mag) in enumerate(adapters):
        A, B = f32(A), f32(B)
        mag = f32(mag) if mag is not None else None
        keep += [A, B, mag]
        arr[i] = _ChainAd(int(dora), int(rank), float(alpha), float(strength), A.ctypes.data, B.ctypes.data,
                          mag.ctypes.data if mag is not None else None)
    return arr, keep


def _chain_sigs(L):
    if getattr(L, "_chain_declared", False):
        return
    I64, I, P = C.c_int64, C.c_int, C.c_void_p
    L.orc_chain_merge.restype = None
    L.orc_chain_merge.argtypes = [f32p, I64, I64, I, P, f32p]
    L.orc_chain_fold.restype = None
    L.orc_chain_fold.argtypes = [f32p, I64, I64, I, P, f32p, f32p, f32p]
    L.orc_chain_forward.restype = None
    L.orc_chain_forward.argtypes = [f32p, I64, f32p, I64, I64, I, P, C.c_void_p, f32p]
    L._chain_declared = True


def chain_merge(W, adapters):
    """apply_loras' sequential merge of the chain into W_eff [out][in]"""
    L = lib()
    _chain_sigs(L)
    W = f32(W)
    out_, in_ = W.shape
    arr, keep = _chain(adapters)
    Weff = np.empty_like(W)
    L.orc_chain_merge(W, in_, out_, len(adapters), C.cast(arr, C.c_void_p), Weff)
    return Weff


def chain_fold(W, adapters):
    """build_functional_lora's constants: (base_scale [out], B' [out][R], scales [n_active])"""
    L = lib()
    _chain_sigs(L)
    W = f32(W)
    out_, in_ = W.shape
    act = [a for a in adapters if a[3] != 0.0]
    R = sum(a[1] for a in act)
    arr, keep = _chain(adapters)
    c0, Bp, sc = np.empty(out_, np.float32), np.empty((out_, max(R, 1)), np.float32), np.empty(max(len(act), 1), np.float32)
    L.orc_chain_fold(W, in_, out_, len(adapters), C.cast(arr, C.c_void_p), c0, Bp, sc)
    return c0, Bp[:, :R], sc[:len(act)]


def chain_forward(X, W, adapters, bias=None):
    """Y [N][out] = base_scale * (X W^T) + sum_k s_k (X A_k^T) B'_k^T (+ bias), double accumulation"""
    L = lib()
    _chain_sigs(L)
    X, W = f32(X), f32(W)
    out_, in_ = W.shape
    arr, keep = _chain(adapters)
    b = f32(bias) if bias is not None else None
    Y = np.empty((X.shape[0], out_), np.float32)
    L.orc_chain_forward(X, X.shape[0], W, in_, out_, len(adapters), C.cast(arr, C.c_void_p), _p(b), Y)
    return Y
