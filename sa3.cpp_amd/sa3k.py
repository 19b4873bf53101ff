"""Python binding of the sa3k C ABI (include/sa3k.h) over ctypes.

This is plumbing for the test and benchmark harnesses: it loads the in-tree libsa3k.so (built by
sa3.cpp_amd/build.py), owns device buffers and converts numpy arrays. It never falls back to
another implementation: when the library or a GPU is missing it raises.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsa3k.so")

SA3K_OK = 0
TYPE_F32, TYPE_F16, TYPE_Q8_0, TYPE_BF16 = 0, 1, 8, 30
PREC_F32, PREC_BF16 = 0, 1

_lib = None


class Sa3kError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"sa3k error {code}: {msg}")
        self.code = code


class AdamWParams(C.Structure):
    _fields_ = [("learning_rate", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float),
                ("eps", C.c_float), ("weight_decay", C.c_float), ("grad_clip", C.c_float)]


class ChainAdapter(C.Structure):
    _fields_ = [("dora", C.c_int), ("rank", C.c_int), ("alpha", C.c_float), ("strength", C.c_float),
                ("A", C.c_void_p), ("B", C.c_void_p), ("magnitude", C.c_void_p)]


class BlockConfig(C.Structure):
    _fields_ = [("dim", C.c_int), ("heads", C.c_int), ("head_dim", C.c_int), ("inner", C.c_int),
                ("rope_dims", C.c_int), ("window", C.c_int), ("rope_base", C.c_float), ("norm_eps", C.c_float),
                ("qk_eps", C.c_float)]


class BlockWeights(C.Structure):
    _fields_ = [("weight_type", C.c_int), ("W", C.c_void_p * 7), ("bias", C.c_void_p * 7)] + \
               [(n, C.c_void_p) for n in ("ssg", "pre_g", "cross_g", "ff_g", "sq_g", "sk_g", "cq_g", "ck_g")]


BLOCK_VECTORS = ("ssg", "pre_g", "cross_g", "ff_g", "sq_g", "sk_g", "cq_g", "ck_g")


class DitConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("io", "dim", "depth", "heads", "head_dim", "cond_dim", "mem_tokens", "rope_dims",
                                       "time_dim", "inner", "window")] + \
               [(n, C.c_float) for n in ("rope_base", "norm_eps", "qk_eps", "time_min_freq", "time_max_freq")] + \
               [("local_dim", C.c_int)]


class DitTrain(C.Structure):
    _fields_ = [("rank", C.c_int), ("alpha", C.c_float), ("dora", C.c_int), ("scope", C.c_int), ("batch", C.c_int),
                ("frames", C.c_int), ("ctx_tokens", C.c_int), ("recompute", C.c_int)]


SCOPE_CORE, SCOPE_FULL = 0, 1


def dit_config(io, dim, depth, heads, cond_dim, mem_tokens, time_dim, inner, window=0, rope_dims=32, local_dim=0):
    return DitConfig(io, dim, depth, heads, 64, cond_dim, mem_tokens, rope_dims, time_dim, inner, window,
                     1e4, 1e-5, 1e-6, 0.5, 1e4, local_dim)


def block_target_dims(dim, inner):
    """(in, out) of the 7 adapted linears of a block, in target order"""
    return [(dim, 5 * dim), (dim, dim), (dim, 2 * dim), (dim, 3 * dim), (dim, dim), (dim, 2 * inner), (inner, dim)]


def _declare(lib):
    P, I64, I, F, D = C.c_void_p, C.c_int64, C.c_int, C.c_float, C.c_double
    sig = {
        "sa3k_create": (P, [I, C.c_char_p, I]),
        "sa3k_destroy": (None, [P]),
        "sa3k_last_error": (C.c_char_p, [P]),
        "sa3k_version": (C.c_char_p, []),
        "sa3k_malloc": (I, [P, C.c_size_t, C.POINTER(P)]),
        "sa3k_free": (I, [P, P]),
        "sa3k_upload": (I, [P, P, P, C.c_size_t]),
        "sa3k_download": (I, [P, P, P, C.c_size_t]),
        "sa3k_copy_d2d": (I, [P, P, P, C.c_size_t]),
        "sa3k_memset": (I, [P, P, I, C.c_size_t]),
        "sa3k_sync": (I, [P]),
        "sa3k_set_option": (I, [P, C.c_char_p, I]),
        "sa3k_get_option": (I, [P, C.c_char_p, C.POINTER(I)]),
        "sa3k_option_name": (C.c_char_p, [I]),
        "sa3k_timer_start": (I, [P]),
        "sa3k_timer_stop": (I, [P, C.POINTER(F)]),
        "sa3k_profile_enable": (I, [P, I]),
        "sa3k_profile_reset": (I, [P]),
        "sa3k_profile_report": (I, [P, C.c_char_p, I]),
        "sa3k_adamw_clip": (I, [P, P, P, P, P, I64, C.POINTER(AdamWParams), I, I, C.POINTER(D)]),
        "sa3k_adamw_clip_scale": (I, [P, C.POINTER(D), C.POINTER(F)]),
        "sa3k_average_and_clip": (I, [P, P, I64, I, F, C.POINTER(D)]),
        "sa3k_q8_0_dequant": (I, [P, P, P, I64]),
        "sa3k_q8_0_quantize": (I, [P, P, P, I64]),
        "sa3k_gemm_nt": (I, [P, I, I, P, I64, I, P, I64, P, I64, I64, I64, I64, F, P, P, P, I64, I]),
        "sa3k_gemm_nt_noalloc": (I, [P, I, I, P, I64, I, P, I64, P, I64, I64, I64, I64, F, P, P, P, I64, I]),
        "sa3k_weight_create": (I, [P, I, I64, I64, P, I, C.POINTER(P)]),
        "sa3k_weight_destroy": (I, [P, P]),
        "sa3k_weight_drop_working_copy": (I, [P, P]),
        "sa3k_weight_row_norm_sq": (I, [P, P, F, P]),
        "sa3k_weight_row_norms": (I, [P, P, P]),
        "sa3k_row_norms": (I, [P, I, I64, I64, P, I, F, P]),
        "sa3k_lin_create": (I, [P, P, I, I, I64, C.POINTER(P)]),
        "sa3k_lin_destroy": (I, [P, P]),
        "sa3k_lin_prepare": (I, [P, P, P, P, F, I, P, P]),
        "sa3k_lin_forward": (I, [P, P, I, P, I64, P, P]),
        "sa3k_lin_backward": (I, [P, P, I, P, I64, P, P, I, P, P, P]),
        "sa3k_lora_chain_create": (I, [P, P, I, C.POINTER(ChainAdapter), I64, C.POINTER(P)]),
        "sa3k_lora_chain_destroy": (I, [P, P]),
        "sa3k_lora_chain_forward": (I, [P, P, I, P, I64, P, P]),
        "sa3k_lora_chain_constants": (I, [P, P, P, P, C.POINTER(I)]),
        "sa3k_diff_attn_fwd": (I, [P, P, P, P, P, P, I, I, I, I, I, I, F, P, P, P, P, P]),
        "sa3k_diff_attn_bwd": (I, [P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, F, P, P, P, P, P, P, P]),
        "sa3k_block_create": (I, [P, C.POINTER(BlockConfig), C.POINTER(BlockWeights), I, I64, I64, C.POINTER(P)]),
        "sa3k_block_destroy": (I, [P, P]),
        "sa3k_block_base_norm_sq": (I, [P, P, I, C.POINTER(P)]),
        "sa3k_block_ws_create": (I, [P, C.POINTER(BlockConfig), I, I, I, C.POINTER(P)]),
        "sa3k_block_ws_destroy": (I, [P, P]),
        "sa3k_block_prepare": (I, [P, P, P, P, P, F, I]),
        "sa3k_block_forward": (I, [P, P, P, P, P, P, P]),
        "sa3k_block_backward": (I, [P, P, P, P, P, P, P, P, P, P]),
        "sa3k_dit_create": (I, [P, C.POINTER(DitConfig), I, C.POINTER(P)]),
        "sa3k_dit_destroy": (I, [P, P]),
        "sa3k_dit_tensor_count": (I, [P, P, C.POINTER(I)]),
        "sa3k_dit_tensor_info": (I, [P, P, I, C.c_char_p, I, C.POINTER(I64), C.POINTER(I64), C.POINTER(I)]),
        "sa3k_dit_set_tensor": (I, [P, P, C.c_char_p, P, I64]),
        "sa3k_dit_init_random": (I, [P, P, C.c_uint64, F]),
        "sa3k_dit_setup": (I, [P, P, C.POINTER(DitTrain)]),
        "sa3k_dit_weight_row_norms": (I, [P, P, C.c_char_p, I, F, P]),
        "sa3k_dit_arena": (I, [P, P, I, C.POINTER(P), C.POINTER(I64)]),
        "sa3k_dit_target_count": (I, [P, P, C.POINTER(I)]),
        "sa3k_dit_target_info": (I, [P, P, I, C.c_char_p, I, C.POINTER(I64), C.POINTER(I64), C.POINTER(I64),
                                     C.POINTER(I64), C.POINTER(I64)]),
        "sa3k_dit_adapters_init": (I, [P, P, C.c_uint64, F]),
        "sa3k_dit_adapters_changed": (I, [P, P]),
        "sa3k_dit_accumulate": (I, [P, P, P, P, P, P, P, P, P]),
        "sa3k_dit_apply_adamw": (I, [P, P, C.POINTER(AdamWParams), I, C.POINTER(D)]),
        "sa3k_dit_forward": (I, [P, P, P, P, P, P, P]),
        "sa3k_dit_eval_loss": (I, [P, P, P, P, P, P, P, P, C.POINTER(D)]),
        "sa3k_dit_set_graphs": (I, [P, P, I]),
        "sa3k_dit_get_graphs": (I, [P, P, P]),
        "sa3k_dit_set_local": (I, [P, P, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return sig


def load_library(path=None):
    """Load libsa3k.so (cached). Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is missing: run python sa3.cpp_amd/build.py first")
    lib = C.CDLL(path)
    _declare(lib)
    _lib = lib
    return lib


def declared_symbols(header=None):
    """Every sa3k_* function name declared in include/sa3k.h."""
    import re
    header = header or os.path.join(os.path.dirname(HERE), "include", "sa3k.h")
    text = open(header).read()
    return sorted(set(re.findall(r"SA3K_API\s+[^;(]*?\b(sa3k_\w+)\s*\(", text)))


class DeviceArray:
    """A device allocation with a numpy shape/dtype, owned by a Context."""

    def __init__(self, ctx, ptr, shape, dtype, owner=True):
        self.ctx, self.ptr = ctx, ptr
        self.shape = tuple(shape)
        self.dtype = np.dtype(dtype)
        self.owner = owner

    @property
    def nbytes(self):
        return int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize

    @property
    def size(self):
        return int(np.prod(self.shape, dtype=np.int64))

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        self.ctx.check(self.ctx.lib.sa3k_download(self.ctx.h, out.ctypes.data, self.ptr, self.nbytes))
        return out

    def view(self, offset_elems, shape, dtype=None):
        dtype = np.dtype(dtype or self.dtype)
        return DeviceArray(self.ctx, self.ptr + offset_elems * self.dtype.itemsize, shape, dtype, owner=False)

    def free(self):
        if self.owner and self.ptr:
            self.ctx.lib.sa3k_free(self.ctx.h, self.ptr)
        self.ptr = 0

    def __del__(self):
        try:
            if self.owner and self.ptr and self.ctx.h:
                self.ctx.lib.sa3k_free(self.ctx.h, self.ptr)
        except Exception:
            pass


class Context:
    def __init__(self, device=0, lib_path=None):
        self.lib = load_library(lib_path)
        err = C.create_string_buffer(512)
        self.h = self.lib.sa3k_create(device, err, 512)
        if not self.h:
            raise Sa3kError(-1, err.value.decode(errors="replace"))

    def check(self, rc):
        if rc != SA3K_OK:
            raise Sa3kError(rc, self.lib.sa3k_last_error(self.h).decode(errors="replace"))

    def close(self):
        if self.h:
            self.lib.sa3k_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- memory
    def empty(self, shape, dtype=np.float32):
        shape = (shape,) if np.isscalar(shape) else tuple(shape)
        nbytes = int(np.prod(shape, dtype=np.int64)) * np.dtype(dtype).itemsize
        p = C.c_void_p()
        self.check(self.lib.sa3k_malloc(self.h, nbytes, C.byref(p)))
        return DeviceArray(self, p.value, shape, dtype)

    def zeros(self, shape, dtype=np.float32):
        a = self.empty(shape, dtype)
        self.check(self.lib.sa3k_memset(self.h, a.ptr, 0, a.nbytes))
        return a

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        a = self.empty(arr.shape, arr.dtype)
        self.check(self.lib.sa3k_upload(self.h, a.ptr, arr.ctypes.data, arr.nbytes))
        return a

    def copy_into(self, dst, arr):
        arr = np.ascontiguousarray(arr, dtype=dst.dtype)
        assert arr.nbytes == dst.nbytes
        self.check(self.lib.sa3k_upload(self.h, dst.ptr, arr.ctypes.data, arr.nbytes))

    def copy_d2d(self, dst, src, nbytes):
        self.check(self.lib.sa3k_copy_d2d(self.h, dst.ptr, src.ptr, nbytes))

    def sync(self):
        self.check(self.lib.sa3k_sync(self.h))

    def set_option(self, name, value):
        self.check(self.lib.sa3k_set_option(self.h, name.encode(), int(value)))

    def get_option(self, name):
        v = C.c_int()
        self.check(self.lib.sa3k_get_option(self.h, name.encode(), C.byref(v)))
        return v.value

    def options(self):
        """{name: value} of every option of this context"""
        names = []
        while True:
            n = self.lib.sa3k_option_name(len(names))
            if not n:
                break
            names.append(n.decode())
        return {n: self.get_option(n) for n in names}

    def set_options(self, opts):
        for n, v in opts.items():
            self.set_option(n, v)

    def timer_start(self):
        self.check(self.lib.sa3k_timer_start(self.h))

    def timer_stop(self):
        ms = C.c_float()
        self.check(self.lib.sa3k_timer_stop(self.h, C.byref(ms)))
        return ms.value

    # -- per-kernel event timing
    def profile(self, on=True):
        self.check(self.lib.sa3k_profile_enable(self.h, 1 if on else 0))

    def profile_reset(self):
        self.check(self.lib.sa3k_profile_reset(self.h))

    def profile_report(self, with_work=False):
        """{scope name: (launches, total_ms)} or, with_work, (launches, total_ms, algorithmic work)"""
        buf = C.create_string_buffer(1 << 16)
        self.check(self.lib.sa3k_profile_report(self.h, buf, 1 << 16))
        out = {}
        for line in buf.value.decode().splitlines():
            name, cnt, ms, work = line.rsplit(" ", 3)
            out[name] = (int(cnt), float(ms), float(work)) if with_work else (int(cnt), float(ms))
        return out

    # -- K6
    def adamw_clip(self, p, g, m, v, hp, step, count=1, want_norm=False):
        hpv = AdamWParams(*hp) if not isinstance(hp, AdamWParams) else hp
        norm = C.c_double()
        self.check(self.lib.sa3k_adamw_clip(self.h, p.ptr, g.ptr, m.ptr, v.ptr, p.size, C.byref(hpv),
                                            int(step), int(count), C.byref(norm) if want_norm else None))
        return norm.value if want_norm else None

    def adamw_clip_scale(self):
        n, s = C.c_double(), C.c_float()
        self.check(self.lib.sa3k_adamw_clip_scale(self.h, C.byref(n), C.byref(s)))
        return n.value, s.value

    # -- Q8_0
    def q8_0_dequant(self, blocks, out, n):
        self.check(self.lib.sa3k_q8_0_dequant(self.h, blocks.ptr, out.ptr, int(n)))

    def q8_0_quantize(self, x, blocks, n):
        self.check(self.lib.sa3k_q8_0_quantize(self.h, x.ptr, blocks.ptr, int(n)))

    # -- GEMM
    def gemm_nt(self, A, B, M, N, K, prec=PREC_BF16, a_type=TYPE_F32, b_type=TYPE_F32, lda=None, ldb=None,
                B_scales=None, ldbs=0, alpha=1.0, colscale=None, bias=None, C=None, ldc=None, accumulate=False,
                noalloc=False):
        fn = self.lib.sa3k_gemm_nt_noalloc if noalloc else self.lib.sa3k_gemm_nt
        self.check(fn(
            self.h, prec, a_type, A.ptr, lda if lda is not None else K, b_type, B.ptr,
            ldb if ldb is not None else K, B_scales.ptr if B_scales is not None else None, ldbs,
            M, N, K, alpha, colscale.ptr if colscale is not None else None,
            bias.ptr if bias is not None else None, C.ptr, ldc if ldc is not None else N, int(accumulate)))

    # -- weights and adapted linears
    def weight(self, W, wtype=TYPE_F32):
        """W: numpy [out][in] f32 / f16 / bf16-as-uint16 array, or (blocks uint8, in, out) for Q8_0"""
        if wtype == TYPE_Q8_0:
            blocks, in_, out_ = W
            data = np.ascontiguousarray(blocks, np.uint8)
        else:
            data = np.ascontiguousarray(W)
            out_, in_ = data.shape
        h = C.c_void_p()
        self.check(self.lib.sa3k_weight_create(self.h, wtype, in_, out_, data.ctypes.data, 0, C.byref(h)))
        return Weight(self, h.value, in_, out_, wtype)

    def lora_chain(self, weight, adapters, max_tokens):
        """adapters: [(dora, rank, alpha, strength, A DeviceArray, B DeviceArray, magnitude DeviceArray | None)]"""
        arr = (ChainAdapter * max(1, len(adapters)))()
        for i, (dora, rank, alpha, strength, A, B, mag) in enumerate(adapters):
            arr[i] = ChainAdapter(int(dora), int(rank), float(alpha), float(strength), A.ptr, B.ptr,
                                  mag.ptr if mag is not None else None)
        h = C.c_void_p()
        self.check(self.lib.sa3k_lora_chain_create(self.h, weight.h, len(adapters), arr, max_tokens, C.byref(h)))
        return LoraChain(self, h.value, weight)

    def lin(self, weight, rank, prec, max_tokens):
        h = C.c_void_p()
        self.check(self.lib.sa3k_lin_create(self.h, weight.h, rank, prec, max_tokens, C.byref(h)))
        return Lin(self, h.value, weight, rank, prec)


class Weight:
    def __init__(self, ctx, h, in_, out_, wtype):
        self.ctx, self.h, self.in_, self.out_, self.wtype = ctx, h, in_, out_, wtype

    def row_norm_sq(self, eps=1e-12):
        y = self.ctx.empty(self.out_)
        self.ctx.check(self.ctx.lib.sa3k_weight_row_norm_sq(self.ctx.h, self.h, eps, y.ptr))
        return y

    def row_norms(self):
        y = self.ctx.empty(self.out_)
        self.ctx.check(self.ctx.lib.sa3k_weight_row_norms(self.ctx.h, self.h, y.ptr))
        return y

    def drop_working_copy(self):
        self.ctx.check(self.ctx.lib.sa3k_weight_drop_working_copy(self.ctx.h, self.h))

    def destroy(self):
        if self.h:
            self.ctx.check(self.ctx.lib.sa3k_weight_destroy(self.ctx.h, self.h))
            self.h = None


class LoraChain:
    def __init__(self, ctx, h, weight):
        self.ctx, self.h, self.weight = ctx, h, weight

    def forward(self, X, N, Y, bias=None, x_type=TYPE_F32):
        self.ctx.check(self.ctx.lib.sa3k_lora_chain_forward(self.ctx.h, self.h, x_type, X.ptr, N,
                                                            bias.ptr if bias is not None else None, Y.ptr))

    def constants(self):
        """(base_scale [out], B' [out][R]) as numpy, or (None, None) for an empty chain"""
        R = C.c_int()
        self.ctx.check(self.ctx.lib.sa3k_lora_chain_constants(self.ctx.h, self.h, None, None, C.byref(R)))
        if R.value == 0:
            return None, None
        out_ = self.weight.out_
        c0, Bp = self.ctx.empty(out_), self.ctx.empty((out_, R.value))
        self.ctx.check(self.ctx.lib.sa3k_lora_chain_constants(self.ctx.h, self.h, c0.ptr, Bp.ptr, None))
        return c0.numpy(), Bp.numpy()

    def destroy(self):
        if self.h:
            self.ctx.check(self.ctx.lib.sa3k_lora_chain_destroy(self.ctx.h, self.h))
            self.h = None


class Lin:
    def __init__(self, ctx, h, weight, rank, prec):
        self.ctx, self.h, self.weight, self.rank, self.prec = ctx, h, weight, rank, prec

    def prepare(self, A, B, scale, dora=False, mag=None, bnsq=None):
        self.ctx.check(self.ctx.lib.sa3k_lin_prepare(self.ctx.h, self.h, A.ptr if A is not None else None,
                                                     B.ptr if B is not None else None, scale, int(dora),
                                                     mag.ptr if mag is not None else None,
                                                     bnsq.ptr if bnsq is not None else None))

    def forward(self, X, N, Y, bias=None, x_type=TYPE_F32):
        self.ctx.check(self.ctx.lib.sa3k_lin_forward(self.ctx.h, self.h, x_type, X.ptr, N,
                                                     bias.ptr if bias is not None else None, Y.ptr))

    def backward(self, X, N, dY, dX, dA, dB, dm=None, dx_accumulate=False, x_type=TYPE_F32):
        self.ctx.check(self.ctx.lib.sa3k_lin_backward(self.ctx.h, self.h, x_type, X.ptr, N, dY.ptr,
                                                      dX.ptr if dX is not None else None, int(dx_accumulate),
                                                      dA.ptr, dB.ptr, dm.ptr if dm is not None else None))

    def destroy(self):
        if self.h:
            self.ctx.check(self.ctx.lib.sa3k_lin_destroy(self.ctx.h, self.h))
            self.h = None


def _ptr_array(arrs):
    return (C.c_void_p * len(arrs))(*[a.ptr if a is not None else None for a in arrs])


class Block:
    """One DiT block (sa3k_block_*). W: list of 7 host arrays as accepted by Context.weight
    (numpy [out][in], or (blocks, in, out) for Q8_0), bias: 7 host f32 arrays or None, vecs: dict
    of the 8 block vectors (ssg, pre_g, ...)."""

    def __init__(self, ctx, cfg, W, bias, vecs, rank, max_tokens, max_ctx, wtype=TYPE_F32):
        self.ctx, self.cfg = ctx, cfg
        self.keep = []
        bw = BlockWeights()
        bw.weight_type = wtype
        for t in range(7):
            data = np.ascontiguousarray(W[t][0] if wtype == TYPE_Q8_0 else W[t])
            self.keep.append(data)
            bw.W[t] = data.ctypes.data
            if bias[t] is not None:
                b = np.ascontiguousarray(bias[t], np.float32)
                self.keep.append(b)
                bw.bias[t] = b.ctypes.data
        for n in BLOCK_VECTORS:
            v = np.ascontiguousarray(vecs[n], np.float32)
            self.keep.append(v)
            setattr(bw, n, v.ctypes.data)
        h = C.c_void_p()
        ctx.check(ctx.lib.sa3k_block_create(ctx.h, C.byref(cfg), C.byref(bw), rank, max_tokens, max_ctx, C.byref(h)))
        self.h = h.value
        self.keep = []

    def base_norm_sq(self, t):
        p = C.c_void_p()
        self.ctx.check(self.ctx.lib.sa3k_block_base_norm_sq(self.ctx.h, self.h, t, C.byref(p)))
        return p.value

    def prepare(self, A, B, scale, dora=False, mag=None):
        self.ctx.check(self.ctx.lib.sa3k_block_prepare(self.ctx.h, self.h, _ptr_array(A), _ptr_array(B),
                                                       _ptr_array(mag) if dora else None, scale, int(dora)))

    def forward(self, ws, x, context, gcond, out):
        # the backward reads x and context again: the workspace keeps them alive until then
        ws.inputs = (x, context, gcond)
        self.ctx.check(self.ctx.lib.sa3k_block_forward(self.ctx.h, self.h, ws.h, x.ptr, context.ptr, gcond.ptr, out.ptr))

    def backward(self, ws, dout, dx, dcontext, dgcond, dA, dB, dm=None):
        self.ctx.check(self.ctx.lib.sa3k_block_backward(self.ctx.h, self.h, ws.h, dout.ptr, dx.ptr, dcontext.ptr,
                                                        dgcond.ptr, _ptr_array(dA), _ptr_array(dB),
                                                        _ptr_array(dm) if dm is not None else None))

    def destroy(self):
        if self.h:
            self.ctx.check(self.ctx.lib.sa3k_block_destroy(self.ctx.h, self.h))
            self.h = None


class BlockWorkspace:
    def __init__(self, ctx, cfg, B, S, Ctx):
        self.ctx = ctx
        h = C.c_void_p()
        ctx.check(ctx.lib.sa3k_block_ws_create(ctx.h, C.byref(cfg), B, S, Ctx, C.byref(h)))
        self.h = h.value
        self.inputs = None

    def destroy(self):
        if self.h:
            self.ctx.check(self.ctx.lib.sa3k_block_ws_destroy(self.ctx.h, self.h))
            self.h = None
        self.inputs = None


class Dit:
    """The DiT training step (sa3k_dit_*): named tensors, setup, adapter arena, accumulate / AdamW."""

    def __init__(self, ctx, cfg, wtype=TYPE_F16):
        self.ctx, self.cfg, self.wtype = ctx, cfg, wtype
        h = C.c_void_p()
        ctx.check(ctx.lib.sa3k_dit_create(ctx.h, C.byref(cfg), wtype, C.byref(h)))
        self.h = h.value
        self.train = None

    def tensors(self):
        """[(name, rows, cols, type)]"""
        L, out = self.ctx.lib, []
        n = C.c_int()
        self.ctx.check(L.sa3k_dit_tensor_count(self.ctx.h, self.h, C.byref(n)))
        buf = C.create_string_buffer(256)
        r, c, t = C.c_int64(), C.c_int64(), C.c_int()
        for i in range(n.value):
            self.ctx.check(L.sa3k_dit_tensor_info(self.ctx.h, self.h, i, buf, 256, C.byref(r), C.byref(c), C.byref(t)))
            out.append((buf.value.decode(), r.value, c.value, t.value))
        return out

    def set_tensor(self, name, arr):
        a = np.ascontiguousarray(arr)
        self.ctx.check(self.ctx.lib.sa3k_dit_set_tensor(self.ctx.h, self.h, name.encode(), a.ctypes.data, a.nbytes))

    def init_random(self, seed, w_sd=0.02):
        self.ctx.check(self.ctx.lib.sa3k_dit_init_random(self.ctx.h, self.h, seed, w_sd))

    def setup(self, rank, alpha, dora, scope, batch, frames, ctx_tokens, recompute=False):
        self.train = DitTrain(rank, alpha, int(dora), scope, batch, frames, ctx_tokens, int(recompute))
        self.ctx.check(self.ctx.lib.sa3k_dit_setup(self.ctx.h, self.h, C.byref(self.train)))

    def arena(self, which=0):
        """0 params, 1 grads, 2 m, 3 v: a non-owning DeviceArray view"""
        p, n = C.c_void_p(), C.c_int64()
        self.ctx.check(self.ctx.lib.sa3k_dit_arena(self.ctx.h, self.h, which, C.byref(p), C.byref(n)))
        return DeviceArray(self.ctx, p.value, (n.value,), np.float32, owner=False)

    def targets(self):
        """[(name, in, out, off_a, off_b, off_m)] in arena order"""
        L, out = self.ctx.lib, []
        n = C.c_int()
        self.ctx.check(L.sa3k_dit_target_count(self.ctx.h, self.h, C.byref(n)))
        buf = C.create_string_buffer(256)
        v = [C.c_int64() for _ in range(5)]
        for i in range(n.value):
            self.ctx.check(L.sa3k_dit_target_info(self.ctx.h, self.h, i, buf, 256, *[C.byref(x) for x in v]))
            out.append((buf.value.decode(),) + tuple(x.value for x in v))
        return out

    def adapters_init(self, seed, b_sd=0.0):
        self.ctx.check(self.ctx.lib.sa3k_dit_adapters_init(self.ctx.h, self.h, seed, b_sd))

    def adapters_changed(self):
        self.ctx.check(self.ctx.lib.sa3k_dit_adapters_changed(self.ctx.h, self.h))

    def accumulate(self, x_t, target, t, cross, glob, loss_weight=None, want_loss=True):
        B = self.train.batch
        loss = (C.c_double * B)()
        self.ctx.check(self.ctx.lib.sa3k_dit_accumulate(self.ctx.h, self.h, x_t.ptr, target.ptr, t.ptr, cross.ptr,
                                                        glob.ptr, loss_weight.ptr if loss_weight is not None else None,
                                                        loss if want_loss else None))
        return np.array(loss[:]) if want_loss else None

    def eval_loss(self, x_t, target, t, cross, glob, loss_weight=None):
        loss = (C.c_double * self.train.batch)()
        self.ctx.check(self.ctx.lib.sa3k_dit_eval_loss(self.ctx.h, self.h, x_t.ptr, target.ptr, t.ptr, cross.ptr,
                                                       glob.ptr, loss_weight.ptr if loss_weight is not None else None,
                                                       loss))
        return np.array(loss[:])

    def apply_adamw(self, hp, step, want_norm=False):
        p = AdamWParams(*hp)
        nrm = C.c_double(0.0)
        self.ctx.check(self.ctx.lib.sa3k_dit_apply_adamw(self.ctx.h, self.h, C.byref(p), step,
                                                         C.byref(nrm) if want_norm else None))
        return nrm.value if want_norm else None

    def set_graphs(self, on):
        self.ctx.check(self.ctx.lib.sa3k_dit_set_graphs(self.ctx.h, self.h, int(on)))

    def graphs(self):
        """whether the accumulate step replays captured graphs (0 once a capture has failed)"""
        on = C.c_int(0)
        self.ctx.check(self.ctx.lib.sa3k_dit_get_graphs(self.ctx.h, self.h, C.byref(on)))
        return on.value

    def set_local(self, local):
        """bind the inpaint local conditioning [B][T][local_dim] (device buffer) or None"""
        self._local = local   # keeps the buffer alive while bound
        self.ctx.check(self.ctx.lib.sa3k_dit_set_local(self.ctx.h, self.h, local.ptr if local is not None else None))

    def forward(self, x_t, t, cross, glob, velocity):
        self.ctx.check(self.ctx.lib.sa3k_dit_forward(self.ctx.h, self.h, x_t.ptr, t.ptr, cross.ptr, glob.ptr,
                                                     velocity.ptr))

    def destroy(self):
        if self.h:
            self.ctx.check(self.ctx.lib.sa3k_dit_destroy(self.ctx.h, self.h))
            self.h = None


def attn_fwd(ctx, q1, k1, q2, k2, v, B, H, Sq, Sk, window=0, scale=0.125):
    """device bf16 inputs [B*H][S][64]; returns (o, o1, o2, lse1, lse2) device arrays"""
    o = ctx.empty((B, Sq, H * 64), np.uint16)
    o1, o2 = ctx.empty((B * H, Sq, 64), np.uint16), ctx.empty((B * H, Sq, 64), np.uint16)
    l1, l2 = ctx.empty((B * H, Sq)), ctx.empty((B * H, Sq))
    ctx.check(ctx.lib.sa3k_diff_attn_fwd(ctx.h, q1.ptr, k1.ptr, q2.ptr, k2.ptr, v.ptr, B, H, Sq, Sk, 64, window,
                                         scale, o.ptr, o1.ptr, o2.ptr, l1.ptr, l2.ptr))
    return o, o1, o2, l1, l2


def attn_bwd(ctx, q1, k1, q2, k2, v, o1, o2, l1, l2, dO, B, H, Sq, Sk, window=0, scale=0.125):
    """dO f32 device [B][Sq][H*64]; returns dict of f32 device gradients"""
    BH = B * H
    dOh, dn = ctx.empty((BH, Sq, 64), np.uint16), ctx.empty((2, BH, Sq))
    g = {k: ctx.empty((BH, Sq if k in ("dq1", "dq2") else Sk, 64)) for k in ("dq1", "dk1", "dq2", "dk2", "dv")}
    ctx.check(ctx.lib.sa3k_diff_attn_bwd(ctx.h, q1.ptr, k1.ptr, q2.ptr, k2.ptr, v.ptr, o1.ptr, o2.ptr, l1.ptr, l2.ptr,
                                         dO.ptr, B, H, Sq, Sk, 64, window, scale, dOh.ptr, dn.ptr, g["dq1"].ptr,
                                         g["dk1"].ptr, g["dq2"].ptr, g["dk2"].ptr, g["dv"].ptr))
    return g
