"""ctypes binding of the oracle's DiT block (orc_block_fwd / orc_block_bwd). TEST INFRASTRUCTURE
ONLY, like the rest of oracle/. Weights are passed as a dict of float32 numpy arrays:
ssg [6*dim], pre_g/cross_g/ff_g [dim], sq_g/sk_g/cq_g/ck_g [64], W[t] [out][in], bias[t] (t = 5, 6),
A[t] [r][in], B[t] [out][r], mag[t] / bnsq[t] [out] (dora), for the 7 targets
0 self.qkv, 1 self.out, 2 cross.q, 3 cross.kv, 4 cross.out, 5 ff.proj, 6 ff.out."""
import ctypes as C

import numpy as np

from oracle import f32, lib

P7 = C.c_void_p * 7


class OrcBlock(C.Structure):
    _fields_ = [("B", C.c_int), ("S", C.c_int), ("Ctx", C.c_int), ("dim", C.c_int), ("heads", C.c_int),
                ("inner", C.c_int), ("rope_dims", C.c_int), ("window", C.c_int),
                ("rope_base", C.c_float), ("norm_eps", C.c_float), ("qk_eps", C.c_float),
                ("ssg", C.c_void_p), ("pre_g", C.c_void_p), ("cross_g", C.c_void_p), ("ff_g", C.c_void_p),
                ("sq_g", C.c_void_p), ("sk_g", C.c_void_p), ("cq_g", C.c_void_p), ("ck_g", C.c_void_p),
                ("W", P7), ("bias", P7), ("A", P7), ("Bm", P7), ("mag", P7), ("bnsq", P7),
                ("rank", C.c_int), ("dora", C.c_int), ("scale", C.c_float),
                ("ladd", C.c_void_p), ("dladd", C.c_void_p)]


def _declare():
    L = lib()
    if not getattr(L, "_block_declared", False):
        L.orc_block_fwd.restype = None
        L.orc_block_fwd.argtypes = [C.POINTER(OrcBlock), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_block_bwd.restype = None
        L.orc_block_bwd.argtypes = [C.POINTER(OrcBlock), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        L._block_declared = True
    return L


def make(cfg, w):
    """cfg: dict B, S, Ctx, dim, heads, inner, window, rank, alpha, dora (+ rope_dims, base, eps)"""
    keep = []

    def p(a):
        if a is None:
            return None
        a = f32(a)
        keep.append(a)
        return a.ctypes.data

    st = OrcBlock(cfg["B"], cfg["S"], cfg["Ctx"], cfg["dim"], cfg["heads"], cfg["inner"], cfg.get("rope_dims", 32),
                  cfg.get("window", 0), cfg.get("rope_base", 1e4), cfg.get("norm_eps", 1e-5), cfg.get("qk_eps", 1e-6),
                  p(w["ssg"]), p(w["pre_g"]), p(w["cross_g"]), p(w["ff_g"]), p(w["sq_g"]), p(w["sk_g"]),
                  p(w["cq_g"]), p(w["ck_g"]),
                  P7(*[p(w["W"][t]) for t in range(7)]), P7(*[p(w["bias"][t]) for t in range(7)]),
                  P7(*[p(w["A"][t]) for t in range(7)]), P7(*[p(w["B"][t]) for t in range(7)]),
                  P7(*[p(w["mag"][t]) for t in range(7)]), P7(*[p(w["bnsq"][t]) for t in range(7)]),
                  cfg["rank"], int(cfg["dora"]), cfg["alpha"] / cfg["rank"] if cfg["rank"] else 1.0)
    return st, keep


def block_fwd(cfg, w, x, ctx, gcond):
    st, keep = make(cfg, w)
    x, ctx, gcond = f32(x), f32(ctx), f32(gcond)
    out = np.empty_like(x)
    _declare().orc_block_fwd(C.byref(st), x.ctypes.data, ctx.ctypes.data, gcond.ctypes.data, out.ctypes.data)
    return out


def block_bwd(cfg, w, x, ctx, gcond, dout):
    st, keep = make(cfg, w)
    x, ctx, gcond, dout = f32(x), f32(ctx), f32(gcond), f32(dout)
    dx, dctx, dg = np.empty_like(x), np.empty_like(ctx), np.empty_like(gcond)
    r = cfg["rank"]
    dA = [np.zeros_like(f32(w["A"][t])) for t in range(7)]
    dB = [np.zeros_like(f32(w["B"][t])) for t in range(7)]
    dm = [np.zeros(f32(w["W"][t]).shape[0], np.float32) for t in range(7)]
    arr = lambda lst: P7(*[a.ctypes.data for a in lst])
    _declare().orc_block_bwd(C.byref(st), x.ctypes.data, ctx.ctypes.data, gcond.ctypes.data, dout.ctypes.data,
                             dx.ctypes.data, dctx.ctypes.data, dg.ctypes.data, arr(dA), arr(dB), arr(dm))
    return dict(dx=dx, dctx=dctx, dgcond=dg, dA=dA, dB=dB, dm=dm)


def random_block(seed, B, S, Ctx, dim, heads, inner, rank, alpha, dora, window=0, w_sd=0.02, b_sd=0.01):
    """seeded synthetic block weights/inputs (Philox), float32"""
    g = np.random.Generator(np.random.Philox(seed))
    nd = lambda shape, sd: g.normal(0, sd, shape).astype(np.float32)
    outs = [5 * dim, dim, 2 * dim, 3 * dim, dim, 2 * inner, dim]
    ins = [dim, dim, dim, dim, dim, dim, inner]
    w = dict(ssg=nd(6 * dim, 0.1), pre_g=1 + nd(dim, 0.1), cross_g=1 + nd(dim, 0.1), ff_g=1 + nd(dim, 0.1),
             sq_g=1 + nd(64, 0.1), sk_g=1 + nd(64, 0.1), cq_g=1 + nd(64, 0.1), ck_g=1 + nd(64, 0.1))
    w["W"] = [nd((o, i), w_sd) for o, i in zip(outs, ins)]
    w["bias"] = [None, None, None, None, None, nd(outs[5], 0.02), nd(outs[6], 0.02)]
    w["A"] = [g.uniform(-1 / np.sqrt(i), 1 / np.sqrt(i), (rank, i)).astype(np.float32) for i in ins]
    w["B"] = [nd((o, rank), b_sd) for o in outs]
    if dora:
        w["mag"] = [(np.sqrt((W.astype(np.float64) ** 2).sum(1)) * (1 + 0.05 * g.standard_normal(W.shape[0]))).astype(np.float32)
                    for W in w["W"]]
        w["bnsq"] = [((W.astype(np.float64) ** 2).sum(1) + W.shape[1] * 1e-12).astype(np.float32) for W in w["W"]]
    else:
        w["mag"] = [None] * 7
        w["bnsq"] = [None] * 7
    cfg = dict(B=B, S=S, Ctx=Ctx, dim=dim, heads=heads, inner=inner, window=window, rank=rank, alpha=alpha, dora=dora)
    x = nd((B, S, dim), 1.0)
    ctx = nd((B, Ctx, dim), 1.0)
    gcond = nd((B, 6 * dim), 0.1)
    return cfg, w, x, ctx, gcond
