"""ctypes binding of the oracle's whole-DiT loss (orc_dit_loss). TEST INFRASTRUCTURE ONLY, like
the rest of oracle/.

A model is a dict of float32 numpy arrays keyed by the reference's GGUF tensor names
(dit.memory_tokens, dit.pre_conv.weight, dit.<l>.self.qkv.weight, dit.<l>.ssg, ...), adapters a
dict weight name -> (A [r][in], B [out][r], magnitude [out] or None) for the selected targets.
A config with local_dim > 0 adds the inpaint local-conditioning linears dit.<l>.local.{0,2}
(weights and biases, src/dit.h:244-254); the step inputs then carry "local" [B][T][local_dim].
"""
import ctypes as C

import numpy as np

from oracle import f32, lib
from block_binding import OrcBlock, P7

BLOCK_TARGETS = ["self.qkv", "self.out", "cross.q", "cross.kv", "cross.out", "ff.proj", "ff.out"]
BLOCK_VECTORS = {"ssg": "ssg", "pre_g": "pre_norm.gamma", "cross_g": "cross_norm.gamma", "ff_g": "ff_norm.gamma",
                 "sq_g": "self.q_norm.gamma", "sk_g": "self.k_norm.gamma", "cq_g": "cross.q_norm.gamma",
                 "ck_g": "cross.k_norm.gamma"}
# head/tail linears in the oracle's order (ORC_PRE_CONV ... ORC_POST_CONV)
HEAD_TARGETS = ["pre_conv", "proj_in", "time_embed.0", "time_embed.2", "global_embed.0", "global_embed.2",
                "gce.0", "gce.2", "cond_embed.0", "cond_embed.2", "proj_out", "post_conv"]
HEAD_BIAS = {"time_embed.0", "time_embed.2", "gce.0", "gce.2"}


class OrcLin(C.Structure):
    _fields_ = [("W", C.c_void_p), ("bias", C.c_void_p), ("A", C.c_void_p), ("B", C.c_void_p),
                ("mag", C.c_void_p), ("bnsq", C.c_void_p), ("in_", C.c_int), ("out", C.c_int)]


class OrcDit(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("B", "T", "Ctx", "io", "dim", "heads", "inner", "depth", "mem", "cond_dim",
                                       "time_dim", "rope_dims", "window")] + \
               [(n, C.c_float) for n in ("rope_base", "norm_eps", "qk_eps", "time_min_freq", "time_max_freq")] + \
               [("blocks", C.c_void_p), ("head", OrcLin * 12), ("memory_tokens", C.c_void_p),
                ("rank", C.c_int), ("dora", C.c_int), ("scale", C.c_float),
                ("local_dim", C.c_int), ("local", C.c_void_p), ("local_cond", C.c_void_p)]


def tensor_shapes(cfg):
    """name -> shape of every model tensor"""
    d, io, I, cd, td = cfg["dim"], cfg["io"], cfg["inner"], cfg["cond_dim"], cfg["time_dim"]
    s = {"dit.memory_tokens": (cfg["mem"], d), "dit.pre_conv.weight": (io, io), "dit.proj_in.weight": (d, io),
         "dit.proj_out.weight": (io, d), "dit.post_conv.weight": (io, io),
         "dit.time_embed.0.weight": (d, td), "dit.time_embed.0.bias": (d,), "dit.time_embed.2.weight": (d, d),
         "dit.time_embed.2.bias": (d,), "dit.global_embed.0.weight": (d, cd), "dit.global_embed.2.weight": (d, d),
         "dit.gce.0.weight": (d, d), "dit.gce.0.bias": (d,), "dit.gce.2.weight": (6 * d, d),
         "dit.gce.2.bias": (6 * d,), "dit.cond_embed.0.weight": (d, cd), "dit.cond_embed.2.weight": (d, d)}
    outs = [5 * d, d, 2 * d, 3 * d, d, 2 * I, d]
    ins = [d, d, d, d, d, d, I]
    for l in range(cfg["depth"]):
        p = f"dit.{l}."
        for t, o, i in zip(BLOCK_TARGETS, outs, ins):
            s[p + t + ".weight"] = (o, i)
        s[p + "ff.proj.bias"] = (2 * I,)
        s[p + "ff.out.bias"] = (d,)
        s[p + "ssg"] = (6 * d,)
        for k, n in BLOCK_VECTORS.items():
            if k != "ssg":
                s[p + n] = (d,) if k in ("pre_g", "cross_g", "ff_g") else (64,)
        if cfg.get("local_dim", 0) > 0:
            s[p + "local.0.weight"] = (d, cfg["local_dim"])
            s[p + "local.0.bias"] = (d,)
            s[p + "local.2.weight"] = (d, d)
            s[p + "local.2.bias"] = (d,)
    return s


def target_names(cfg, scope="full"):
    """adapted weight names in the reference's order (sorted, src/train_lora.h:99-121)"""
    names = [f"dit.{l}.{t}.weight" for l in range(cfg["depth"]) for t in BLOCK_TARGETS]
    if scope == "full":
        names += [f"dit.{t}.weight" for t in HEAD_TARGETS]
        if cfg.get("local_dim", 0) > 0:   # "core" drops local.{0,2} (src/train_lora.h:85-89)
            names += [f"dit.{l}.local.{k}.weight" for l in range(cfg["depth"]) for k in (0, 2)]
    return sorted(names)


def random_dit(seed, cfg, scope="full", w_sd=0.05, b_sd=0.05):
    """seeded synthetic model, adapters and step inputs (Philox), float32"""
    g = np.random.Generator(np.random.Philox(seed))
    nd = lambda shape, sd: g.normal(0, sd, shape).astype(np.float32)
    tensors = {}
    for name, shape in tensor_shapes(cfg).items():
        if name.endswith(".gamma"):
            tensors[name] = 1 + nd(shape, 0.1)
        elif name.endswith(".ssg"):
            tensors[name] = nd(shape, 0.1)
        elif name.endswith(".bias"):
            tensors[name] = nd(shape, 0.02)
        elif name == "dit.memory_tokens":
            tensors[name] = nd(shape, 1.0)
        else:
            tensors[name] = nd(shape, w_sd)
    r = cfg["rank"]
    adapters = {}
    for name in target_names(cfg, scope):
        o, i = tensors[name].shape
        A = g.uniform(-1 / np.sqrt(i), 1 / np.sqrt(i), (r, i)).astype(np.float32)
        Bm = nd((o, r), b_sd)
        W = tensors[name].astype(np.float64)
        mag = (np.sqrt((W ** 2).sum(1)) * (1 + 0.05 * g.standard_normal(o))).astype(np.float32) if cfg["dora"] else None
        adapters[name] = (A, Bm, mag)
    B, T, Ctx = cfg["B"], cfg["T"], cfg["Ctx"]
    inputs = dict(x_t=nd((B, T, cfg["io"]), 1.0), target=nd((B, T, cfg["io"]), 1.0),
                  t=g.uniform(0, 1, B).astype(np.float32), cross=nd((B, Ctx, cfg["cond_dim"]), 1.0),
                  glob=nd((B, cfg["cond_dim"]), 1.0))
    if cfg.get("local_dim", 0) > 0:
        inputs["local"] = nd((B, T, cfg["local_dim"]), 1.0)
    return tensors, adapters, inputs


def expo_features(t, dim, lo, hi):
    L = lib()
    L.orc_expo_features.restype = None
    L.orc_expo_features.argtypes = [C.c_float, C.c_void_p, C.c_int, C.c_float, C.c_float]
    out = np.zeros(dim, np.float32)
    L.orc_expo_features(t, out.ctypes.data, dim, lo, hi)
    return out


def bnsq_of(W):
    W = W.astype(np.float64)
    return ((W ** 2).sum(1) + W.shape[1] * 1e-12).astype(np.float32)


def dit_loss(cfg, tensors, adapters, inputs, loss_weight=None, grad=True):
    """returns (loss [B] float64, velocity [B][T][io], grads: name -> (dA, dB, dm or None))"""
    keep = []

    def p(a):
        if a is None:
            return None
        a = f32(a)
        keep.append(a)
        return a.ctypes.data

    L = lib()
    if not getattr(L, "_dit_declared", False):
        L.orc_dit_loss.restype = None
        L.orc_dit_loss.argtypes = [C.POINTER(OrcDit)] + [C.c_void_p] * 17
        L._dit_declared = True
    dora = int(cfg["dora"])
    depth = cfg["depth"]
    blocks = (OrcBlock * max(depth, 1))()
    for l in range(depth):
        pre = f"dit.{l}."
        b = blocks[l]
        for k, n in BLOCK_VECTORS.items():
            setattr(b, k, p(tensors[pre + n]))
        Ws, bs, As, Bs, ms, ns = [], [], [], [], [], []
        for t in BLOCK_TARGETS:
            wn = pre + t + ".weight"
            Ws.append(p(tensors[wn]))
            bias = tensors.get(pre + t + ".bias")
            bs.append(p(bias))
            A, Bm, mag = adapters[wn]
            As.append(p(A))
            Bs.append(p(Bm))
            ms.append(p(mag) if dora else None)
            ns.append(p(bnsq_of(tensors[wn])) if dora else None)
        b.W, b.bias, b.A, b.Bm, b.mag, b.bnsq = P7(*Ws), P7(*bs), P7(*As), P7(*Bs), P7(*ms), P7(*ns)
    st = OrcDit()
    for k in ("B", "T", "Ctx", "io", "dim", "heads", "inner", "depth", "mem", "cond_dim", "time_dim"):
        setattr(st, k, cfg[k])
    st.rope_dims, st.window = cfg.get("rope_dims", 32), cfg.get("window", 0)
    st.rope_base, st.norm_eps, st.qk_eps = cfg.get("rope_base", 1e4), cfg.get("norm_eps", 1e-5), cfg.get("qk_eps", 1e-6)
    st.time_min_freq, st.time_max_freq = cfg.get("time_min_freq", 0.5), cfg.get("time_max_freq", 1e4)
    st.blocks = C.cast(blocks, C.c_void_p)
    st.memory_tokens = p(tensors["dit.memory_tokens"])
    st.rank, st.dora, st.scale = cfg["rank"], dora, cfg["alpha"] / cfg["rank"]
    for i, t in enumerate(HEAD_TARGETS):
        wn = f"dit.{t}.weight"
        W = tensors[wn]
        ad = adapters.get(wn)
        bias = tensors.get(f"dit.{t}.bias") if t in HEAD_BIAS else None
        st.head[i] = OrcLin(p(W), p(bias), p(ad[0]) if ad else None, p(ad[1]) if ad else None,
                            p(ad[2]) if (ad and dora) else None, p(bnsq_of(W)) if (ad and dora) else None,
                            W.shape[1], W.shape[0])
    ldim = cfg.get("local_dim", 0)
    lnames = [f"dit.{l}.local.{k}.weight" for l in range(depth) for k in (0, 2)] if ldim > 0 else []
    locs = (OrcLin * max(len(lnames), 1))()
    for i, wn in enumerate(lnames):
        W = tensors[wn]
        ad = adapters.get(wn)
        locs[i] = OrcLin(p(W), p(tensors[wn[:-len("weight")] + "bias"]), p(ad[0]) if ad else None,
                         p(ad[1]) if ad else None, p(ad[2]) if (ad and dora) else None,
                         p(bnsq_of(W)) if (ad and dora) else None, W.shape[1], W.shape[0])
    use_local = ldim > 0 and inputs.get("local") is not None
    st.local_dim = ldim if use_local else 0
    st.local = C.cast(locs, C.c_void_p) if use_local else None
    st.local_cond = p(inputs["local"]) if use_local else None
    B = cfg["B"]
    loss = np.zeros(B, np.float64)
    vel = np.zeros((B, cfg["T"], cfg["io"]), np.float32)
    grads = {n: (np.zeros_like(a[0]), np.zeros_like(a[1]), np.zeros_like(a[2]) if dora else None)
             for n, a in adapters.items()}
    arr = lambda lst: (C.c_void_p * len(lst))(*lst)
    ptr = lambda a: a.ctypes.data if a is not None else None
    if grad:
        bl = [f"dit.{l}.{t}.weight" for l in range(depth) for t in BLOCK_TARGETS]
        hd = [f"dit.{t}.weight" for t in HEAD_TARGETS]
        pick = lambda names, j: arr([ptr(grads[n][j]) if n in grads else None for n in names])
        gargs = [pick(bl, 0), pick(bl, 1), pick(bl, 2), pick(hd, 0), pick(hd, 1), pick(hd, 2)]
        gargs += [pick(lnames, 0), pick(lnames, 1), pick(lnames, 2)] if lnames else [None] * 3
    else:
        gargs = [None] * 9
    x, tg, t, cr, gl = (f32(inputs[k]) for k in ("x_t", "target", "t", "cross", "glob"))
    lw = f32(loss_weight) if loss_weight is not None else None
    L.orc_dit_loss(C.byref(st), x.ctypes.data, tg.ctypes.data, t.ctypes.data, cr.ctypes.data, gl.ctypes.data,
                   lw.ctypes.data if lw is not None else None, vel.ctypes.data, loss.ctypes.data, *gargs)
    return loss, vel, grads
