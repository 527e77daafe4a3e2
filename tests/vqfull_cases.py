"""Quantizer cases for the full multiscale VQ (src/vq.c): the reference's
config fields and a state dict under the reference's weight names, plus a
driver of the reference's own vq_load / vq_z_to_idx / vq_idx_to_zhats
(compiled into oracle/_ref/libref.so) through its C structs."""
import ctypes

import numpy as np

import ncmhip
import oracle as O


def make_case(seed, B, levels, V, D, phi=None, ratio=0.5, down=None, up=None, gaps=False, norm=(0, 0),
              refine=()):
    """phi: None (off) or the quant_resi_share_mode (0 per level, 1 shared, k
    partially shared); down/up: strides of the learned level-0 cascade (their
    product maps L to levels[0]); gaps: conv module indices skip the
    parameter-free GroupNorm modules; refine: levels with down+up refine convs."""
    rng = np.random.default_rng(seed)
    n = len(levels)
    cfg = dict(n_qlevels=n, levels=list(levels), vq_vocab=[V] * n, vq_embed_dim=D, quant_resi_ratio=0.0,
               quant_resi_enabled=0, quant_resi_share_mode=0, learned_l1_sampling=0, learned_l1_norm=norm[0],
               learned_l1_norm_final=norm[1], learned_all_sampling=0)
    w = {}

    def conv(name, k, scale=1.0):
        w[name + ".weight"] = (rng.standard_normal((D, D, k)) * scale / np.sqrt(D * k)).astype(np.float32)
        w[name + ".bias"] = (rng.standard_normal(D) * 0.02).astype(np.float32)

    for i in range(n):
        E = (rng.standard_normal((V, D)) / np.sqrt(D)).astype(np.float32)
        E[V - 1] = E[2]   # exact duplicate: ties resolve to the lower index
        w[f"embeddings.{i}.weight"] = E
    if phi is not None:
        cfg.update(quant_resi_enabled=1, quant_resi_ratio=float(ratio), quant_resi_share_mode=phi)
        nphi = n if phi == 0 else (1 if phi == 1 else phi)
        for i in range(nphi):
            conv(f"quant_resi.{i}", 3, 0.5)
    if down:
        cfg["learned_l1_sampling"] = 1
        step = 2 if gaps else 1
        for j, s in enumerate(down):
            conv(f"learned_down_l1.{j * step}", s)
        for j, s in enumerate(up):
            conv(f"learned_up_l1.{j * step}", s)
    if refine:
        cfg["learned_all_sampling"] = 1
        for i in refine:
            conv(f"learned_down_refine.{i}", 3, 0.3)
            conv(f"learned_up_refine.{i}", 3, 0.3)
    z = rng.standard_normal((B, levels[-1], D)).astype(np.float32)
    return cfg, w, z


def ncm_config(cfg):
    """The reference NCMConfig (ncm.h:75-137) with the quantizer fields set."""
    c = ncmhip.NCMConfig()
    for k, v in cfg.items():
        if k in ("levels", "vq_vocab"):
            arr = getattr(c, k)
            for i, x in enumerate(v):
                arr[i] = x
        else:
            setattr(c, k, v)
    return c


def weight_store(tensors):
    """A WeightStore over (name, TensorS) pairs; returns (store, keepalive)."""
    items = (ncmhip.NamedTensor * len(tensors))()
    for i, (name, t) in enumerate(tensors):
        items[i].name = name.encode()
        items[i].t = ctypes.pointer(t)
    return ncmhip.WeightStore(items, len(tensors)), items


def host_tensor(a):
    t = ncmhip.TensorS()
    t.data = a.ctypes.data
    for i, s in enumerate(a.shape):
        t.shape[i] = s
    t.ndim = a.ndim
    t.n = a.size
    return t


_ref_ready = False


def ref_vq(cfg, w, z, B, soft=None):
    """The reference's own vq_load + vq_z_to_idx + vq_idx_to_zhats (CPU build):
    returns (idx, zhats [n_levels][B][L][D]).  soft = (soft_levels, tau,
    seed): the codes come from its vq_z_to_idx_soft instead, and the rng
    state after is returned third."""
    global _ref_ready
    R = O.ref()
    if not _ref_ready:
        R.vq_load.restype = ctypes.c_void_p
        R.vq_load.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_char_p]
        R.vq_z_to_idx.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        R.vq_z_to_idx_soft.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                       ctypes.c_double, ctypes.c_void_p]
        R.vq_idx_to_zhats.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        R.vq_free.argtypes = [ctypes.c_void_p]
        R.arena_init.argtypes = [ctypes.c_size_t]
        R.arena_init(8 << 30)
        _ref_ready = True
    arrays = {k: np.ascontiguousarray(v, np.float32) for k, v in w.items()}
    tens = [(k, host_tensor(a)) for k, a in arrays.items()]
    ws, keep = weight_store(tens)
    c = ncm_config(cfg)
    vq = R.vq_load(ctypes.byref(c), ctypes.byref(ws), b"")
    n, L, D = cfg["n_qlevels"], cfg["levels"][cfg["n_qlevels"] - 1], cfg["vq_embed_dim"]
    z = np.ascontiguousarray(z, np.float32)
    idx = np.zeros((B, sum(cfg["levels"][:n])), np.int32)
    R.arena_reset()
    rng = ctypes.c_ulonglong(soft[2] if soft else 0)
    if soft:
        R.vq_z_to_idx_soft(vq, z.ctypes.data, B, idx.ctypes.data, soft[0], soft[1], ctypes.byref(rng))
    else:
        R.vq_z_to_idx(vq, z.ctypes.data, B, idx.ctypes.data)
    zh = np.empty((n, B, L, D), np.float32)
    ptrs = (ctypes.c_void_p * n)(*[zh[i].ctypes.data for i in range(n)])
    R.arena_reset()
    R.vq_idx_to_zhats(vq, idx.ctypes.data, B, ptrs)
    R.vq_free(vq)
    return (idx, zh, rng.value) if soft else (idx, zh)


def ref_vq_ema(cfg, w, z, codes, B, decay, eps, steps=1):
    """The reference's own vq_ema_update (vq.c:697-790), `steps` calls with the
    same z and codes, on copies of the weights: returns the codebooks after
    (its vq_load binds them in place, vq.c:90)."""
    ref_vq(cfg, w, z, B)   # argtypes and arena
    R = O.ref()
    R.vq_ema_update.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_double,
                                ctypes.c_double]
    arrays = {k: np.array(v, np.float32, copy=True) for k, v in w.items()}
    tens = [(k, host_tensor(a)) for k, a in arrays.items()]
    ws, keep = weight_store(tens)
    c = ncm_config(cfg)
    vq = R.vq_load(ctypes.byref(c), ctypes.byref(ws), b"")
    z = np.ascontiguousarray(z, np.float32)
    codes = np.ascontiguousarray(codes, np.int32)
    for _ in range(steps):
        R.arena_reset()
        R.vq_ema_update(vq, z.ctypes.data, codes.ctypes.data, B, decay, eps)
    R.vq_free(vq)
    return [arrays[f"embeddings.{i}.weight"] for i in range(cfg["n_qlevels"])]


def ref_inputs(cfg, w, idx, B):
    """The reference's own vq_idx_to_ncm_input and, level by level from a zero
    z_hat, vq_next_input over the same codes: returns (x [B][T][D],
    [(z_hat, x_next)] per level below the last)."""
    R = O.ref()
    R.vq_next_input.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                ctypes.c_int]
    R.vq_idx_to_ncm_input.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    ref_vq(cfg, w, np.zeros((B, cfg["levels"][cfg["n_qlevels"] - 1], cfg["vq_embed_dim"]), np.float32), B)
    arrays = {k: np.ascontiguousarray(v, np.float32) for k, v in w.items()}
    tens = [(k, host_tensor(a)) for k, a in arrays.items()]
    ws, keep = weight_store(tens)
    c = ncm_config(cfg)
    vq = R.vq_load(ctypes.byref(c), ctypes.byref(ws), b"")
    n, L, D = cfg["n_qlevels"], cfg["levels"][cfg["n_qlevels"] - 1], cfg["vq_embed_dim"]
    idx = np.ascontiguousarray(idx, np.int32)
    x = np.zeros((B, sum(cfg["levels"][1:n]), D), np.float32)
    R.arena_reset()
    R.vq_idx_to_ncm_input(vq, idx.ctypes.data, B, x.ctypes.data)
    steps, zh, base = [], np.zeros((B, L, D), np.float32), 0
    for lv in range(n - 1):
        tl = cfg["levels"][lv]
        codes = np.ascontiguousarray(idx[:, base:base + tl])
        xn = np.zeros((B, cfg["levels"][lv + 1], D), np.float32)
        R.arena_reset()
        R.vq_next_input(vq, codes.ctypes.data, lv, zh.ctypes.data, xn.ctypes.data, B)
        steps.append((zh.copy(), xn))
        base += tl
    R.vq_free(vq)
    return x, steps


# Cases: (name, kwargs).  L = 16 rows per sequence unless stated.
CASES = [
    ("area_linear", dict(B=6, levels=[1, 2, 4, 8, 16], V=64, D=32)),
    ("odd_levels", dict(B=5, levels=[1, 3, 5, 7, 12], V=48, D=24)),
    ("phi_per_level", dict(B=4, levels=[1, 2, 4, 8, 16], V=64, D=32, phi=0, ratio=0.5)),
    ("phi_shared", dict(B=4, levels=[2, 4, 8, 16], V=64, D=32, phi=1, ratio=0.3)),
    ("phi_partial4", dict(B=4, levels=[1, 2, 3, 4, 6, 8, 12, 16], V=40, D=32, phi=4, ratio=0.5)),
    ("l1_cascade", dict(B=4, levels=[1, 4, 8, 16], V=64, D=32, down=[4, 4], up=[4, 4])),
    ("l1_norm_gaps", dict(B=3, levels=[2, 4, 8, 16], V=64, D=32, down=[2, 4], up=[4, 2], gaps=True, norm=(1, 1))),
    ("refine", dict(B=4, levels=[1, 2, 4, 8, 16], V=64, D=32, refine=(1, 3))),
    ("everything", dict(B=3, levels=[1, 2, 4, 8, 16], V=64, D=32, phi=4, ratio=0.5, down=[4, 4], up=[4, 4],
                        norm=(1, 0), refine=(2,))),
]
