"""ctypes binding of the CPU oracle (liboracle.so) and of the reference's own
CPU code compiled from /root/reference (_ref/libref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the library.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libref.so")
KTEST_BIN = os.path.join(HERE, "_ref", "ktest")

vp = ctypes.c_void_p
i64 = ctypes.c_int64
ci = ctypes.c_int


def _ptr(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


_orc = None


def lib():
    global _orc
    if _orc is None:
        if not os.path.exists(ORACLE_LIB):
            raise FileNotFoundError(f"{ORACLE_LIB} not built (make -C oracle)")
        L = ctypes.CDLL(ORACLE_LIB)
        sigs = {
            "orc_linear_fwd": (None, [vp, vp, vp, vp, i64, ci, ci]),
            "orc_linear_bwd": (None, [vp, vp, vp, vp, vp, vp, i64, ci, ci]),
            "orc_l2sq": (None, [vp, vp, vp, i64, i64, ci]),
            "orc_vq_argmin": (None, [vp, vp, vp, i64, ci, ci]),
            "orc_vq_multiscale": (None, [vp, ctypes.POINTER(vp), ctypes.POINTER(ci), ci, ci, ci, ci,
                                         vp, vp, vp]),
            "orc_argmax_row": (ci, [vp, ci]),
            "orc_sample_topkp": (ci, [vp, ci, ctypes.c_float, ci, ctypes.c_float, ctypes.POINTER(ctypes.c_uint64)]),
            "orc_vq_z_to_idx": (None, [vp, vp, ci, vp, vp, vp]),
            "orc_vq_z_to_idx_soft": (None, [vp, vp, ci, vp, vp, vp, ci, ctypes.c_double, vp]),
            "orc_soft_pick": (ci, [vp, ci, ctypes.c_double, vp]),
            "orc_vq_ema_update": (None, [vp, vp, vp, vp, vp, ci, ctypes.c_double, ctypes.c_double]),
            "orc_vq_idx_to_zhats": (None, [vp, vp, ci, vp]),
            "orc_vq_next_input": (None, [vp, vp, ci, vp, vp, ci]),
            "orc_vq_idx_to_ncm_input": (None, [vp, vp, ci, vp]),
            "orc_gelu": (None, [vp, vp, i64]),
            "orc_gelu_tanh": (None, [vp, vp, i64]),
            "orc_silu": (None, [vp, vp, i64]),
            "orc_add": (None, [vp, vp, vp, i64]),
            "orc_rng_next": (ctypes.c_uint64, [ctypes.POINTER(ctypes.c_uint64)]),
            "orc_fill_ktest": (None, [ctypes.POINTER(ctypes.c_uint64), vp, i64]),
            "orc_set_threads": (None, [ci]),
            "orc_rmsnorm": (None, [vp, vp, vp, i64, ci]),
            "orc_layernorm": (None, [vp, vp, vp, vp, i64, ci]),
            "orc_layernorm_eps": (None, [vp, vp, vp, vp, i64, ci, ctypes.c_float]),
            "orc_rope": (None, [vp, vp, vp, i64, ci, ci]),
            "orc_rope_tables_qwen": (None, [ci, ci, ctypes.c_double, vp, vp]),
            "orc_sdpa_gqa": (None, [vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci]),
            "orc_embedding": (None, [vp, vp, vp, i64, ci]),
            "orc_heads_transpose": (None, [vp, vp, ci, i64, ci, ci]),
            "orc_qkv_split": (None, [vp, vp, vp, vp, ci, ci, ci, ci, ci, ci, ci]),
            "orc_head_merge": (None, [vp, vp, ci, ci, ci, ci, ci]),
            "orc_mul": (None, [vp, vp, vp, i64]),
            "orc_scale": (None, [vp, ctypes.c_float, vp, i64]),
            "orc_layernorm_bwd": (None, [vp, vp, vp, vp, vp, vp, i64, ci, ctypes.c_double]),
            "orc_rmsnorm_bwd": (None, [vp, vp, vp, vp, vp, i64, ci]),
            "orc_ce_fwd": (ctypes.c_double, [vp, vp, vp, vp, vp, i64, ci]),
            "orc_ce_bwd": (None, [vp, vp, vp, vp, i64, ci, ctypes.c_double]),
            "orc_adamw": (None, [vp, vp, vp, vp, i64] + [ctypes.c_double] * 7),
            "orc_sched_cosine_warmup": (ctypes.c_double, [ctypes.c_long, ctypes.c_double, ctypes.c_double]),
            "orc_grad_clip": (ctypes.c_double, [ctypes.POINTER(vp), ctypes.POINTER(i64), ci, ctypes.c_double]),
            "orc_sdpa_probs": (None, [vp, vp, vp, vp, ci, ci, ci, ci, ci, ci]),
            "orc_sdpa_bwd": (None, [vp, vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci]),
            "orc_act_bwd": (None, [vp, vp, vp, i64, ci]),
            "orc_mul_bwd": (None, [vp, vp, vp, vp, vp, i64]),
            "orc_rope_bwd": (None, [vp, vp, vp, vp, i64, ci, ci]),
            "orc_embedding_bwd": (None, [vp, vp, i64, ci, vp, ci]),
            "orc_qkv_split_bwd": (None, [vp, vp, vp, vp] + [ci] * 7),
            "orc_head_merge_bwd": (None, [vp, vp] + [ci] * 5),
            "orc_heads_transpose_bwd": (None, [vp, vp] + [ci] * 5),
            "orc_rope_tables_ncp": (None, [ci, ci, ci, vp, vp]),
            "orc_conv1d_btc": (None, [vp, vp, vp, vp] + [ci] * 7),
            "orc_ncp_tied_head": (None, [vp, vp, vp, ctypes.c_float, vp, ci, ci, ci]),
        }
        for n, (r, a) in sigs.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _orc = L
    return _orc


def set_threads(n):
    lib().orc_set_threads(int(n))


def linear_fwd(x, W, b=None):
    x, W = _f32(x), _f32(W)
    b = None if b is None else _f32(b)
    batch, K = x.shape
    M = W.shape[0]
    y = np.empty((batch, M), np.float32)
    lib().orc_linear_fwd(_ptr(x), _ptr(W), _ptr(b), _ptr(y), batch, M, K)
    return y


def linear_bwd(x, W, dy, dx=None, dW=None, db=None, want=("dx", "dW", "db")):
    """Returns (dx, dW, db) accumulated into the given arrays (zeros if None)."""
    x, W, dy = _f32(x), _f32(W), _f32(dy)
    batch, K = x.shape
    M = W.shape[0]
    dx = (np.zeros((batch, K), np.float32) if dx is None else _f32(dx).copy()) if "dx" in want else None
    dW = (np.zeros((M, K), np.float32) if dW is None else _f32(dW).copy()) if "dW" in want else None
    db = (np.zeros(M, np.float32) if db is None else _f32(db).copy()) if "db" in want else None
    lib().orc_linear_bwd(_ptr(x), _ptr(W), _ptr(dy), _ptr(dx), _ptr(dW), _ptr(db), batch, M, K)
    return dx, dW, db


def l2sq(a, b):
    a, b = _f32(a), _f32(b)
    d2 = np.empty((a.shape[0], b.shape[0]), np.float32)
    lib().orc_l2sq(_ptr(a), _ptr(b), _ptr(d2), a.shape[0], b.shape[0], a.shape[1])
    return d2


def vq_argmin(a, E):
    a, E = _f32(a), _f32(E)
    idx = np.empty(a.shape[0], np.int32)
    lib().orc_vq_argmin(_ptr(a), _ptr(E), _ptr(idx), a.shape[0], E.shape[0], a.shape[1])
    return idx


def vq_multiscale(z, Es, B, L):
    """z: [B*L, D]; Es: list of [V_l, D].  Returns (idx [B, n*L], z_hat, z_rest)."""
    z = _f32(z)
    Es = [_f32(e) for e in Es]
    n, D = len(Es), z.shape[1]
    idx = np.empty((B, n * L), np.int32)
    z_hat = np.empty_like(z)
    z_rest = np.empty_like(z)
    eptrs = (vp * n)(*[e.ctypes.data for e in Es])
    vocs = (ci * n)(*[e.shape[0] for e in Es])
    lib().orc_vq_multiscale(_ptr(z), eptrs, vocs, n, B, L, D, _ptr(idx), _ptr(z_hat), _ptr(z_rest))
    return idx, z_hat, z_rest


def sample_topkp(logits, temp, top_k, top_p, rng):
    """kernels.c:782-825 sample_topkp; returns (id, advanced rng state)."""
    x = _f32(logits)
    st = ctypes.c_uint64(rng)
    i = lib().orc_sample_topkp(_ptr(x), x.size, temp, top_k, top_p, ctypes.byref(st))
    return i, st.value


class OrcVq(ctypes.Structure):
    """OrcVq of ncm_oracle.h."""
    _fields_ = [("n_levels", ci), ("D", ci), ("levels", ctypes.POINTER(ci)), ("vocabs", ctypes.POINTER(ci)),
                ("E", ctypes.POINTER(vp)), ("n_phi", ci), ("resi_ratio", ctypes.c_float),
                ("phiW", ctypes.POINTER(vp)), ("phib", ctypes.POINTER(vp)), ("n_down", ci), ("n_up", ci),
                ("downW", ctypes.POINTER(vp)), ("downB", ctypes.POINTER(vp)), ("downK", ctypes.POINTER(ci)),
                ("upW", ctypes.POINTER(vp)), ("upB", ctypes.POINTER(vp)), ("upK", ctypes.POINTER(ci)),
                ("l1_norm", ci), ("l1_norm_final", ci), ("has_all", ci),
                ("drefW", ctypes.POINTER(vp)), ("drefB", ctypes.POINTER(vp)),
                ("urefW", ctypes.POINTER(vp)), ("urefB", ctypes.POINTER(vp))]


def vq_desc(cfg, weights):
    """OrcVq for a quantizer given the reference's config fields (cfg: a dict
    with n_qlevels, levels, vq_vocab, vq_embed_dim, quant_resi_ratio,
    quant_resi_enabled, quant_resi_share_mode, learned_l1_sampling,
    learned_l1_norm, learned_l1_norm_final, learned_all_sampling) and its
    weights by their state-dict names, read as vq_load does (vq.c:76-197).
    Returns (desc, keepalive)."""
    keep = []

    def arr(xs, t=vp):
        a = (t * max(1, len(xs)))(*xs)
        keep.append(a)
        return a

    def f(name):
        a = np.ascontiguousarray(weights[name], np.float32)
        keep.append(a)
        return a.ctypes.data

    n = cfg["n_qlevels"]
    d = OrcVq()
    d.n_levels, d.D = n, cfg["vq_embed_dim"]
    d.levels = arr(list(cfg["levels"][:n]), ci)
    d.vocabs = arr(list(cfg["vq_vocab"][:n]), ci)
    d.E = arr([f(f"embeddings.{i}.weight") for i in range(n)])
    if cfg.get("quant_resi_enabled") and abs(cfg.get("quant_resi_ratio", 0.0)) > 1e-6:
        sm = cfg.get("quant_resi_share_mode", 0)
        nphi = n if sm == 0 else (1 if sm == 1 else sm)
        ws, bs = [], []
        for i in range(nphi):
            w, b = f"quant_resi.{i}.weight", f"quant_resi.{i}.bias"
            if w not in weights and nphi == 1:
                w = "quant_resi.weight"
            if b not in weights and nphi == 1:
                b = "quant_resi.bias"
            ws.append(f(w))
            bs.append(f(b))
        d.n_phi, d.resi_ratio = nphi, cfg["quant_resi_ratio"]
        d.phiW, d.phib = arr(ws), arr(bs)
    if cfg.get("learned_l1_sampling"):
        dw, db, dk, uw, ub, uk = [], [], [], [], [], []
        for s_ in range(16):
            if f"learned_down_l1.{s_}.weight" in weights:
                dw.append(f(f"learned_down_l1.{s_}.weight"))
                db.append(f(f"learned_down_l1.{s_}.bias"))
                dk.append(int(weights[f"learned_down_l1.{s_}.weight"].shape[2]))
            if f"learned_up_l1.{s_}.weight" in weights:
                uw.append(f(f"learned_up_l1.{s_}.weight"))
                ub.append(f(f"learned_up_l1.{s_}.bias"))
                uk.append(int(weights[f"learned_up_l1.{s_}.weight"].shape[2]))
        d.n_down, d.n_up = len(dw), len(uw)
        d.downW, d.downB, d.downK = arr(dw), arr(db), arr(dk, ci)
        d.upW, d.upB, d.upK = arr(uw), arr(ub), arr(uk, ci)
        d.l1_norm, d.l1_norm_final = cfg.get("learned_l1_norm", 0), cfg.get("learned_l1_norm_final", 0)
    if cfg.get("learned_all_sampling"):
        d.has_all = 1
        refs = {k: [None] * n for k in ("dW", "dB", "uW", "uB")}
        for i in range(1, n - 1):
            if f"learned_down_refine.{i}.weight" in weights:
                refs["dW"][i] = f(f"learned_down_refine.{i}.weight")
                refs["dB"][i] = f(f"learned_down_refine.{i}.bias")
            if f"learned_up_refine.{i}.weight" in weights:
                refs["uW"][i] = f(f"learned_up_refine.{i}.weight")
                refs["uB"][i] = f(f"learned_up_refine.{i}.bias")
        d.drefW, d.drefB, d.urefW, d.urefB = (arr(refs[k]) for k in ("dW", "dB", "uW", "uB"))
    return d, keep


def vq_z_to_idx(cfg, weights, z, B):
    """vq_load + vq_z_to_idx (vq.c:76-197, 378-500); returns (idx, z_hat, z_rest)."""
    d, keep = vq_desc(cfg, weights)
    n, L, D = cfg["n_qlevels"], cfg["levels"][cfg["n_qlevels"] - 1], cfg["vq_embed_dim"]
    z = _f32(z)
    idx = np.zeros((B, sum(cfg["levels"][:n])), np.int32)
    zh, zr = np.empty((B, L, D), np.float32), np.empty((B, L, D), np.float32)
    lib().orc_vq_z_to_idx(ctypes.byref(d), _ptr(z), B, _ptr(idx), _ptr(zh), _ptr(zr))
    return idx, zh, zr


def vq_z_to_idx_soft(cfg, weights, z, B, soft_levels, tau, seed):
    """vq_load + vq_z_to_idx_soft (vq.c:388-500) from rng state `seed`;
    returns (idx, z_hat, z_rest, the rng state after)."""
    d, keep = vq_desc(cfg, weights)
    n, L, D = cfg["n_qlevels"], cfg["levels"][cfg["n_qlevels"] - 1], cfg["vq_embed_dim"]
    z = _f32(z)
    idx = np.zeros((B, sum(cfg["levels"][:n])), np.int32)
    zh, zr = np.empty((B, L, D), np.float32), np.empty((B, L, D), np.float32)
    rng = ctypes.c_ulonglong(seed)
    lib().orc_vq_z_to_idx_soft(ctypes.byref(d), _ptr(z), B, _ptr(idx), _ptr(zh), _ptr(zr), soft_levels, tau,
                               ctypes.byref(rng))
    return idx, zh, zr, rng.value


def vq_ema_update(cfg, weights, z, codes, B, decay, eps, steps=1):
    """vq_ema_init + `steps` calls of vq_ema_update (vq.c:677-790) with the
    same z and codes; returns (codebooks after, [n_levels] arrays), the EMA
    counts and sums after."""
    n = cfg["n_qlevels"]
    w2 = {k: np.array(v, np.float32, copy=True) for k, v in weights.items()}
    d, keep = vq_desc(cfg, w2)
    cs = [np.ones(cfg["vq_vocab"][i], np.float32) for i in range(n)]
    ws = [np.array(w2[f"embeddings.{i}.weight"], np.float32, copy=True) for i in range(n)]
    csp = (vp * n)(*[a.ctypes.data for a in cs])
    wsp = (vp * n)(*[a.ctypes.data for a in ws])
    z = _f32(z)
    codes = np.ascontiguousarray(codes, np.int32)
    for _ in range(steps):
        lib().orc_vq_ema_update(ctypes.byref(d), csp, wsp, _ptr(z), _ptr(codes), B, decay, eps)
    return [w2[f"embeddings.{i}.weight"] for i in range(n)], cs, ws


def soft_pick(d, tau, seed):
    """One row's soft draw (vq.c:402-431): (index or -1, rng state after)."""
    d = _f32(d)
    rng = ctypes.c_ulonglong(seed)
    j = lib().orc_soft_pick(_ptr(d), d.size, tau, ctypes.byref(rng))
    return j, rng.value


def vq_idx_to_zhats(cfg, weights, idx, B):
    """vq_idx_to_zhats (vq.c:502-552): z_hat after every level, [n_levels][B][L][D]."""
    d, keep = vq_desc(cfg, weights)
    n, L, D = cfg["n_qlevels"], cfg["levels"][cfg["n_qlevels"] - 1], cfg["vq_embed_dim"]
    idx = np.ascontiguousarray(idx, np.int32)
    out = np.empty((n, B, L, D), np.float32)
    lib().orc_vq_idx_to_zhats(ctypes.byref(d), _ptr(idx), B, _ptr(out))
    return out


def vq_next_input(cfg, weights, codes, level, z_hat, B):
    """vq_next_input (vq.c:554-597): returns (z_hat + the level's contribution,
    area(that -> levels[level + 1]))."""
    d, keep = vq_desc(cfg, weights)
    codes = np.ascontiguousarray(codes, np.int32)
    zh = np.array(z_hat, np.float32, copy=True, order="C")
    x = np.empty((B, cfg["levels"][level + 1], cfg["vq_embed_dim"]), np.float32)
    lib().orc_vq_next_input(ctypes.byref(d), _ptr(codes), level, _ptr(zh), _ptr(x), B)
    return zh, x


def vq_idx_to_ncm_input(cfg, weights, idx, B):
    """vq_idx_to_ncm_input (vq.c:601-670): [B][total - levels[0]][D]."""
    d, keep = vq_desc(cfg, weights)
    n = cfg["n_qlevels"]
    idx = np.ascontiguousarray(idx, np.int32)
    x = np.empty((B, sum(cfg["levels"][1:n]), cfg["vq_embed_dim"]), np.float32)
    lib().orc_vq_idx_to_ncm_input(ctypes.byref(d), _ptr(idx), B, _ptr(x))
    return x


def ref_sample_topkp(logits, temp, top_k, top_p, rng):
    """The reference's own sample_topkp (kernels.c, compiled into _ref/libref.so)."""
    x = _f32(logits)
    st = ctypes.c_uint64(rng)
    i = ref().sample_topkp(_ptr(x), x.size, temp, top_k, top_p, ctypes.byref(st))
    return i, st.value


def argmax_row(x):
    x = _f32(x)
    return lib().orc_argmax_row(_ptr(x), x.size)


def act(name, x):
    x = _f32(x)
    y = np.empty_like(x)
    getattr(lib(), "orc_" + name)(_ptr(x), _ptr(y), x.size)
    return y


def rmsnorm(x, w):
    x = _f32(x)
    w = None if w is None else _f32(w)
    y = np.empty_like(x)
    lib().orc_rmsnorm(_ptr(x), _ptr(w), _ptr(y), x.shape[0], x.shape[1])
    return y


def layernorm(x, w, b, eps=None):
    """eps None: layernorm_fwd (1e-6 double); else layernorm_eps_fwd(eps)."""
    x = _f32(x)
    w = None if w is None else _f32(w)
    b = None if b is None else _f32(b)
    y = np.empty_like(x)
    if eps is None:
        lib().orc_layernorm(_ptr(x), _ptr(w), _ptr(b), _ptr(y), x.shape[0], x.shape[1])
    else:
        lib().orc_layernorm_eps(_ptr(x), _ptr(w), _ptr(b), _ptr(y), x.shape[0], x.shape[1], eps)
    return y


def rope(x, cos_t, sin_t, T):
    """x: [rows, hd] with row position = row % T; returns a rotated copy."""
    x = _f32(x).copy()
    lib().orc_rope(_ptr(x), _ptr(_f32(cos_t)), _ptr(_f32(sin_t)), x.shape[0], T, x.shape[1])
    return x


def rope_tables_qwen(T, hd, theta):
    c = np.empty((T, hd), np.float32)
    s_ = np.empty((T, hd), np.float32)
    lib().orc_rope_tables_qwen(T, hd, theta, _ptr(c), _ptr(s_))
    return c, s_


def sdpa_gqa(q, k, v, mask=None):
    """q [B,Hq,Tq,hd], k/v [B,Hkv,Tkv,hd], mask [Tq,Tkv] or None."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, Hq, Tq, hd = q.shape
    Hkv, Tkv = k.shape[1], k.shape[2]
    m = None if mask is None else _f32(mask)
    out = np.empty_like(q)
    lib().orc_sdpa_gqa(_ptr(q), _ptr(k), _ptr(v), _ptr(m), _ptr(out), B, Hq, Hkv, Tq, Tkv, hd)
    return out


def embedding(W, idx):
    W = _f32(W)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    y = np.empty((idx.size, W.shape[1]), np.float32)
    lib().orc_embedding(_ptr(W), _ptr(idx), _ptr(y), idx.size, W.shape[1])
    return y


def heads_transpose(x, B, T, H, hd):
    x = _f32(x)
    y = np.empty((B, H, T, hd), np.float32)
    lib().orc_heads_transpose(_ptr(x), _ptr(y), B, T, H, hd)
    return y


def qkv_split(x, B, T, C, H, hd, K, rep):
    x = _f32(x)
    outs = [np.empty((B, H, T, hd), np.float32) for _ in range(3)]
    lib().orc_qkv_split(_ptr(x), *[_ptr(o) for o in outs], B, T, C, H, hd, K, rep)
    return tuple(outs)


def head_merge(ctx, B, T, C, H, hd):
    ctx = _f32(ctx)
    y = np.empty((B, T, C), np.float32)
    lib().orc_head_merge(_ptr(ctx), _ptr(y), B, T, C, H, hd)
    return y


def mul(a, b):
    a, b = _f32(a), _f32(b)
    y = np.empty_like(a)
    lib().orc_mul(_ptr(a), _ptr(b), _ptr(y), a.size)
    return y


def scale(x, s_):
    x = _f32(x)
    y = np.empty_like(x)
    lib().orc_scale(_ptr(x), s_, _ptr(y), x.size)
    return y


def _grad(g0, shape):
    return np.zeros(shape, np.float32) if g0 is None else _f32(g0).copy()


def layernorm_bwd(x, w, dy, dx0=None, dw0=None, db0=None, eps=1e-6, want=("dx", "dw", "db")):
    """train_tape.c:569-634; returns (dx, dw, db) accumulated onto the given
    starting gradients (zeros by default); grads not in `want` are None."""
    x, dy = _f32(x), _f32(dy)
    w = None if w is None else _f32(w)
    rows, C = x.shape
    dx = _grad(dx0, (rows, C)) if "dx" in want else None
    dw = _grad(dw0, C) if "dw" in want else None
    db = _grad(db0, C) if "db" in want else None
    lib().orc_layernorm_bwd(_ptr(x), _ptr(w), _ptr(dy), _ptr(dx), _ptr(dw), _ptr(db), rows, C, eps)
    return dx, dw, db


def rmsnorm_bwd(x, w, dy, dx0=None, dw0=None, want=("dx", "dw")):
    x, dy = _f32(x), _f32(dy)
    w = None if w is None else _f32(w)
    rows, C = x.shape
    dx = _grad(dx0, (rows, C)) if "dx" in want else None
    dw = _grad(dw0, C) if "dw" in want else None
    lib().orc_rmsnorm_bwd(_ptr(x), _ptr(w), _ptr(dy), _ptr(dx), _ptr(dw), rows, C)
    return dx, dw


def ce_fwd(logits, tgt, wm=None):
    """t_ce: returns (loss, probs, cnt)."""
    logits = _f32(logits)
    tgt = np.ascontiguousarray(tgt, np.int32)
    wm = None if wm is None else _f32(wm)
    rows, V = logits.shape
    probs = np.empty_like(logits)
    loss = np.zeros(1, np.float32)
    cnt = lib().orc_ce_fwd(_ptr(logits), _ptr(tgt), _ptr(wm), _ptr(loss), _ptr(probs), rows, V)
    return float(loss[0]), probs, cnt


def ce_bwd(probs, tgt, wm, inv, dl0=None):
    probs = _f32(probs)
    tgt = np.ascontiguousarray(tgt, np.int32)
    wm = None if wm is None else _f32(wm)
    dl = _grad(dl0, probs.shape)
    lib().orc_ce_bwd(_ptr(probs), _ptr(tgt), _ptr(wm), _ptr(dl), probs.shape[0], probs.shape[1], inv)
    return dl


def adamw(p, g, m, v, lr, b1, b2, b1t, b2t, eps, wd):
    """Returns updated copies (p, m, v)."""
    p, m, v = _f32(p).copy(), _f32(m).copy(), _f32(v).copy()
    g = _f32(g)
    lib().orc_adamw(_ptr(p), _ptr(g), _ptr(m), _ptr(v), p.size, lr, b1, b2, b1t, b2t, eps, wd)
    return p, m, v


def sched_cosine_warmup(step, warmup, total):
    return lib().orc_sched_cosine_warmup(step, warmup, total)


def grad_clip(grads, max_norm=1.0):
    """Returns (gnorm, clipped copies)."""
    gs = [_f32(g).copy() for g in grads]
    ptrs = (vp * len(gs))(*[g.ctypes.data for g in gs])
    ns = (i64 * len(gs))(*[g.size for g in gs])
    gn = lib().orc_grad_clip(ptrs, ns, len(gs), max_norm)
    return gn, gs


def sdpa_probs(q, k, mask=None):
    q, k = _f32(q), _f32(k)
    B, H, Tq, hd = q.shape
    Hkv, Tkv = k.shape[1], k.shape[2]
    m = None if mask is None else _f32(mask)
    P = np.empty((B, H, Tq, Tkv), np.float32)
    lib().orc_sdpa_probs(_ptr(q), _ptr(k), _ptr(m), _ptr(P), B, H, Hkv, Tq, Tkv, hd)
    return P


def sdpa_bwd(q, k, v, P, dy, dq0=None, dk0=None, dv0=None):
    q, k, v, P, dy = _f32(q), _f32(k), _f32(v), _f32(P), _f32(dy)
    B, H, Tq, hd = q.shape
    Hkv, Tkv = k.shape[1], k.shape[2]
    dq, dk, dv = _grad(dq0, q.shape), _grad(dk0, k.shape), _grad(dv0, v.shape)
    lib().orc_sdpa_bwd(_ptr(q), _ptr(k), _ptr(v), _ptr(P), _ptr(dy), _ptr(dq), _ptr(dk), _ptr(dv),
                       B, H, Hkv, Tq, Tkv, hd)
    return dq, dk, dv


ACT_BWD = {"gelu": 0, "silu": 1, "gelu_tanh": 2}


def act_bwd(name, x, dy, dx0=None):
    x, dy = _f32(x), _f32(dy)
    dx = _grad(dx0, x.shape)
    lib().orc_act_bwd(_ptr(x), _ptr(dy), _ptr(dx), x.size, ACT_BWD[name])
    return dx


def mul_bwd(a, b, dy, da0=None, db0=None):
    a, b, dy = _f32(a), _f32(b), _f32(dy)
    da, db = _grad(da0, a.shape), _grad(db0, b.shape)
    lib().orc_mul_bwd(_ptr(a), _ptr(b), _ptr(dy), _ptr(da), _ptr(db), a.size)
    return da, db


def rope_bwd(g, cos_t, sin_t, T, dx0=None):
    """g: [rows, hd] gradient of the rotated rows (position row % T)."""
    g = _f32(g)
    dx = _grad(dx0, g.shape)
    lib().orc_rope_bwd(_ptr(g), _ptr(_f32(cos_t)), _ptr(_f32(sin_t)), _ptr(dx), g.shape[0], T, g.shape[1])
    return dx


def embedding_bwd(dy, idx, V, dW0=None):
    dy = _f32(dy)
    idx = np.ascontiguousarray(idx, np.int32)
    D = dy.shape[1]
    dW = _grad(dW0, (V, D))
    lib().orc_embedding_bwd(_ptr(dy), _ptr(idx), idx.size, D, _ptr(dW), V)
    return dW


def qkv_split_bwd(gq, gk, gv, B, T, C, H, hd, K, rep, dx0=None):
    gq, gk, gv = [None if g is None else _f32(g) for g in (gq, gk, gv)]
    dx = _grad(dx0, (B, T, C + 2 * K * hd))
    lib().orc_qkv_split_bwd(_ptr(gq), _ptr(gk), _ptr(gv), _ptr(dx), B, T, C, H, hd, K, rep)
    return dx


def head_merge_bwd(dy, B, T, C, H, hd, dx0=None):
    dy = _f32(dy)
    dx = _grad(dx0, (B, H, T, hd))
    lib().orc_head_merge_bwd(_ptr(dy), _ptr(dx), B, T, C, H, hd)
    return dx


def heads_transpose_bwd(dy, B, T, C, H, hd, dx0=None):
    dy = _f32(dy)
    dx = _grad(dx0, (B, T, C))
    lib().orc_heads_transpose_bwd(_ptr(dy), _ptr(dx), B, T, C, H, hd)
    return dx


def ktest_fill(state, n):
    """tests/ktest_kernels.c:8-12 generator; returns (values, new_state)."""
    st = ctypes.c_uint64(state)
    out = np.empty(n, np.float32)
    lib().orc_fill_ktest(ctypes.byref(st), _ptr(out), n)
    return out, st.value


# ---- the reference itself (only where /root/reference was compiled) ----
_ref = None


def ref_available():
    return os.path.exists(REF_LIB)


def ref():
    global _ref
    if _ref is None:
        L = ctypes.CDLL(REF_LIB, mode=os.RTLD_LAZY)
        sigs = {
            "linear_fwd": (None, [vp, vp, vp, vp, i64, ci, ci]),
            "rowwise_l2sq": (None, [vp, vp, vp, i64, i64, ci]),
            "argmax_row": (ci, [vp, ci]),
            "sample_topkp": (ci, [vp, ci, ctypes.c_float, ci, ctypes.c_float, ctypes.POINTER(ctypes.c_uint64)]),
            "gelu_fwd": (None, [vp, vp, i64]),
            "gelu_tanh_fwd": (None, [vp, vp, i64]),
            "silu_fwd": (None, [vp, vp, i64]),
            "refg_linear_bwd": (None, [vp, vp, vp, vp, vp, vp, vp, ctypes.c_longlong, ci, ci]),
            "refg_vq_multiscale": (ci, [vp, vp, vp, ci, ci, ci, ci, vp, vp, vp]),
            "rmsnorm_fwd": (None, [vp, vp, vp, i64, ci]),
            "layernorm_fwd": (None, [vp, vp, vp, vp, i64, ci]),
            "layernorm_eps_fwd": (None, [vp, vp, vp, vp, i64, ci, ctypes.c_float]),
            "rope_apply_gqa": (None, [vp, vp, vp, vp, ci, ci, ci, ci, ci]),
            "sdpa_fwd_gqa": (None, [vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ci]),
            "sdpa_fwd": (None, [vp, vp, vp, vp, vp, ci, ci, ci, ci, ci]),
            "embedding_fwd": (None, [vp, vp, vp, i64, ci]),
            "heads_transpose_fwd_b": (None, [vp, vp, ci, i64, ci, ci]),
            "qkv_split_fwd": (None, [vp, vp, vp, vp, ci, ci, ci, ci, ci, ci, ci]),
            "head_merge_fwd": (None, [vp, vp, ci, ci, ci, ci, ci]),
            "mul_fwd": (None, [vp, vp, vp, i64]),
            "scale_fwd": (None, [vp, ctypes.c_float, vp, i64]),
            "add_fwd": (None, [vp, vp, vp, i64]),
            "refg_ln_bwd": (None, [vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_longlong, ci, ctypes.c_double]),
            "refg_rmsn_bwd": (None, [vp, vp, vp, vp, vp, vp, ctypes.c_longlong, ci]),
            "refg_ce": (None, [vp, vp, vp, vp, vp, vp, ctypes.c_longlong, ci, ctypes.c_double]),
            "refg_sdpa_bwd": (None, [vp] * 10 + [ci] * 6),
            "refg_act_bwd": (None, [ci, vp, vp, vp, vp, ctypes.c_longlong]),
            "refg_mul_bwd": (None, [vp] * 6 + [ctypes.c_longlong]),
            "refg_rope_bwd": (None, [vp] * 10 + [ci] * 5),
            "refg_embed_bwd": (None, [vp, vp, ci, vp, vp, vp, ctypes.c_longlong, ci]),
            "refg_split_bwd": (None, [vp] * 8 + [ci] * 7),
            "refg_merge_bwd": (None, [ci, vp, vp, vp, vp] + [ci] * 5),
            "refg_qwen_open": (vp, [ctypes.c_char_p, ci, ci, ci, ci, ci, ctypes.c_double]),
            "refg_qwen_forward": (ci, [vp, vp, ci, ci, vp]),
            "refg_qwen_generate": (ci, [vp, vp, ci, ci, vp]),
            "refg_qwen_close": (None, [vp]),
            "refg_ncp_forward": (ci, [vp, ci, vp, vp, ci, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(vp),
                                      vp, vp, ci, vp, vp, ci, vp]),
        }
        for n, (r, a) in sigs.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _ref = L
    return _ref


def ref_linear_fwd(x, W, b=None):
    x, W = _f32(x), _f32(W)
    b = None if b is None else _f32(b)
    y = np.empty((x.shape[0], W.shape[0]), np.float32)
    ref().linear_fwd(_ptr(x), _ptr(W), _ptr(b), _ptr(y), x.shape[0], W.shape[0], x.shape[1])
    return y


def ref_linear_bwd(x, W, b, dy, dx0=None, dW0=None, db0=None):
    x, W, dy = _f32(x), _f32(W), _f32(dy)
    b = None if b is None else _f32(b)
    batch, K = x.shape
    M = W.shape[0]
    dx = np.zeros((batch, K), np.float32) if dx0 is None else _f32(dx0).copy()
    dW = np.zeros((M, K), np.float32) if dW0 is None else _f32(dW0).copy()
    db = np.zeros(M, np.float32) if db0 is None else _f32(db0).copy()
    ref().refg_linear_bwd(_ptr(x), _ptr(W), _ptr(b), _ptr(dy), _ptr(dx), _ptr(dW),
                          _ptr(db) if b is not None else None, batch, M, K)
    return dx, dW, (db if b is not None else None)


def ref_l2sq(a, b):
    a, b = _f32(a), _f32(b)
    d2 = np.empty((a.shape[0], b.shape[0]), np.float32)
    ref().rowwise_l2sq(_ptr(a), _ptr(b), _ptr(d2), a.shape[0], b.shape[0], a.shape[1])
    return d2


def ref_call(name, *arrays_and_ints):
    """Calls a reference kernels.c function; numpy arrays are passed by pointer."""
    args = [a.ctypes.data if isinstance(a, np.ndarray) else a for a in arrays_and_ints]
    return getattr(ref(), name)(*args)


def ref_vq_multiscale(z, Es, B, L):
    z = _f32(z)
    Es = [_f32(e) for e in Es]
    n, D = len(Es), z.shape[1]
    flat = np.ascontiguousarray(np.concatenate([e.reshape(-1) for e in Es]))
    vocs = np.array([e.shape[0] for e in Es], np.int32)
    idx = np.empty((B, n * L), np.int32)
    z_hat = np.empty_like(z)
    z_rest = np.empty_like(z)
    rc = ref().refg_vq_multiscale(_ptr(z), _ptr(flat), _ptr(vocs), n, B, L, D, _ptr(idx),
                                  _ptr(z_hat), _ptr(z_rest))
    assert rc == 0
    return idx, z_hat, z_rest


def ref_ln_bwd(x, w, b, dy, dx0=None, dw0=None, db0=None, eps=None):
    """Reference tape, one TOP_LN (eps None) or TOP_LNE record."""
    x, dy = _f32(x), _f32(dy)
    w = None if w is None else _f32(w)
    b = None if b is None else _f32(b)
    rows, C = x.shape
    y = np.empty_like(x)
    dx = _grad(dx0, (rows, C))
    dw = _grad(dw0, C) if w is not None else None
    db = _grad(db0, C) if b is not None else None
    ref().refg_ln_bwd(_ptr(x), _ptr(w), _ptr(b), _ptr(dy), _ptr(y), _ptr(dx), _ptr(dw), _ptr(db), rows, C,
                      -1.0 if eps is None else eps)
    return dx, dw, db


def ref_rmsn_bwd(x, w, dy, dx0=None, dw0=None):
    x, dy = _f32(x), _f32(dy)
    w = None if w is None else _f32(w)
    rows, C = x.shape
    y = np.empty_like(x)
    dx = _grad(dx0, (rows, C))
    dw = _grad(dw0, C) if w is not None else None
    ref().refg_rmsn_bwd(_ptr(x), _ptr(w), _ptr(dy), _ptr(y), _ptr(dx), _ptr(dw), rows, C)
    return dx, dw


def ref_ce(logits, tgt, wm=None, weight=1.0, dl0=None):
    """Reference t_ce + backward: (loss, probs, dlogits)."""
    logits = _f32(logits)
    tgt = np.ascontiguousarray(tgt, np.int32)
    wm = None if wm is None else _f32(wm)
    rows, V = logits.shape
    loss = np.zeros(1, np.float32)
    probs = np.empty_like(logits)
    dl = _grad(dl0, logits.shape)
    ref().refg_ce(_ptr(logits), _ptr(tgt), _ptr(wm), _ptr(loss), _ptr(probs), _ptr(dl), rows, V, weight)
    return float(loss[0]), probs, dl


def ref_sdpa_bwd(q, k, v, mask, dy):
    """Reference t_sdpa + TOP_SDPA backward: (o, P, dq, dk, dv)."""
    q, k, v, dy = _f32(q), _f32(k), _f32(v), _f32(dy)
    m = None if mask is None else _f32(mask)
    B, H, Tq, hd = q.shape
    Hkv, Tkv = k.shape[1], k.shape[2]
    o = np.empty_like(q)
    P = np.empty((B, H, Tq, Tkv), np.float32)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    ref().refg_sdpa_bwd(_ptr(q), _ptr(k), _ptr(v), _ptr(m), _ptr(dy), _ptr(o), _ptr(dq), _ptr(dk), _ptr(dv),
                        _ptr(P), B, H, Hkv, Tq, Tkv, hd)
    return o, P, dq, dk, dv


def ref_act_bwd(name, x, dy, dx0=None):
    x, dy = _f32(x), _f32(dy)
    y = np.empty_like(x)
    dx = _grad(dx0, x.shape)
    ref().refg_act_bwd(ACT_BWD[name], _ptr(x), _ptr(dy), _ptr(y), _ptr(dx), x.size)
    return dx


def ref_mul_bwd(a, b, dy, da0=None, db0=None):
    a, b, dy = _f32(a), _f32(b), _f32(dy)
    y = np.empty_like(a)
    da, db = _grad(da0, a.shape), _grad(db0, b.shape)
    ref().refg_mul_bwd(_ptr(a), _ptr(b), _ptr(dy), _ptr(y), _ptr(da), _ptr(db), a.size)
    return da, db


def ref_rope_bwd(xq, xk, cos_t, sin_t, gq, gk):
    xq, xk, gq, gk = _f32(xq), _f32(xk), _f32(gq), _f32(gk)
    B, H, T, hd = xq.shape
    Hkv = xk.shape[1]
    yq, yk = np.empty_like(xq), np.empty_like(xk)
    dxq, dxk = np.zeros_like(xq), np.zeros_like(xk)
    ref().refg_rope_bwd(_ptr(xq), _ptr(xk), _ptr(_f32(cos_t)), _ptr(_f32(sin_t)), _ptr(gq), _ptr(gk), _ptr(yq),
                        _ptr(yk), _ptr(dxq), _ptr(dxk), B, H, Hkv, T, hd)
    return dxq, dxk


def ref_embed_bwd(W, idx, dy, dW0=None):
    W, dy = _f32(W), _f32(dy)
    idx = np.ascontiguousarray(idx, np.int32)
    V, D = W.shape
    y = np.empty((idx.size, D), np.float32)
    dW = _grad(dW0, W.shape)
    ref().refg_embed_bwd(_ptr(W), _ptr(idx), V, _ptr(dy), _ptr(y), _ptr(dW), idx.size, D)
    return dW


def ref_split_bwd(x, gq, gk, gv, B, T, C, H, hd, K, rep):
    x = _f32(x)
    gq, gk, gv = [None if g is None else _f32(g) for g in (gq, gk, gv)]
    qq, kk, vv = [np.empty((B, H, T, hd), np.float32) for _ in range(3)]
    dx = np.zeros_like(x)
    ref().refg_split_bwd(_ptr(x), _ptr(gq), _ptr(gk), _ptr(gv), _ptr(qq), _ptr(kk), _ptr(vv), _ptr(dx),
                         B, T, C, H, hd, K, rep)
    return dx


def ref_merge_bwd(kind, x, dy, B, T, C, H, hd):
    """kind 0: head_merge (x [B,H,T,hd]); kind 1: head split (x [B,T,C])."""
    x, dy = _f32(x), _f32(dy)
    y = np.empty_like(dy)
    dx = np.zeros_like(x)
    ref().refg_merge_bwd(kind, _ptr(x), _ptr(dy), _ptr(y), _ptr(dx), B, T, C, H, hd)
    return dx


# ---- config 5: the taped GPT-2 step (train_gpt2.c:42-180) restated ----
GPT2_BLOCK = ("ln_1.weight", "ln_1.bias", "attn.c_attn.weight", "attn.c_attn.bias", "attn.c_proj.weight",
              "attn.c_proj.bias", "ln_2.weight", "ln_2.bias", "mlp.c_fc.weight", "mlp.c_fc.bias",
              "mlp.c_proj.weight", "mlp.c_proj.bias")


def gpt2_shapes(n_layer, C, V, npos):
    shapes = [(V, C), (npos, C)]
    per = [(C,), (C,), (3 * C, C), (3 * C,), (C, C), (C,), (C,), (C,), (4 * C, C), (4 * C,), (C, 4 * C), (C,)]
    for _ in range(n_layer):
        shapes += per
    return shapes + [(C,), (C,)]


def gpt2_grads(params, n_layer, C, H, V, npos, ids, tgt):
    """Forward of train_gpt2_forward, mean CE on tgt, and the host tape
    backward (train_tape.c:636-1051) over the same records in reverse, every
    op the pinned oracle function of the tape case it follows.  Returns
    (loss, grads in parameter order)."""
    ids = np.ascontiguousarray(ids, np.int32)
    B, T = ids.shape
    R, hd = B * T, C // H
    P = [_f32(p) for p in params]
    tape = []

    def rec(op, out, *ins, **kw):
        tape.append((op, out, ins, kw))
        return out

    pos = np.tile(np.arange(T, dtype=np.int32), B)
    xe = rec("embed", embedding(P[0], ids.reshape(-1)), 0, ids.reshape(-1), V)
    pe = rec("embed", embedding(P[1], pos), 1, pos, npos)
    h = rec("add", xe + pe, xe, pe)
    mask = np.where(np.arange(T)[None, :] <= np.arange(T)[:, None], 0.0, -1e9).astype(np.float32)
    for li in range(n_layer):
        w = list(range(2 + 12 * li, 14 + 12 * li))
        x = h
        ln = rec("ln", layernorm(x, P[w[0]], P[w[1]], eps=np.float32(1e-5)), x, w[0], w[1])
        qkv = rec("linear", linear_fwd(ln, P[w[2]], P[w[3]]), ln, w[2], w[3])
        q, k, v = qkv_split(qkv.reshape(B, T, 3 * C), B, T, C, H, hd, H, 1)
        tape.append(("split", (q, k, v), (qkv,), {}))
        Pm = sdpa_probs(q, k, mask)
        ctx = rec("sdpa", sdpa_gqa(q, k, v, mask), q, k, v, P=Pm)
        mo = rec("merge", head_merge(ctx, B, T, C, H, hd).reshape(R, C), ctx)
        ao = rec("linear", linear_fwd(mo, P[w[4]], P[w[5]]), mo, w[4], w[5])
        x1 = rec("add", x + ao, x, ao)
        mn = rec("ln", layernorm(x1, P[w[6]], P[w[7]], eps=np.float32(1e-5)), x1, w[6], w[7])
        mm = rec("linear", linear_fwd(mn, P[w[8]], P[w[9]]), mn, w[8], w[9])
        m2 = rec("gelu_tanh", act("gelu_tanh", mm), mm)
        mlpo = rec("linear", linear_fwd(m2, P[w[10]], P[w[11]]), m2, w[10], w[11])
        h = rec("add", x1 + mlpo, x1, mlpo)
    n = len(P)
    lnf = rec("ln", layernorm(h, P[n - 2], P[n - 1], eps=np.float32(1e-5)), h, n - 2, n - 1)
    logits = rec("linear", linear_fwd(lnf, P[0], None), lnf, 0, None)
    loss, probs, cnt = ce_fwd(logits, tgt.reshape(-1))
    grads = [np.zeros_like(p) for p in P]
    g = {id(logits): ce_bwd(probs, tgt.reshape(-1), None, 1.0 / cnt)}

    def gget(a):
        if isinstance(a, int):
            return grads[a]
        if id(a) not in g:
            g[id(a)] = np.zeros_like(a)
        return g[id(a)]

    def gset(a, val):
        if isinstance(a, int):
            grads[a][...] = val
        else:
            g[id(a)] = val

    for op, out, ins, kw in reversed(tape):
        if op == "split":
            gq, gk, gv = (g.get(id(o)) for o in out)
            if gq is None and gk is None and gv is None:
                continue
            (a,) = ins
            gset(a, qkv_split_bwd(gq, gk, gv, B, T, C, H, hd, H, 1, gget(a).reshape(B, T, -1)).reshape(a.shape))
            continue
        dy = g.get(id(out))
        if dy is None:
            continue
        if op == "embed":
            wi, idx, VV = ins
            gset(wi, embedding_bwd(dy, idx, VV, gget(wi)))
        elif op == "add":
            a, b = ins
            gset(a, gget(a) + dy)
            gset(b, gget(b) + dy)
        elif op == "ln":
            x, wi, bi = ins
            dx, dw, db = layernorm_bwd(x, P[wi], dy, gget(x), gget(wi), gget(bi), eps=1e-5)
            gset(x, dx); gset(wi, dw); gset(bi, db)
        elif op == "linear":
            x, wi, bi = ins
            want = ("dx", "dW", "db") if bi is not None else ("dx", "dW")
            dx, dW, db = linear_bwd(x, P[wi], dy, gget(x), gget(wi), gget(bi) if bi is not None else None, want)
            gset(x, dx); gset(wi, dW)
            if bi is not None:
                gset(bi, db)
        elif op == "sdpa":
            q, k, v = ins
            dq, dk, dv = sdpa_bwd(q, k, v, kw["P"], dy, gget(q), gget(k), gget(v))
            gset(q, dq); gset(k, dk); gset(v, dv)
        elif op == "merge":
            (a,) = ins
            gset(a, head_merge_bwd(dy.reshape(B, T, C), B, T, C, H, hd, gget(a)))
        elif op == "gelu_tanh":
            (a,) = ins
            gset(a, act_bwd("gelu_tanh", a, dy, gget(a)))
    return loss, grads


def ref_gpt2_grads(params, n_layer, C, H, V, npos, ids, tgt):
    """The reference's own taped step (libref): (loss, grads)."""
    P = [_f32(p) for p in params]
    G = [np.zeros_like(p) for p in P]
    ids = np.ascontiguousarray(ids, np.int32)
    tgt = np.ascontiguousarray(tgt, np.int32)
    B, T = ids.shape
    L = ref()
    f = L.refg_gpt2_grads
    f.restype = ctypes.c_float
    f.argtypes = [ctypes.POINTER(vp), ctypes.POINTER(vp)] + [ci] * 5 + [vp, vp, ci, ci]
    pp = (vp * len(P))(*[p.ctypes.data for p in P])
    gp = (vp * len(G))(*[x.ctypes.data for x in G])
    loss = f(pp, gp, n_layer, C, H, V, npos, _ptr(ids), _ptr(tgt), B, T)
    return float(loss), G


# ---- config 4: qwen_forward (qwen.c:121-190) and greedy generation ----
def qwen_shapes(n_layer, C, H, K, I, V):
    hd = C // H
    per = [(C,), (C, C), (C,), (K * hd, C), (K * hd,), (K * hd, C), (K * hd,), (C, C), (C,), (I, C), (I, C), (C, I)]
    return [(V, C)] + per * n_layer + [(C,)]


def qwen_forward(params, n_layer, C, H, K, I, V, theta, ids, last_only=False, tables=None, cache=None):
    """The reference forward op for op with the pinned oracle functions;
    returns logits [T][V] (or [V] for the last row).  Bit-equal to the
    reference's own qwen_forward (tests/test_oracle_models.py).  cache: a list
    that receives each layer's post-RoPE keys and values ([K][T][hd] each)."""
    ids = np.ascontiguousarray(ids, np.int32)
    T, hd = ids.size, C // H
    P = [_f32(p) for p in params]
    cos_t, sin_t = tables if tables is not None else rope_tables_qwen(T, hd, theta)
    cos_t, sin_t = cos_t[:T], sin_t[:T]
    mask = np.where(np.arange(T)[None, :] <= np.arange(T)[:, None], 0.0, -1e9).astype(np.float32)
    h = embedding(P[0], ids)
    for li in range(n_layer):
        w = P[1 + 12 * li:13 + 12 * li]
        h1 = rmsnorm(h, w[0])
        ql, kl, vl = linear_fwd(h1, w[1], w[2]), linear_fwd(h1, w[3], w[4]), linear_fwd(h1, w[5], w[6])
        qq = heads_transpose(ql.reshape(1, T, C), 1, T, H, hd)
        kk = heads_transpose(kl.reshape(1, T, K * hd), 1, T, K, hd)
        vv = heads_transpose(vl.reshape(1, T, K * hd), 1, T, K, hd)
        qq = rope(qq.reshape(-1, hd), cos_t, sin_t, T).reshape(qq.shape)
        kk = rope(kk.reshape(-1, hd), cos_t, sin_t, T).reshape(kk.shape)
        if cache is not None:
            cache.append((kk[0].copy(), vv[0].copy()))
        ctx = sdpa_gqa(qq, kk, vv, mask)
        mo = head_merge(ctx, 1, T, C, H, hd).reshape(T, C)
        x1 = h + linear_fwd(mo, w[7], None)
        h2 = rmsnorm(x1, w[8])
        gu = mul(act("silu", linear_fwd(h2, w[9], None)), linear_fwd(h2, w[10], None))
        h = x1 + linear_fwd(gu, w[11], None)
    lnf = rmsnorm(h, P[-1])
    if last_only:
        return linear_fwd(lnf[-1:], P[0], None)[0]
    return linear_fwd(lnf, P[0], None)


def qwen_generate(params, n_layer, C, H, K, I, V, theta, prompt, n_new, eos=-1, n_ctx=None):
    """qwen_generate with temp 0 (qwen.c:204-228): full recompute per step,
    argmax_row of the last row; returns (ids, per-step logits)."""
    ids = list(np.asarray(prompt, np.int32))
    tables = rope_tables_qwen(n_ctx or len(ids) + n_new, C // H, theta)
    out, steps = [], []
    for _ in range(n_new):
        lg = qwen_forward(params, n_layer, C, H, K, I, V, theta, np.array(ids, np.int32), True, tables)
        nx = argmax_row(lg)
        steps.append(lg)
        out.append(nx)
        ids.append(nx)
        if nx == eos:
            break
    return out, steps



def qwen_generate_cached(params, n_layer, C, H, K, I, V, theta, prompt, n_new, eos=-1, n_ctx=None, keep=8):
    """qwen_generate with temp 0 (qwen.c:204-228) computing one new row per
    step against cached keys and values instead of the reference's full
    recompute.  Bit-equal to qwen_generate: every op is row-separable (the
    same float operations on the same row), a cached row's key and value
    equal the recomputed ones, and the masked columns the recompute adds
    (-1e9) contribute exact zeros to the max, the sum and the output.
    Returns (ids, per-step (top ids, top logits) of the `keep` largest)."""
    prompt = np.ascontiguousarray(prompt, np.int32)
    hd = C // H
    P = [_f32(p) for p in params]
    tables = rope_tables_qwen(n_ctx or prompt.size + n_new, hd, theta)
    cache = []
    lg = qwen_forward(P, n_layer, C, H, K, I, V, theta, prompt, True, tables, cache)
    kc = [np.concatenate([k, np.zeros((K, n_new, hd), np.float32)], axis=1) for k, _ in cache]
    vc = [np.concatenate([v, np.zeros((K, n_new, hd), np.float32)], axis=1) for _, v in cache]
    out, tops = [], []
    n = prompt.size
    for s in range(n_new):
        top = np.argsort(-lg, kind="stable")[:keep]
        tops.append((top.astype(np.int32), lg[top].copy()))
        nx = argmax_row(lg)
        out.append(nx)
        if nx == eos or s + 1 == n_new:
            break
        # one row at position n for token nx
        cs, sn = tables[0][n:n + 1], tables[1][n:n + 1]
        h = embedding(P[0], np.array([nx], np.int32))
        for li in range(n_layer):
            w = P[1 + 12 * li:13 + 12 * li]
            h1 = rmsnorm(h, w[0])
            q = rope(linear_fwd(h1, w[1], w[2]).reshape(H, hd), cs, sn, 1)
            kc[li][:, n] = rope(linear_fwd(h1, w[3], w[4]).reshape(K, hd), cs, sn, 1)
            vc[li][:, n] = linear_fwd(h1, w[5], w[6]).reshape(K, hd)
            ctx = sdpa_gqa(q.reshape(1, H, 1, hd), kc[li][None, :, :n + 1].copy(),
                           vc[li][None, :, :n + 1].copy())
            x1 = h + linear_fwd(ctx.reshape(1, C), w[7], None)
            h2 = rmsnorm(x1, w[8])
            gu = mul(act("silu", linear_fwd(h2, w[9], None)), linear_fwd(h2, w[10], None))
            h = x1 + linear_fwd(gu, w[11], None)
        lg = linear_fwd(rmsnorm(h, P[-1]), P[0], None)[0]
        n += 1
    return out, tops


# ---- config 1: the NCP transformer forward (ncp.c:184-338) ----
def rope_tables_ncp(S, hd, base):
    c = np.empty((S, hd), np.float32)
    s_ = np.empty((S, hd), np.float32)
    lib().orc_rope_tables_ncp(S, hd, base, _ptr(c), _ptr(s_))
    return c, s_


def ncp_shapes(n_layer, C, H, Kv, I, V):
    hd = C // H
    qkv = C + 2 * Kv * hd
    per = [(C,), (C,), (qkv, C), (qkv,), (C, C), (C,), (C,), (C,), (I, C), (I,), (I, C), (I,), (C, I), (C,)]
    return [(V, C)] + per * n_layer + [(C,), (C,), (V, C), (V,)]


def ncp_forward(params, n_layer, C, H, Kv, I, V, ids, rope_base=10000):
    """ncp_block x n_layer + ln_f + head on one level of S tokens, op for op
    with the pinned oracle functions (None entries = absent biases).  Equal
    bit for bit to the reference's ncp_load + ncp_forward (ncp.c:94-175,
    480-640) on one-hot inputs through wte = params[0]^T, no prefix, levels
    {1, S} (level 0 not a target), a zero level embedding and one untied
    head (tests/test_oracle_models.py)."""
    ids = np.ascontiguousarray(ids, np.int32)
    B, S = ids.shape
    hd, R = C // H, B * S
    P = [None if p is None else _f32(p) for p in params]
    cos_t, sin_t = rope_tables_ncp(S, hd, rope_base)
    nrm = layernorm
    x = embedding(P[0], ids.reshape(-1))
    for li in range(n_layer):
        w = P[1 + 14 * li:15 + 14 * li]
        ln = nrm(x, w[0], w[1])
        qkv = linear_fwd(ln, w[2], w[3])
        q, k, v = qkv_split(qkv.reshape(B, S, -1), B, S, C, H, hd, Kv, H // Kv)
        q = rope(q.reshape(-1, hd), cos_t, sin_t, S).reshape(q.shape)
        k = rope(k.reshape(-1, hd), cos_t, sin_t, S).reshape(k.shape)
        ctx = sdpa_gqa(q, k, v)
        mo = head_merge(ctx, B, S, C, H, hd).reshape(R, C)
        x = x + linear_fwd(mo, w[4], w[5])
        ln = nrm(x, w[6], w[7])
        g = mul(act("silu", linear_fwd(ln, w[8], w[9])), linear_fwd(ln, w[10], w[11]))
        x = x + linear_fwd(g, w[12], w[13])
    n = len(P)
    return linear_fwd(nrm(x, P[n - 4], P[n - 3]), P[n - 2], P[n - 1])


# ---- the reference's own model code (libref: qwen.c via ref_glue_qwen.c, ncp.c) ----
def write_ncm1(path, named):
    """An NCM1 weights file (the layout weights_load reads, tensor.c:69-124):
    "NCM1", u32 count, then per tensor u8 name length, name, u8 ndim, u32
    dims, u64 byte count, float32 data (little-endian)."""
    import struct
    with open(path, "wb") as f:
        f.write(b"NCM1" + struct.pack("<I", len(named)))
        for name, a in named:
            a = _f32(a)
            nb = name.encode()
            f.write(struct.pack("<B", len(nb)) + nb + struct.pack("<B", a.ndim))
            f.write(b"".join(struct.pack("<I", d) for d in a.shape))
            f.write(struct.pack("<Q", a.nbytes))
            f.write(a.tobytes())


def qwen_names(n_layer):
    """The reference's tensor names (qwen.c:59-79) in qwen_shapes order."""
    per = ["input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.q_proj.bias",
           "self_attn.k_proj.weight", "self_attn.k_proj.bias", "self_attn.v_proj.weight", "self_attn.v_proj.bias",
           "self_attn.o_proj.weight", "post_attention_layernorm.weight", "mlp.gate_proj.weight",
           "mlp.up_proj.weight", "mlp.down_proj.weight"]
    return (["model.embed_tokens.weight"] + [f"model.layers.{li}.{n}" for li in range(n_layer) for n in per]
            + ["model.norm.weight"])


class RefQwen:
    """The reference's qwen_open / qwen_forward / qwen_generate on a weights
    file written from params (qwen_shapes order)."""

    def __init__(self, params, n_layer, C, H, K, n_ctx, theta, path):
        write_ncm1(path, list(zip(qwen_names(n_layer), params)))
        self.V = params[0].shape[0]
        self.h = ref().refg_qwen_open(path.encode(), n_layer, H, K, C, n_ctx, theta)
        if not self.h:
            raise RuntimeError("reference qwen_open failed")

    def forward(self, ids, last_only=False):
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty(self.V if last_only else ids.size * self.V, np.float32)
        if ref().refg_qwen_forward(self.h, _ptr(ids), ids.size, int(last_only), _ptr(out)) != self.V:
            raise RuntimeError("reference qwen_forward failed")
        return out if last_only else out.reshape(ids.size, self.V)

    def generate(self, prompt, n_new):
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max(n_new, 1), np.int32)
        n = ref().refg_qwen_generate(self.h, _ptr(prompt), prompt.size, n_new, _ptr(out))
        return [int(v) for v in out[:n]]

    def close(self):
        if self.h:
            ref().refg_qwen_close(self.h)
            self.h = None


# NCMConfig fields refg_ncp_forward reads, in its cfg[] order (ref_glue.c)
NCP_CFG_KEYS = ("n_layer", "n_head", "n_embd", "n_kv_heads", "prefix_len", "query_level0",
                "attn_pattern_block_diag", "use_rope", "rope_base", "use_qk_norm", "puc_enabled", "puc_kernel",
                "shared_output_head", "shared_head_per_level_bias", "untied_head_bias", "tie_heads_to_codebook",
                "use_swiglu", "use_geglu", "use_relu2", "vq_embed_dim", "prefix_pad_token_id")


def ncp_named(params, n_layer, C):
    """The reference's tensor names (ncp.c:189-316, 94-175, 406-478) for the
    oracle's flat ncp parameters, with wte as the [C][V] linear of one-hot
    inputs and a zero level embedding."""
    pre = "gen.transformer."
    per = ["ln_1.weight", "ln_1.bias", "attn.c_attn.weight", "attn.c_attn.bias", "attn.c_proj.weight",
           "attn.c_proj.bias", "ln_2.weight", "ln_2.bias", "mlp.w_gate.weight", "mlp.w_gate.bias",
           "mlp.w_up.weight", "mlp.w_up.bias", "mlp.c_proj.weight", "mlp.c_proj.bias"]
    named = {pre + "wte.weight": params[0].T.copy(), pre + "wle.weight": np.zeros((1, C), np.float32)}
    for li in range(n_layer):
        for j, n in enumerate(per):
            if params[1 + 14 * li + j] is not None:
                named[f"{pre}blocks.{li}.{n}"] = params[1 + 14 * li + j]
    n = len(params)
    for name, p in ((pre + "ln_f.weight", params[n - 4]), (pre + "ln_f.bias", params[n - 3]),
                    ("gen.lm_heads.0.weight", params[n - 2]), ("gen.lm_heads.0.bias", params[n - 1])):
        if p is not None:
            named[name] = p
    return named


def ncp_single_level_cfg(n_layer, C, H, Kv, V, S, rope_base=10000):
    """The NCMConfig fields under which the reference's ncp_forward runs the
    oracle's single-level ncp_forward: one target level of S tokens (level 0
    of length 1 is not a target), no prefix, RoPE, SwiGLU, one untied head,
    one-hot inputs of dimension V."""
    return dict(n_layer=n_layer, n_head=H, n_embd=C, n_kv_heads=Kv, prefix_len=0, query_level0=0,
                attn_pattern_block_diag=1, use_rope=1, rope_base=rope_base, use_swiglu=1, vq_embed_dim=V,
                prefix_pad_token_id=-1, levels=[1, S], vocab_size=[V])


def ref_ncp_forward(cfg, named, x, prefix_ids=None):
    """The reference's ncp_load + ncp_forward (ncp.c:94-175, 480-640).
    cfg: dict of NCP_CFG_KEYS plus levels (list) and vocab_size (list per
    target level); named: dict name -> array; x [B][P+T][D].
    Returns logits [B][T][max vocab]."""
    x = _f32(x)
    B = x.shape[0]
    levels = np.ascontiguousarray(cfg["levels"], np.int32)
    vocabs = np.ascontiguousarray(cfg["vocab_size"], np.int32)
    c = np.ascontiguousarray([int(cfg.get(k, 0)) for k in NCP_CFG_KEYS], np.int32)
    lvl_first = 0 if cfg.get("query_level0", 0) else 1
    T = int(levels.sum()) - (0 if lvl_first == 0 else int(levels[0]))
    names = list(named)
    arrs = [_f32(named[n]) for n in names]
    cn = (ctypes.c_char_p * len(names))(*[n.encode() for n in names])
    dp = (vp * len(arrs))(*[a.ctypes.data for a in arrs])
    shapes = np.zeros((len(arrs), 4), np.int64)
    ndims = np.ascontiguousarray([a.ndim for a in arrs], np.int32)
    for i, a in enumerate(arrs):
        shapes[i, :a.ndim] = a.shape
    pids = None if prefix_ids is None else np.ascontiguousarray(prefix_ids, np.int32)
    out = np.empty((B, T, int(vocabs.max())), np.float32)
    rc = ref().refg_ncp_forward(_ptr(c), levels.size, _ptr(levels), _ptr(vocabs), vocabs.size, cn, dp,
                                _ptr(shapes), _ptr(ndims), len(arrs), _ptr(x), _ptr(pids), B, _ptr(out))
    if rc:
        raise RuntimeError("reference ncp_forward failed")
    return out


# ---- the multi-level NCP forward (ncp.c:94-175, 184-358, 361-403, 406-640) ----
def conv1d_btc(x, W, b, K, stride, pad):
    """conv1d_fwd (kernels.c:546-566) on [B][T][Cin] rows; W [Cout][Cin][K]."""
    x, W = _f32(x), _f32(W)
    b = None if b is None else _f32(b)
    B, T, Cin = x.shape
    Cout = W.shape[0]
    To = (T + 2 * pad - K) // stride + 1
    y = np.empty((B, To, Cout), np.float32)
    lib().orc_conv1d_btc(_ptr(x), _ptr(W), _ptr(b), _ptr(y), B, T, Cin, Cout, K, stride, pad)
    return y


def _expf(v):
    """glibc's expf, as the reference's head_logits calls it (ncp.c:460)."""
    f = ctypes.CDLL("libm.so.6").expf
    f.restype = ctypes.c_float
    f.argtypes = [ctypes.c_float]
    return f(float(v))


def ncp_build_mask(cfg, S):
    """build_full_mask (ncp.c:361-386): [S][S] additive, 0 or -inf."""
    P = cfg.get("prefix_len", 0)
    levels = list(cfg["levels"])
    first = 0 if cfg.get("query_level0", 0) else 1
    lvl = np.concatenate([np.full(levels[k], k) for k in range(first, len(levels))]).astype(np.int64)
    m = np.zeros((S, S), np.float32)
    m[:P, P:] = -np.inf
    li, lj = lvl[:, None], lvl[None, :]
    tgt = (li == lj) if cfg.get("attn_pattern_block_diag", 0) else (li >= lj)
    m[P:, P:] = np.where(tgt, 0.0, -np.inf).astype(np.float32)
    return m


def _ncp_block(cfg, named, li, x, B, S, mask, cos_t, sin_t):
    """ncp_block (ncp.c:184-345) on x [B*S][C], returning the new x."""
    C, H, nkv = cfg["n_embd"], cfg["n_head"], cfg["n_kv_heads"]
    hd = C // H
    pre = f"gen.transformer.blocks.{li}."
    g = named.get
    ln = layernorm(x, named[pre + "ln_1.weight"], g(pre + "ln_1.bias"))
    qkv = linear_fwd(ln, named[pre + "attn.c_attn.weight"], g(pre + "attn.c_attn.bias"))
    qq, kk, vv = qkv_split(qkv.reshape(B, S, -1), B, S, C, H, hd, nkv, H // nkv)
    if cfg.get("use_qk_norm", 0):
        qq = rmsnorm(qq.reshape(-1, hd), named[pre + "attn.q_norm.weight"]).reshape(qq.shape)
        kk = rmsnorm(kk.reshape(-1, hd), named[pre + "attn.k_norm.weight"]).reshape(kk.shape)
    if cfg.get("use_rope", 0):
        qq = rope(qq.reshape(-1, hd), cos_t, sin_t, S).reshape(qq.shape)
        kk = rope(kk.reshape(-1, hd), cos_t, sin_t, S).reshape(kk.shape)
    ctx = sdpa_gqa(qq, kk, vv, mask)
    mo = head_merge(ctx, B, S, C, H, hd).reshape(B * S, C)
    x = x + linear_fwd(mo, named[pre + "attn.c_proj.weight"], g(pre + "attn.c_proj.bias"))
    mn = layernorm(x, named[pre + "ln_2.weight"], g(pre + "ln_2.bias"))
    if cfg.get("use_swiglu", 0) or cfg.get("use_geglu", 0):
        gt = linear_fwd(mn, named[pre + "mlp.w_gate.weight"], g(pre + "mlp.w_gate.bias"))
        up = linear_fwd(mn, named[pre + "mlp.w_up.weight"], g(pre + "mlp.w_up.bias"))
        gt = act("silu" if cfg.get("use_swiglu", 0) else "gelu", gt)
        h = gt * up
    else:
        h = linear_fwd(mn, named[pre + "mlp.c_fc.weight"], g(pre + "mlp.c_fc.bias"))
        if cfg.get("use_relu2", 0):
            r = np.where(h > 0, h, np.float32(0)).astype(np.float32)
            h = r * r
        else:
            h = act("gelu", h)
    return x + linear_fwd(h, named[pre + "mlp.c_proj.weight"], g(pre + "mlp.c_proj.bias"))


def ncp_head(cfg, named, k, slice_):
    """head_logits (ncp.c:406-478) of target level k on rows slice_ [R][C]."""
    g = named.get
    first = 0 if cfg.get("query_level0", 0) else 1
    V = list(cfg["vocab_size"])[k]
    if cfg.get("shared_output_head", 0):
        # the level's vocabulary is the first V rows of the shared head
        b = (named[f"gen.lm_heads.biases.{k}"] if cfg.get("shared_head_per_level_bias", 0)
             else named["gen.lm_heads.head.bias"] if cfg.get("untied_head_bias", 0) else None)
        return linear_fwd(slice_, _f32(named["gen.lm_heads.head.weight"])[:V], None if b is None else _f32(b)[:V])
    if cfg.get("tie_heads_to_codebook", 0):
        z = linear_fwd(slice_, named[f"gen.lm_heads.{k}.proj.weight"], g(f"gen.lm_heads.{k}.proj.bias"))
        E = _f32(named[f"tok.vq.embeddings.{k + first}.weight"])
        invT = _expf(np.asarray(named[f"gen.lm_heads.{k}.log_inv_T"], np.float32).reshape(-1)[0])
        bias = g(f"gen.lm_heads.{k}.bias")
        bias = None if bias is None else _f32(bias)
        V, Dd = E.shape
        out = np.empty((z.shape[0], V), np.float32)
        lib().orc_ncp_tied_head(_ptr(z), _ptr(E), _ptr(bias), invT, _ptr(out), z.shape[0], V, Dd)
        return out
    return linear_fwd(slice_, named[f"gen.lm_heads.{k}.weight"], g(f"gen.lm_heads.{k}.bias"))


def ncp_forward_levels(cfg, named, x, prefix_ids=None):
    """ncp_forward (ncp.c:480-640) op for op with the pinned oracle
    functions: x [B][P+T][D] -> logits [B][T][max vocab] (-inf past a
    level's vocabulary).  cfg / named as ref_ncp_forward takes them."""
    x = _f32(x)
    B = x.shape[0]
    C, H, D = cfg["n_embd"], cfg["n_head"], cfg["vq_embed_dim"]
    hd = C // H
    P = cfg.get("prefix_len", 0)
    first = 0 if cfg.get("query_level0", 0) else 1
    tl = list(cfg["levels"])[first:]
    T = sum(tl)
    S = P + T
    use_rope = cfg.get("use_rope", 0)
    pos = list(range(P)) + [t for lk in tl for t in range(lk)]
    cos_t = sin_t = None
    if use_rope:
        cs, sn = rope_tables_ncp(max(pos) + 1, hd, cfg["rope_base"])
        cos_t, sin_t = cs[pos].copy(), sn[pos].copy()
    wle = _f32(named["gen.transformer.wle.weight"])
    lvl_pos = np.concatenate([np.repeat(wle[k:k + 1], lk, axis=0) for k, lk in enumerate(tl)])
    if not use_rope:
        wpe = _f32(named["gen.transformer.wpe.weight"])
        lvl_pos = lvl_pos + np.concatenate([wpe[:lk] for lk in tl])
    zpre, xt = x[:, :P].copy(), x[:, P:].copy()
    if cfg.get("puc_enabled", 0):
        Kc, off = cfg["puc_kernel"], 0
        for k, lk in enumerate(tl):
            co = conv1d_btc(xt[:, off:off + lk], named[f"gen.post_upsample_convs.{k}.weight"],
                            named[f"gen.post_upsample_convs.{k}.bias"], Kc, 1, Kc // 2)
            xt[:, off:off + lk] = xt[:, off:off + lk] + co[:, :lk]
            off += lk
    wte, wteb = named["gen.transformer.wte.weight"], named.get("gen.transformer.wte.bias")
    pemb = linear_fwd(zpre.reshape(-1, D), wte, wteb).reshape(B, P, C)
    xe = linear_fwd(xt.reshape(-1, D), wte, wteb).reshape(B, T, C) + lvl_pos[None]
    if not use_rope:
        pemb = pemb + _f32(named["gen.transformer.wpe.weight"])[:P][None]
    h = np.concatenate([pemb, xe], axis=1)
    mask = ncp_build_mask(cfg, S)
    pad = cfg.get("prefix_pad_token_id", -1)
    n_layer = cfg["n_layer"]

    def run_stack(hb, nb, m):
        hb = hb.reshape(nb * S, C)
        for li in range(n_layer):
            hb = _ncp_block(cfg, named, li, hb, nb, S, m, cos_t, sin_t)
        return layernorm(hb, named["gen.transformer.ln_f.weight"], named.get("gen.transformer.ln_f.bias"))

    pids = None if prefix_ids is None else np.asarray(prefix_ids, np.int32).reshape(B, P)
    if pad >= 0 and pids is not None and (pids == pad).any():
        outs = []
        for b in range(B):
            mb = mask.copy()
            mb[:, :P][:, pids[b] == pad] = -np.inf
            outs.append(run_stack(h[b:b + 1], 1, mb))
        h = np.concatenate(outs).reshape(B, S, C)
    else:
        h = run_stack(h, B, mask).reshape(B, S, C)
    vocabs = list(cfg["vocab_size"])[:len(tl)]
    logits = np.full((B, T, max(vocabs)), -np.inf, np.float32)
    off = 0
    for k, lk in enumerate(tl):
        lg = ncp_head(cfg, named, k, h[:, P + off:P + off + lk].reshape(B * lk, C))
        logits[:, off:off + lk, :vocabs[k]] = lg.reshape(B, lk, vocabs[k])
        off += lk
    return logits
