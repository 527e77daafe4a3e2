"""Pins the oracle's training rows (norm backward, softmax-CE, SDPA backward,
AdamW, schedule, clip): bit-equality with the reference's own tape compiled
from source (where /root/reference was built), plus float64 finite
differences and closed forms that a dropped term or a wrong index fails."""
import numpy as np
import pytest

import oracle as O
from conftest import bits_equal

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference not compiled here")


def rnd(seed, *shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


# ------------------------------------------------------------------ vs the reference tape
@needs_ref
@pytest.mark.parametrize("eps", [None, 1e-5])
@pytest.mark.parametrize("affine", [True, False])
def test_ln_bwd_vs_reference(eps, affine):
    rows, C = 37, 96
    x, dy = rnd(1, rows, C) * 2 + 0.5, rnd(2, rows, C)
    w, b = (rnd(3, C), rnd(4, C)) if affine else (None, None)
    dx0, dw0, db0 = rnd(5, rows, C), rnd(6, C), rnd(7, C)
    rdx, rdw, rdb = O.ref_ln_bwd(x, w, b, dy, dx0, dw0, db0, eps=eps)
    want = ("dx", "dw", "db") if affine else ("dx",)
    dx, dw, db = O.layernorm_bwd(x, w, dy, dx0, dw0, db0, eps=1e-6 if eps is None else eps, want=want)
    assert bits_equal(dx, rdx)
    if affine:
        assert bits_equal(dw, rdw) and bits_equal(db, rdb)


@needs_ref
@pytest.mark.parametrize("weighted", [True, False])
def test_rmsn_bwd_vs_reference(weighted):
    rows, C = 29, 128
    x, dy = rnd(8, rows, C), rnd(9, rows, C)
    w = rnd(10, C) if weighted else None
    dx0, dw0 = rnd(11, rows, C), rnd(12, C)
    rdx, rdw = O.ref_rmsn_bwd(x, w, dy, dx0, dw0)
    dx, dw = O.rmsnorm_bwd(x, w, dy, dx0, dw0, want=("dx", "dw") if weighted else ("dx",))
    assert bits_equal(dx, rdx)
    if weighted:
        assert bits_equal(dw, rdw)


@needs_ref
@pytest.mark.parametrize("masked", [False, True])
def test_ce_vs_reference(masked):
    rows, V = 23, 300
    logits = rnd(13, rows, V, scale=3.0)
    tgt = np.random.default_rng(14).integers(0, V, rows).astype(np.int32)
    wm = None
    if masked:
        wm = np.random.default_rng(15).uniform(0.5, 2.0, rows).astype(np.float32)
        wm[[2, 7]] = 0.0
    dl0 = rnd(16, rows, V)
    rloss, rprobs, rdl = O.ref_ce(logits, tgt, wm, weight=0.7, dl0=dl0)
    loss, probs, cnt = O.ce_fwd(logits, tgt, wm)
    dl = O.ce_bwd(probs, tgt, wm, 0.7 / cnt, dl0)
    assert np.float32(loss) == np.float32(rloss)
    assert bits_equal(probs, rprobs) and bits_equal(dl, rdl)


@needs_ref
@pytest.mark.parametrize("B,H,Hkv,Tq,Tkv,hd,causal", [(2, 4, 4, 9, 9, 16, True), (1, 6, 2, 7, 11, 8, False),
                                                     (2, 14, 2, 5, 5, 64, True)])
def test_sdpa_bwd_vs_reference(B, H, Hkv, Tq, Tkv, hd, causal):
    q, k, v = rnd(17, B, H, Tq, hd), rnd(18, B, Hkv, Tkv, hd), rnd(19, B, Hkv, Tkv, hd)
    dy = rnd(20, B, H, Tq, hd)
    mask = None
    if causal:
        mask = np.where(np.arange(Tkv)[None, :] > np.arange(Tq)[:, None] + (Tkv - Tq), -1e9, 0).astype(np.float32)
    o, P, rdq, rdk, rdv = O.ref_sdpa_bwd(q, k, v, mask, dy)
    assert bits_equal(O.sdpa_probs(q, k, mask), P)
    dq, dk, dv = O.sdpa_bwd(q, k, v, P, dy)
    assert bits_equal(dq, rdq) and bits_equal(dk, rdk) and bits_equal(dv, rdv)


# ------------------------------------------------------------------ float64 mathematics
def ln64(x, w, b, eps):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def rms64(x, w):
    return x / np.sqrt((x ** 2).mean(-1, keepdims=True) + 1e-6) * w


def num_grad(f, x, h=1e-6):
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        xp, xm = x.copy(), x.copy()
        xp[i] += h
        xm[i] -= h
        g[i] = (f(xp) - f(xm)) / (2 * h)
    return g


def test_ln_bwd_finite_differences():
    rows, C, eps = 3, 12, 1e-5
    x, w, b, dy = (rnd(21, rows, C).astype(np.float64), rnd(22, C).astype(np.float64),
                   rnd(23, C).astype(np.float64), rnd(24, rows, C).astype(np.float64))
    dx, dw, db = O.layernorm_bwd(x, w, dy, eps=eps)
    assert np.allclose(dx, num_grad(lambda z: np.sum(dy * ln64(z, w, b, eps)), x), atol=2e-5)
    assert np.allclose(dw, num_grad(lambda z: np.sum(dy * ln64(x, z, b, eps)), w), atol=2e-5)
    assert np.allclose(db, dy.sum(0), atol=1e-5)
    assert np.max(np.abs(dx.sum(-1))) < 1e-5        # LN input grads sum to zero per row


def test_rmsn_bwd_finite_differences():
    rows, C = 3, 16
    x, w, dy = rnd(25, rows, C).astype(np.float64), rnd(26, C).astype(np.float64), rnd(27, rows, C).astype(np.float64)
    dx, dw = O.rmsnorm_bwd(x, w, dy)
    assert np.allclose(dx, num_grad(lambda z: np.sum(dy * rms64(z, w)), x), atol=2e-5)
    assert np.allclose(dw, num_grad(lambda z: np.sum(dy * rms64(x, z)), w), atol=2e-5)


def test_ce_closed_forms():
    rows, V = 9, 50
    logits = rnd(28, rows, V, scale=2.0)
    tgt = np.random.default_rng(29).integers(0, V, rows).astype(np.int32)
    loss, probs, cnt = O.ce_fwd(logits, tgt)
    l64 = logits.astype(np.float64)
    lse = np.log(np.exp(l64 - l64.max(-1, keepdims=True)).sum(-1)) + l64.max(-1)
    assert cnt == rows
    assert abs(loss - np.mean(lse - l64[np.arange(rows), tgt])) < 1e-5
    assert np.max(np.abs(probs.sum(-1) - 1)) < 1e-5
    dl = O.ce_bwd(probs, tgt, None, 1.0 / cnt)
    assert np.max(np.abs(dl.sum(-1))) < 1e-6          # (p - onehot) sums to zero
    onehot = np.eye(V)[tgt]
    assert np.allclose(dl, (np.exp(l64 - lse[:, None]) - onehot) / rows, atol=1e-7)


def test_adamw_step_one_closed_form():
    n, lr, wd, eps = 1000, 3e-4, 0.1, 1e-8
    p, g = rnd(30, n), rnd(31, n)
    z = np.zeros(n, np.float32)
    b1, b2 = 0.9, 0.95
    p1, m1, v1 = O.adamw(p, g, z, z, lr, b1, b2, 1 - b1, 1 - b2, eps, wd)
    # m-hat = g and v-hat = g^2 at step 1
    want = p.astype(np.float64) * (1 - lr * wd) - lr * g / (np.abs(g) + eps)
    assert np.max(np.abs(p1 - want)) < 1e-6
    assert np.allclose(m1, 0.1 * g, rtol=1e-6) and np.allclose(v1, 0.05 * g.astype(np.float64) ** 2, rtol=1e-6)
    # zero gradient: pure decay, moments stay zero
    p2, m2, v2 = O.adamw(p, z, z, z, lr, b1, b2, 1 - b1, 1 - b2, eps, wd)
    assert np.allclose(p2, p.astype(np.float64) * (1 - lr * wd), rtol=1.2e-7, atol=0) and not m2.any() and not v2.any()


@needs_ref
def test_adamw_and_schedule_vs_reference_step():
    """orc_adamw with the learning rate of orc_sched_cosine_warmup against the
    reference's own adamw_new + adamw_step (train.c:18-145, its host loop and
    static schedule), three steps through warm-up, per-tensor lr multipliers."""
    import ctypes
    import ncmhip
    mem = {k: ncmhip._SIGS[k] for k in ("tensor_alloc", "tensor_free", "mem_h2d", "mem_d2h")}
    R = ncmhip.bind(O.ref(), {**ncmhip.FORMAT_SIGS, **mem})
    shapes = [(13, 7), (29,), (4, 3, 5)]
    ps = [rnd(40 + i, *sh) for i, sh in enumerate(shapes)]
    items = (ncmhip.NamedTensor * len(ps))()
    for i, p in enumerate(ps):
        t = R.tensor_alloc(p.ndim, (ctypes.c_int64 * 4)(*p.shape, *([0] * (4 - p.ndim))))
        items[i].name = f"t{i}".encode()
        items[i].t = ctypes.cast(t, ctypes.POINTER(ncmhip.TensorS))
        R.mem_h2d(items[i].t.contents.data, p.ctypes.data, p.nbytes)
    ws = ncmhip.WeightStore(items, len(ps))
    op = ctypes.cast(R.adamw_new(ctypes.byref(ws), None), ctypes.POINTER(ncmhip.AdamW))
    o = op.contents
    o.wd = 0.1
    lrm = [1.0, 0.5, 3.0]
    for i, m in enumerate(lrm):
        o.lr[i] = m
    mine = [(p.copy(), np.zeros_like(p), np.zeros_like(p)) for p in ps]
    base_lr, warmup, total = 3e-4, 2.0, 10.0
    for step in range(1, 4):
        gs = [rnd(50 + 10 * step + i, *sh) for i, sh in enumerate(shapes)]
        for i, g in enumerate(gs):
            ctypes.memmove(o.g[i], g.ctypes.data, g.nbytes)
        R.adamw_step(op, base_lr, warmup, total)
        lr = base_lr * O.sched_cosine_warmup(step, warmup, total)
        b1t, b2t = 1.0 - 0.9 ** step, 1.0 - 0.95 ** step
        mine = [O.adamw(p, g, m, v, lr * lrm[i], 0.9, 0.95, b1t, b2t, 1e-8, 0.1)
                for i, ((p, m, v), g) in enumerate(zip(mine, gs))]
    assert o.step == 3
    for i, (p, m, v) in enumerate(mine):
        got = [np.empty_like(p) for _ in range(3)]
        R.mem_d2h(got[0].ctypes.data, items[i].t.contents.data, p.nbytes)
        ctypes.memmove(got[1].ctypes.data, o.m[i], p.nbytes)
        ctypes.memmove(got[2].ctypes.data, o.v[i], p.nbytes)
        assert bits_equal(got[0], p) and bits_equal(got[1], m) and bits_equal(got[2], v)
    R.adamw_free(op)
    for i in range(len(ps)):
        R.tensor_free(ctypes.cast(items[i].t, ctypes.c_void_p))


def test_schedule_closed_forms():
    assert O.sched_cosine_warmup(50, 100, 1000) == 0.5
    assert O.sched_cosine_warmup(100, 100, 1000) == 1.0
    assert abs(O.sched_cosine_warmup(550, 100, 1000) - 0.5) < 1e-15
    assert O.sched_cosine_warmup(1000, 100, 1000) == 0.0
    assert O.sched_cosine_warmup(3, 0, 10) == pytest.approx(0.5 * (1 + np.cos(np.pi * 0.3)), abs=1e-15)


def test_grad_clip():
    gs = [rnd(32, 100), rnd(33, 7, 3)]
    norm64 = np.sqrt(sum(float(np.sum(g.astype(np.float64) ** 2)) for g in gs))
    gn, out = O.grad_clip(gs, 1.0)
    assert abs(gn - norm64) < 1e-12 * norm64
    assert abs(np.sqrt(sum(float(np.sum(g.astype(np.float64) ** 2)) for g in out)) - 1.0) < 1e-6
    small = [g * np.float32(1e-3) for g in gs]
    gn2, out2 = O.grad_clip(small, 1.0)
    assert gn2 < 1.0 and all(bits_equal(a, b) for a, b in zip(out2, small))


def sdpa64(q, k, v, mask):
    rep = q.shape[1] // k.shape[1]
    kk, vv = np.repeat(k, rep, axis=1), np.repeat(v, rep, axis=1)
    s = q @ kk.transpose(0, 1, 3, 2) / np.sqrt(q.shape[-1]) + mask
    p = np.exp(s - s.max(-1, keepdims=True))
    return (p / p.sum(-1, keepdims=True)) @ vv


def test_sdpa_bwd_finite_differences():
    B, H, Hkv, T, hd = 1, 4, 2, 5, 8
    q, k, v, dy = (rnd(34, B, H, T, hd).astype(np.float64), rnd(35, B, Hkv, T, hd).astype(np.float64),
                   rnd(36, B, Hkv, T, hd).astype(np.float64), rnd(37, B, H, T, hd).astype(np.float64))
    mask = np.where(np.arange(T)[None, :] > np.arange(T)[:, None], -1e9, 0.0)
    P = O.sdpa_probs(q, k, mask)
    dq, dk, dv = O.sdpa_bwd(q, k, v, P, dy)
    loss = lambda qq, kk, vv: np.sum(dy * sdpa64(qq, kk, vv, mask))
    assert np.allclose(dq, num_grad(lambda z: loss(z, k, v), q), atol=2e-5)
    assert np.allclose(dk, num_grad(lambda z: loss(q, z, v), k), atol=2e-5)
    assert np.allclose(dv, num_grad(lambda z: loss(q, k, z), v), atol=2e-5)


# ------------------------------------------------------------------ remaining tape ops
@needs_ref
@pytest.mark.parametrize("name", ["gelu", "silu", "gelu_tanh"])
def test_act_bwd_vs_reference(name):
    x = np.concatenate([rnd(60, 3000, scale=3.0), np.array([0.0, -0.0, 20.0, -20.0], np.float32)])
    dy, dx0 = rnd(61, x.size), rnd(62, x.size)
    assert bits_equal(O.act_bwd(name, x, dy, dx0), O.ref_act_bwd(name, x, dy, dx0))


@needs_ref
def test_mul_rope_embed_vs_reference():
    a, b, dy = rnd(63, 999), rnd(64, 999), rnd(65, 999)
    da0, db0 = rnd(66, 999), rnd(67, 999)
    for u, v in zip(O.mul_bwd(a, b, dy, da0, db0), O.ref_mul_bwd(a, b, dy, da0, db0)):
        assert bits_equal(u, v)
    B, H, Hkv, T, hd = 2, 6, 2, 9, 16
    c, s = O.rope_tables_qwen(T, hd, 1e4)
    xq, xk, gq, gk = rnd(68, B, H, T, hd), rnd(69, B, Hkv, T, hd), rnd(70, B, H, T, hd), rnd(71, B, Hkv, T, hd)
    rq, rk = O.ref_rope_bwd(xq, xk, c, s, gq, gk)
    assert bits_equal(O.rope_bwd(gq.reshape(-1, hd), c, s, T).reshape(gq.shape), rq)
    assert bits_equal(O.rope_bwd(gk.reshape(-1, hd), c, s, T).reshape(gk.shape), rk)
    V, D, n = 50, 24, 300
    W = rnd(72, V, D)
    idx = np.random.default_rng(73).integers(0, V, n).astype(np.int32)
    dy, dW0 = rnd(74, n, D), rnd(75, V, D)
    assert bits_equal(O.embedding_bwd(dy, idx, V, dW0), O.ref_embed_bwd(W, idx, dy, dW0))


@needs_ref
@pytest.mark.parametrize("B,T,C,H,hd,K,rep", [(2, 5, 64, 4, 16, 4, 1), (1, 7, 96, 6, 16, 2, 3)])
def test_split_merge_bwd_vs_reference(B, T, C, H, hd, K, rep):
    x = rnd(76, B, T, C + 2 * K * hd)
    gq, gk, gv = rnd(77, B, H, T, hd), rnd(78, B, H, T, hd), rnd(79, B, H, T, hd)
    assert bits_equal(O.qkv_split_bwd(gq, gk, gv, B, T, C, H, hd, K, rep),
                      O.ref_split_bwd(x, gq, gk, gv, B, T, C, H, hd, K, rep))
    assert bits_equal(O.qkv_split_bwd(None, gk, None, B, T, C, H, hd, K, rep),
                      O.ref_split_bwd(x, None, gk, None, B, T, C, H, hd, K, rep))
    ctx, dy = rnd(80, B, H, T, hd), rnd(81, B, T, C)
    assert bits_equal(O.head_merge_bwd(dy, B, T, C, H, hd), O.ref_merge_bwd(0, ctx, dy, B, T, C, H, hd))
    xs, dys = rnd(82, B, T, C), rnd(83, B, H, T, hd)
    assert bits_equal(O.heads_transpose_bwd(dys, B, T, C, H, hd), O.ref_merge_bwd(1, xs, dys, B, T, C, H, hd))


def test_act_bwd_finite_differences():
    x = rnd(84, 200, scale=2.5).astype(np.float64)
    dy = np.ones_like(x)
    fns = {"gelu": lambda z: 0.5 * z * (1 + np.vectorize(__import__("math").erf)(z / np.sqrt(2))),
           "silu": lambda z: z / (1 + np.exp(-z)),
           "gelu_tanh": lambda z: 0.5 * z * (1 + np.tanh(np.sqrt(2 / np.pi) * (z + 0.044715 * z ** 3)))}
    for name, f in fns.items():
        h = 1e-6
        num = (f(x + h) - f(x - h)) / (2 * h)
        assert np.max(np.abs(O.act_bwd(name, x, dy) - num)) < 1e-6


def test_layout_bwd_are_adjoints():
    """<dy, f(x)> = <f^T(dy), x> for the permutations and the GQA split."""
    B, T, C, H, hd, K, rep = 2, 3, 24, 6, 4, 2, 3
    x = rnd(85, B, T, C + 2 * K * hd).astype(np.float64)
    gq, gk, gv = rnd(86, B, H, T, hd), rnd(87, B, H, T, hd), rnd(88, B, H, T, hd)
    q, k, v = O.qkv_split(x, B, T, C, H, hd, K, rep)
    lhs = sum(float(np.sum(g.astype(np.float64) * y)) for g, y in ((gq, q), (gk, k), (gv, v)))
    rhs = float(np.sum(O.qkv_split_bwd(gq, gk, gv, B, T, C, H, hd, K, rep).astype(np.float64) * x))
    assert abs(lhs - rhs) < 1e-4
    ctx, dy = rnd(89, B, H, T, hd), rnd(90, B, T, C)
    assert abs(float(np.sum(dy * O.head_merge(ctx, B, T, C, H, hd))) -
               float(np.sum(O.head_merge_bwd(dy, B, T, C, H, hd) * ctx))) < 1e-4
    W = rnd(91, 10, 3)
    idx = np.array([3, 3, 0, 9, 3], np.int32)
    dye = rnd(92, 5, 3)
    assert abs(float(np.sum(dye * O.embedding(W, idx))) - float(np.sum(O.embedding_bwd(dye, idx, 10) * W))) < 1e-5


# ------------------------------------------------------------------ config 5: the whole taped step
def gpt2_case(seed, n_layer, C, H, V, npos, B, T):
    rng = np.random.default_rng(seed)
    params = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in O.gpt2_shapes(n_layer, C, V, npos)]
    for i, s in enumerate(O.gpt2_shapes(n_layer, C, V, npos)):   # LayerNorm gains near 1
        if len(s) == 1 and s[0] == C and (i >= len(params) - 2 or (i - 2) % 12 in (0, 6)):
            params[i] += 1.0
    ids = rng.integers(0, V, (B, T)).astype(np.int32)
    tgt = rng.integers(0, V, (B, T)).astype(np.int32)
    return params, ids, tgt


@needs_ref
@pytest.mark.parametrize("n_layer,C,H,V,npos,B,T", [(2, 32, 4, 50, 16, 2, 9), (1, 64, 2, 40, 8, 3, 8)])
def test_gpt2_step_vs_reference(n_layer, C, H, V, npos, B, T):
    params, ids, tgt = gpt2_case(7, n_layer, C, H, V, npos, B, T)
    rloss, rg = O.ref_gpt2_grads(params, n_layer, C, H, V, npos, ids, tgt)
    loss, g = O.gpt2_grads(params, n_layer, C, H, V, npos, ids, tgt)
    assert np.float32(loss) == np.float32(rloss)
    for a, b in zip(g, rg):
        assert bits_equal(a, b)
