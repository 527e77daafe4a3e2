"""GPU training-step rows against the oracle (the reference's tape backward and
optimizer restated on the CPU).

Bars (gradients: the north-star max-abs 1e-3, asserted tighter here):
  norm backward dx, dw, db      maxrel 1e-5 (fp64 in both; RMSNorm dw 1e-4:
                                the reference sums it in float)
  CE probs / loss               maxrel 1e-6;  ce_bwd bit-exact from equal probs
  SDPA probs                    max-abs 1e-6
  SDPA backward dq, dk, dv      max-abs 1e-4 and maxrel 1e-4 (fp32 MFMA sums
                                against the reference's fp64/float mix)
  AdamW                         bit-exact over several steps
  clip                          norm rel 1e-12, gradients within 1 ulp
"""
import ctypes

import numpy as np
import pytest

import ncmhip
import oracle as O
from conftest import bits_equal, maxrel

pytestmark = pytest.mark.gpu
D = ncmhip.DeviceBuffer


@pytest.fixture(scope="module", autouse=True)
def device():
    ncmhip.init(0)
    print("[gpu] train tests on device 0", flush=True)


def rnd(seed, *shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def up(a):
    return None if a is None else D.from_numpy(a)


# ---------------------------------------------------------------- norms
@pytest.mark.parametrize("rows,C", [(1, 1), (37, 96), (300, 65), (4096, 768), (129, 896), (70, 1024), (33, 1028)])
@pytest.mark.parametrize("eps,affine", [(1e-6, True), (1e-5, True), (1e-6, False)])
def test_layernorm_bwd(rows, C, eps, affine):
    x, dy = rnd(1, rows, C) * 2 + 0.3, rnd(2, rows, C)
    w = rnd(3, C) if affine else None
    dx0, dw0, db0 = rnd(4, rows, C), rnd(5, C), rnd(6, C)
    want = ("dx", "dw", "db") if affine else ("dx",)
    rdx, rdw, rdb = O.layernorm_bwd(x, w, dy, dx0, dw0, db0, eps=eps, want=want)
    dx, dw, db = up(dx0), up(dw0) if affine else None, up(db0) if affine else None
    ncmhip.call("layernorm_bwd", up(x), up(w), up(dy), dx, dw, db, rows, C, eps)
    assert maxrel(dx.numpy(), rdx) <= 1e-5
    if affine:
        assert maxrel(dw.numpy(), rdw) <= 1e-5 and maxrel(db.numpy(), rdb) <= 1e-5


@pytest.mark.parametrize("rows,C", [(1, 1), (29, 128), (5184, 256), (2048, 896), (45, 1024)])
@pytest.mark.parametrize("weighted", [True, False])
def test_rmsnorm_bwd(rows, C, weighted):
    x, dy = rnd(7, rows, C), rnd(8, rows, C)
    w = rnd(9, C) if weighted else None
    dx0, dw0 = rnd(10, rows, C), rnd(11, C)
    rdx, rdw = O.rmsnorm_bwd(x, w, dy, dx0, dw0, want=("dx", "dw") if weighted else ("dx",))
    dx, dw = up(dx0), up(dw0) if weighted else None
    ncmhip.call("rmsnorm_bwd", up(x), up(w), up(dy), dx, dw, rows, C)
    assert maxrel(dx.numpy(), rdx) <= 1e-5
    if weighted:
        assert maxrel(dw.numpy(), rdw) <= 1e-4


def test_norm_bwd_param_only():
    rows, C = 200, 64
    x, dy, w = rnd(12, rows, C), rnd(13, rows, C), rnd(14, C)
    _, rdw, rdb = O.layernorm_bwd(x, w, dy, want=("dw", "db"))
    dw, db = D.from_numpy(np.zeros(C, np.float32)), D.from_numpy(np.zeros(C, np.float32))
    ncmhip.call("layernorm_bwd", up(x), up(w), up(dy), None, dw, db, rows, C, 1e-6)
    assert maxrel(dw.numpy(), rdw) <= 1e-5 and maxrel(db.numpy(), rdb) <= 1e-5


# ---------------------------------------------------------------- cross-entropy
@pytest.mark.parametrize("rows,V", [(1, 16), (81, 16), (512, 4096), (37, 1000)])
@pytest.mark.parametrize("masked", [False, True])
def test_ce(rows, V, masked):
    logits = rnd(15, rows, V, scale=3.0)
    tgt = np.random.default_rng(16).integers(0, V, rows).astype(np.int32)
    wm = None
    if masked:
        wm = np.random.default_rng(17).uniform(0.5, 2.0, rows).astype(np.float32)
        wm[::3] = 0.0
        if rows == 1:
            wm[0] = 1.5
    rloss, rprobs, cnt = O.ce_fwd(logits, tgt, wm)
    dlg, dtg, dwm = up(logits), up(tgt), up(wm)
    loss, probs = D.empty(1), D.empty((rows, V))
    ncmhip.call("ce_fwd", dlg, dtg, dwm, loss, probs, rows, V)
    assert maxrel(probs.numpy(), rprobs) <= 1e-6
    assert abs(float(loss.numpy()[0]) - rloss) <= 1e-6 * (abs(rloss) + 1)
    # backward from the oracle's probs: the same float/double operations
    dl0 = rnd(18, rows, V)
    rdl = O.ce_bwd(rprobs, tgt, wm, 0.7 / cnt, dl0)
    dl = up(dl0)
    ncmhip.call("ce_bwd", up(rprobs), dtg, dwm, dl, rows, V, 0.7 / cnt)
    assert bits_equal(dl.numpy(), rdl)
    # fused forward + backward
    dl2, loss2 = up(dl0), D.empty(1)
    ncmhip.call("ce_fwd_bwd", dlg, dtg, dwm, loss2, dl2, rows, V, 0.7)
    assert np.max(np.abs(dl2.numpy() - rdl)) <= 1e-6
    assert abs(float(loss2.numpy()[0]) - rloss) <= 1e-6 * (abs(rloss) + 1)


# ---------------------------------------------------------------- optimizer
def test_adamw_bitexact_over_steps():
    n = 100003
    p, m, v = rnd(19, n) * 0.02, np.zeros(n, np.float32), np.zeros(n, np.float32)
    dp, dm, dv = up(p), up(m), up(v)
    b1, b2, eps, wd = 0.9, 0.95, 1e-8, 0.1
    for step in range(1, 4):
        g = rnd(20 + step, n)
        lr = 3e-4 * O.sched_cosine_warmup(step, 2, 10)
        b1t, b2t = 1 - b1 ** step, 1 - b2 ** step
        p, m, v = O.adamw(p, g, m, v, lr, b1, b2, b1t, b2t, eps, wd)
        ncmhip.call("adamw_update", dp, up(g), dm, dv, n, lr, b1, b2, b1t, b2t, eps, wd)
    assert bits_equal(dp.numpy(), p) and bits_equal(dm.numpy(), m) and bits_equal(dv.numpy(), v)


def test_schedule_matches_oracle():
    lib = ncmhip.load()
    for step, w, t in [(0, 100, 1000), (50, 100, 1000), (100, 100, 1000), (777, 100, 1000), (1200, 100, 1000),
                       (5, 0, 10)]:
        assert lib.sched_cosine_warmup(step, w, t) == O.sched_cosine_warmup(step, w, t)


@pytest.mark.parametrize("scale", [1.0, 1e-4])
def test_grad_clip(scale):
    gs = [rnd(30, 1000) * scale, rnd(31, 768, 3) * scale, rnd(32, 5) * scale, np.zeros(0, np.float32)]
    gn, ref = O.grad_clip(gs, 1.0)
    bufs = [D.from_numpy(g) if g.size else None for g in gs]
    ptrs = (ctypes.c_void_p * 4)(*[b.ptr if b else None for b in bufs])
    ns = (ctypes.c_int64 * 4)(*[g.size for g in gs])
    got = ncmhip.call("grad_clip_global", ptrs, ns, 4, 1.0)
    assert abs(got - gn) <= 1e-12 * gn
    for b, r in zip(bufs, ref):
        if b is not None:
            assert maxrel(b.numpy(), r) <= 2e-7


# ---------------------------------------------------------------- attention
def causal(Tq, Tkv):
    return np.where(np.arange(Tkv)[None, :] > np.arange(Tq)[:, None] + (Tkv - Tq), -1e9, 0).astype(np.float32)


@pytest.mark.parametrize("B,H,Hkv,Tq,Tkv,hd,masked", [
    (2, 12, 12, 128, 128, 64, True),    # GPT-2 heads
    (1, 14, 2, 81, 84, 64, False),
    (1, 4, 2, 81, 81, 64, True),        # NCP heads, Tkv % 4 != 0 (row kernel)
    (2, 3, 3, 17, 40, 32, True),
])
def test_sdpa_probs(B, H, Hkv, Tq, Tkv, hd, masked):
    q, k = rnd(40, B, H, Tq, hd), rnd(41, B, Hkv, Tkv, hd)
    mask = causal(Tq, Tkv) if masked else None
    ref = O.sdpa_probs(q, k, mask)
    P = D.empty(ref.shape)
    ncmhip.call("sdpa_probs_gqa", up(q), up(k), up(mask), P, B, H, Hkv, Tq, Tkv, hd)
    assert np.max(np.abs(P.numpy() - ref)) <= 1e-6


@pytest.mark.parametrize("B,H,Hkv,Tq,Tkv,hd", [
    (2, 12, 12, 256, 256, 64),          # GPT-2 heads (MFMA path)
    (1, 14, 2, 128, 128, 64),           # Qwen heads, GQA fan-in
    (1, 4, 2, 81, 81, 64),              # NCP heads: Tkv % 4 != 0 -> row kernels
    (1, 4, 4, 70, 100, 64),             # ragged tiles, Tq != Tkv
    (2, 6, 3, 33, 33, 32),              # generic head size
    (1, 2, 1, 9, 20, 128),
])
def test_sdpa_bwd(B, H, Hkv, Tq, Tkv, hd):
    q, k, v = rnd(42, B, H, Tq, hd), rnd(43, B, Hkv, Tkv, hd), rnd(44, B, Hkv, Tkv, hd)
    dO = rnd(45, B, H, Tq, hd)
    P = O.sdpa_probs(q, k, causal(Tq, Tkv))
    dq0, dk0, dv0 = rnd(46, *q.shape), rnd(47, *k.shape), rnd(48, *v.shape)
    rdq, rdk, rdv = O.sdpa_bwd(q, k, v, P, dO, dq0, dk0, dv0)
    dq, dk, dv = up(dq0), up(dk0), up(dv0)
    ncmhip.call("sdpa_bwd_gqa", up(q), up(k), up(v), up(P), up(dO), dq, dk, dv, B, H, Hkv, Tq, Tkv, hd)
    for got, ref in ((dq, rdq), (dk, rdk), (dv, rdv)):
        g = got.numpy()
        assert np.max(np.abs(g - ref)) <= 1e-4 and maxrel(g, ref) <= 1e-4


def test_sdpa_bwd_partial_outputs():
    B, H, Hkv, T, hd = 1, 4, 2, 64, 64
    q, k, v, dO = rnd(50, B, H, T, hd), rnd(51, B, Hkv, T, hd), rnd(52, B, Hkv, T, hd), rnd(53, B, H, T, hd)
    P = O.sdpa_probs(q, k, None)
    rdq, rdk, rdv = O.sdpa_bwd(q, k, v, P, dO)
    dv = D.from_numpy(np.zeros_like(v))
    ncmhip.call("sdpa_bwd_gqa", up(q), up(k), up(v), up(P), up(dO), None, None, dv, B, H, Hkv, T, T, hd)
    assert np.max(np.abs(dv.numpy() - rdv)) <= 1e-4
    dq = D.from_numpy(np.zeros_like(q))
    ncmhip.call("sdpa_bwd_gqa", up(q), up(k), up(v), up(P), up(dO), dq, None, None, B, H, Hkv, T, T, hd)
    assert np.max(np.abs(dq.numpy() - rdq)) <= 1e-4


# ---------------------------------------------------------------- remaining tape ops (bit-exact
# except the fp64 transcendentals of the activation backward: <= 1 ulp)
@pytest.mark.parametrize("name", ["gelu", "silu", "gelu_tanh"])
def test_act_bwd(name):
    x = np.concatenate([rnd(100, 100000, scale=3.0), np.array([0.0, -0.0, 20.0, -20.0], np.float32)])
    dy, dx0 = rnd(101, x.size), rnd(102, x.size)
    ref = O.act_bwd(name, x, dy, dx0)
    dx = up(dx0)
    ncmhip.call(name + "_bwd", up(x), up(dy), dx, x.size)
    got = dx.numpy()
    ulp = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert int(ulp.max()) <= 1


def test_mul_rope_embed_bwd():
    n = 4097
    a, b, dy, da0, db0 = rnd(103, n), rnd(104, n), rnd(105, n), rnd(106, n), rnd(107, n)
    rda, rdb = O.mul_bwd(a, b, dy, da0, db0)
    da, db = up(da0), up(db0)
    ncmhip.call("mul_bwd", up(a), up(b), up(dy), da, db, n)
    assert bits_equal(da.numpy(), rda) and bits_equal(db.numpy(), rdb)

    B, H, Hkv, T, hd = 2, 14, 2, 37, 64
    c, s = O.rope_tables_qwen(T, hd, 1e6)
    gq, gk, q0, k0 = rnd(108, B, H, T, hd), rnd(109, B, Hkv, T, hd), rnd(110, B, H, T, hd), rnd(111, B, Hkv, T, hd)
    dxq, dxk = up(q0), up(k0)
    ncmhip.call("rope_bwd_gqa", up(gq), up(gk), up(c), up(s), dxq, dxk, B, H, Hkv, T, hd)
    assert bits_equal(dxq.numpy(), O.rope_bwd(gq.reshape(-1, hd), c, s, T, q0.reshape(-1, hd)).reshape(q0.shape))
    assert bits_equal(dxk.numpy(), O.rope_bwd(gk.reshape(-1, hd), c, s, T, k0.reshape(-1, hd)).reshape(k0.shape))

    for V, D, nrow in [(4096, 768, 16384), (512, 768, 16384), (16, 256, 5184), (100, 5, 7)]:
        idx = np.random.default_rng(V + nrow).integers(0, V, nrow).astype(np.int32)
        dye, dW0 = rnd(112, nrow, D), rnd(113, V, D)
        dW = up(dW0)
        ncmhip.call("embedding_bwd", up(dye), idx.ctypes.data, nrow, D, dW, V)
        assert bits_equal(dW.numpy(), O.embedding_bwd(dye, idx, V, dW0))


@pytest.mark.parametrize("B,T,C,H,hd,K,rep", [(2, 33, 768, 12, 64, 12, 1), (1, 17, 896, 14, 64, 2, 7),
                                               (3, 5, 64, 4, 16, 1, 4)])
def test_split_merge_bwd(B, T, C, H, hd, K, rep):
    gq, gk, gv = rnd(114, B, H, T, hd), rnd(115, B, H, T, hd), rnd(116, B, H, T, hd)
    dx0 = rnd(117, B, T, C + 2 * K * hd)
    dx = up(dx0)
    ncmhip.call("qkv_split_bwd", up(gq), up(gk), up(gv), dx, B, T, C, H, hd, K, rep)
    assert bits_equal(dx.numpy(), O.qkv_split_bwd(gq, gk, gv, B, T, C, H, hd, K, rep, dx0))
    dy, c0 = rnd(118, B, T, C), rnd(119, B, H, T, hd)
    dc = up(c0)
    ncmhip.call("head_merge_bwd", up(dy), dc, B, T, C, H, hd)
    assert bits_equal(dc.numpy(), O.head_merge_bwd(dy, B, T, C, H, hd, c0))
    dys, x0 = rnd(120, B, H, T, hd), rnd(121, B, T, C)
    dxs = up(x0)
    ncmhip.call("heads_transpose_bwd", up(dys), dxs, B, T, C, H, hd)
    assert bits_equal(dxs.numpy(), O.heads_transpose_bwd(dys, B, T, C, H, hd, x0))


def test_layout_rows_partial_heads():
    """A qkv row whose q part is wider than H*hd (its tail unused) on the
    row-blocked layout path, with a missing q gradient.  (Merged rows are
    exactly H*hd wide: the reference's head_merge_fwd writes H*hd columns.)"""
    B, T, H, hd, K, rep = 2, 5, 4, 16, 2, 2
    C = 80
    x = rnd(130, B, T, C + 2 * K * hd)
    outs = [D.empty((B, H, T, hd)) for _ in range(3)]
    ncmhip.call("qkv_split_fwd", up(x), *outs, B, T, C, H, hd, K, rep)
    for g, r in zip(outs, O.qkv_split(x, B, T, C, H, hd, K, rep)):
        assert bits_equal(g.numpy(), r)
    gk, gv = rnd(131, B, H, T, hd), rnd(132, B, H, T, hd)
    dx0 = rnd(133, B, T, C + 2 * K * hd)
    dx = up(dx0)
    ncmhip.call("qkv_split_bwd", None, up(gk), up(gv), dx, B, T, C, H, hd, K, rep)
    assert bits_equal(dx.numpy(), O.qkv_split_bwd(None, gk, gv, B, T, C, H, hd, K, rep, dx0))


# ---------------------------------------------------------------- the tape's recomputing SDPA backward
class _PMap(ctypes.Structure):
    _fields_ = [("params", ctypes.c_void_p), ("grads", ctypes.c_void_p), ("sizes", ctypes.c_void_p),
                ("n", ctypes.c_int)]


@pytest.mark.parametrize("B,H,Hkv,Tq,Tkv,hd,kind", [
    (2, 12, 12, 512, 512, 64, "causal"),    # config 5 heads and length, the generated causal mask
    (2, 12, 12, 512, 512, 64, "mask"),      # the same with the reference's -1e9 mask read from memory
    (1, 14, 2, 100, 164, 64, "causal"),     # GQA, Tq < Tkv (bottom-right causal), ragged tiles
    (1, 4, 2, 96, 96, 64, "random"),        # an arbitrary additive mask
    (1, 4, 2, 81, 81, 64, "causal"),        # Tkv % 4 != 0: stored probabilities, as the reference
    (2, 6, 3, 33, 33, 32, "causal"),        # hd != 64: stored probabilities
])
def test_tape_sdpa_backward(B, H, Hkv, Tq, Tkv, hd, kind):
    """One SDPA record on the device tape (ncm_t_sdpa / ncm_t_sdpa_causal) and
    its backward against the oracle's restatement of t_sdpa + its backward
    case (train_tape.c:289-313, 936-1051), upstream gradient dO."""
    lib = ncmhip.load()
    q, k, v = rnd(60, B, H, Tq, hd), rnd(61, B, Hkv, Tkv, hd), rnd(62, B, Hkv, Tkv, hd)
    dO = rnd(63, B, H, Tq, hd)
    if kind == "random":
        mask = np.where(np.random.default_rng(64).random((Tq, Tkv)) < 0.3, -1e9, 0.0).astype(np.float32)
        mask[:, 0] = 0.0
    else:
        mask = causal(Tq, Tkv)
    P = O.sdpa_probs(q, k, mask)
    rdq, rdk, rdv = O.sdpa_bwd(q, k, v, P, dO)
    qd, kd, vd, od = up(q), up(k), up(v), D.empty(q.shape)
    gq, gk, gv, go = (D.from_numpy(np.zeros_like(a)) for a in (q, k, v, dO))
    go.upload(dO)
    md = up(mask)
    tape = lib.ncm_tape_new()
    try:
        if kind == "causal":
            lib.ncm_t_sdpa_causal(tape, qd.ptr, kd.ptr, vd.ptr, od.ptr, B, H, Hkv, Tq, Tkv, hd)
        else:
            lib.ncm_t_sdpa(tape, qd.ptr, kd.ptr, vd.ptr, md.ptr, od.ptr, B, H, Hkv, Tq, Tkv, hd)
        ncmhip.check()
        assert np.max(np.abs(od.numpy() - O.sdpa_gqa(q, k, v, mask))) <= 1e-5
        ptrs = (ctypes.c_void_p * 4)(od.ptr, qd.ptr, kd.ptr, vd.ptr)
        grads = (ctypes.c_void_p * 4)(go.ptr, gq.ptr, gk.ptr, gv.ptr)
        sizes = (ctypes.c_int64 * 4)(dO.size, q.size, k.size, v.size)
        pm = _PMap(ctypes.cast(ptrs, ctypes.c_void_p), ctypes.cast(grads, ctypes.c_void_p),
                   ctypes.cast(sizes, ctypes.c_void_p), 4)
        lib.ncm_tape_backward(tape, ctypes.byref(pm))
        ncmhip.check()
        for got, ref in ((gq, rdq), (gk, rdk), (gv, rdv)):
            g = got.numpy()
            assert np.max(np.abs(g - ref)) <= 1e-4 and maxrel(g, ref) <= 1e-4, (kind, float(np.max(np.abs(g - ref))))
    finally:
        lib.ncm_tape_free(tape)


# ---------------------------------------------------------------- fused linear records
@pytest.mark.parametrize("R,K,M", [(300, 96, 128), (130, 768, 3072), (6, 64, 96)])
def test_tape_fused_linear_records(R, K, M):
    """ncm_t_linear_act (the GEMM also writing the pre-activation) and
    ncm_t_linear_res (the residual summed in the GEMM epilogue, the linear
    output never stored) against the unfused records ncm_t_linear +
    ncm_t_gelu_tanh and ncm_t_linear + ncm_t_add: outputs and every gradient
    bit for bit, from one seeded output gradient.  Shapes: whole GEMM tiles,
    a split-K forward (fixup epilogue), and a batch of at most 8 (the GEMV
    path)."""
    lib = ncmhip.load()
    x, W, b, res, g = rnd(70, R, K), rnd(71, M, K), rnd(72, M), rnd(73, R, M), rnd(74, R, M)

    def run(records, outs, inputs):
        """records(tape, bufs); the seeded gradient goes to outs[-1]; returns
        the outputs and the gradients of the inputs."""
        bufs = {n: up(a) for n, a in inputs.items()}
        for n, shape in outs:
            bufs[n] = D.empty(shape)
        grads = {n: D.from_numpy(np.zeros_like(a)) for n, a in inputs.items()}
        gy = up(g)
        tape = lib.ncm_tape_new()
        try:
            records(tape, bufs)
            ncmhip.check()
            names = list(inputs) + [outs[-1][0]]
            ptrs = (ctypes.c_void_p * len(names))(*[bufs[n].ptr for n in names])
            gp = (ctypes.c_void_p * len(names))(*[grads[n].ptr for n in inputs] + [gy.ptr])
            sizes = (ctypes.c_int64 * len(names))(*[inputs[n].size for n in inputs] + [g.size])
            pm = _PMap(ctypes.cast(ptrs, ctypes.c_void_p), ctypes.cast(gp, ctypes.c_void_p),
                       ctypes.cast(sizes, ctypes.c_void_p), len(names))
            lib.ncm_tape_backward(tape, ctypes.byref(pm))
            ncmhip.check()
            return {n: bufs[n].numpy() for n, _ in outs}, {n: grads[n].numpy() for n in inputs}
        finally:
            lib.ncm_tape_free(tape)

    ins = {"x": x, "W": W, "b": b}
    o1, g1 = run(lambda t, f: (lib.ncm_t_linear(t, f["x"].ptr, f["W"].ptr, f["b"].ptr, f["pre"].ptr, R, M, K),
                               lib.ncm_t_gelu_tanh(t, f["pre"].ptr, f["y"].ptr, R * M)),
                 [("pre", (R, M)), ("y", (R, M))], ins)
    o2, g2 = run(lambda t, f: lib.ncm_t_linear_act(t, f["x"].ptr, f["W"].ptr, f["b"].ptr, f["pre"].ptr,
                                                   f["y"].ptr, R, M, K, 2),
                 [("pre", (R, M)), ("y", (R, M))], ins)
    for n in o1:
        assert bits_equal(o1[n], o2[n]), n
    for n in g1:
        assert bits_equal(g1[n], g2[n]), n
    assert np.any(g1["x"])

    ins = {"x": x, "W": W, "b": b, "res": res}
    o1, g1 = run(lambda t, f: (lib.ncm_t_linear(t, f["x"].ptr, f["W"].ptr, f["b"].ptr, f["ao"].ptr, R, M, K),
                               lib.ncm_t_add(t, f["res"].ptr, f["ao"].ptr, f["y"].ptr, R * M)),
                 [("ao", (R, M)), ("y", (R, M))], ins)
    o2, g2 = run(lambda t, f: lib.ncm_t_linear_res(t, f["x"].ptr, f["W"].ptr, f["b"].ptr, f["res"].ptr,
                                                   f["y"].ptr, R, M, K),
                 [("y", (R, M))], ins)
    assert bits_equal(o1["y"], o2["y"])
    for n in g1:
        assert bits_equal(g1[n], g2[n]), n
    assert bits_equal(g1["res"], g)


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("R,K0,K1,M", [(300, 64, 96, 128), (130, 768, 3072, 768), (33, 20, 36, 52), (6, 32, 64, 48)])
def test_tape_activation_backward_in_dx_gemm(kind, R, K0, K1, M):
    """linear -> activation -> linear on the tape: when nothing else reads the
    activation's output, the second linear's dX GEMM applies the activation
    backward in its epilogue and that gradient is never stored.  Against the
    same tape with the activation output's gradient requested (which keeps the
    two records apart): every gradient bit for bit, including the
    pre-activation's.  Shapes: whole tiles, the GPT-2 MLP widths (split-K
    fixup), ragged tiles, and a batch of at most 8 (no fusion)."""
    lib = ncmhip.load()
    x, W1, b1 = rnd(80, R, K0), rnd(81, K1, K0, scale=0.2), rnd(82, K1)
    W2, b2, g = rnd(83, M, K1, scale=0.2), rnd(84, M), rnd(85, R, M)
    act = (lib.ncm_t_gelu, lib.ncm_t_silu, lib.ncm_t_gelu_tanh)[kind]

    def run(keep_h):
        ins = {"x": x, "W1": W1, "b1": b1, "W2": W2, "b2": b2}
        bufs = {n: up(a) for n, a in ins.items()}
        pre, h, y = D.empty((R, K1)), D.empty((R, K1)), D.empty((R, M))
        grads = {n: D.from_numpy(np.zeros_like(a)) for n, a in ins.items()}
        gy, gh = up(g), D.from_numpy(np.zeros((R, K1), np.float32))
        tape = lib.ncm_tape_new()
        try:
            lib.ncm_t_linear(tape, bufs["x"].ptr, bufs["W1"].ptr, bufs["b1"].ptr, pre.ptr, R, K1, K0)
            act(tape, pre.ptr, h.ptr, R * K1)
            lib.ncm_t_linear(tape, h.ptr, bufs["W2"].ptr, bufs["b2"].ptr, y.ptr, R, M, K1)
            ncmhip.check()
            keys = [bufs[n].ptr for n in ins] + [y.ptr] + ([h.ptr] if keep_h else [])
            gps = [grads[n].ptr for n in ins] + [gy.ptr] + ([gh.ptr] if keep_h else [])
            sz = [a.size for a in ins.values()] + [g.size] + ([R * K1] if keep_h else [])
            n = len(keys)
            pm = _PMap(ctypes.cast((ctypes.c_void_p * n)(*keys), ctypes.c_void_p),
                       ctypes.cast((ctypes.c_void_p * n)(*gps), ctypes.c_void_p),
                       ctypes.cast((ctypes.c_int64 * n)(*sz), ctypes.c_void_p), n)
            lib.ncm_tape_backward(tape, ctypes.byref(pm))
            ncmhip.check()
            gpre = np.empty((R, K1), np.float32)
            lib.mem_d2h(gpre.ctypes.data, lib.ncm_tape_grad(tape, pre.ptr), gpre.nbytes)
            ncmhip.check()
            return {n: grads[n].numpy() for n in ins} | {"pre": gpre}
        finally:
            lib.ncm_tape_free(tape)

    fused, apart = run(False), run(True)
    for n in apart:
        assert bits_equal(fused[n], apart[n]), n
    assert np.any(apart["pre"]) and np.any(apart["x"])


@pytest.mark.parametrize("B,T,C,H,hd,K", [(2, 128, 128, 2, 64, 2), (3, 64, 192, 3, 64, 3), (2, 192, 256, 4, 64, 2),
                                          (2, 70, 128, 2, 64, 2), (2, 40, 128, 4, 32, 4), (1, 6, 128, 2, 64, 2)])
def test_tape_qkv_projection_to_heads(B, T, C, H, hd, K):
    """ncm_t_linear_qkvsplit (the c_attn GEMM storing q, k, v in the
    attention's head-major layout from its epilogue) against ncm_t_linear +
    ncm_t_qkvsplit: q, k, v and the gradients of x, W and b bit for bit, from
    seeded q, k, v gradients.  Shapes: sequences of 128 and 64 tokens (every
    tile one [64 t][64 d] block of q, k or v), and the fallbacks (GQA, whose
    split repeats each kv head for its query heads; T = 70, whose tiles would
    span two sequences; hd 32; 6 rows).  q, k and v are [B][H][T][hd]."""
    lib = ncmhip.load()
    R, N = B * T, C + 2 * K * hd
    x, W, b = rnd(90, R, C), rnd(91, N, C, scale=0.1), rnd(92, N)
    gq, gk, gv = rnd(93, B, H, T, hd), rnd(94, B, H, T, hd), rnd(95, B, H, T, hd)

    def run(fused):
        ins = {"x": x, "W": W, "b": b}
        bufs = {n: up(a) for n, a in ins.items()}
        qkv, qq, kk, vv = D.empty((R, N)), D.empty((B, H, T, hd)), D.empty((B, H, T, hd)), D.empty((B, H, T, hd))
        grads = {n: D.from_numpy(np.zeros_like(a)) for n, a in ins.items()}
        gbuf = [up(gq), up(gk), up(gv)]
        tape = lib.ncm_tape_new()
        try:
            if fused:
                lib.ncm_t_linear_qkvsplit(tape, bufs["x"].ptr, bufs["W"].ptr, bufs["b"].ptr, qkv.ptr, qq.ptr, kk.ptr,
                                          vv.ptr, B, T, C, H, hd, K, H // K)
            else:
                lib.ncm_t_linear(tape, bufs["x"].ptr, bufs["W"].ptr, bufs["b"].ptr, qkv.ptr, R, N, C)
                lib.ncm_t_qkvsplit(tape, qkv.ptr, qq.ptr, kk.ptr, vv.ptr, B, T, C, H, hd, K, H // K)
            ncmhip.check()
            keys = [bufs[n].ptr for n in ins] + [qq.ptr, kk.ptr, vv.ptr]
            gps = [grads[n].ptr for n in ins] + [g.ptr for g in gbuf]
            sz = [a.size for a in ins.values()] + [gq.size, gk.size, gv.size]
            n = len(keys)
            pm = _PMap(ctypes.cast((ctypes.c_void_p * n)(*keys), ctypes.c_void_p),
                       ctypes.cast((ctypes.c_void_p * n)(*gps), ctypes.c_void_p),
                       ctypes.cast((ctypes.c_int64 * n)(*sz), ctypes.c_void_p), n)
            lib.ncm_tape_backward(tape, ctypes.byref(pm))
            ncmhip.check()
            return [qq.numpy(), kk.numpy(), vv.numpy()], {n: grads[n].numpy() for n in ins}
        finally:
            lib.ncm_tape_free(tape)

    (o1, g1), (o2, g2) = run(False), run(True)
    for a, c in zip(o1, o2):
        assert bits_equal(a, c)
    for n in g1:
        assert bits_equal(g1[n], g2[n]), n
    assert np.any(o1[0]) and np.any(g1["x"])


@pytest.mark.parametrize("B,T,C,H,causal", [(2, 128, 128, 2, 1), (2, 96, 192, 3, 0), (1, 70, 128, 2, 1)])
def test_tape_attention_gradients_into_qkv_rows(B, T, C, H, causal):
    """split -> attention on the tape with nothing else reading q, k and v:
    the attention's backward writes its gradients straight into the qkv rows'
    gradient (the split's backward is skipped).  Against the same tape with
    q's gradient requested, which keeps the two records apart: the gradients
    of x, W and b bit for bit (ctx's gradient seeded)."""
    lib = ncmhip.load()
    hd, R = 64, B * T
    N = 3 * C
    x, W, b = rnd(100, R, C), rnd(101, N, C, scale=0.1), rnd(102, N)
    g = rnd(103, B, H, T, hd)
    mask = np.where(np.arange(T)[None, :] <= np.arange(T)[:, None], 0.0, -1e9).astype(np.float32)

    def run(keep_q):
        ins = {"x": x, "W": W, "b": b}
        bufs = {n: up(a) for n, a in ins.items()}
        qkv, qq, kk, vv, ctx = (D.empty((R, N)), D.empty((B, H, T, hd)), D.empty((B, H, T, hd)),
                                D.empty((B, H, T, hd)), D.empty((B, H, T, hd)))
        md = up(mask)
        grads = {n: D.from_numpy(np.zeros_like(a)) for n, a in ins.items()}
        gctx, gqb = up(g), D.from_numpy(np.zeros((B, H, T, hd), np.float32))
        tape = lib.ncm_tape_new()
        try:
            lib.ncm_t_linear(tape, bufs["x"].ptr, bufs["W"].ptr, bufs["b"].ptr, qkv.ptr, R, N, C)
            lib.ncm_t_qkvsplit(tape, qkv.ptr, qq.ptr, kk.ptr, vv.ptr, B, T, C, H, hd, H, 1)
            if causal:
                lib.ncm_t_sdpa_causal(tape, qq.ptr, kk.ptr, vv.ptr, ctx.ptr, B, H, H, T, T, hd)
            else:
                lib.ncm_t_sdpa(tape, qq.ptr, kk.ptr, vv.ptr, md.ptr, ctx.ptr, B, H, H, T, T, hd)
            ncmhip.check()
            keys = [bufs[n].ptr for n in ins] + [ctx.ptr] + ([qq.ptr] if keep_q else [])
            gps = [grads[n].ptr for n in ins] + [gctx.ptr] + ([gqb.ptr] if keep_q else [])
            sz = [a.size for a in ins.values()] + [g.size] + ([g.size] if keep_q else [])
            n = len(keys)
            pm = _PMap(ctypes.cast((ctypes.c_void_p * n)(*keys), ctypes.c_void_p),
                       ctypes.cast((ctypes.c_void_p * n)(*gps), ctypes.c_void_p),
                       ctypes.cast((ctypes.c_int64 * n)(*sz), ctypes.c_void_p), n)
            lib.ncm_tape_backward(tape, ctypes.byref(pm))
            ncmhip.check()
            return {n: grads[n].numpy() for n in ins}
        finally:
            lib.ncm_tape_free(tape)

    fused, apart = run(False), run(True)
    for n in apart:
        assert bits_equal(fused[n], apart[n]), n
    assert np.any(apart["x"])


@pytest.mark.parametrize("B,T,H,M", [(2, 128, 2, 96), (3, 64, 4, 256), (1, 70, 2, 64)])
def test_tape_merge_then_linear_dx_to_heads(B, T, H, M):
    """head merge -> linear on the tape with nothing else reading the merged
    rows: the linear's dX GEMM writes the heads' gradient directly (the merge's
    backward is skipped).  Against the same tape with the merged rows'
    gradient requested (which keeps the records apart): the gradients of ctx,
    W and b bit for bit.  T = 70: rows of a tile in two sequences (no fusion)."""
    lib = ncmhip.load()
    hd, R, C = 64, B * T, 64 * H
    ctx, W, b, g = rnd(110, B, H, T, hd), rnd(111, M, C, scale=0.1), rnd(112, M), rnd(113, R, M)

    def run(keep_mo):
        ins = {"ctx": ctx, "W": W, "b": b}
        bufs = {n: up(a) for n, a in ins.items()}
        mo, y = D.empty((R, C)), D.empty((R, M))
        grads = {n: D.from_numpy(np.zeros_like(a)) for n, a in ins.items()}
        gy, gmo = up(g), D.from_numpy(np.zeros((R, C), np.float32))
        tape = lib.ncm_tape_new()
        try:
            lib.ncm_t_headmerge(tape, bufs["ctx"].ptr, mo.ptr, B, T, C, H, hd)
            lib.ncm_t_linear(tape, mo.ptr, bufs["W"].ptr, bufs["b"].ptr, y.ptr, R, M, C)
            ncmhip.check()
            keys = [bufs[n].ptr for n in ins] + [y.ptr] + ([mo.ptr] if keep_mo else [])
            gps = [grads[n].ptr for n in ins] + [gy.ptr] + ([gmo.ptr] if keep_mo else [])
            sz = [a.size for a in ins.values()] + [g.size] + ([R * C] if keep_mo else [])
            n = len(keys)
            pm = _PMap(ctypes.cast((ctypes.c_void_p * n)(*keys), ctypes.c_void_p),
                       ctypes.cast((ctypes.c_void_p * n)(*gps), ctypes.c_void_p),
                       ctypes.cast((ctypes.c_int64 * n)(*sz), ctypes.c_void_p), n)
            lib.ncm_tape_backward(tape, ctypes.byref(pm))
            ncmhip.check()
            return {n: grads[n].numpy() for n in ins}
        finally:
            lib.ncm_tape_free(tape)

    fused, apart = run(False), run(True)
    for n in apart:
        assert bits_equal(fused[n], apart[n]), n
    assert np.any(apart["ctx"])


@pytest.mark.parametrize("B,H,T", [(2, 3, 128), (1, 4, 100), (2, 2, 36)])
def test_tape_attention_writing_merged_rows(B, H, T):
    """ncm_t_sdpa_causal_merge (the attention writing the merged rows itself,
    its backward reading them as O) against ncm_t_sdpa_causal +
    ncm_t_headmerge: the merged output and the q, k, v gradients bit for bit
    from a seeded gradient of the merged rows."""
    lib = ncmhip.load()
    hd = 64
    q, k, v, g = rnd(120, B, H, T, hd), rnd(121, B, H, T, hd), rnd(122, B, H, T, hd), rnd(123, B * T, H * hd)

    def run(fused):
        ins = {"q": q, "k": k, "v": v}
        bufs = {n: up(a) for n, a in ins.items()}
        ctx, mo = D.empty((B, H, T, hd)), D.empty((B * T, H * hd))
        grads = {n: D.from_numpy(np.zeros_like(a)) for n, a in ins.items()}
        gmo = up(g)
        tape = lib.ncm_tape_new()
        try:
            if fused:
                lib.ncm_t_sdpa_causal_merge(tape, bufs["q"].ptr, bufs["k"].ptr, bufs["v"].ptr, ctx.ptr, mo.ptr, B, H,
                                            H, T, hd)
            else:
                lib.ncm_t_sdpa_causal(tape, bufs["q"].ptr, bufs["k"].ptr, bufs["v"].ptr, ctx.ptr, B, H, H, T, T, hd)
                lib.ncm_t_headmerge(tape, ctx.ptr, mo.ptr, B, T, H * hd, H, hd)
            ncmhip.check()
            keys = [bufs[n].ptr for n in ins] + [mo.ptr]
            gps = [grads[n].ptr for n in ins] + [gmo.ptr]
            sz = [a.size for a in ins.values()] + [g.size]
            n = len(keys)
            pm = _PMap(ctypes.cast((ctypes.c_void_p * n)(*keys), ctypes.c_void_p),
                       ctypes.cast((ctypes.c_void_p * n)(*gps), ctypes.c_void_p),
                       ctypes.cast((ctypes.c_int64 * n)(*sz), ctypes.c_void_p), n)
            lib.ncm_tape_backward(tape, ctypes.byref(pm))
            ncmhip.check()
            return mo.numpy(), {n: grads[n].numpy() for n in ins}
        finally:
            lib.ncm_tape_free(tape)

    (o1, g1), (o2, g2) = run(False), run(True)
    assert bits_equal(o1, o2)
    for n in g1:
        assert bits_equal(g1[n], g2[n]), n
    assert np.any(g1["q"])


@pytest.mark.parametrize("norm", ["ln", "rms"])
@pytest.mark.parametrize("R,C", [(300, 128), (130, 768), (33, 52), (7, 1040)])
@pytest.mark.parametrize("shape", ["read", "unread", "shared"])
def test_tape_residual_gradient_into_norm(norm, R, C, shape):
    """The residual gradient of ncm_t_linear_res whose next reader (backward
    order) is the norm of that residual: its first write is folded into the
    norm's dX pass.  Against ncm_t_linear + ncm_t_add (two operands, never
    deferred): output and every gradient bit for bit.  s = 1.5 x is the
    residual (an intermediate, so its gradient is new at the add).  Shapes:
    the norm output feeding the linear ("read"), the norm output unread (the
    norm record is skipped and still owes the write), s also scaled into the
    linear's input between the norm and the add ("shared": no deferral).
    C 52 and 1040 take the unfused norm backward."""
    lib = ncmhip.load()
    x, W, b = rnd(130, R, C), rnd(131, C, C), rnd(132, C)
    lw, lb, x2, g = rnd(133, C) + 1.0, rnd(134, C), rnd(135, R, C), rnd(136, R, C)

    def run(fused):
        ins = {"x": x, "W": W, "b": b, "lw": lw, "x2": x2}
        if norm == "ln":
            ins["lb"] = lb
        bufs = {n: up(a) for n, a in ins.items()}
        s, h, t2, ao, y = (D.empty((R, C)) for _ in range(5))
        grads = {n: D.from_numpy(np.zeros_like(a)) for n, a in ins.items()}
        gy = up(g)
        tape = lib.ncm_tape_new()
        try:
            lib.ncm_t_scale(tape, bufs["x"].ptr, 1.5, s.ptr, R * C)
            if norm == "ln":
                lib.ncm_t_layernorm(tape, s.ptr, bufs["lw"].ptr, bufs["lb"].ptr, h.ptr, R, C)
            else:
                lib.ncm_t_rmsnorm(tape, s.ptr, bufs["lw"].ptr, h.ptr, R, C)
            if shape == "read":
                lin_in = h
            elif shape == "unread":
                lin_in = bufs["x2"]
            else:
                lib.ncm_t_scale(tape, s.ptr, 0.5, t2.ptr, R * C)
                lib.ncm_t_add(tape, h.ptr, t2.ptr, ao.ptr, R * C)
                lin_in = ao
                ao = D.empty((R, C))
            if fused:
                lib.ncm_t_linear_res(tape, lin_in.ptr, bufs["W"].ptr, bufs["b"].ptr, s.ptr, y.ptr, R, C, C)
            else:
                lib.ncm_t_linear(tape, lin_in.ptr, bufs["W"].ptr, bufs["b"].ptr, ao.ptr, R, C, C)
                lib.ncm_t_add(tape, s.ptr, ao.ptr, y.ptr, R * C)
            ncmhip.check()
            keys = [bufs[n].ptr for n in ins] + [y.ptr]
            gps = [grads[n].ptr for n in ins] + [gy.ptr]
            sz = [a.size for a in ins.values()] + [g.size]
            n = len(keys)
            pm = _PMap(ctypes.cast((ctypes.c_void_p * n)(*keys), ctypes.c_void_p),
                       ctypes.cast((ctypes.c_void_p * n)(*gps), ctypes.c_void_p),
                       ctypes.cast((ctypes.c_int64 * n)(*sz), ctypes.c_void_p), n)
            lib.ncm_tape_backward(tape, ctypes.byref(pm))
            ncmhip.check()
            return y.numpy(), {n: grads[n].numpy() for n in ins}
        finally:
            lib.ncm_tape_free(tape)

    (o1, g1), (o2, g2) = run(False), run(True)
    assert bits_equal(o1, o2)
    for n in g1:
        assert bits_equal(g1[n], g2[n]), n
    assert np.any(g1["x"]) and np.any(g1["W"])
