"""Config 5 end to end: the device tape running the taped GPT-2 step of
train_gpt2.c (forward, mean CE, backward, clip, AdamW) against the oracle's
restatement of the same step (bit-identical to the reference's own tape on
the CPU).  Bar: the north-star gradient bar max-abs 1e-3, asserted here as
max-abs 2e-5 and relative L2 error 1e-4 per parameter tensor.  Updated
parameters: AdamW divides each coordinate by its own gradient scale, so a
coordinate whose gradient is near eps = 1e-8 turns fp32 rounding of that
gradient into a visible share of its step; the bar is therefore stated on
the update: max-abs difference <= 2% of the summed learning rate and
relative L2 error of the total update <= 1e-3.  The key slice of
attn.c_attn.bias is left out of the L2 check: its true gradient is exactly
zero (a bias on every key shifts all of a query's scores by the same amount,
which softmax ignores), so both sides feed pure rounding noise to Adam."""
import ctypes

import numpy as np
import pytest

import ncmhip
import oracle as O

pytestmark = pytest.mark.gpu
D = ncmhip.DeviceBuffer


@pytest.fixture(scope="module", autouse=True)
def device():
    ncmhip.init(0)
    ncmhip.load().arena_init(4 << 30)
    ncmhip.check()
    print("[gpu] gpt2 tests on device 0", flush=True)


def case(seed, n_layer, C, H, V, npos, B, T):
    rng = np.random.default_rng(seed)
    shapes = O.gpt2_shapes(n_layer, C, V, npos)
    params = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in shapes]
    for i, s in enumerate(shapes):
        if len(s) == 1 and s[0] == C and (i >= len(params) - 2 or (i - 2) % 12 in (0, 6)):
            params[i] += 1.0
    return params, rng.integers(0, V, (B, T)).astype(np.int32), rng.integers(0, V, (B, T)).astype(np.int32)


def close(got, ref):
    err = float(np.max(np.abs(got - ref))) if ref.size else 0.0
    rel = float(np.linalg.norm((got - ref).ravel()) / max(np.linalg.norm(ref.ravel()), 1e-30))
    return err <= 2e-5 and rel <= 1e-4, (err, rel)


class PMap(ctypes.Structure):
    """NcmPMap {float **params; float **grads; int64_t *sizes; int n}"""
    _fields_ = [("params", ctypes.c_void_p), ("grads", ctypes.c_void_p), ("sizes", ctypes.c_void_p),
                ("n", ctypes.c_int)]

    def __init__(self, p, g, s, n):
        self._keep = (p, g, s)
        super().__init__(ctypes.cast(p, ctypes.c_void_p), ctypes.cast(g, ctypes.c_void_p),
                         ctypes.cast(s, ctypes.c_void_p), n)


CASES = [(2, 768, 12, 4096, 512, 2, 128),     # C5 widths, 2 layers, MFMA attention
         (1, 64, 4, 50, 16, 2, 9)]            # ragged: row attention kernels


@pytest.mark.parametrize("n_layer,C,H,V,npos,B,T", CASES)
def test_gpt2_grads(n_layer, C, H, V, npos, B, T):
    lib = ncmhip.load()
    params, ids, tgt = case(11, n_layer, C, H, V, npos, B, T)
    rloss, rgrads = O.gpt2_grads(params, n_layer, C, H, V, npos, ids, tgt)
    cfg = ncmhip.Gpt2Config(n_layer, C, H, V, npos)
    P = [D.from_numpy(p) for p in params]
    G = [D.from_numpy(np.zeros_like(p)) for p in params]
    tape = lib.ncm_tape_new()
    try:
        lib.arena_reset()
        logits = lib.ncm_gpt2_forward(tape, ctypes.byref(cfg), ncmhip.ptr_array(P), ids.ctypes.data, B, T)
        ncmhip.check()
        loss = D.empty(1)
        lib.ncm_t_ce(tape, logits, tgt.ctypes.data, None, loss.ptr, None, B * T, V, 1.0)
        sizes = (ctypes.c_int64 * len(P))(*[p.size for p in params])
        pmap = PMap(ncmhip.ptr_array(P), ncmhip.ptr_array(G), sizes, len(P))
        lib.ncm_tape_backward(tape, ctypes.byref(pmap))
        ncmhip.check()
        assert abs(float(loss.numpy()[0]) - rloss) <= 1e-5 * abs(rloss)
        for i, (g, r) in enumerate(zip(G, rgrads)):
            ok, why = close(g.numpy(), r)
            assert ok, (i, why)
    finally:
        lib.ncm_tape_free(tape)


@pytest.mark.parametrize("n_layer,C,H,V,npos,B,T", CASES)
def test_gpt2_grads_reused_tape(n_layer, C, H, V, npos, B, T):
    """The backward writes most activation gradients instead of accumulating
    them into cleared buffers, and reuses those buffers across steps: a step
    on other ids in between must not leak into the next step's gradients
    (bit for bit equal to the first run on the same ids)."""
    lib = ncmhip.load()
    params, ids, tgt = case(13, n_layer, C, H, V, npos, B, T)
    _, ids2, tgt2 = case(14, n_layer, C, H, V, npos, B, T)
    cfg = ncmhip.Gpt2Config(n_layer, C, H, V, npos)
    P = [D.from_numpy(p) for p in params]
    sizes = (ctypes.c_int64 * len(P))(*[p.size for p in params])
    tape = lib.ncm_tape_new()
    try:
        runs = []
        for x, y in ((ids, tgt), (ids2, tgt2), (ids, tgt)):
            G = [D.from_numpy(np.zeros_like(p)) for p in params]
            lib.ncm_tape_clear(tape)
            lib.arena_reset()
            logits = lib.ncm_gpt2_forward(tape, ctypes.byref(cfg), ncmhip.ptr_array(P), x.ctypes.data, B, T)
            loss = D.empty(1)
            lib.ncm_t_ce(tape, logits, y.ctypes.data, None, loss.ptr, None, B * T, V, 1.0)
            lib.ncm_tape_backward(tape, ctypes.byref(PMap(ncmhip.ptr_array(P), ncmhip.ptr_array(G), sizes, len(P))))
            ncmhip.check()
            runs.append([g.numpy() for g in G])
        for i, (a, c) in enumerate(zip(runs[0], runs[2])):
            assert np.array_equal(a.view(np.uint32), c.view(np.uint32)), i
        assert any(not np.array_equal(a, b) for a, b in zip(runs[0], runs[1]))
    finally:
        lib.ncm_tape_free(tape)


def test_gpt2_train_steps():
    lib = ncmhip.load()
    n_layer, C, H, V, npos, B, T = 1, 256, 4, 512, 64, 2, 64
    params, ids, tgt = case(12, n_layer, C, H, V, npos, B, T)
    cfg = ncmhip.Gpt2Config(n_layer, C, H, V, npos)
    P = [D.from_numpy(p) for p in params]
    G = [D.from_numpy(np.zeros_like(p)) for p in params]
    M = [D.from_numpy(np.zeros_like(p)) for p in params]
    Vm = [D.from_numpy(np.zeros_like(p)) for p in params]
    p_ref = [p.copy() for p in params]
    m_ref = [np.zeros_like(p) for p in params]
    v_ref = [np.zeros_like(p) for p in params]
    tape = lib.ncm_tape_new()
    gn = ctypes.c_double()
    try:
        for step in (1, 2):
            loss = lib.ncm_gpt2_train_step(tape, ctypes.byref(cfg), ncmhip.ptr_array(P), ncmhip.ptr_array(G),
                                           ncmhip.ptr_array(M), ncmhip.ptr_array(Vm), ids.ctypes.data,
                                           tgt.ctypes.data, B, T, step, 3e-4, 1.0, 10.0, 0.1, ctypes.byref(gn))
            ncmhip.check()
            rloss, rg = O.gpt2_grads(p_ref, n_layer, C, H, V, npos, ids, tgt)
            rgn, rg = O.grad_clip(rg, 1.0)
            assert abs(loss - rloss) <= 1e-5 * abs(rloss) and abs(gn.value - rgn) <= 1e-4 * rgn
            lr = 3e-4 * O.sched_cosine_warmup(step, 1.0, 10.0)
            b1t, b2t = 1 - 0.9 ** step, 1 - 0.95 ** step
            for i in range(len(p_ref)):
                p_ref[i], m_ref[i], v_ref[i] = O.adamw(p_ref[i], rg[i], m_ref[i], v_ref[i], lr, 0.9, 0.95, b1t, b2t,
                                                       1e-8, 0.1)
        lr_sum = sum(3e-4 * O.sched_cosine_warmup(s, 1.0, 10.0) for s in (1, 2))
        for i, (p, r, p0) in enumerate(zip(P, p_ref, params)):
            got = p.numpy()
            assert float(np.max(np.abs(got - r))) <= 0.02 * lr_sum, i
            du, dr = (got - p0).astype(np.float64), (r - p0).astype(np.float64)
            if i >= 2 and i < len(P) - 2 and (i - 2) % 12 == 3:
                du, dr = np.delete(du, np.s_[C:2 * C]), np.delete(dr, np.s_[C:2 * C])
            assert np.linalg.norm((du - dr).ravel()) <= 1e-3 * np.linalg.norm(dr.ravel()), i
        assert all(not g.numpy().any() for g in G)   # gradients zeroed after the update
    finally:
        lib.ncm_tape_free(tape)
