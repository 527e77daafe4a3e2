"""The full multiscale quantizer on the device (vq_load + vq_z_to_idx +
vq_idx_to_zhats over device tensors) against the oracle restatement of
src/vq.c, which is pinned to the reference's own functions: codes, z_hat,
z_rest and every level's z_hat bit for bit."""
import ctypes

import numpy as np
import pytest

import ncmhip
import oracle as O
from conftest import bits_equal
from vqfull_cases import CASES, make_case, ncm_config, ref_vq, weight_store

pytestmark = pytest.mark.gpu
D_ = ncmhip.DeviceBuffer


@pytest.fixture(scope="module", autouse=True)
def device():
    ncmhip.init(0)
    print("[gpu] full quantizer tests on device 0", flush=True)


class DevVq:
    """vq_load over a WeightStore of device tensors built here."""

    def __init__(self, cfg, w):
        self.lib = ncmhip.load()
        self.bufs, tens = [], []
        for k, a in w.items():
            b = D_.from_numpy(np.ascontiguousarray(a, np.float32))
            t = ncmhip.TensorS()
            t.data = b.ptr
            for i, s in enumerate(a.shape):
                t.shape[i] = s
            t.ndim, t.n = a.ndim, a.size
            self.bufs.append(b)
            tens.append((k, t))
        self.tens = tens
        self.ws, self.items = weight_store(tens)
        self.cfg = ncm_config(cfg)
        self.vq = self.lib.vq_load(ctypes.byref(self.cfg), ctypes.byref(self.ws), b"")
        ncmhip.check()
        n = cfg["n_qlevels"]
        self.n, self.L, self.D, self.total = n, cfg["levels"][n - 1], cfg["vq_embed_dim"], sum(cfg["levels"][:n])

    def z_to_idx(self, z, B):
        zd = D_.from_numpy(z)
        idx = D_.empty((B, self.total), np.int32)
        zh, zr = D_.empty((B, self.L, self.D)), D_.empty((B, self.L, self.D))
        self.lib.vq_z_to_idx_dev(self.vq, zd.ptr, B, idx.ptr, zh.ptr, zr.ptr)
        ncmhip.check()
        host = np.zeros((B, self.total), np.int32)
        self.lib.vq_z_to_idx(self.vq, zd.ptr, B, host.ctypes.data)   # the drop-in: host codes
        ncmhip.check()
        return idx.numpy(), zh.numpy(), zr.numpy(), host

    def zhats(self, idx, B):
        outs = [D_.empty((B, self.L, self.D)) for _ in range(self.n)]
        ptrs = (ctypes.c_void_p * self.n)(*[o.ptr for o in outs])
        idx = np.ascontiguousarray(idx, np.int32)
        self.lib.vq_idx_to_zhats(self.vq, idx.ctypes.data, B, ptrs)
        ncmhip.check()
        return np.stack([o.numpy() for o in outs])

    def next_input(self, codes, level, z_hat, B, nlen):
        zd = D_.from_numpy(np.ascontiguousarray(z_hat, np.float32))
        x = D_.empty((B, nlen, self.D))
        codes = np.ascontiguousarray(codes, np.int32)
        self.lib.vq_next_input(self.vq, codes.ctypes.data, level, zd.ptr, x.ptr, B)
        ncmhip.check()
        return zd.numpy(), x.numpy()

    def ncm_input(self, idx, B):
        T = self.total - self.lib.vq_level_len(self.vq, 0)
        x = D_.empty((B, max(T, 1), self.D))
        idx = np.ascontiguousarray(idx, np.int32)
        self.lib.vq_idx_to_ncm_input(self.vq, idx.ctypes.data, B, x.ptr)
        ncmhip.check()
        return x.numpy()[:, :T]

    def close(self):
        self.lib.vq_free(self.vq)


@pytest.mark.parametrize("name,kw", CASES, ids=[c[0] for c in CASES])
def test_matches_oracle(name, kw):
    cfg, w, z = make_case(7, **kw)
    B = kw["B"]
    print(f"[gpu] vqfull case {name}", flush=True)
    want_idx, want_zh, want_zr = O.vq_z_to_idx(cfg, w, z, B)
    q = DevVq(cfg, w)
    try:
        assert q.lib.vq_total_codes(q.vq) == q.total and q.lib.vq_Ltotal(q.vq) == q.L
        assert q.lib.vq_nlevels(q.vq) == q.n and q.lib.vq_Ddim(q.vq) == q.D
        idx, zh, zr, host = q.z_to_idx(z, B)
        assert np.array_equal(idx, want_idx) and np.array_equal(host, want_idx)
        assert bits_equal(zh, want_zh) and bits_equal(zr, want_zr)
        assert bits_equal(q.zhats(idx, B), O.vq_idx_to_zhats(cfg, w, idx, B))
    finally:
        q.close()


def test_larger_case_with_phi():
    # 8192 rows of D = 256, five levels 1..16, 1024 codes, partially shared Phi
    cfg, w, z = make_case(11, B=512, levels=[1, 2, 4, 8, 16], V=1024, D=256, phi=4, ratio=0.5)
    print("[gpu] vqfull larger case", flush=True)
    want_idx, want_zh, want_zr = O.vq_z_to_idx(cfg, w, z, 512)
    q = DevVq(cfg, w)
    try:
        idx, zh, zr, host = q.z_to_idx(z, 512)
        assert np.array_equal(idx, want_idx)
        assert bits_equal(zh, want_zh) and bits_equal(zr, want_zr)
    finally:
        q.close()


def test_zero_sequences_and_negative_zero_bias():
    """All-zero sequences through convs whose biases hold -0.0: a conv output
    that ends exactly at zero keeps the reference's sign (the kernel's
    fallback path for chains ending at +-0)."""
    cfg, w, z = make_case(13, B=3, levels=[1, 2, 4, 8, 16], V=32, D=32, phi=1, ratio=0.5, refine=(2,))
    z[1] = 0.0
    for name in ("quant_resi.0.bias", "learned_down_refine.2.bias", "learned_up_refine.2.bias"):
        b = w[name].copy()
        b[::3] = -0.0
        b[1::3] = 0.0
        w[name] = b
    want_idx, want_zh, want_zr = O.vq_z_to_idx(cfg, w, z, 3)
    q = DevVq(cfg, w)
    try:
        idx, zh, zr, host = q.z_to_idx(z, 3)
        assert np.array_equal(idx, want_idx)
        assert bits_equal(zh, want_zh) and bits_equal(zr, want_zr)
        assert bits_equal(q.zhats(idx, 3), O.vq_idx_to_zhats(cfg, w, idx, 3))
    finally:
        q.close()


@pytest.mark.parametrize("name,kw", CASES, ids=[c[0] for c in CASES])
def test_next_input_and_ncm_input_match_oracle(name, kw):
    """vq_next_input threaded through the levels and vq_idx_to_ncm_input, over
    the oracle's codes, bit for bit."""
    cfg, w, z = make_case(7, **kw)
    B = kw["B"]
    print(f"[gpu] vq inputs case {name}", flush=True)
    idx, _, _ = O.vq_z_to_idx(cfg, w, z, B)
    q = DevVq(cfg, w)
    try:
        assert bits_equal(q.ncm_input(idx, B), O.vq_idx_to_ncm_input(cfg, w, idx, B))
        zh, zh_dev, base = np.zeros_like(z), np.zeros_like(z), 0
        for lv in range(q.n - 1):
            tl, nlen = cfg["levels"][lv], cfg["levels"][lv + 1]
            codes = idx[:, base:base + tl]
            zh, xn = O.vq_next_input(cfg, w, codes, lv, zh, B)
            zh_dev, xn_dev = q.next_input(codes, lv, zh_dev, B, nlen)
            assert bits_equal(zh_dev, zh) and bits_equal(xn_dev, xn)
            base += tl
    finally:
        q.close()


def test_next_input_refuses_the_last_level():
    cfg, w, z = make_case(3, B=2, levels=[1, 4, 16], V=8, D=16)
    q = DevVq(cfg, w)
    try:
        with pytest.raises(ncmhip.NcmError, match="vq_next_input"):
            q.next_input(np.zeros((2, 16), np.int32), 2, z, 2, 16)
    finally:
        q.close()


@pytest.mark.parametrize("name,kw", [CASES[0], CASES[2], CASES[5], CASES[8]],
                         ids=[CASES[i][0] for i in (0, 2, 5, 8)])
@pytest.mark.parametrize("soft_levels,tau", [(2, 0.5), (5, 0.05), (9, 2.0), (0, 0.5)])
def test_soft_assignment_matches_oracle(name, kw, soft_levels, tau):
    """vq_z_to_idx_soft (vq.c:388-437) through the drop-in entry point: codes
    and the rng state after equal to the oracle's (which equals the
    reference's own from the same seed).  soft_levels 0 is vq_z_to_idx with
    the rng untouched."""
    cfg, w, z = make_case(7, **kw)
    B, seed = kw["B"], 0x9E3779B97F4A7C15
    print(f"[gpu] vq soft case {name} levels {soft_levels} tau {tau}", flush=True)
    want_idx, _, _, want_rng = O.vq_z_to_idx_soft(cfg, w, z, B, soft_levels, tau, seed)
    q = DevVq(cfg, w)
    try:
        zd = D_.from_numpy(z)
        idx = np.zeros((B, q.total), np.int32)
        rng = ctypes.c_ulonglong(seed)
        q.lib.vq_z_to_idx_soft(q.vq, zd.ptr, B, idx.ctypes.data, soft_levels, tau, ctypes.byref(rng))
        ncmhip.check()
        assert np.array_equal(idx, want_idx)
        assert rng.value == want_rng
        if soft_levels == 0:
            assert rng.value == seed and np.array_equal(idx, O.vq_z_to_idx(cfg, w, z, B)[0])
    finally:
        q.close()


def test_soft_assignment_larger_rows():
    """2048 rows at the last level, 512 codes: every row drawn on the device,
    the same codes and rng state as the oracle."""
    cfg, w, z = make_case(11, B=128, levels=[1, 2, 4, 8, 16], V=512, D=64)
    seed = 88172645463325252
    print("[gpu] vq soft larger case", flush=True)
    want_idx, _, _, want_rng = O.vq_z_to_idx_soft(cfg, w, z, 128, 5, 0.3, seed)
    q = DevVq(cfg, w)
    try:
        zd = D_.from_numpy(z)
        idx = np.zeros((128, q.total), np.int32)
        rng = ctypes.c_ulonglong(seed)
        q.lib.vq_z_to_idx_soft(q.vq, zd.ptr, 128, idx.ctypes.data, 5, 0.3, ctypes.byref(rng))
        ncmhip.check()
        assert np.array_equal(idx, want_idx) and rng.value == want_rng
    finally:
        q.close()


@pytest.mark.parametrize("name,kw", [CASES[0], CASES[1], CASES[3], CASES[5], CASES[8]],
                         ids=[CASES[i][0] for i in (0, 1, 3, 5, 8)])
def test_ema_update_matches_oracle(name, kw):
    """vq_ema_update (vq.c:677-790) twice in a row through the drop-in entry
    point: every codebook the state was loaded with, rewritten in place, bit
    for bit with the oracle's (which equals the reference's own); the codes
    are the argmin codes of the same input."""
    cfg, w, z = make_case(7, **kw)
    B = kw["B"]
    print(f"[gpu] vq ema case {name}", flush=True)
    idx, _, _ = O.vq_z_to_idx(cfg, w, z, B)
    want, _, _ = O.vq_ema_update(cfg, w, z, idx, B, 0.9, 1e-5, steps=2)
    q = DevVq(cfg, w)
    try:
        zd = D_.from_numpy(z)
        codes = np.ascontiguousarray(idx, np.int32)
        for _ in range(2):
            q.lib.vq_ema_update(q.vq, zd.ptr, codes.ctypes.data, B, 0.9, 1e-5)
            ncmhip.check()
        bufs = dict(zip([k for k, _ in q.tens], q.bufs))
        for lv in range(q.n):
            assert bits_equal(bufs[f"embeddings.{lv}.weight"].numpy(), want[lv]), lv
        bad = codes.copy()
        bad[0, 0] = cfg["vq_vocab"][0]
        with pytest.raises(ncmhip.NcmError, match="vq_ema_update"):
            q.lib.vq_ema_update(q.vq, zd.ptr, bad.ctypes.data, B, 0.9, 1e-5)
            ncmhip.check()
    finally:
        q.close()


def test_ema_update_larger_rows():
    """128 sequences (2048 rows at the last level), 512 codes, D 64: the
    codebooks after one update equal the oracle's."""
    cfg, w, z = make_case(13, B=128, levels=[1, 2, 4, 8, 16], V=512, D=64)
    print("[gpu] vq ema larger case", flush=True)
    idx, _, _ = O.vq_z_to_idx(cfg, w, z, 128)
    want, _, _ = O.vq_ema_update(cfg, w, z, idx, 128, 0.99, 1e-5)
    q = DevVq(cfg, w)
    try:
        zd = D_.from_numpy(z)
        q.lib.vq_ema_update(q.vq, zd.ptr, np.ascontiguousarray(idx, np.int32).ctypes.data, 128, 0.99, 1e-5)
        ncmhip.check()
        bufs = dict(zip([k for k, _ in q.tens], q.bufs))
        for lv in range(q.n):
            assert bits_equal(bufs[f"embeddings.{lv}.weight"].numpy(), want[lv]), lv
    finally:
        q.close()


def test_ema_init_failure_leaves_no_half_state():
    """An allocation failure at the second level of the EMA set-up releases
    the first level too: the update reports it and changes nothing, and the
    next update (allocations working again) builds the state whole and gives
    the oracle's codebooks."""
    name, kw = CASES[0]
    cfg, w, z = make_case(7, **kw)
    B = kw["B"]
    print(f"[gpu] vq ema rollback on case {name}", flush=True)
    idx, _, _ = O.vq_z_to_idx(cfg, w, z, B)
    want, _, _ = O.vq_ema_update(cfg, w, z, idx, B, 0.9, 1e-5)
    q = DevVq(cfg, w)
    assert q.n >= 2
    try:
        zd = D_.from_numpy(z)
        codes = np.ascontiguousarray(idx, np.int32)
        bufs = dict(zip([k for k, _ in q.tens], q.bufs))
        before = [bufs[f"embeddings.{lv}.weight"].numpy() for lv in range(q.n)]
        q.lib.ncm_hip_fail_alloc_after(1)
        try:
            with pytest.raises(ncmhip.NcmError, match="vq_ema_init: level 1"):
                q.lib.vq_ema_update(q.vq, zd.ptr, codes.ctypes.data, B, 0.9, 1e-5)
                ncmhip.check()
        finally:
            q.lib.ncm_hip_fail_alloc_after(-1)
        for lv in range(q.n):
            assert bits_equal(bufs[f"embeddings.{lv}.weight"].numpy(), before[lv]), lv
        q.lib.vq_ema_update(q.vq, zd.ptr, codes.ctypes.data, B, 0.9, 1e-5)
        ncmhip.check()
        for lv in range(q.n):
            assert bits_equal(bufs[f"embeddings.{lv}.weight"].numpy(), want[lv]), lv
    finally:
        q.close()


def _soft_state_drawing_half():
    """A xorshift64 state (vq.c:425's 13/7/17 form) whose next step gives
    u = (x >> 11) 2^-53 = 0.5 exactly: the three steps undone in reverse."""
    m = (1 << 64) - 1
    y = 1 << 63
    y = (y ^ (y << 17) ^ (y << 34) ^ (y << 51)) & m
    t = y
    for s in range(7, 64, 7):
        t ^= y >> s
    y = t
    y = (y ^ (y << 13) ^ (y << 26) ^ (y << 39) ^ (y << 52)) & m
    x = y
    x ^= (x << 13) & m
    x ^= x >> 7
    x ^= (x << 17) & m
    assert x >> 11 == 1 << 52
    return y


def test_soft_draw_on_a_running_sum_is_decided_on_the_host():
    """Codewords e_j (one-hot) and z = 0 make every level-0 distance 1.0, so
    every weight is exp(0) = 1 and the first row's draw 0.5 * V lands exactly
    on a running sum: the device marks it, the host decides it with glibc's
    exp, and codes and rng state equal the oracle's and the reference's."""
    V, D, B, levels = 16, 32, 4, [1, 2, 4]
    cfg, w, _ = make_case(3, B=B, levels=levels, V=V, D=D)
    w["embeddings.0.weight"] = np.eye(V, D, dtype=np.float32)
    z = np.zeros((B, levels[-1], D), np.float32)
    seed = _soft_state_drawing_half()
    print("[gpu] vq soft draw on a running sum", flush=True)
    want_idx, _, _, want_rng = O.vq_z_to_idx_soft(cfg, w, z, B, 3, 0.5, seed)
    assert want_idx[0, 0] == V // 2
    q = DevVq(cfg, w)
    try:
        zd = D_.from_numpy(z)
        idx = np.zeros((B, q.total), np.int32)
        rng = ctypes.c_ulonglong(seed)
        q.lib.vq_z_to_idx_soft(q.vq, zd.ptr, B, idx.ctypes.data, 3, 0.5, ctypes.byref(rng))
        ncmhip.check()
        host_rows = q.lib.ncm_vq_soft_host_rows()
        print(f"[gpu] rows decided on the host: {host_rows}", flush=True)
        assert host_rows >= 1
        assert np.array_equal(idx, want_idx) and rng.value == want_rng
        if O.ref_available():
            ridx, _, rrng = ref_vq(cfg, w, z, B, soft=(3, 0.5, seed))
            assert np.array_equal(idx, ridx) and rng.value == rrng
    finally:
        q.close()
