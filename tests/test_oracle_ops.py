"""Oracle pinning for the norm / RoPE / SDPA / layout / elementwise rows:
the reference's kernel checksum harness (tests/ktest_kernels.c), bit-equality
with the reference compiled from source, and closed forms."""
import os

import numpy as np
import pytest

import oracle as O
from conftest import GOLDEN, bits_equal

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference not compiled here")


def _ktest_lines():
    out = {}
    for line in open(os.path.join(GOLDEN, "ktest_cpu.txt")):
        if " sum=" in line:
            out[line.split()[0]] = line.strip()
    return out


def _chk(name, v):
    v = np.asarray(v, np.float32).reshape(-1)
    s = float(np.cumsum(v.astype(np.float64))[-1])
    mx = float(np.max(np.abs(v.astype(np.float64))))
    return "%s sum=%.6f maxabs=%.6f first=%.6f %.6f %.6f %.6f" % (name, s, mx, v[0], v[1], v[2], v[3])


def _ktest_arrays():
    """The inputs tests/ktest_kernels.c:33-77 draws, in its order."""
    st = 0x12345678
    out = []

    def mk(n):
        nonlocal st
        v, st = O.ktest_fill(st, n)
        out.append(v)
        return v
    ln = [mk(256), mk(64), mk(64), mk(256)]
    rms = [mk(256), mk(64), mk(256)]
    act = [mk(512), mk(512)]
    rope = [mk(1024), mk(1024), mk(512), mk(512)]
    sdpa = [mk(256), mk(384), mk(384), mk(96), mk(256)]
    return ln, rms, act, rope, sdpa


def test_ktest_norms_activations():
    ln, rms, act, _, _ = _ktest_arrays()
    lines = _ktest_lines()
    assert _chk("layernorm", O.layernorm(ln[0].reshape(4, 64), ln[1], ln[2])) == lines["layernorm"]
    assert _chk("rmsnorm", O.rmsnorm(rms[0].reshape(4, 64), rms[1])) == lines["rmsnorm"]
    assert _chk("gelu", O.act("gelu", act[0])) == lines["gelu"]
    assert _chk("silu", O.act("silu", act[0])) == lines["silu"]


def test_ktest_rope():
    _, _, _, (q, k, co, si), _ = _ktest_arrays()
    lines = _ktest_lines()
    # rope_apply(q, k, co, si, B=1, H=2, T=16, hd=32)
    assert _chk("rope_q", O.rope(q.reshape(32, 32), co.reshape(16, 32), si.reshape(16, 32), 16)) == lines["rope_q"]
    assert _chk("rope_k", O.rope(k.reshape(32, 32), co.reshape(16, 32), si.reshape(16, 32), 16)) == lines["rope_k"]


def test_ktest_sdpa():
    _, _, _, _, (q, k, v, m, _) = _ktest_arrays()
    mask = np.where(m > 0, np.float32(0.0), np.float32(-np.inf)).astype(np.float32)
    out = O.sdpa_gqa(q.reshape(1, 2, 8, 16), k.reshape(1, 2, 12, 16), v.reshape(1, 2, 12, 16), mask.reshape(8, 12))
    assert _chk("sdpa", out) == _ktest_lines()["sdpa"]


@needs_ref
def test_vs_reference_norms_rope():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((37, 96)).astype(np.float32)
    w = rng.standard_normal(96).astype(np.float32)
    b = rng.standard_normal(96).astype(np.float32)
    y = np.empty_like(x)
    O.ref_call("rmsnorm_fwd", x, w, y, 37, 96)
    assert bits_equal(y, O.rmsnorm(x, w))
    O.ref_call("layernorm_fwd", x, w, b, y, 37, 96)
    assert bits_equal(y, O.layernorm(x, w, b))
    O.ref_call("layernorm_eps_fwd", x, w, b, y, 37, 96, 1e-5)
    assert bits_equal(y, O.layernorm(x, w, b, 1e-5))
    B, H, K, T, hd = 2, 4, 2, 9, 64
    c, s = O.rope_tables_qwen(T, hd, 1e6)
    q = rng.standard_normal((B, H, T, hd)).astype(np.float32)
    k = rng.standard_normal((B, K, T, hd)).astype(np.float32)
    q2, k2 = q.copy(), k.copy()
    O.ref_call("rope_apply_gqa", q2, k2, c, s, B, H, K, T, hd)
    assert bits_equal(q2.reshape(-1, hd), O.rope(q.reshape(-1, hd), c, s, T))
    assert bits_equal(k2.reshape(-1, hd), O.rope(k.reshape(-1, hd), c, s, T))


@needs_ref
@pytest.mark.parametrize("Hq,Hkv,causal", [(4, 2, True), (4, 4, False), (6, 1, True)])
def test_vs_reference_sdpa(Hq, Hkv, causal):
    rng = np.random.default_rng(Hq * 10 + Hkv)
    B, Tq, Tkv, hd = 2, 11, 11, 64
    q = rng.standard_normal((B, Hq, Tq, hd)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, Tkv, hd)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, Tkv, hd)).astype(np.float32)
    mask = None
    if causal:
        mask = np.where(np.arange(Tkv)[None, :] <= np.arange(Tq)[:, None], 0.0, -1e9).astype(np.float32)
    out = np.empty_like(q)
    O.ref_call("sdpa_fwd_gqa", q, k, v, mask, out, B, Hq, Hkv, Tq, Tkv, hd)
    assert bits_equal(out, O.sdpa_gqa(q, k, v, mask))
    if Hq == Hkv:
        out2 = np.empty_like(q)
        O.ref_call("sdpa_fwd", q, k, v, mask, out2, B, Hq, Tq, Tkv, hd)
        assert bits_equal(out2, out)


@needs_ref
def test_vs_reference_layout_elementwise():
    rng = np.random.default_rng(3)
    B, T, H, hd, K = 2, 5, 4, 8, 2
    C = H * hd
    x = rng.standard_normal((B, T, C)).astype(np.float32)
    y = np.empty((B, H, T, hd), np.float32)
    O.ref_call("heads_transpose_fwd_b", x, y, B, T, H, hd)
    assert bits_equal(y, O.heads_transpose(x, B, T, H, hd))
    qkv = rng.standard_normal((B, T, C + 2 * K * hd)).astype(np.float32)
    refs = [np.empty((B, H, T, hd), np.float32) for _ in range(3)]
    O.ref_call("qkv_split_fwd", qkv, *refs, B, T, C, H, hd, K, H // K)
    for a, r in zip(O.qkv_split(qkv, B, T, C, H, hd, K, H // K), refs):
        assert bits_equal(a, r)
    ctx = rng.standard_normal((B, H, T, hd)).astype(np.float32)
    o = np.empty((B, T, C), np.float32)
    O.ref_call("head_merge_fwd", ctx, o, B, T, C, H, hd)
    assert bits_equal(o, O.head_merge(ctx, B, T, C, H, hd))
    W = rng.standard_normal((50, 16)).astype(np.float32)
    idx = rng.integers(0, 50, 23).astype(np.int32)
    e = np.empty((23, 16), np.float32)
    O.ref_call("embedding_fwd", W, idx, e, 23, 16)
    assert bits_equal(e, O.embedding(W, idx))
    a, bb = rng.standard_normal(100).astype(np.float32), rng.standard_normal(100).astype(np.float32)
    m = np.empty(100, np.float32)
    O.ref_call("mul_fwd", a, bb, m, 100)
    assert bits_equal(m, O.mul(a, bb))
    O.ref_call("scale_fwd", a, 0.37, m, 100)
    assert bits_equal(m, O.scale(a, 0.37))


# ------------------------------------------------------------- closed forms
def test_rmsnorm_constant_row():
    """RMSNorm of c*1 is sign(c) * w / sqrt(1 + 1e-6/c^2) (up to the float
    rounding of the scale)."""
    C = 64
    w = np.linspace(-2, 2, C).astype(np.float32)
    for c in (3.0, -0.5, 1e-2):
        x = np.full((1, C), c, np.float32)
        want = np.sign(c) * w / np.sqrt(1 + 1e-6 / c ** 2)
        assert np.max(np.abs(O.rmsnorm(x, w)[0] - want)) < 1e-6 * np.max(np.abs(w)) + 1e-7


def test_layernorm_constant_row_is_bias():
    x = np.full((3, 48), 2.5, np.float32)
    w = np.arange(48, dtype=np.float32)
    b = np.linspace(-1, 1, 48).astype(np.float32)
    assert bits_equal(O.layernorm(x, w, b), np.tile(b, (3, 1)))


def test_rope_position_zero_and_norm():
    T, hd = 8, 64
    c, s = O.rope_tables_qwen(T, hd, 1e4)
    assert np.all(c[0] == 1) and np.all(s[0] == 0)
    x = np.random.default_rng(4).standard_normal((T, hd)).astype(np.float32)
    y = O.rope(x, c, s, T)
    assert bits_equal(y[0], x[0])
    h = hd // 2
    nx = x[:, :h] ** 2 + x[:, h:] ** 2
    ny = y[:, :h].astype(np.float64) ** 2 + y[:, h:].astype(np.float64) ** 2
    assert np.max(np.abs(nx - ny) / (nx + 1)) < 1e-5


def test_sdpa_closed_forms():
    rng = np.random.default_rng(5)
    B, H, T, hd = 1, 2, 6, 16
    k = rng.standard_normal((B, H, T, hd)).astype(np.float32)
    v = rng.standard_normal((B, H, T, hd)).astype(np.float32)
    # q = 0: uniform weights -> mean of V
    out = O.sdpa_gqa(np.zeros((B, H, 3, hd), np.float32), k, v)
    assert np.max(np.abs(out - v.mean(axis=2, keepdims=True))) < 1e-6
    # a single key: the output is that value row
    out = O.sdpa_gqa(rng.standard_normal((B, H, 3, hd)).astype(np.float32), k[:, :, :1], v[:, :, :1])
    assert np.max(np.abs(out - v[:, :, :1])) < 1e-6
    # causal row 0 sees only key 0
    q = rng.standard_normal((B, H, T, hd)).astype(np.float32)
    mask = np.where(np.arange(T)[None, :] <= np.arange(T)[:, None], 0.0, -np.inf).astype(np.float32)
    out = O.sdpa_gqa(q, k, v, mask)
    assert np.max(np.abs(out[:, :, 0] - v[:, :, 0])) < 1e-6
    # GQA with Hq = 2 Hkv equals MHA on duplicated K/V
    k1, v1 = k[:, :1], v[:, :1]
    gq = O.sdpa_gqa(q, k1, v1, mask)
    mh = O.sdpa_gqa(q, np.repeat(k1, 2, axis=1), np.repeat(v1, 2, axis=1), mask)
    assert bits_equal(gq, mh)


def test_layout_index_formulas_on_iota():
    """heads_transpose is the [B,T,H,hd] -> [B,H,T,hd] axis swap, qkv_split
    slices the fused row (kv head h // rep), head_merge inverts
    heads_transpose, embedding gathers rows: checked on iota data, where any
    wrong index shows up as a wrong value."""
    B, T, H, hd, K = 2, 3, 4, 5, 2
    C, rep = H * hd, H // K
    x = np.arange(B * T * C, dtype=np.float32).reshape(B, T, C)
    ht = O.heads_transpose(x, B, T, H, hd)
    assert bits_equal(ht, x.reshape(B, T, H, hd).transpose(0, 2, 1, 3))
    assert bits_equal(O.head_merge(ht, B, T, C, H, hd), x)
    qkv = np.arange(B * T * (C + 2 * K * hd), dtype=np.float32).reshape(B, T, -1)
    q, k, v = O.qkv_split(qkv, B, T, C, H, hd, K, rep)
    kv_of = np.arange(H) // rep
    assert bits_equal(q, qkv[..., :C].reshape(B, T, H, hd).transpose(0, 2, 1, 3))
    assert bits_equal(k, qkv[..., C:C + K * hd].reshape(B, T, K, hd)[:, :, kv_of].transpose(0, 2, 1, 3))
    assert bits_equal(v, qkv[..., C + K * hd:].reshape(B, T, K, hd)[:, :, kv_of].transpose(0, 2, 1, 3))
    W = np.arange(30, dtype=np.float32).reshape(10, 3)
    idx = np.array([9, 0, 4, 4], np.int32)
    assert bits_equal(O.embedding(W, idx), W[idx])


def test_sdpa_brute_force_float64():
    """Two-pass float64 softmax(QK^T/sqrt(hd) + mask)V on small shapes."""
    rng = np.random.default_rng(6)
    B, Hq, Hkv, Tq, Tkv, hd = 2, 4, 2, 5, 7, 8
    q = rng.standard_normal((B, Hq, Tq, hd)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, Tkv, hd)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, Tkv, hd)).astype(np.float32)
    mask = rng.standard_normal((Tq, Tkv)).astype(np.float32)
    kk = np.repeat(k, Hq // Hkv, axis=1).astype(np.float64)
    vv = np.repeat(v, Hq // Hkv, axis=1).astype(np.float64)
    s = q.astype(np.float64) @ kk.transpose(0, 1, 3, 2) / np.sqrt(hd) + mask
    p = np.exp(s - s.max(-1, keepdims=True))
    want = (p / p.sum(-1, keepdims=True)) @ vv
    assert np.max(np.abs(O.sdpa_gqa(q, k, v, mask) - want)) < 2e-6


def test_ncp_rope_tables():
    """build_rope (ncp.c:80-92): position 0 is the identity, the first pair's
    angle is the position itself, cos^2 + sin^2 = 1; the library's host
    table builder gives the same bits."""
    import ctypes
    import ncmhip
    S, hd = 81, 64
    c, s = O.rope_tables_ncp(S, hd, 10000)
    assert np.all(c[0] == 1) and np.all(s[0] == 0)
    assert bits_equal(c[:, 0], np.cos(np.arange(S, dtype=np.float64)).astype(np.float32))
    assert np.max(np.abs(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2 - 1)) < 1e-6
    assert bits_equal(c[:, :32], c[:, 32:])
    lc, ls = np.empty_like(c), np.empty_like(s)
    assert ncmhip.load().ncm_ncp_rope_tables(S, hd, 10000, lc.ctypes.data, ls.ctypes.data) == 0
    assert bits_equal(lc, c) and bits_equal(ls, s)
