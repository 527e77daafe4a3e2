"""GPU norms, RoPE, SDPA-GQA, head layout, embedding and elementwise kernels
against the oracle (kernels.c restated on the CPU).

Bars: layout / embedding / RoPE / add / mul / scale bit-exact (same float
operations, no contraction); norms and activations within a few ulp (fp64
reduction in another order, fp64 transcendental); SDPA max-abs 1e-5 and
maxrel 1e-5 (online softmax, hardware exp)."""
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
    print("[gpu] ops tests on device 0", flush=True)


def rnd(seed, *shape, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def run(name, outs, *args):
    ncmhip.call(name, *args)
    return [o.numpy() for o in outs]


# ---------------------------------------------------------------- norms
@pytest.mark.parametrize("rows,C", [(1, 1), (7, 896), (129, 4864), (300, 65), (64, 768)])
@pytest.mark.parametrize("weighted", [True, False])
def test_rmsnorm(rows, C, weighted):
    x, w = rnd(rows * C, rows, C), (rnd(C, C) if weighted else None)
    y = D.empty((rows, C))
    (got,) = run("rmsnorm_fwd", [y], D.from_numpy(x), None if w is None else D.from_numpy(w), y, rows, C)
    assert maxrel(got, O.rmsnorm(x, w)) <= 1e-6


@pytest.mark.parametrize("rows,C", [(1, 1), (9, 768), (513, 1024), (33, 100)])
@pytest.mark.parametrize("eps", [None, 1e-5])
def test_layernorm(rows, C, eps):
    x, w, b = rnd(rows + C, rows, C, scale=3.0) + 1.5, rnd(1, C), rnd(2, C)
    y = D.empty((rows, C))
    if eps is None:
        (got,) = run("layernorm_fwd", [y], D.from_numpy(x), D.from_numpy(w), D.from_numpy(b), y, rows, C)
    else:
        (got,) = run("layernorm_eps_fwd", [y], D.from_numpy(x), D.from_numpy(w), D.from_numpy(b), y, rows, C, eps)
    assert maxrel(got, O.layernorm(x, w, b, eps)) <= 1e-6


def test_layernorm_no_affine():
    x = rnd(5, 17, 256)
    y = D.empty(x.shape)
    (got,) = run("layernorm_fwd", [y], D.from_numpy(x), None, None, y, 17, 256)
    assert maxrel(got, O.layernorm(x, None, None)) <= 1e-6


# ---------------------------------------------------------------- elementwise
@pytest.mark.parametrize("n", [1, 255, 4097, 1 << 20])
def test_add_mul_scale_bitexact(n):
    a, b = rnd(n, n), rnd(n + 1, n)
    da, db, y = D.from_numpy(a), D.from_numpy(b), D.empty(n)
    assert bits_equal(run("add_fwd", [y], da, db, y, n)[0], a + b)
    assert bits_equal(run("mul_fwd", [y], da, db, y, n)[0], O.mul(a, b))
    assert bits_equal(run("scale_fwd", [y], da, np.float32(0.125).item(), y, n)[0], O.scale(a, 0.125))
    y.upload(b)
    assert bits_equal(run("add_inplace_fwd", [y], y, da, n)[0], b + a)


@pytest.mark.parametrize("name", ["silu", "gelu", "gelu_tanh"])
def test_activations(name):
    x = np.concatenate([rnd(3, 50000, scale=4.0), np.array([0.0, -0.0, 30.0, -30.0, 1e-8], np.float32)])
    y = D.empty(x.size)
    (got,) = run(name + "_fwd", [y], D.from_numpy(x), y, x.size)
    ref = O.act(name, x)
    ulp = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert maxrel(got, ref) <= 1e-6
    # gelu's 1 + erff(x/sqrt2) cancels for x < -1 (kernels.c:190), so an ulp of
    # erff there is many ulp of the tiny result; elsewhere both agree to 2 ulp.
    ok = (x >= -1.0) if name == "gelu" else (np.abs(ref) > 1e-30)
    assert int(ulp[ok].max()) <= 2


# ---------------------------------------------------------------- RoPE
@pytest.mark.parametrize("B,H,K,T,hd", [(1, 14, 2, 37, 64), (2, 4, 4, 5, 128), (1, 2, 1, 300, 64), (3, 1, 1, 1, 8)])
def test_rope_gqa_bitexact(B, H, K, T, hd):
    cos_t, sin_t = O.rope_tables_qwen(T, hd, 1e6)
    q, k = rnd(1, B, H, T, hd), rnd(2, B, K, T, hd)
    dq, dk = D.from_numpy(q), D.from_numpy(k)
    got_q, got_k = run("rope_apply_gqa", [dq, dk], dq, dk, D.from_numpy(cos_t), D.from_numpy(sin_t), B, H, K, T, hd)
    assert bits_equal(got_q, O.rope(q.reshape(-1, hd), cos_t, sin_t, T).reshape(q.shape))
    assert bits_equal(got_k, O.rope(k.reshape(-1, hd), cos_t, sin_t, T).reshape(k.shape))


def test_rope_q_only():
    T, hd = 11, 64
    cos_t, sin_t = O.rope_tables_qwen(T, hd, 1e4)
    q = rnd(9, 1, 3, T, hd)
    dq = D.from_numpy(q)
    (got,) = run("rope_apply", [dq], dq, None, D.from_numpy(cos_t), D.from_numpy(sin_t), 1, 3, T, hd)
    assert bits_equal(got, O.rope(q.reshape(-1, hd), cos_t, sin_t, T).reshape(q.shape))


# ---------------------------------------------------------------- layout / embedding
@pytest.mark.parametrize("B,T,H,hd", [(1, 7, 12, 64), (2, 33, 14, 64), (3, 1, 2, 5)])
def test_heads_transpose_bitexact(B, T, H, hd):
    x = rnd(B * T, B, T, H * hd)
    y = D.empty((B, H, T, hd))
    (got,) = run("heads_transpose_fwd_b", [y], D.from_numpy(x), y, B, T, H, hd)
    assert bits_equal(got, O.heads_transpose(x, B, T, H, hd))
    if B == 1:
        (got1,) = run("heads_transpose_fwd", [y], D.from_numpy(x), y, T, H, hd)
        assert bits_equal(got1, got)


@pytest.mark.parametrize("B,T,C,H,hd,K,rep", [(2, 9, 768, 12, 64, 12, 1), (1, 17, 896, 14, 64, 2, 7),
                                               (3, 4, 64, 4, 16, 1, 4)])
def test_qkv_split_head_merge_bitexact(B, T, C, H, hd, K, rep):
    x = rnd(C + T, B, T, C + 2 * K * hd)
    outs = [D.empty((B, H, T, hd)) for _ in range(3)]
    got = run("qkv_split_fwd", outs, D.from_numpy(x), *outs, B, T, C, H, hd, K, rep)
    for g, r in zip(got, O.qkv_split(x, B, T, C, H, hd, K, rep)):
        assert bits_equal(g, r)
    ctx = rnd(5, B, H, T, hd)
    y = D.empty((B, T, C))
    (m,) = run("head_merge_fwd", [y], D.from_numpy(ctx), y, B, T, C, H, hd)
    assert bits_equal(m, O.head_merge(ctx, B, T, C, H, hd))


def test_embedding_bitexact():
    V, Dm, n = 1000, 896, 77
    W = rnd(1, V, Dm)
    idx = np.random.default_rng(2).integers(0, V, n).astype(np.int32)
    idx[:3] = [0, V - 1, 5]
    y = D.empty((n, Dm))
    (got,) = run("embedding_fwd", [y], D.from_numpy(W), D.from_numpy(idx), y, n, Dm)
    assert bits_equal(got, O.embedding(W, idx))
    bad = idx.copy()
    bad[[4, 9]] = [V, -3]
    (gv,) = run("embedding_fwd_v", [y], D.from_numpy(W), V, D.from_numpy(bad), y, n, Dm)
    ref = O.embedding(W, np.where((bad < 0) | (bad >= V), 0, bad))
    assert bits_equal(gv, ref)


# ---------------------------------------------------------------- SDPA
def causal_mask(Tq, Tkv):
    """-1e9 above the diagonal, bottom-right aligned (qwen.c:130-138 when Tq == Tkv)."""
    off = Tkv - Tq
    m = np.zeros((Tq, Tkv), np.float32)
    m[np.arange(Tkv)[None, :] > np.arange(Tq)[:, None] + off] = -1e9
    return m


def gpu_sdpa(q, k, v, mask=None, causal=False, offset_bytes=0):
    B, Hq, Tq, hd = q.shape
    Hkv, Tkv = k.shape[1], k.shape[2]
    bufs = []
    for a in (q, k, v):
        if offset_bytes:
            b = D.empty(a.size + 4)
            raw = np.zeros(a.size + 4, np.float32)
            raw[offset_bytes // 4:offset_bytes // 4 + a.size] = a.ravel()
            b.upload(raw)
            bufs.append((b, b.ptr + offset_bytes))
        else:
            b = D.from_numpy(a)
            bufs.append((b, b))
    out = D.empty(q.shape)
    (dq, _), (dk, _), (dv, _) = bufs
    args = [p for _, p in bufs]
    if causal:
        ncmhip.call("sdpa_fwd_gqa_causal", *args, out, B, Hq, Hkv, Tq, Tkv, hd)
    else:
        ncmhip.call("sdpa_fwd_gqa", *args, None if mask is None else D.from_numpy(mask), out, B, Hq, Hkv, Tq, Tkv, hd)
    return out.numpy()


def check_sdpa(got, ref, tol=1e-5):
    assert np.all(np.isfinite(got))
    assert float(np.max(np.abs(got - ref))) <= tol and maxrel(got, ref) <= tol


@pytest.mark.parametrize("B,Hq,Hkv,Tq,Tkv,hd", [
    (1, 14, 2, 128, 128, 64),    # Qwen2.5-0.5B prefill heads
    (2, 12, 12, 77, 77, 64),     # GPT-2 heads, ragged T
    (1, 14, 2, 1, 300, 64),      # decode step
    (1, 4, 1, 65, 200, 64),
    (2, 3, 3, 19, 40, 32),       # generic row kernel
    (1, 2, 1, 9, 130, 128),
    (1, 2, 2, 3, 5, 256),
])
def test_sdpa_vs_oracle(B, Hq, Hkv, Tq, Tkv, hd):
    q, k, v = rnd(1, B, Hq, Tq, hd), rnd(2, B, Hkv, Tkv, hd), rnd(3, B, Hkv, Tkv, hd)
    check_sdpa(gpu_sdpa(q, k, v), O.sdpa_gqa(q, k, v))


@pytest.mark.parametrize("B,Hq,Hkv,Tq,Tkv,hd", [(1, 14, 2, 200, 200, 64), (2, 12, 12, 64, 64, 64),
                                               (1, 14, 2, 7, 135, 64), (1, 14, 2, 1, 64, 64),
                                               (1, 4, 2, 33, 33, 48)])
def test_sdpa_causal(B, Hq, Hkv, Tq, Tkv, hd):
    q, k, v = rnd(4, B, Hq, Tq, hd), rnd(5, B, Hkv, Tkv, hd), rnd(6, B, Hkv, Tkv, hd)
    m = causal_mask(Tq, Tkv)
    ref = O.sdpa_gqa(q, k, v, m)
    check_sdpa(gpu_sdpa(q, k, v, mask=m), ref)
    check_sdpa(gpu_sdpa(q, k, v, causal=True), ref)


def test_sdpa_key_split():
    """Grids that cannot fill the chip cut each query tile's keys into parts
    merged afterwards: a causal 1024-token single sequence (up to 8 parts per
    tile), and a masked long-key case where whole parts are masked out (their
    max is -inf and they must weigh nothing), head-major and merged output."""
    B, Hq, Hkv, T = 1, 4, 2, 1024
    q, k, v = rnd(40, B, Hq, T, 64), rnd(41, B, Hkv, T, 64), rnd(42, B, Hkv, T, 64)
    check_sdpa(gpu_sdpa(q, k, v, causal=True), O.sdpa_gqa(q, k, v, causal_mask(T, T)))
    Tq, Tkv = 100, 700
    q, k, v = rnd(43, 1, 2, Tq, 64), rnd(44, 1, 1, Tkv, 64), rnd(45, 1, 1, Tkv, 64)
    m = np.zeros((Tq, Tkv), np.float32)
    m[:, 128:384] = -np.inf
    m[::3, 500:] = -np.inf
    ref = O.sdpa_gqa(q, k, v, m)
    check_sdpa(gpu_sdpa(q, k, v, mask=m), ref)
    out = D.empty((1, Tq, 2 * 64))
    ncmhip.call("sdpa_fwd_gqa_merged", D.from_numpy(q), D.from_numpy(k), D.from_numpy(v), D.from_numpy(m), out, 1,
                2, 1, Tq, Tkv, 64)
    check_sdpa(out.numpy().reshape(1, Tq, 2, 64).transpose(0, 2, 1, 3), ref)


def test_sdpa_additive_mask_and_large_scores():
    B, Hq, Hkv, Tq, Tkv, hd = 1, 4, 2, 70, 90, 64
    q, k, v = rnd(7, B, Hq, Tq, hd, scale=4.0), rnd(8, B, Hkv, Tkv, hd, scale=4.0), rnd(9, B, Hkv, Tkv, hd)
    m = rnd(10, Tq, Tkv, scale=3.0)
    # scores of magnitude ~16 from fp32 dot products carry ~1e-5 relative
    # error, which the softmax passes on to the output
    check_sdpa(gpu_sdpa(q, k, v, mask=m), O.sdpa_gqa(q, k, v, m), tol=1e-4)


def test_sdpa_unaligned_pointers_take_row_kernel():
    q, k, v = rnd(11, 1, 2, 30, 64), rnd(12, 1, 2, 50, 64), rnd(13, 1, 2, 50, 64)
    check_sdpa(gpu_sdpa(q, k, v, offset_bytes=4), O.sdpa_gqa(q, k, v))


def test_sdpa_mha_alias_matches_gqa():
    q, k, v = rnd(14, 2, 3, 20, 64), rnd(15, 2, 3, 20, 64), rnd(16, 2, 3, 20, 64)
    out = D.empty(q.shape)
    ncmhip.call("sdpa_fwd", D.from_numpy(q), D.from_numpy(k), D.from_numpy(v), None, out, 2, 3, 20, 20, 64)
    assert bits_equal(out.numpy(), gpu_sdpa(q, k, v))


@pytest.mark.parametrize("Hq,Hkv,hd", [(14, 3, 64), (2, 2, 300), (2, 0, 64)])
def test_sdpa_rejects_bad_shapes(Hq, Hkv, hd):
    q = D.empty(1024)
    with pytest.raises(ncmhip.NcmError):
        ncmhip.call("sdpa_fwd_gqa", q, q, q, None, q, 1, Hq, Hkv, 1, 1, hd)


def test_sdpa_causal_rejects_more_queries_than_keys():
    q = D.empty(64 * 64)
    with pytest.raises(ncmhip.NcmError):
        ncmhip.call("sdpa_fwd_gqa_causal", q, q, q, q, 1, 1, 1, 8, 4, 64)
