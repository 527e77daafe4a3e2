"""Fused entry points against the unfused sequences they replace, bit for bit
on the device: linear_fwd_glu = linear_fwd_ep(act) then mul_fwd (ncp.c:301-310);
qkv_split_rope_fwd = qkv_split_fwd then rope_apply (ncp.c:213-236);
sdpa_fwd_gqa_merged = sdpa_fwd_gqa then head_merge_fwd (ncp.c:248-260).  The
unfused entry points are each pinned to the oracle in their own tests."""
import numpy as np
import pytest

import ncmhip
import oracle as O
from conftest import bits_equal

pytestmark = pytest.mark.gpu
D = ncmhip.DeviceBuffer


@pytest.fixture(scope="module", autouse=True)
def device():
    ncmhip.init(0)
    print("[gpu] fused entry points on device 0", flush=True)


@pytest.mark.parametrize("batch,M,K,act", [(5184, 1024, 256, 1), (333, 100, 96, 1), (7, 64, 32, 1), (1, 48, 64, 2),
                                           (130, 77, 40, 3), (64, 256, 256, 0)])
def test_linear_glu_matches_unfused(batch, M, K, act):
    print(f"[gpu] glu batch={batch} M={M} K={K} act={act}", flush=True)
    rng = np.random.default_rng(batch + M)
    x = rng.standard_normal((batch, K)).astype(np.float32)
    W = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    b = (rng.standard_normal(M) * 0.1).astype(np.float32)
    u = rng.standard_normal((batch, M)).astype(np.float32)
    lib = ncmhip.load()
    dx, dW, db, du = D.from_numpy(x), D.from_numpy(W), D.from_numpy(b), D.from_numpy(u)
    y, g = D.empty((batch, M)), D.empty((batch, M))
    lib.linear_fwd_glu(dx.ptr, dW.ptr, db.ptr, du.ptr, y.ptr, batch, M, K, act)
    lib.linear_fwd_ep(dx.ptr, dW.ptr, db.ptr, None, g.ptr, batch, M, K, act)
    lib.mul_fwd(g.ptr, du.ptr, g.ptr, batch * M)
    ncmhip.check()
    assert bits_equal(y.numpy(), g.numpy())
    if act == 1:   # and the oracle: silu(x W^T + b) * u
        ref = O.mul(O.act("silu", O.linear_fwd(x, W, b)), u)
        np.testing.assert_allclose(y.numpy(), ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("batch,M,K,act,bias", [(5184, 1024, 256, 1, True), (2048, 4864, 896, 1, False),
                                                (300, 200, 96, 2, True), (70, 40, 8, 1, True), (5, 64, 32, 1, True),
                                                (4096, 130, 36, 3, False)])
def test_linear_gated_matches_glu_path(batch, M, K, act, bias):
    """One launch for both products (when its tiles fill the CUs) against the up
    GEMM followed by the multiply-epilogue gate GEMM: bit for bit where neither
    of those splits K (the same MFMA sequence per output), else within the
    oracle's tolerance."""
    print(f"[gpu] gated batch={batch} M={M} K={K} act={act}", flush=True)
    rng = np.random.default_rng(batch * 7 + M)
    x = rng.standard_normal((batch, K)).astype(np.float32)
    Wg = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    Wu = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
    bg = (rng.standard_normal(M) * 0.1).astype(np.float32) if bias else None
    bu = (rng.standard_normal(M) * 0.1).astype(np.float32) if bias else None
    lib = ncmhip.load()
    dx, dg, du = D.from_numpy(x), D.from_numpy(Wg), D.from_numpy(Wu)
    dbg, dbu = (D.from_numpy(bg), D.from_numpy(bu)) if bias else (None, None)
    pg, pu = (dbg.ptr, dbu.ptr) if bias else (None, None)
    y, u, g = D.empty((batch, M)), D.empty((batch, M)), D.empty((batch, M))
    lib.linear_fwd_gated(dx.ptr, dg.ptr, pg, du.ptr, pu, y.ptr, batch, M, K, act)
    lib.linear_fwd(dx.ptr, du.ptr, pu, u.ptr, batch, M, K)
    lib.linear_fwd_glu(dx.ptr, dg.ptr, pg, u.ptr, g.ptr, batch, M, K, act)
    ncmhip.check()
    got = y.numpy()
    if ncmhip.linear_plan("fwd", batch, M, K)[1] == 1:
        assert bits_equal(got, g.numpy())
    name = {1: "silu", 2: "gelu", 3: "gelu_tanh"}[act]
    ref = O.mul(O.act(name, O.linear_fwd(x, Wg, bg)), O.linear_fwd(x, Wu, bu))
    np.testing.assert_allclose(got, ref, rtol=2e-4, atol=2e-4)


def test_linear_glu_refuses_an_aliased_multiplier():
    lib = ncmhip.load()
    x, W, y = D.empty((16, 8)), D.empty((4, 8)), D.empty((16, 4))
    with pytest.raises(ncmhip.NcmError, match="multiplier"):
        lib.linear_fwd_glu(x.ptr, W.ptr, None, y.ptr, y.ptr, 16, 4, 8, 1)
        ncmhip.check()


@pytest.mark.parametrize("B,T,H,Kv,hd", [(64, 81, 4, 2, 64), (3, 17, 6, 3, 32), (2, 5, 4, 4, 10)])
def test_qkv_split_rope_matches_unfused(B, T, H, Kv, hd):
    print(f"[gpu] split+rope B={B} T={T} H={H} Kv={Kv} hd={hd}", flush=True)
    rng = np.random.default_rng(T * H)
    C = H * hd
    qkv = rng.standard_normal((B, T, C + 2 * Kv * hd)).astype(np.float32)
    cos = rng.uniform(-1, 1, (T, hd)).astype(np.float32)
    sin = rng.uniform(-1, 1, (T, hd)).astype(np.float32)
    lib = ncmhip.load()
    din, dc, ds = D.from_numpy(qkv), D.from_numpy(cos), D.from_numpy(sin)
    f = [D.empty((B, H, T, hd)) for _ in range(3)]
    u = [D.empty((B, H, T, hd)) for _ in range(3)]
    lib.qkv_split_rope_fwd(din.ptr, f[0].ptr, f[1].ptr, f[2].ptr, dc.ptr, ds.ptr, B, T, C, H, hd, Kv, H // Kv)
    lib.qkv_split_fwd(din.ptr, u[0].ptr, u[1].ptr, u[2].ptr, B, T, C, H, hd, Kv, H // Kv)
    lib.rope_apply(u[0].ptr, u[1].ptr, dc.ptr, ds.ptr, B, H, T, hd)
    ncmhip.check()
    for a, b in zip(f, u):
        assert bits_equal(a.numpy(), b.numpy())


@pytest.mark.parametrize("B,Hq,Hkv,Tq,Tkv,hd,masked", [(64, 4, 4, 81, 81, 64, False), (2, 6, 2, 70, 90, 64, True),
                                                      (3, 4, 2, 9, 9, 40, False)])
def test_sdpa_merged_matches_unfused(B, Hq, Hkv, Tq, Tkv, hd, masked):
    print(f"[gpu] sdpa merged B={B} Hq={Hq} Hkv={Hkv} Tq={Tq} Tkv={Tkv} hd={hd}", flush=True)
    rng = np.random.default_rng(Tq + Tkv)
    q = rng.standard_normal((B, Hq, Tq, hd)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, Tkv, hd)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, Tkv, hd)).astype(np.float32)
    mask = np.where(rng.random((Tq, Tkv)) < 0.2, -1e9, 0.0).astype(np.float32) if masked else None
    lib = ncmhip.load()
    dq, dk, dv = D.from_numpy(q), D.from_numpy(k), D.from_numpy(v)
    dm = D.from_numpy(mask) if masked else None
    mp = dm.ptr if masked else None
    out, ctx, mo = D.empty((B, Tq, Hq * hd)), D.empty((B, Hq, Tq, hd)), D.empty((B, Tq, Hq * hd))
    lib.sdpa_fwd_gqa_merged(dq.ptr, dk.ptr, dv.ptr, mp, out.ptr, B, Hq, Hkv, Tq, Tkv, hd)
    lib.sdpa_fwd_gqa(dq.ptr, dk.ptr, dv.ptr, mp, ctx.ptr, B, Hq, Hkv, Tq, Tkv, hd)
    lib.head_merge_fwd(ctx.ptr, mo.ptr, B, Tq, Hq * hd, Hq, hd)
    ncmhip.check()
    assert bits_equal(out.numpy(), mo.numpy())
