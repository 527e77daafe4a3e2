"""GPU parity of the linear layer (MFMA GEMM / GEMV) against the CPU oracle,
which is bit-identical to the reference's CPU path.  Contract (north star):
GEMM outputs within |got - ref| <= 1e-4 (|ref| + 1)."""
import numpy as np
import pytest

import ncmhip
import oracle as O
from conftest import bits_equal, maxrel

pytestmark = pytest.mark.gpu
TOL = 1e-4
SHAPES = [(768, 2304), (768, 3072), (3072, 768), (896, 4864), (4864, 896)]  # (K, N)
D = ncmhip.DeviceBuffer


@pytest.fixture(scope="module", autouse=True)
def device():
    ncmhip.init(0)
    print(f"[gpu] linear tests on device 0", flush=True)


def sweep_inputs(seed, M, K, N):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    b = (rng.standard_normal(N) * 0.02).astype(np.float32)
    return rng, x, W, b


def gpu_fwd(x, W, b, res=None, act="none"):
    batch, K = x.shape
    N = W.shape[0]
    y = D.empty((batch, N))
    ncmhip.linear_fwd(D.from_numpy(x), D.from_numpy(W), None if b is None else D.from_numpy(b), y,
                      batch, N, K, res=None if res is None else D.from_numpy(res), act=act)
    return y.numpy()


def gpu_bwd(x, W, dy, dx0, dW0, db0):
    batch, K = x.shape
    N = W.shape[0]
    dx, dW, db = (None if a is None else D.from_numpy(a) for a in (dx0, dW0, db0))
    ncmhip.linear_bwd(D.from_numpy(x), D.from_numpy(W), D.from_numpy(dy), dx, dW, db, batch, N, K)
    return tuple(None if a is None else a.numpy() for a in (dx, dW, db))


def test_golden_vectors(golden):
    g = golden("linear_ref.npz")
    for i in range(int(g["n_cases"])):
        p = f"c{i}_"
        b = g[p + "b"] if p + "b" in g else None
        assert maxrel(gpu_fwd(g[p + "x"], g[p + "W"], b), g[p + "y"]) <= TOL, i
        db0 = g[p + "db0"] if b is not None else None
        dx, dW, db = gpu_bwd(g[p + "x"], g[p + "W"], g[p + "dy"], g[p + "dx0"], g[p + "dW0"], db0)
        assert maxrel(dx, g[p + "dx"]) <= TOL, i
        assert maxrel(dW, g[p + "dW"]) <= TOL, i
        if b is not None:
            assert maxrel(db, g[p + "db"]) <= TOL, i


@pytest.mark.parametrize("M", [1, 64, 512])
@pytest.mark.parametrize("K,N", SHAPES)
def test_sweep_forward(M, K, N):
    _, x, W, b = sweep_inputs(M * 7 + K + N, M, K, N)
    err = maxrel(gpu_fwd(x, W, b), O.linear_fwd(x, W, b))
    assert err <= TOL, err


@pytest.mark.parametrize("K,N", SHAPES)
def test_sweep_forward_4096_sampled(K, N):
    """Full M=4096 on the GPU; rows are independent, so the oracle checks a
    random sample of them at full K and N."""
    rng, x, W, b = sweep_inputs(4096 + K + N, 4096, K, N)
    y = gpu_fwd(x, W, b)
    rows = np.sort(rng.choice(4096, 48, replace=False))
    err = maxrel(y[rows], O.linear_fwd(x[rows], W, b))
    assert err <= TOL, err


@pytest.mark.parametrize("M", [1, 64, 512])
@pytest.mark.parametrize("K,N", SHAPES)
def test_sweep_backward(M, K, N):
    rng, x, W, _ = sweep_inputs(M * 11 + K + N, M, K, N)
    dy = rng.standard_normal((M, N)).astype(np.float32)
    g0 = [rng.standard_normal(s).astype(np.float32) for s in ((M, K), (N, K), (N,))]
    got = gpu_bwd(x, W, dy, *g0)
    want = O.linear_bwd(x, W, dy, *g0)
    for name, a, r in zip(("dx", "dW", "db"), got, want):
        err = maxrel(a, r)
        assert err <= TOL, (name, err)


@pytest.mark.parametrize("K,N", SHAPES)
def test_sweep_backward_4096_sampled(K, N):
    """dX rows depend on their own dY row; dW row m on dY[:, m]: both are
    checked on samples at full size."""
    rng, x, W, _ = sweep_inputs(8192 + K + N, 4096, K, N)
    dy = rng.standard_normal((4096, N)).astype(np.float32)
    dx, dW, db = gpu_bwd(x, W, dy, np.zeros((4096, K), np.float32), np.zeros((N, K), np.float32),
                         np.zeros(N, np.float32))
    rows = np.sort(rng.choice(4096, 24, replace=False))
    ref_dx, _, _ = O.linear_bwd(x[rows], W, dy[rows], want=("dx",))
    assert maxrel(dx[rows], ref_dx) <= TOL
    ms = np.sort(rng.choice(N, 8, replace=False))
    _, ref_dW, ref_db = O.linear_bwd(x, W[ms], dy[:, ms], want=("dW", "db"))
    assert maxrel(dW[ms], ref_dW) <= TOL
    assert maxrel(db[ms], ref_db) <= TOL


@pytest.mark.parametrize("act", ["silu", "gelu", "gelu_tanh"])
@pytest.mark.parametrize("M", [3, 200])
def test_fused_epilogues(act, M):
    rng, x, W, b = sweep_inputs(17 + M, M, 256, 384)
    res = rng.standard_normal((M, 384)).astype(np.float32)
    got = gpu_fwd(x, W, b, res=res, act=act)
    want = O.act(act, O.linear_fwd(x, W, b)) + res
    assert maxrel(got, want) <= TOL
    got = gpu_fwd(x, W, b, act=act)
    assert maxrel(got, O.act(act, O.linear_fwd(x, W, b))) <= TOL


def test_in_place_residual():
    rng, x, W, b = sweep_inputs(5, 130, 96, 96)
    h = rng.standard_normal((130, 96)).astype(np.float32)
    hd = D.from_numpy(h)
    ncmhip.linear_fwd(D.from_numpy(x), D.from_numpy(W), D.from_numpy(b), hd, 130, 96, 96, res=hd)
    assert maxrel(hd.numpy(), h + O.linear_fwd(x, W, b)) <= TOL


@pytest.mark.parametrize("batch,M,K", [(2, 33, 17), (3, 100, 97), (5, 7, 1), (8, 40, 130), (9, 64, 64),
                                       (17, 1, 64), (130, 1000, 130), (257, 129, 31), (1, 5, 4864)])
def test_edge_shapes(batch, M, K):
    rng, x, W, b = sweep_inputs(batch * M + K, batch, K, M)
    assert maxrel(gpu_fwd(x, W, b), O.linear_fwd(x, W, b)) <= TOL
    dy = rng.standard_normal((batch, M)).astype(np.float32)
    z = [np.zeros(s, np.float32) for s in ((batch, K), (M, K), (M,))]
    for a, r in zip(gpu_bwd(x, W, dy, *z), O.linear_bwd(x, W, dy)):
        assert maxrel(a, r) <= TOL


def test_unaligned_pointers():
    """Sub-buffer views that are not 16-byte aligned take the scalar path."""
    rng, x, W, b = sweep_inputs(99, 70, 128, 64)
    lib = ncmhip.load()
    xb = D.from_numpy(np.concatenate([[0.0], x.reshape(-1)]).astype(np.float32))
    Wb = D.from_numpy(np.concatenate([[0.0], W.reshape(-1)]).astype(np.float32))
    y = D.empty((70, 64))
    lib.linear_fwd(xb.ptr + 4, Wb.ptr + 4, D.from_numpy(b).ptr, y.ptr, 70, 64, 128)
    ncmhip.check()
    assert maxrel(y.numpy(), O.linear_fwd(x, W, b)) <= TOL


def test_zero_batch_is_a_no_op():
    y = D.from_numpy(np.full((4, 8), 7.0, np.float32))
    ncmhip.linear_fwd(D.empty((4, 16)), D.empty((8, 16)), None, y, 0, 8, 16)
    assert np.all(y.numpy() == 7.0)


def test_exact_integer_products():
    """|partial sums| < 2^24: fp32 MFMA accumulation is exact in any order, so
    the GPU must equal the exact product bit for bit (catches any layout or
    k-permutation error that a tolerance could hide)."""
    rng = np.random.default_rng(21)
    for (M, K, N) in ((512, 768, 640), (64, 3072, 256), (1, 896, 500)):
        x = rng.integers(-4, 5, (M, K)).astype(np.float32)
        W = rng.integers(-4, 5, (N, K)).astype(np.float32)
        exact = (x.astype(np.int64) @ W.T.astype(np.int64)).astype(np.float32)
        assert bits_equal(gpu_fwd(x, W, None), exact)
        dy = rng.integers(-4, 5, (M, N)).astype(np.float32)
        dx, dW, db = gpu_bwd(x, W, dy, np.zeros((M, K), np.float32), np.zeros((N, K), np.float32),
                             np.zeros(N, np.float32))
        assert bits_equal(dx, (dy.astype(np.int64) @ W.astype(np.int64)).astype(np.float32))
        assert bits_equal(dW, (dy.T.astype(np.int64) @ x.astype(np.int64)).astype(np.float32))
        assert bits_equal(db, dy.astype(np.int64).sum(0).astype(np.float32))


def test_bias_gradient_batch_sizes():
    """db over batch sizes on both sides of the one-launch column sum's limits
    (16 waves, 512 rows) and column counts that are not whole 64-column
    blocks or 16-byte aligned rows; accumulated onto a non-zero db."""
    rng = np.random.default_rng(23)
    for rows in (1, 15, 16, 17, 100, 511, 512, 513, 1100):
        for N in (1, 63, 130, 2304):
            K = 8
            x = rng.standard_normal((rows, K)).astype(np.float32)
            W = rng.standard_normal((N, K)).astype(np.float32)
            db0 = rng.standard_normal(N).astype(np.float32)
            dyi = rng.integers(-4, 5, (rows, N)).astype(np.float32)
            _, _, db = gpu_bwd(x, W, dyi, None, None, np.zeros(N, np.float32))
            assert bits_equal(db, dyi.astype(np.int64).sum(0).astype(np.float32)), (rows, N)
            dy = rng.standard_normal((rows, N)).astype(np.float32)
            _, _, db = gpu_bwd(x, W, dy, None, None, db0)
            _, _, ref = O.linear_bwd(x, W, dy, db=db0, want=("db",))
            assert maxrel(db, ref) <= TOL, (rows, N)


def test_bias_gradient_inside_dw():
    """With dW requested (aligned rows), db is summed by the dW GEMM itself
    from the dy slabs of its first tile column: whole tiles write it, split
    tiles leave fp64 partials per segment that the fixup adds in segment
    order.  Row counts that are not whole slabs, 4-aligned column counts that
    are not whole 64-row tiles, both plans; accumulated onto a non-zero db.
    Integer data: every sum is exact, so db and dW are compared bit for bit."""
    rng = np.random.default_rng(29)
    segs_seen = set()
    for rows, N, K in ((9, 68, 8), (100, 132, 64), (513, 2304, 768), (4096, 132, 8), (1100, 200, 256),
                       (16384, 200, 64)):
        kernel, segs = ncmhip.linear_plan("dwdb", rows, N, K)
        # (the instance that skips the slabs past a partial last group of four where rows % 128 != 0)
        assert kernel == ("gemm_64x64_dwb_v" if rows % 128 == 0 else "gemm_64x64_dwbt_v"), (rows, kernel)
        segs_seen.add(segs > 1)
        x = rng.integers(-4, 5, (rows, K)).astype(np.float32)
        W = rng.integers(-4, 5, (N, K)).astype(np.float32)
        dy = rng.integers(-4, 5, (rows, N)).astype(np.float32)
        db0 = rng.integers(-50, 51, N).astype(np.float32)
        _, dW, db = gpu_bwd(x, W, dy, None, np.zeros((N, K), np.float32), db0)
        assert bits_equal(db, (db0.astype(np.int64) + dy.astype(np.int64).sum(0)).astype(np.float32)), (rows, N)
        assert bits_equal(dW, (dy.T.astype(np.int64) @ x.astype(np.int64)).astype(np.float32)), (rows, N)
        if rows <= 1100:
            dyf = rng.standard_normal((rows, N)).astype(np.float32)
            dbf = rng.standard_normal(N).astype(np.float32)
            _, _, got = gpu_bwd(x, W, dyf, None, np.zeros((N, K), np.float32), dbf)
            _, _, ref = O.linear_bwd(x, W, dyf, db=dbf, want=("db",))
            assert maxrel(got, ref) <= TOL, (rows, N)
    assert segs_seen == {False, True}


def test_bias_gradient_inside_rank_update():
    """Batch <= 8 with dW requested: the rank-update dW kernel (vectorised and
    scalar rows) adds db from the dy values it loads, in the same fp64 order
    as the column-sum kernel, so db equals the db-only call's bit for bit and
    dW, db equal the oracle's (the reference's host sums) bit for bit."""
    rng = np.random.default_rng(31)
    for rows in (1, 2, 5, 8):
        for N, K in ((1, 8), (63, 12), (130, 7), (2304, 768)):
            assert ncmhip.linear_plan("dwdb", rows, N, K)[0] == ("dw_rank_v" if K % 4 == 0 else "dw_rank_s")
            x = rng.standard_normal((rows, K)).astype(np.float32)
            W = rng.standard_normal((N, K)).astype(np.float32)
            dy = rng.standard_normal((rows, N)).astype(np.float32)
            db0 = rng.standard_normal(N).astype(np.float32)
            dW0 = rng.standard_normal((N, K)).astype(np.float32)
            _, dW, db = gpu_bwd(x, W, dy, None, dW0, db0)
            _, _, db_only = gpu_bwd(x, W, dy, None, None, db0)
            _, ref_dW, ref_db = O.linear_bwd(x, W, dy, dW=dW0, db=db0, want=("dW", "db"))
            assert bits_equal(db, db_only), (rows, N, K)
            assert bits_equal(db, ref_db) and bits_equal(dW, ref_dW), (rows, N, K)


def test_run_to_run_determinism():
    rng, x, W, b = sweep_inputs(3, 512, 3072, 768)
    a = gpu_fwd(x, W, b)
    c = gpu_fwd(x, W, b)
    assert bits_equal(a, c)


@pytest.mark.parametrize("batch,K,ns", [(2048, 896, (896, 128, 128)), (100, 64, (64, 128, 40)),
                                        (300, 256, (128, 64, 64)), (6, 32, (64, 64, 8)), (50, 36, (60, 64, 64))])
def test_three_products_one_launch(batch, K, ns):
    """ncm_linear_fwd3 (the Qwen prefill's q | k | v projections): three
    products of the same x in one GEMM launch, each tile column inside one
    product, against the oracle per product; a ragged last product, a product
    without bias, and the fallbacks (a batch of at most 8, a first width that
    is not whole tiles)."""
    import ctypes
    lib = ncmhip.load()
    rng = np.random.default_rng(batch + K)
    x = rng.standard_normal((batch, K)).astype(np.float32)
    Ws = [(rng.standard_normal((n, K)) / np.sqrt(K)).astype(np.float32) for n in ns]
    bs = [(rng.standard_normal(n) * 0.1).astype(np.float32) if g != 1 else None for g, n in enumerate(ns)]
    xd, Wd = D.from_numpy(x), [D.from_numpy(W) for W in Ws]
    bd = [None if b is None else D.from_numpy(b) for b in bs]
    yd = [D.empty((batch, n)) for n in ns]
    P3 = ctypes.c_void_p * 3
    fn = lib.ncm_linear_fwd3
    fn.restype = None
    fn.argtypes = [ctypes.c_void_p, P3, P3, P3, ctypes.c_int * 3, ctypes.c_int64, ctypes.c_int]
    fn(xd.ptr, P3(*[w.ptr for w in Wd]), P3(*[None if b is None else b.ptr for b in bd]),
       P3(*[y.ptr for y in yd]), (ctypes.c_int * 3)(*ns), batch, K)
    ncmhip.check()
    for g in range(3):
        assert maxrel(yd[g].numpy(), O.linear_fwd(x, Ws[g], bs[g])) <= TOL, g
