"""The 128 x 128-tile GEMM kernels (gemm_128x128_*_v) against exact integer
products and the oracle, forced onto shapes with ragged tiles through
ncm_hip_set_gemm_tiles(128); the training step (fused forward, head-major,
dX-through-activation and dW+db kernels) on them against the oracle; and
the cost model's choice at the config-5 shapes."""
import numpy as np
import pytest

import ncmhip
import oracle as O
from conftest import bits_equal, maxrel
from test_gpu_gpt2 import CASES as GPT2_CASES
from test_gpu_gpt2 import test_gpt2_grads as gpt2_step

pytestmark = pytest.mark.gpu
D = ncmhip.DeviceBuffer


@pytest.fixture(scope="module", autouse=True)
def device():
    ncmhip.init(0)
    ncmhip.load().arena_init(4 << 30)
    ncmhip.check()
    print("[gpu] 128x128 GEMM tests on device 0", flush=True)


@pytest.fixture
def big_tiles():
    lib = ncmhip.load()
    lib.ncm_hip_set_gemm_tiles(128)
    yield
    lib.ncm_hip_set_gemm_tiles(0)


def fwd(x, W, b=None, res=None, act="none"):
    M, K = x.shape
    N = W.shape[0]
    y = D.empty((M, N))
    ncmhip.linear_fwd(D.from_numpy(x), D.from_numpy(W), None if b is None else D.from_numpy(b), y, M, N, K,
                      res=None if res is None else D.from_numpy(res), act=act)
    return y.numpy()


def bwd(x, W, dy, dx0, dW0, db0):
    M, K = x.shape
    N = W.shape[0]
    dx, dW, db = (None if a is None else D.from_numpy(a) for a in (dx0, dW0, db0))
    ncmhip.linear_bwd(D.from_numpy(x), D.from_numpy(W), D.from_numpy(dy), dx, dW, db, M, N, K)
    return tuple(None if a is None else a.numpy() for a in (dx, dW, db))


@pytest.mark.parametrize("M,K,N", [(300, 200, 260), (128, 32, 128), (1000, 768, 2304), (136, 4, 132),
                                   (260, 1028, 384)])
def test_big_tiles_exact_integer_products(big_tiles, M, K, N):
    """|partial sums| < 2^24: exact in any order, so forward, dX, dW and db
    must equal the integer products bit for bit, partial tiles included."""
    kern = ncmhip.linear_plan("fwd", M, N, K)[0]
    print(f"[gpu] {M}x{K}->{N}: {kern}, {ncmhip.linear_plan('dx', M, N, K)[0]}, "
          f"{ncmhip.linear_plan('dwdb', M, N, K)[0]}", flush=True)
    assert kern == "gemm_128x128_fwd_v"
    assert ncmhip.linear_plan("dx", M, N, K)[0] == "gemm_128x128_dx_v"
    assert ncmhip.linear_plan("dwdb", M, N, K)[0] == "gemm_128x128_dwb_v"
    rng = np.random.default_rng(M + K + N)
    x = rng.integers(-4, 5, (M, K)).astype(np.float32)
    W = rng.integers(-4, 5, (N, K)).astype(np.float32)
    assert bits_equal(fwd(x, W), (x.astype(np.int64) @ W.T.astype(np.int64)).astype(np.float32))
    dy = rng.integers(-4, 5, (M, N)).astype(np.float32)
    dx0 = rng.integers(-9, 10, (M, K)).astype(np.float32)
    dW0 = rng.integers(-9, 10, (N, K)).astype(np.float32)
    db0 = rng.integers(-9, 10, N).astype(np.float32)
    dx, dW, db = bwd(x, W, dy, dx0, dW0, db0)
    i64 = np.int64
    assert bits_equal(dx, (dx0.astype(i64) + dy.astype(i64) @ W.astype(i64)).astype(np.float32))
    assert bits_equal(dW, (dW0.astype(i64) + dy.T.astype(i64) @ x.astype(i64)).astype(np.float32))
    assert bits_equal(db, (db0.astype(i64) + dy.astype(i64).sum(0)).astype(np.float32))


@pytest.mark.parametrize("act", ["none", "silu", "gelu", "gelu_tanh"])
def test_big_tiles_epilogues_vs_oracle(big_tiles, act):
    rng = np.random.default_rng(5)
    M, K, N = 260, 384, 200
    x = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    b = (rng.standard_normal(N) * 0.02).astype(np.float32)
    res = rng.standard_normal((M, N)).astype(np.float32)
    want = O.linear_fwd(x, W, b)
    if act != "none":
        want = O.act(act, want)
    assert maxrel(fwd(x, W, b, res=res, act=act), want + res) <= 1e-4
    dy = rng.standard_normal((M, N)).astype(np.float32)
    g0 = [rng.standard_normal(s).astype(np.float32) for s in ((M, K), (N, K), (N,))]
    for name, a, r in zip(("dx", "dW", "db"), bwd(x, W, dy, *g0), O.linear_bwd(x, W, dy, *g0)):
        assert maxrel(a, r) <= 1e-4, name


def test_big_tiles_training_step(big_tiles):
    """The 2-layer GPT-2 step at config-5 widths (T = 128: the head-major
    q | k | v forward and the c_proj dX into the heads' gradient take 128-row
    tiles too) on 128 x 128 tiles, against the oracle at the step test's bar."""
    gpt2_step(*GPT2_CASES[0])


def test_cost_model_choice():
    """The cost model keeps 64 x 64 tiles for the config-5 and linear-sweep
    products (K <= 3072: the 128 x 128 tiles' fixed cost per tile is not paid
    back) and takes the 128 x 128 tiles for long reductions over whole pairs
    of tiles per CU."""
    for op, R, M, K in (("fwd", 16384, 2304, 768), ("fwd", 16384, 3072, 768), ("dx", 16384, 768, 3072),
                        ("fwd", 4096, 3072, 768), ("dx", 4096, 768, 3072)):
        kern = ncmhip.linear_plan(op, R, M, K)[0]
        print(f"[gpu] {op} {R} x {K}->{M}: {kern}", flush=True)
        assert kern.startswith("gemm_64x64_"), (op, R, M, K, kern)
    for op, R, M, K in (("fwd", 8192, 1024, 8192), ("dx", 8192, 8192, 1024)):
        kern = ncmhip.linear_plan(op, R, M, K)[0]
        print(f"[gpu] {op} {R} x {K}->{M}: {kern}", flush=True)
        assert kern.startswith("gemm_128x128_"), (op, R, M, K, kern)
