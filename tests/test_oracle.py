"""The CPU oracle pinned against the reference: its own kernel checksum
harness (tests/ktest_kernels.c), golden vectors written by the reference's
CPU code, the reference compiled from source (where present), and results
that the mathematics fixes (exact integer arithmetic, closed forms, brute
force)."""
import os

import numpy as np
import pytest

import oracle as O
from conftest import GOLDEN, bits_equal


# ---------------------------------------------------------------- ktest KATs
def _ktest_lines():
    out = {}
    for line in open(os.path.join(GOLDEN, "ktest_cpu.txt")):
        if " sum=" in line:
            out[line.split()[0]] = line.strip()
    return out


def _chk_line(name, v):
    v = np.asarray(v, np.float32).reshape(-1)
    s = float(np.cumsum(v.astype(np.float64))[-1])
    mx = float(np.max(np.abs(v.astype(np.float64))))
    return "%s sum=%.6f maxabs=%.6f first=%.6f %.6f %.6f %.6f" % (name, s, mx, v[0], v[1], v[2], v[3])


def _ktest_inputs():
    """Replays the generator order of tests/ktest_kernels.c:33-103 up to the
    l2sq and linear cases and returns their inputs."""
    st = 0x12345678
    seq = {}

    def mk(n):
        nonlocal st
        v, st = O.ktest_fill(st, n)
        return v
    for n in (256, 64, 64, 256, 256, 64, 256, 512, 512, 1024, 1024, 512, 512,
              256, 384, 384, 96, 256, 256, 48, 4, 256):
        mk(n)
    seq["l2_a"], seq["l2_b"] = mk(16 * 32), mk(8 * 32)
    mk(16 * 8)
    seq["x"], seq["W"], seq["b"] = mk(8 * 64), mk(128 * 64), mk(128)
    return seq


def test_ktest_linear_checksum():
    seq = _ktest_inputs()
    y = O.linear_fwd(seq["x"].reshape(8, 64), seq["W"].reshape(128, 64), seq["b"])
    assert _chk_line("linear", y) == _ktest_lines()["linear"]


def test_ktest_l2sq_checksum():
    seq = _ktest_inputs()
    d2 = O.l2sq(seq["l2_a"].reshape(16, 32), seq["l2_b"].reshape(8, 32))
    assert _chk_line("l2sq", d2) == _ktest_lines()["l2sq"]


# ---------------------------------------------------------- golden vectors
def test_golden_linear(golden):
    g = golden("linear_ref.npz")
    for i in range(int(g["n_cases"])):
        p = f"c{i}_"
        b = g[p + "b"] if p + "b" in g else None
        assert bits_equal(O.linear_fwd(g[p + "x"], g[p + "W"], b), g[p + "y"]), i
        db0 = g[p + "db0"] if b is not None else None
        dx, dW, db = O.linear_bwd(g[p + "x"], g[p + "W"], g[p + "dy"], g[p + "dx0"], g[p + "dW0"], db0,
                                  want=("dx", "dW", "db") if b is not None else ("dx", "dW"))
        assert bits_equal(dx, g[p + "dx"]), i
        assert bits_equal(dW, g[p + "dW"]), i
        if b is not None:
            assert bits_equal(db, g[p + "db"]), i


def test_golden_vq(golden):
    g = golden("vq_ref.npz")
    B, L = int(g["B"]), int(g["L"])
    Es = [g[f"E{i}"] for i in range(3)]
    idx, z_hat, z_rest = O.vq_multiscale(g["z"], Es, B, L)
    assert np.array_equal(idx, g["idx"])
    assert bits_equal(z_hat, g["z_hat"]) and bits_equal(z_rest, g["z_rest"])
    # planted row 5 = E0[77] = E0[90]: distance 0, lowest index wins
    assert idx[0, 5] == 77
    assert bits_equal(O.l2sq(g["l2_a"], g["l2_b"]), g["l2_d2"])


# ------------------------------------------- the reference compiled here
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference not compiled here")


@needs_ref
@pytest.mark.parametrize("seed", [1, 2])
def test_vs_reference_linear(seed):
    rng = np.random.default_rng(seed)
    batch, M, K = 67, 96, 181
    x = rng.standard_normal((batch, K)).astype(np.float32)
    W = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal(M).astype(np.float32)
    dy = rng.standard_normal((batch, M)).astype(np.float32)
    assert bits_equal(O.linear_fwd(x, W, b), O.ref_linear_fwd(x, W, b))
    ours = O.linear_bwd(x, W, dy)
    theirs = O.ref_linear_bwd(x, W, b, dy)
    for a, r in zip(ours, theirs):
        assert bits_equal(a, r)


@needs_ref
def test_vs_reference_vq_multiscale():
    rng = np.random.default_rng(7)
    B, L, D, V = 3, 50, 48, 200
    z = rng.standard_normal((B * L, D)).astype(np.float32)
    Es = [(rng.standard_normal((V, D)) / np.sqrt(D)).astype(np.float32) for _ in range(4)]
    Es[1][150] = Es[1][20]
    a = O.vq_multiscale(z, Es, B, L)
    r = O.ref_vq_multiscale(z, Es, B, L)
    assert np.array_equal(a[0], r[0])
    assert bits_equal(a[1], r[1]) and bits_equal(a[2], r[2])


# ------------------------------------------------- what mathematics fixes
def test_linear_exact_integers():
    """Small integer operands: every fp64 partial sum is exact, so the oracle
    must equal the exact integer product (catches transposed operands, wrong
    strides, dropped bias)."""
    rng = np.random.default_rng(3)
    batch, M, K = 23, 31, 300
    x = rng.integers(-8, 9, (batch, K))
    W = rng.integers(-8, 9, (M, K))
    b = rng.integers(-50, 51, M)
    y = O.linear_fwd(x.astype(np.float32), W.astype(np.float32), b.astype(np.float32))
    assert np.array_equal(y.astype(np.int64), x @ W.T + b)
    dy = rng.integers(-8, 9, (batch, M))
    dx0 = rng.integers(-5, 6, (batch, K))
    dx, dW, db = O.linear_bwd(x.astype(np.float32), W.astype(np.float32), dy.astype(np.float32),
                              dx0.astype(np.float32))
    assert np.array_equal(dx.astype(np.int64), dx0 + dy @ W)
    assert np.array_equal(dW.astype(np.int64), dy.T @ x)
    assert np.array_equal(db.astype(np.int64), dy.sum(0))


def test_linear_bias_only_and_identity():
    rng = np.random.default_rng(4)
    b = rng.standard_normal(17).astype(np.float32)
    assert bits_equal(O.linear_fwd(np.zeros((3, 9), np.float32), rng.standard_normal((17, 9)), b),
                      np.tile(b, (3, 1)))
    x = rng.standard_normal((5, 12)).astype(np.float32)
    assert bits_equal(O.linear_fwd(x, np.eye(12, dtype=np.float32)), x)


def test_linear_rounding_is_single():
    """fp64 accumulation then one rounding: equals float32(exact sum) when the
    exact sum is representable in fp64 (small dyadic inputs)."""
    rng = np.random.default_rng(5)
    x = (rng.integers(-1000, 1000, (4, 64)) / 1024.0).astype(np.float32)
    W = (rng.integers(-1000, 1000, (8, 64)) / 4096.0).astype(np.float32)
    exact = (x.astype(np.float64) @ W.T.astype(np.float64)).astype(np.float32)
    assert bits_equal(O.linear_fwd(x, W), exact)


def test_l2sq_brute_force():
    rng = np.random.default_rng(6)
    a = rng.integers(-20, 21, (13, 40)).astype(np.float32)
    b = rng.integers(-20, 21, (17, 40)).astype(np.float32)
    exact = ((a[:, None, :].astype(np.int64) - b[None, :, :]) ** 2).sum(-1)
    assert np.array_equal(O.l2sq(a, b).astype(np.int64), exact)


def test_vq_argmin_ties_brute_force():
    """Integer data make many exact distance ties: the code must be the lowest
    index of the minimum (numpy argmin returns the first occurrence)."""
    rng = np.random.default_rng(8)
    a = rng.integers(-2, 3, (300, 6)).astype(np.float32)
    E = rng.integers(-2, 3, (64, 6)).astype(np.float32)
    d = ((a[:, None, :].astype(np.int64) - E[None, :, :]) ** 2).sum(-1)
    assert np.array_equal(O.vq_argmin(a, E), d.argmin(1))
    assert (d.min(1)[:, None] == d).sum(1).max() > 1  # ties do occur


def test_vq_multiscale_integer_invariants():
    rng = np.random.default_rng(9)
    B, L, D = 2, 40, 8
    z = rng.integers(-6, 7, (B * L, D)).astype(np.float32)
    Es = [rng.integers(-3, 4, (16, D)).astype(np.float32) for _ in range(3)]
    idx, z_hat, z_rest = O.vq_multiscale(z, Es, B, L)
    assert np.array_equal(z_hat + z_rest, z)
    rest = z.astype(np.int64)
    for lv, E in enumerate(Es):
        d = ((rest[:, None, :] - E[None].astype(np.int64)) ** 2).sum(-1)
        codes = d.argmin(1)
        got = idx[:, lv * L:(lv + 1) * L].reshape(-1)
        assert np.array_equal(got, codes)
        rest = rest - E[codes].astype(np.int64)
    assert np.array_equal(z_rest.astype(np.int64), rest)


def test_argmax_semantics():
    assert O.argmax_row(np.array([1, 3, 3, 2], np.float32)) == 1
    assert O.argmax_row(np.array([np.nan, 3, 4], np.float32)) == 0
    assert O.argmax_row(np.array([1, np.nan, 4, 4], np.float32)) == 2
    assert O.argmax_row(np.array([-np.inf, -np.inf], np.float32)) == 0


def test_activations_closed_form():
    import math
    x = np.linspace(-6, 6, 2001).astype(np.float32)
    xd = x.astype(np.float64)
    silu = xd / (1 + np.exp(-xd))
    gelu = 0.5 * xd * (1 + np.array([math.erf(v / math.sqrt(2)) for v in xd]))
    gtanh = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3)))
    for name, ref in (("silu", silu), ("gelu", gelu), ("gelu_tanh", gtanh)):
        assert np.max(np.abs(O.act(name, x) - ref)) < 2e-6, name


def test_thread_count_invariance():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((40, 70)).astype(np.float32)
    W = rng.standard_normal((50, 70)).astype(np.float32)
    dy = rng.standard_normal((40, 50)).astype(np.float32)
    O.set_threads(1)
    a = O.linear_fwd(x, W), O.linear_bwd(x, W, dy)
    O.set_threads(8)
    b = O.linear_fwd(x, W), O.linear_bwd(x, W, dy)
    assert bits_equal(a[0], b[0])
    for p, q in zip(a[1], b[1]):
        assert bits_equal(p, q)
