"""Oracle pinning for sample_topkp (src/kernels.c:782-825): the reference's
own function compiled from source (ids and the advanced rng state, bit for
bit), the golden draws it wrote, and closed forms a wrong sort direction,
tie order, nucleus rule or rng step would break.  Plus the library's
argument checks, which need no GPU."""
import numpy as np
import pytest

import ncmhip
import oracle as O
from conftest import GOLDEN

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference not compiled here")


def sample_row(gen):
    """tests/golden/gen_golden.py sample_row: the ktest generator times scale."""
    seed, V, scale, ties = gen
    x, _ = O.ktest_fill(int(seed), int(V))
    x = (x * np.float32(scale)).astype(np.float32)
    return (np.round(x * 2) / 2).astype(np.float32) if ties else x


def golden_cases():
    g = np.load(f"{GOLDEN}/sample_ref.npz", allow_pickle=False)
    for i in range(int(g["n_cases"])):
        x = g[f"c{i}_x"] if f"c{i}_x" in g else sample_row(g[f"c{i}_gen"])
        temp, k, p = g[f"c{i}_cfg"]
        yield i, x, float(temp), int(k), float(p), [int(v) for v in g[f"c{i}_rng"]], [int(v) for v in g[f"c{i}_ids"]]


def test_oracle_matches_golden_draws():
    n = 0
    for i, x, temp, k, p, sts, ids in golden_cases():
        s = sts[0]
        for d in range(4):
            j, s = O.sample_topkp(x, temp, k, p, s)
            assert (j, s) == (ids[d], sts[d + 1]), (i, d)
        n += 1
    assert n == 8


@needs_ref
def test_oracle_matches_reference_random():
    rng = np.random.default_rng(5)
    for t in range(150):
        V = int(rng.integers(1, 4000)) if t % 6 else 151936
        x = (rng.standard_normal(V) * rng.uniform(0.1, 6)).astype(np.float32)
        if t % 3 == 0:
            x = np.round(x).astype(np.float32)
        if t % 7 == 0:
            x[rng.integers(0, V)] = -0.0
        temp = float(rng.choice([0.0, -1.0, 0.25, 0.7, 1.0, 1.7]))
        k = int(rng.choice([0, 1, 2, 7, 50, V, V + 5]))
        p = float(rng.choice([0.0, 0.3, 0.9, 0.97, 1.0, 3.0]))
        st = int(rng.integers(1, 2 ** 63))
        assert O.sample_topkp(x, temp, k, p, st) == O.ref_sample_topkp(x, temp, k, p, st), t


def test_greedy_when_temperature_not_positive():
    x = np.array([0.5, 2.0, -1.0, 2.0], np.float32)
    for temp in (0.0, -2.0, float("nan")):
        assert O.sample_topkp(x, temp, 0, 1.0, 77) == (1, 77)   # first maximum, rng untouched


def test_top_k_one_is_the_first_maximum():
    x = np.array([0.5, 3.0, 3.0, 1.0], np.float32)
    for st in range(1, 40):
        j, s = O.sample_topkp(x, 1.0, 1, 1.0, st)
        assert j == 1 and s != st   # the tie resolves to the lower index; one rng step


def test_two_point_frequencies():
    # w = (0, ln 3): q = (1/4, 3/4) for indices (0, 1)
    x = np.array([0.0, np.log(3.0)], np.float32)
    s, hits, n = 12345, 0, 4000
    for _ in range(n):
        j, s = O.sample_topkp(x, 1.0, 0, 1.0, s)
        hits += j == 1
    assert abs(hits - 0.75 * n) < 4 * np.sqrt(n * 0.75 * 0.25)


def test_nucleus_rule():
    # q = (0.5, 0.3, 0.2): F_r = cum_r - q_r = (-0.5, 0.2, 0.6).  top_p 0.1 cuts
    # after rank 0 (only index of 0.5 survives); top_p 0.5 keeps two ranks.
    w = np.log(np.array([0.3, 0.5, 0.2]))
    x = w.astype(np.float32)
    s = 9
    for _ in range(50):
        j, s = O.sample_topkp(x, 1.0, 0, 0.1, s)
        assert j == 1
    seen = set()
    for _ in range(200):
        j, s = O.sample_topkp(x, 1.0, 0, 0.5, s)
        seen.add(j)
    assert seen == {0, 1}


def test_rng_is_one_xorshift_step():
    x = np.zeros(10, np.float32)
    st = 0x1234567
    _, s = O.sample_topkp(x, 1.0, 0, 1.0, st)
    s2 = np.uint64(st)
    s2 ^= s2 >> np.uint64(12)
    s2 ^= (s2 << np.uint64(25)) & np.uint64(0xFFFFFFFFFFFFFFFF)
    s2 ^= s2 >> np.uint64(27)
    assert s == int(s2)


def test_library_argument_checks():
    ncmhip.load()
    x = np.zeros(4, np.float32)
    with pytest.raises(ncmhip.NcmError, match="top_p"):
        ncmhip.sample_topkp(x, 1.0, 0, -0.5, 1)
    with pytest.raises(ncmhip.NcmError, match="V <= 262144"):
        ncmhip.sample_topkp(np.zeros(262145, np.float32), 1.0, 0, 1.0, 1)
    # greedy stays on the host row (the reference's argmax_row), rng untouched
    assert ncmhip.sample_topkp(np.array([1, 4, 4], np.float32), 0.0, 0, 1.0, 5) == (1, 5, 0)


def test_library_rng_next_is_the_reference_generator():
    import ctypes
    lib = ncmhip.load()
    a, b = ctypes.c_uint64(99), ctypes.c_uint64(99)
    for _ in range(5):
        assert lib.rng_next(ctypes.byref(a)) == O.lib().orc_rng_next(ctypes.byref(b))
        assert a.value == b.value
