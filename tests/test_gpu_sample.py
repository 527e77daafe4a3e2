"""GPU sampler (sample_topkp_dev, sample_topkp) against the oracle and the
reference's golden draws: the same id and the same advanced rng state, with
the certification flag 0 (a flag of 1 marks a draw inside the rounding
bound of a cumulative boundary, where the device and glibc exp could
disagree; such draws are counted and must stay rare)."""
import numpy as np
import pytest

import ncmhip
import oracle as O
from test_oracle_sample import golden_cases

pytestmark = pytest.mark.gpu
D = ncmhip.DeviceBuffer


@pytest.fixture(scope="module", autouse=True)
def device():
    ncmhip.init(0)
    print("[gpu] sampler tests on device 0", flush=True)


class DevSampler:
    def __init__(self, x):
        self.V = x.size
        self.x = D.from_numpy(np.ascontiguousarray(x, np.float32))
        self.rng = D.empty(1, np.uint64)
        self.out = D.empty(1, np.int32)
        self.flag = D.empty(1, np.int32)

    def draw(self, temp, k, p, st=None):
        if st is not None:
            self.rng.upload(np.array([st], np.uint64))
        ncmhip.sample_topkp_dev(self.x, self.V, temp, k, p, self.rng, self.out, self.flag)
        return int(self.out.numpy()[0]), int(self.rng.numpy()[0]), int(self.flag.numpy()[0])


def test_golden_draws_device_and_host_entry():
    for i, x, temp, k, p, sts, ids in golden_cases():
        print(f"[gpu] golden case {i}: V={x.size} temp={temp} k={k} p={p}", flush=True)
        s = DevSampler(x)
        st = sts[0]
        s.rng.upload(np.array([st], np.uint64))
        for d in range(4):
            j, st_dev, fl = s.draw(temp, k, p)   # the device rng chains draw to draw
            assert fl == 0 and (j, st_dev) == (ids[d], sts[d + 1]), (i, d, j, fl)
            jh, st_h, flh = ncmhip.sample_topkp(x, temp, k, p, sts[d])
            assert flh == 0 and (jh, st_h) == (ids[d], sts[d + 1]), (i, d, jh)


def test_random_rows_match_oracle():
    rng = np.random.default_rng(11)
    flagged = 0
    n = 0
    for t in range(90):
        V = int(rng.choice([1, 2, 3, 100, 1023, 1024, 1025, 2047, 2049, 5000, 40000, 151936, 262144]))
        x = (rng.standard_normal(V) * rng.uniform(0.05, 8)).astype(np.float32)
        if t % 3 == 0:
            x = np.round(x * rng.choice([1, 4])).astype(np.float32)   # ties
        if t % 5 == 0:
            x[rng.integers(0, V, size=min(V, 7))] = np.float32(-0.0)
        temp = float(rng.choice([0.05, 0.3, 0.7, 1.0, 2.5]))
        k = int(rng.choice([0, 0, 1, 2, 40, 1000, 1500, V, V + 1]))
        p = float(rng.choice([0.0, 0.5, 0.9, 0.95, 1.0, 1.0, 2.0]))
        st = int(rng.integers(1, 2 ** 63))
        want = O.sample_topkp(x, temp, k, p, st)
        j, s, fl = DevSampler(x).draw(temp, k, p, st)
        assert fl in (0, 1), (t, fl)
        assert s == want[1], t
        if fl:
            flagged += 1
            continue
        assert j == want[0], (t, V, temp, k, p, j, want[0])
        n += 1
    assert flagged <= 2 and n >= 85


def test_consecutive_draws_on_one_row():
    x = (np.random.default_rng(3).standard_normal(151936) * 3).astype(np.float32)
    s = DevSampler(x)
    st = 0xC0FFEE
    s.rng.upload(np.array([st], np.uint64))
    for d in range(20):
        want = O.sample_topkp(x, 0.8, 0, 0.9, st)
        j, st_dev, fl = s.draw(0.8, 0, 0.9)
        assert fl == 0 and (j, st_dev) == want, d
        st = want[1]


def test_greedy_path_leaves_rng():
    x = np.array([0.25, 7.0, 7.0, -3.0], np.float32)
    s = DevSampler(x)
    for temp in (0.0, -1.0):
        assert s.draw(temp, 0, 1.0, 42) == (1, 42, 0)


def test_non_finite_rows_are_flagged():
    x = np.zeros(3000, np.float32)
    x[17] = np.inf
    j, st, fl = DevSampler(x).draw(1.0, 0, 1.0, 5)
    assert fl == 2 and 0 <= j < 3000


M64 = (1 << 64) - 1
XS_MUL = 0x2545F4914F6CDD1D


def state_drawing_half():
    """An xorshift64* state whose next draw gives U = 0.5 exactly (output
    2^63): the multiplier is inverted mod 2^64 and the three xorshift steps
    undone in reverse order."""
    y = (1 << 63) * pow(XS_MUL, -1, 1 << 64) & M64
    y ^= (y >> 27) ^ (y >> 54)                                      # x ^= x >> 27
    y = (y ^ (y << 25) ^ (y << 50)) & M64                           # x ^= x << 25
    y ^= (y >> 12) ^ (y >> 24) ^ (y >> 36) ^ (y >> 48) ^ (y >> 60)  # x ^= x >> 12
    return y


def reference_draw(x, temp, k, p, st):
    if O.ref_available():
        return O.ref_sample_topkp(x, temp, k, p, st)
    pytest.skip("oracle/_ref/libref.so (the reference's sampler) is not built here")


def test_host_entry_redraws_on_a_cumulative_boundary():
    """u lands exactly on a cumulative sum (four equal logits, U = 0.5): the
    device cannot certify such a draw, and the host entry point must return
    the reference's own pick and rng state."""
    st = state_drawing_half()
    assert (O.sample_topkp(np.zeros(4, np.float32), 1.0, 0, 1.0, st)[1] * XS_MUL & M64) >> 11 == 1 << 52
    for V, hot in ((4, [0, 1, 2, 3]), (151936, [5, 77, 140000, 151935])):
        x = np.full(V, -1e4, np.float32)
        x[hot] = 3.0
        for temp, k, p in ((1.0, 0, 1.0), (0.7, 0, 0.99), (1.0, 4, 1.0), (1.0, 1000, 0.9)):
            want = reference_draw(x, temp, k, p, st)
            j, s2, fl = DevSampler(x).draw(temp, k, p, st)
            assert fl == 1 and s2 == want[1], (V, temp, k, p, fl)
            got = ncmhip.sample_topkp(x, temp, k, p, st)
            print(f"[gpu] boundary V={V} temp={temp} k={k} p={p}: device {j}, host entry {got[0]}, "
                  f"reference {want[0]}", flush=True)
            assert got == (want[0], want[1], 1), (V, temp, k, p, got, want)


@pytest.mark.parametrize("kind", ["inf", "nan", "neg_inf_mix", "all_nan"])
def test_host_entry_non_finite_rows_match_reference(kind):
    rng = np.random.default_rng(17)
    x = rng.standard_normal(3000).astype(np.float32)
    if kind == "inf":
        x[[17, 2500]] = np.inf
    elif kind == "nan":
        x[[3, 900, 2999]] = np.nan
    elif kind == "neg_inf_mix":
        x[[0, 1, 2]] = -np.inf
        x[1500] = np.inf
        x[10] = np.nan
    else:
        x[:] = np.nan
    for temp, k, p, st in ((1.0, 0, 1.0, 5), (0.5, 40, 0.9, 12345), (2.0, 0, 0.0, 99)):
        want = reference_draw(x, temp, k, p, st)
        got = ncmhip.sample_topkp(x, temp, k, p, st)
        assert got[:2] == want and got[2] == 2, (kind, temp, k, p, got, want)
