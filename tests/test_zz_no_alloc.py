"""vq_argmin_noalloc (the allocation-free VQ search) against vq_argmin: the
same codes bit for bit, on two calls in a row, the second smaller, so that
whatever the first call left in the shared fixed scratch cannot leak into the
second.  The data plant exact ties (duplicated codewords), near ties and
rows on codewords, so the pair and full rescore lists in the scratch are
used, not only the certified path."""
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
    print("[gpu] no-alloc vq tests on device 0", flush=True)


def tie_heavy(rows, V, Dm, seed):
    """Integer-valued codebook with duplicates, rows on / between codewords."""
    rng = np.random.default_rng(seed)
    E = rng.integers(-3, 4, size=(V, Dm)).astype(np.float32)
    E[V // 2:V // 2 + 8] = E[3:11]                     # duplicated codewords: lowest index wins
    a = rng.integers(-3, 4, size=(rows, Dm)).astype(np.float32)
    pick = rng.integers(0, V, size=rows // 3)
    a[:rows // 3] = E[pick]                             # rows on codewords (often duplicated ones)
    j, k = rng.integers(0, V, size=(2, rows // 6))
    a[rows // 3:rows // 3 + rows // 6] = 0.5 * (E[j] + E[k])   # midpoints: exact two-way ties
    a[rows - rows // 6:] += rng.standard_normal((rows // 6, Dm)).astype(np.float32) * 1e-3
    return a, E


def run_both(a, E):
    rows, Dm = a.shape
    V = E.shape[0]
    ad, Ed = D.from_numpy(a), D.from_numpy(E)
    want = D.empty(rows, np.int32)
    got = D.from_numpy(np.full(rows, -7, np.int32))
    assert ncmhip.vq_argmin_noalloc(ad, Ed, got, rows, V, Dm) == 0
    ncmhip.vq_argmin(ad, Ed, want, rows, V, Dm)
    return got.numpy(), want.numpy()


def hip_free_bytes():
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_noalloc_matches_vq_argmin_twice():
    # call 1, then a smaller call 2 on the same fixed scratch
    for rows, V, Dm, seed in ((20000, 1500, 96, 1), (3001, 700, 40, 2)):
        print(f"[gpu] noalloc rows={rows} V={V} D={Dm}", flush=True)
        a, E = tie_heavy(rows, V, Dm, seed)
        got, want = run_both(a, E)
        assert np.array_equal(got, want), f"rows={rows}: {int((got != want).sum())} codes differ"
    # the small call against the CPU reference restatement too
    assert np.array_equal(got, O.vq_argmin(a, E))


def test_noalloc_random_then_smaller():
    rng = np.random.default_rng(5)
    for rows, V, Dm in ((65536, 4096, 256), (777, 4096, 256)):
        print(f"[gpu] noalloc random rows={rows} V={V} D={Dm}", flush=True)
        a = rng.standard_normal((rows, Dm)).astype(np.float32)
        E = (rng.standard_normal((V, Dm)) / np.sqrt(Dm)).astype(np.float32)
        got, want = run_both(a, E)
        assert np.array_equal(got, want)


def test_noalloc_allocates_nothing():
    # warm the kernels up first, then a shape whose workspace would need
    # more than any earlier search in this process (200000 rows x 32 B)
    a, E = tie_heavy(64, 512, 64, 3)
    run_both(a, E)
    ncmhip.sync()
    rng = np.random.default_rng(9)
    rows, V, Dm = 200000, 512, 64
    a = rng.standard_normal((rows, Dm)).astype(np.float32)
    E = (rng.standard_normal((V, Dm)) / 8).astype(np.float32)
    ad, Ed, idx = D.from_numpy(a), D.from_numpy(E), D.empty(rows, np.int32)
    ncmhip.sync()
    before = hip_free_bytes()
    assert ncmhip.vq_argmin_noalloc(ad, Ed, idx, rows, V, Dm) == 0
    ncmhip.sync()
    after = hip_free_bytes()
    assert after == before, f"device free memory moved by {before - after} bytes"
    want = D.empty(rows, np.int32)
    ncmhip.vq_argmin(ad, Ed, want, rows, V, Dm)
    assert np.array_equal(idx.numpy(), want.numpy())


def test_noalloc_refuses_beyond_limits():
    a, E = D.empty((4, 8)), D.empty((4, 8))
    idx = D.empty(4, np.int32)
    with pytest.raises(ncmhip.NcmError, match="limits"):
        ncmhip.vq_argmin_noalloc(a, E, idx, (1 << 18) + 1, 4, 8)
    with pytest.raises(ncmhip.NcmError, match="limits"):
        ncmhip.vq_argmin_noalloc(a, E, idx, 4, (1 << 16) + 1, 8)
