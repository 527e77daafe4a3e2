"""Config 1: the NCP transformer forward at its full size (4 layers, d 256,
4 query / 2 kv heads, SwiGLU 1024, vocab 16, 64 boards x 81 tokens) on the
device against the oracle's op-for-op restatement of ncp_block, which is
bit-equal to the reference's own ncp_forward (tests/test_oracle_models.py).
Bar: logits max-abs 1e-3 (north star), asserted as 1e-4."""
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
    ncmhip.load().arena_init(2 << 30)
    ncmhip.check()
    print("[gpu] ncp tests on device 0", flush=True)


def ncp_weights(seed, n_layer, C, H, Kv, I, V, biases=True):
    """N(0, 0.02) matrices and biases; norm gains 1, norm biases 0 (the
    tools/mkinit.py convention)."""
    rng = np.random.default_rng(seed)
    shapes = O.ncp_shapes(n_layer, C, H, Kv, I, V)
    ps = []
    n = len(shapes)
    for i, s in enumerate(shapes):
        j = (i - 1) % 14 if 1 <= i < n - 4 else None
        if j in (0, 6) or i == n - 4:
            ps.append(np.ones(s, np.float32))
        elif j in (1, 7) or i == n - 3:
            ps.append(np.zeros(s, np.float32))
        elif len(s) == 1 and not biases:
            ps.append(None)
        else:
            ps.append((0.02 * rng.standard_normal(s)).astype(np.float32))
    return ps


@pytest.mark.parametrize("biases", [True, False])
def test_ncp_forward_full_size(biases):
    n_layer, C, H, Kv, I, V, B, S = 4, 256, 4, 2, 1024, 16, 64, 81
    params = ncp_weights(1, n_layer, C, H, Kv, I, V, biases)
    ids = np.random.default_rng(2).integers(0, V, (B, S)).astype(np.int32)
    ref = O.ncp_forward(params, n_layer, C, H, Kv, I, V, ids)
    bufs = [None if p is None else D.from_numpy(p) for p in params]
    cfg = ncmhip.NcpConfig(n_layer, C, H, Kv, I, V, 10000)
    lib = ncmhip.load()
    p = lib.ncm_ncp_forward(ctypes.byref(cfg), ncmhip.ptr_array(bufs), ids.ctypes.data, B, S)
    ncmhip.check()
    got = np.empty((B * S, V), np.float32)
    lib.mem_d2h(got.ctypes.data, p, got.nbytes)
    ncmhip.check()
    assert float(np.max(np.abs(got - ref))) <= 1e-4
