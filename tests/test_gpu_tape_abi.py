"""The tape at link level: tests/_build/tape_check, a GPT-2 training step
written against the reference's own src/ncm.h (tests/c/tape_check.c: the
t_* calls of train_gpt2.c:42-147 and tape_backward(tp, &pm, 0) of
:146-159) and linked to libncmhip_tape.so + libncmhip.so, with no library-
specific call.  Its loss and gradients are checked against the oracle's
taped step (bit-equal to the reference's own train_gpt2_forward + t_ce +
tape_backward_host) at the GPT-2 step test's bar, and bit for bit against
the library's own ncm_gpt2_forward driver, whose fused records give the
unfused records' values."""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import ncmhip
import oracle as O
from conftest import ROOT

pytestmark = pytest.mark.gpu
BIN = os.path.join(ROOT, "tests", "_build", "tape_check")
D = ncmhip.DeviceBuffer


class PMap(ctypes.Structure):
    _fields_ = [("params", ctypes.c_void_p), ("grads", ctypes.c_void_p), ("sizes", ctypes.c_void_p),
                ("n", ctypes.c_int)]

    def __init__(self, p, g, s, n):
        self._keep = (p, g, s)
        super().__init__(ctypes.cast(p, ctypes.c_void_p), ctypes.cast(g, ctypes.c_void_p),
                         ctypes.cast(s, ctypes.c_void_p), n)


def driver_grads(params, n_layer, C, H, V, npos, ids, tgt):
    lib = ncmhip.load()
    lib.arena_init(2 << 30)
    B, T = ids.shape
    P = [D.from_numpy(p) for p in params]
    G = [D.from_numpy(np.zeros_like(p)) for p in params]
    tape = lib.ncm_tape_new()
    try:
        lib.arena_reset()
        cfg = ncmhip.Gpt2Config(n_layer, C, H, V, npos)
        logits = lib.ncm_gpt2_forward(tape, ctypes.byref(cfg), ncmhip.ptr_array(P), ids.ctypes.data, B, T)
        ncmhip.check()
        loss = D.empty(1)
        lib.ncm_t_ce(tape, logits, tgt.ctypes.data, None, loss.ptr, None, B * T, V, 1.0)
        sizes = (ctypes.c_int64 * len(P))(*[p.size for p in params])
        lib.ncm_tape_backward(tape, ctypes.byref(PMap(ncmhip.ptr_array(P), ncmhip.ptr_array(G), sizes, len(P))))
        ncmhip.check()
        return float(loss.numpy()[0]), [g.numpy() for g in G]
    finally:
        lib.ncm_tape_free(tape)


@pytest.mark.parametrize("n_layer,C,H,V,npos,B,T", [(2, 128, 2, 300, 64, 2, 64), (1, 96, 3, 50, 16, 2, 9)])
def test_trainer_against_reference_header(tmp_path, n_layer, C, H, V, npos, B, T):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} not built (tests/c/Makefile needs /root/reference at build time)")
    ncmhip.init(0)
    rng = np.random.default_rng(31)
    shapes = O.gpt2_shapes(n_layer, C, V, npos)
    params = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in shapes]
    for i, s in enumerate(shapes):
        if len(s) == 1 and s[0] == C and (i >= len(params) - 2 or (i - 2) % 12 in (0, 6)):
            params[i] += np.float32(1.0)
    ids = rng.integers(0, V, (B, T)).astype(np.int32)
    tgt = rng.integers(0, V, (B, T)).astype(np.int32)
    (tmp_path / "dims.txt").write_text(f"{n_layer} {C} {H} {V} {npos} {B} {T}")
    np.concatenate([p.reshape(-1) for p in params]).astype(np.float32).tofile(tmp_path / "params.bin")
    ids.tofile(tmp_path / "ids.bin")
    tgt.tofile(tmp_path / "tgt.bin")
    print(f"[gpu] tape_check {n_layer} layers C={C} T={T}", flush=True)
    r = subprocess.run([BIN, str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "tape_check: ok" in r.stdout
    loss = float(np.fromfile(tmp_path / "loss.bin", np.float32)[0])
    flat = np.fromfile(tmp_path / "grads.bin", np.float32)
    grads, off = [], 0
    for p in params:
        grads.append(flat[off:off + p.size].reshape(p.shape))
        off += p.size
    assert off == flat.size

    rloss, rgrads = O.gpt2_grads(params, n_layer, C, H, V, npos, ids, tgt)
    assert abs(loss - rloss) <= 1e-5 * abs(rloss)
    for i, (g, rg) in enumerate(zip(grads, rgrads)):
        err = float(np.max(np.abs(g - rg)))
        rel = float(np.linalg.norm((g - rg).ravel()) / max(np.linalg.norm(rg.ravel()), 1e-30))
        assert err <= 2e-5 and rel <= 1e-4, (i, err, rel)

    dloss, dgrads = driver_grads(params, n_layer, C, H, V, npos, ids, tgt)
    assert dloss == loss
    for i, (g, dg) in enumerate(zip(grads, dgrads)):
        assert np.array_equal(g.view(np.uint32), dg.view(np.uint32)), i
