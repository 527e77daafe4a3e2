"""The drop-in at link level: tests/_build/dropin_check, a C program compiled
against the reference's own src/ncm.h (tests/c/Makefile) and linked to
libncmhip.so, calls tensor_alloc / tensor_to_backend / tensor_to_host,
arena_init / arena_alloc / arena_reset, mem_h2d, backend_to_host,
linear_fwd, rowwise_l2sq, sdpa_fwd_gqa, rmsnorm_fwd, layernorm_fwd and
argmax_row through the reference prototypes (ncm.h:29-56, 141-199), with no
library-specific initialisation.  Its outputs are checked against the
reference-written golden vectors (tests/golden/linear_ref.npz,
vq_ref.npz) and the oracle."""
import os
import subprocess

import numpy as np
import pytest

import oracle as O
from conftest import ROOT, bits_equal, maxrel

pytestmark = pytest.mark.gpu
BIN = os.path.join(ROOT, "tests", "_build", "dropin_check")


def test_c_caller_through_reference_header(golden, tmp_path):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} not built (tests/c/Makefile needs /root/reference at build time)")
    lin = golden("linear_ref.npz")
    vq = golden("vq_ref.npz")
    x, W, b, y_ref = lin["c4_x"], lin["c4_W"], lin["c4_b"], lin["c4_y"]     # batch 130, 64 -> 136, with bias
    a, e, d2_ref = vq["l2_a"], vq["l2_b"], vq["l2_d2"]
    rng = np.random.default_rng(21)
    B, Hq, Hkv, Tq, Tkv, hd = 2, 6, 2, 37, 37, 64
    q = rng.standard_normal((B, Hq, Tq, hd)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, Tkv, hd)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, Tkv, hd)).astype(np.float32)
    mask = np.where(np.arange(Tkv)[None, :] <= np.arange(Tq)[:, None], 0.0, -1e9).astype(np.float32)
    nr, nc = 33, 200
    xr = rng.standard_normal((nr, nc)).astype(np.float32)
    wr = (1.0 + 0.1 * rng.standard_normal(nc)).astype(np.float32)
    br = (0.1 * rng.standard_normal(nc)).astype(np.float32)
    nv = 151936
    logits = rng.standard_normal(nv).astype(np.float32)
    logits[[5000, 120000]] = 9.5                     # a tie: the lower index wins
    dims = [x.shape[0], W.shape[0], W.shape[1], 1, a.shape[0], e.shape[0], a.shape[1],
            B, Hq, Hkv, Tq, Tkv, hd, nr, nc, nv]
    (tmp_path / "dims.txt").write_text(" ".join(str(int(d)) for d in dims))
    for name, arr in (("W", W), ("x", x), ("b", b), ("a", a), ("e", e), ("q", q), ("k", k), ("v", v),
                      ("mask", mask), ("xr", xr), ("wr", wr), ("br", br), ("logits", logits)):
        np.ascontiguousarray(arr, np.float32).tofile(tmp_path / f"{name}.bin")
    print("[gpu] dropin_check", flush=True)
    r = subprocess.run([BIN, str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "dropin_check: ok" in r.stdout

    def out(name, shape, dtype=np.float32):
        return np.fromfile(tmp_path / f"{name}.bin", dtype).reshape(shape)

    assert maxrel(out("y", y_ref.shape), y_ref) <= 1e-4
    assert bits_equal(out("d2", d2_ref.shape), d2_ref)
    assert float(np.max(np.abs(out("o", q.shape) - O.sdpa_gqa(q, k, v, mask)))) <= 1e-5
    assert maxrel(out("rms", xr.shape), O.rmsnorm(xr, wr)) <= 1e-6
    assert maxrel(out("ln", xr.shape), O.layernorm(xr, wr, br)) <= 1e-6
    assert int(out("argmax", (1,), np.int32)[0]) == O.argmax_row(logits) == 5000
