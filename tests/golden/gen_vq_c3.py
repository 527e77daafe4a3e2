"""Writes tests/golden/vq_c3_codes.npz: the CPU result of BASELINE config 3
(65536 vectors of dim 256, 4 residual scales of 4096 codes) on the seeded
inputs of tests/model_data.py: every code (uint16 [4][65536], scale-major)
and the SHA-256 of the final z_hat and z_rest bytes.

The codes come from oracle.vq_multiscale, the restatement of vq.c:388-500
with identity resampling (kernels.c:753-770 distances, strict-< scan, float
residual updates).  Where the reference was compiled here
(oracle/_ref/libref.so), its own vq_load + vq_z_to_idx over the same
codebooks is run too and must give the same codes, z_hat and z_rest.

Run from the repository root: NCM_ARENA_MB=8192 python tests/golden/gen_vq_c3.py
(the reference's scratch arena must hold the four 1 GiB distance matrices;
about 1-2 minutes on 8 cores for the oracle, ~2 more for the reference)."""
import hashlib
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

import oracle as O  # noqa: E402
import model_data as MD  # noqa: E402


def main():
    t0 = time.time()
    z, Es = MD.vq_c3_inputs()
    R, S = MD.C3["R"], MD.C3["S"]
    idx, z_hat, z_rest = O.vq_multiscale(z, Es, 1, R)
    print(f"oracle done in {time.time() - t0:.0f} s", flush=True)
    if O.ref_available():
        ridx, rh, rr = O.ref_vq_multiscale(z, Es, 1, R)
        same = (np.array_equal(ridx, idx) and np.array_equal(rh.view(np.uint32), z_hat.view(np.uint32))
                and np.array_equal(rr.view(np.uint32), z_rest.view(np.uint32)))
        print(f"reference done in {time.time() - t0:.0f} s: equal to the oracle: {same}", flush=True)
        if not same:
            raise SystemExit("the oracle and the reference disagree; no fixture written")
    codes = idx.reshape(S, R).astype(np.uint16)
    out = os.path.join(ROOT, "tests", "golden", "vq_c3_codes.npz")
    np.savez_compressed(out, codes=codes, z_hat_sha256=hashlib.sha256(z_hat.tobytes()).hexdigest(),
                        z_rest_sha256=hashlib.sha256(z_rest.tobytes()).hexdigest())
    print(f"wrote {out} in {time.time() - t0:.0f} s", flush=True)


if __name__ == "__main__":
    main()
