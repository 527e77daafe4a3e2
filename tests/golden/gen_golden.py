"""Writes the golden fixtures of tests/golden from the REFERENCE's own CPU code.

Run in the build container, where /root/reference exists and
`make -C oracle` has compiled oracle/_ref/{libref.so,ktest} from the
reference sources.  The fixtures are data only (inputs and the reference's
outputs); the GPU box, which has no /root/reference, checks the oracle and
the HIP library against them.

    python tests/golden/gen_golden.py
"""
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402


def linear_cases(rng):
    # (batch, M, K): odd K, K % 4 != 0, batch 1, tile-edge shapes
    shapes = [(5, 24, 40), (33, 70, 130), (40, 64, 96), (1, 150, 97), (130, 136, 64), (9, 130, 72)]
    out = {}
    for i, (batch, M, K) in enumerate(shapes):
        x = rng.standard_normal((batch, K)).astype(np.float32)
        W = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
        b = (rng.standard_normal(M) * 0.02).astype(np.float32) if i % 2 == 0 else None
        dy = rng.standard_normal((batch, M)).astype(np.float32)
        dx0 = rng.standard_normal((batch, K)).astype(np.float32)
        dW0 = rng.standard_normal((M, K)).astype(np.float32)
        db0 = rng.standard_normal(M).astype(np.float32)
        y = O.ref_linear_fwd(x, W, b)
        dx, dW, db = O.ref_linear_bwd(x, W, b, dy, dx0, dW0, db0)
        p = f"c{i}_"
        out.update({p + "x": x, p + "W": W, p + "dy": dy, p + "dx0": dx0, p + "dW0": dW0,
                    p + "y": y, p + "dx": dx, p + "dW": dW})
        if b is not None:
            out.update({p + "b": b, p + "db0": db0, p + "db": db})
    out["n_cases"] = np.array(len(shapes))
    return out


def vq_case(rng):
    B, L, D, V, n = 4, 32, 64, 128, 3
    z = rng.standard_normal((B * L, D)).astype(np.float32)
    Es = []
    for lv in range(n):
        E = (rng.standard_normal((V, D)) / np.sqrt(D)).astype(np.float32)
        # exact duplicates (ties must resolve to the lower index) and a
        # codeword planted on a row so its distance is exactly 0
        E[V - 1] = E[3]
        E[V - 2] = E[40]
        if lv == 0:
            E[77] = z[5]
            E[90] = z[5]
        Es.append(E)
    idx, z_hat, z_rest = O.ref_vq_multiscale(z, Es, B, L)
    out = {"z": z, "idx": idx, "z_hat": z_hat, "z_rest": z_rest, "B": np.array(B), "L": np.array(L)}
    for lv, E in enumerate(Es):
        out[f"E{lv}"] = E
    a = rng.standard_normal((20, 32)).astype(np.float32)
    bb = rng.standard_normal((48, 32)).astype(np.float32)
    out["l2_a"], out["l2_b"], out["l2_d2"] = a, bb, O.ref_l2sq(a, bb)
    return out


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref/libref.so missing: run make -C oracle where /root/reference exists")
    rng = np.random.default_rng(20261201)
    np.savez_compressed(os.path.join(HERE, "linear_ref.npz"), **linear_cases(rng))
    np.savez_compressed(os.path.join(HERE, "vq_ref.npz"), **vq_case(rng))
    kt = subprocess.run([O.KTEST_BIN], check=True, capture_output=True, text=True).stdout
    with open(os.path.join(HERE, "ktest_cpu.txt"), "w") as f:
        f.write(kt)
    print("wrote linear_ref.npz vq_ref.npz ktest_cpu.txt")


if __name__ == "__main__":
    main()
