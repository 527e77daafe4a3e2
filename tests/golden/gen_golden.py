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


def sample_row(seed, V, scale, ties):
    """A logits row from the reference's ktest generator (tests/ktest_kernels.c:8-12,
    values in [-2, 2)) times scale; rounded to halves when ties is set."""
    x, _ = O.ktest_fill(int(seed), int(V))
    x = (x * np.float32(scale)).astype(np.float32)
    return (np.round(x * 2) / 2).astype(np.float32) if ties else x


def sample_cases():
    """Rows for sample_topkp (kernels.c:782-825): ties (rounded logits),
    temperatures, top-k, nucleus settings and the full Qwen vocabulary.  The
    full-vocabulary rows are stored as their generator seed (sample_row)."""
    rng = np.random.default_rng(20261202)
    cfg = [(1.0, 0, 1.0), (0.7, 0, 0.9), (1.3, 40, 1.0), (0.5, 5, 0.5), (1.0, 1, 1.0), (2.0, 0, 0.0),
           (0.8, 1000, 0.95), (1.0, 0, 1.0)]
    out = {}
    for i, (temp, k, p) in enumerate(cfg):
        if i in (0, 1, 7):
            gen = np.array([int(rng.integers(1, 2 ** 62)), 151936, rng.uniform(1.0, 4.0), i % 2], np.float64)
            x = sample_row(*gen)
            out[f"c{i}_gen"] = gen
        else:
            V = int(rng.integers(2, 5000))
            x = (rng.standard_normal(V) * rng.uniform(0.5, 4.0)).astype(np.float32)
            if i % 2:
                x = np.round(x * 2).astype(np.float32) / 2   # many exact ties
            out[f"c{i}_x"] = x
        st = int(rng.integers(1, 2 ** 63))
        ids, sts = [], []
        s = st
        for _ in range(4):   # four draws in a row from the same row
            j, s = O.ref_sample_topkp(x, temp, k, p, s)
            ids.append(j)
            sts.append(s)
        out.update({f"c{i}_cfg": np.array([temp, k, p], np.float64),
                    f"c{i}_rng": np.array([st] + sts, np.uint64), f"c{i}_ids": np.array(ids, np.int32)})
    out["n_cases"] = np.array(len(cfg))
    return out


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref/libref.so missing: run make -C oracle where /root/reference exists")
    rng = np.random.default_rng(20261201)
    np.savez_compressed(os.path.join(HERE, "linear_ref.npz"), **linear_cases(rng))
    np.savez_compressed(os.path.join(HERE, "vq_ref.npz"), **vq_case(rng))
    np.savez_compressed(os.path.join(HERE, "sample_ref.npz"), **sample_cases())
    kt = subprocess.run([O.KTEST_BIN], check=True, capture_output=True, text=True).stdout
    with open(os.path.join(HERE, "ktest_cpu.txt"), "w") as f:
        f.write(kt)
    print("wrote linear_ref.npz vq_ref.npz sample_ref.npz ktest_cpu.txt")


if __name__ == "__main__":
    main()
