"""Writes tests/golden/gpt2_c5_grads.npz: the CPU result of one config-5
training step's forward, mean cross-entropy and backward (12 layers, d 768,
12 heads, vocab 4096, 32 x 512 tokens) on the seeded weights of
tests/model_data.py.

The step is oracle.gpt2_grads: the forward of train_gpt2_forward
(train_gpt2.c:42-147), t_ce (train_tape.c:442-481) and the host tape backward
(train_tape.c:636-1051) over the same records; tests/test_oracle_models.py
pins it bit for bit against the reference's own train_gpt2.c + train_tape.c
compiled from source.

Stored (gradients are 88.5 M floats, too large for a fixture):
- loss (float64 of the float the oracle returns);
- per parameter tensor, in oracle.gpt2_shapes order: the float64 L2 norm of
  its gradient; four checksums sum(g * s_j) against seeded +-1 vectors
  s_j = model_data.grad_probe_signs(n, 7000 + 10 i + j), each of which a
  wrong element moves by its error; 64 sampled flat indices (the first and
  last element plus 62 seeded draws) and the gradient values there.

Run from the repository root: python tests/golden/gen_gpt2_c5.py
(about 65 minutes on 8 cores, 32 GB of memory)."""
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

import oracle as O  # noqa: E402
import model_data as MD  # noqa: E402

NPROBE, NSAMPLE = 4, 64


def summarise(grads):
    n = len(grads)
    norms = np.zeros(n)
    probes = np.zeros((n, NPROBE))
    idx = np.zeros((n, NSAMPLE), np.int64)
    val = np.zeros((n, NSAMPLE), np.float32)
    for i, g in enumerate(grads):
        f = g.reshape(-1)
        g64 = f.astype(np.float64)
        norms[i] = np.sqrt(np.dot(g64, g64))
        for j in range(NPROBE):
            probes[i, j] = np.dot(g64, MD.grad_probe_signs(f.size, 7000 + 10 * i + j))
        rng = np.random.default_rng(9000 + i)
        pick = np.concatenate([[0, f.size - 1], rng.choice(f.size, NSAMPLE - 2, replace=False)])
        idx[i] = pick
        val[i] = f[pick]
    return norms, probes, idx, val


def main():
    t0 = time.time()
    params, ids, tgt = MD.gpt2_c5_weights()
    c = MD.C5
    loss, grads = O.gpt2_grads(params, c["n_layer"], c["C"], c["H"], c["V"], c["npos"], ids, tgt)
    print(f"step done in {time.time() - t0:.0f} s: loss {loss:.9g}", flush=True)
    norms, probes, idx, val = summarise(grads)
    out = os.path.join(ROOT, "tests", "golden", "gpt2_c5_grads.npz")
    np.savez_compressed(out, loss=np.float64(loss), norms=norms, probes=probes, idx=idx, val=val)
    print(f"wrote {out} in {time.time() - t0:.0f} s; smallest gradient norm {norms.min():.3e}", flush=True)


if __name__ == "__main__":
    main()
