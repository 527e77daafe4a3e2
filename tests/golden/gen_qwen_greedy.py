"""Writes tests/golden/qwen_greedy_c4.npz: the CPU greedy generation of config 4
(24 layers, d 896, 14/2 heads, FFN 4864, vocab 151936, 2048-token prompt,
256 steps) on the seeded weights of tests/model_data.py.

The generation is oracle.qwen_generate_cached: the reference's arithmetic
(every op bit-equal to the reference's kernels) with a KV cache, which is
bit-equal to the reference's full-recompute qwen_generate (qwen.c:204-228);
tests/test_oracle_models.py pins both equalities against the reference's own
qwen.c.  The full recompute itself would take hours at this size.

Stored per step: the 8 largest logits and their ids (descending, ties by
index), so the GPU test can measure its logit error where the argmax is
decided and report the smallest top-2 gap.

Run from the repository root: python tests/golden/gen_qwen_greedy.py
(about 5-10 minutes on 8 cores)."""
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
    params = MD.qwen_weights(MD.C4_SEED, **MD.C4)
    prompt = MD.c4_prompt()
    print(f"weights ready in {time.time() - t0:.1f} s", flush=True)
    ids, tops = O.qwen_generate_cached(params, theta=MD.C4_THETA, prompt=prompt, n_new=MD.C4_NEW,
                                       n_ctx=MD.C4_CTX, keep=8, **MD.C4)
    top_ids = np.stack([t[0] for t in tops]).astype(np.int32)
    top_vals = np.stack([t[1] for t in tops]).astype(np.float32)
    gaps = top_vals[:, 0].astype(np.float64) - top_vals[:, 1]
    out = os.path.join(ROOT, "tests", "golden", "qwen_greedy_c4.npz")
    np.savez_compressed(out, ids=np.asarray(ids, np.int32), top_ids=top_ids, top_vals=top_vals,
                        seed=MD.C4_SEED, n_new=MD.C4_NEW)
    print(f"{len(ids)} ids in {time.time() - t0:.1f} s; min top-2 gap {gaps.min():.3e} at step "
          f"{int(gaps.argmin())}; first ids {ids[:8]}", flush=True)


if __name__ == "__main__":
    main()
