"""Seeded synthetic weights and inputs shared by the GPU tests, the golden
fixture scripts and the benchmark (the same seed gives the same arrays on any
machine with this numpy)."""
import numpy as np

import oracle as O


def qwen_weights(seed, n_layer, C, H, K, I, V, scale=0.02):
    """Qwen2 parameters in oracle.qwen_shapes order: matrices and q/k/v biases
    N(0, scale^2), RMSNorm gains 1 + N(0, 0.02^2); float32 draws."""
    rng = np.random.default_rng(seed)
    shapes = O.qwen_shapes(n_layer, C, H, K, I, V)
    ps = []
    for i, s in enumerate(shapes):
        z = rng.standard_normal(s, dtype=np.float32)
        if len(s) == 1 and s[0] == C and (i == len(shapes) - 1 or (i - 1) % 12 in (0, 8)):
            ps.append((np.float32(1.0) + np.float32(0.02) * z).astype(np.float32))
        else:
            ps.append((np.float32(scale) * z).astype(np.float32))
    return ps


# Config 4 (BASELINE): Qwen2-0.5B shape, 2048-token prompt, 256 greedy steps.
C4 = dict(n_layer=24, C=896, H=14, K=2, I=4864, V=151936)
C4_THETA = 1e6
C4_SEED = 41
C4_PROMPT = 2048
C4_NEW = 256
C4_CTX = 2304


def c4_prompt():
    return np.random.default_rng(C4_SEED + 1).integers(0, C4["V"], C4_PROMPT).astype(np.int32)
