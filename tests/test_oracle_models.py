"""The oracle's model compositions against the reference's own model code
(libref: qwen.c through oracle/ref_glue_qwen.c, ncp.c), bit for bit:

- qwen_forward (oracle.py) vs qwen_open + qwen_forward (qwen.c:43-190), all
  rows and last row only;
- qwen_generate (full recompute) vs qwen_generate (qwen.c:204-228), ids and
  per-step logits;
- qwen_generate_cached (one row per step against cached keys/values) vs the
  full-recompute qwen_generate, and vs the reference's generation;
- ncp_forward (one level of token ids) vs ncp_load + ncp_forward
  (ncp.c:94-175, 480-640) on one-hot inputs through wte = table^T.

A slip in the composition (weight order, the q/k/v biases, the RoPE table
convention, the mask, the last-row head, the residual order) changes bits in
one of these."""
import os

import numpy as np
import pytest

import model_data as MD
import oracle as O
from conftest import bits_equal

pytestmark = pytest.mark.skipif(not os.path.exists(O.REF_LIB), reason="oracle/_ref/libref.so not built")


def qwen_params(seed, n_layer, C, H, K, I, V, scale):
    rng = np.random.default_rng(seed)
    shapes = O.qwen_shapes(n_layer, C, H, K, I, V)
    ps = []
    for i, s in enumerate(shapes):
        if len(s) == 1 and s[0] == C and (i == len(shapes) - 1 or (i - 1) % 12 in (0, 8)):
            ps.append((1.0 + 0.02 * rng.standard_normal(s)).astype(np.float32))   # RMSNorm gains
        else:
            ps.append((scale * rng.standard_normal(s)).astype(np.float32))
    return ps


QCFG = dict(n_layer=2, C=64, H=4, K=2, I=96, V=300)


@pytest.fixture(scope="module")
def ref_qwen(tmp_path_factory):
    made = []

    def make(params, n_ctx, theta, **cfg):
        path = str(tmp_path_factory.mktemp("qwen") / "w.ncm")
        m = O.RefQwen(params, cfg["n_layer"], cfg["C"], cfg["H"], cfg["K"], n_ctx, theta, path)
        made.append(m)
        return m
    yield make
    for m in made:
        m.close()


@pytest.mark.parametrize("theta,T", [(1e6, 13), (1e4, 32)])
def test_qwen_forward_matches_reference(ref_qwen, theta, T):
    params = qwen_params(1, scale=0.1, **QCFG)
    ids = np.random.default_rng(2).integers(0, QCFG["V"], T).astype(np.int32)
    r = ref_qwen(params, 32, theta, **QCFG)
    assert bits_equal(O.qwen_forward(params, theta=theta, ids=ids, **QCFG), r.forward(ids))
    assert bits_equal(O.qwen_forward(params, theta=theta, ids=ids, last_only=True, **QCFG),
                      r.forward(ids, last_only=True))


def test_qwen_forward_gqa_ratios_match_reference(ref_qwen):
    cfg = dict(n_layer=1, C=96, H=6, K=3, I=64, V=77)        # 2 query heads per kv head, hd 16
    params = qwen_params(3, scale=0.2, **cfg)
    ids = np.random.default_rng(4).integers(0, cfg["V"], 9).astype(np.int32)
    r = ref_qwen(params, 16, 1e6, **cfg)
    assert bits_equal(O.qwen_forward(params, theta=1e6, ids=ids, **cfg), r.forward(ids))


def test_qwen_generate_matches_reference(ref_qwen):
    params = qwen_params(5, scale=0.3, **QCFG)
    prompt = np.random.default_rng(6).integers(0, QCFG["V"], 11).astype(np.int32)
    n_new, n_ctx = 10, 32
    r = ref_qwen(params, n_ctx, 1e6, **QCFG)
    want = r.generate(prompt, n_new)
    assert len(set(want)) > 3                      # a generation that moves, not one repeated id
    ids, steps = O.qwen_generate(params, theta=1e6, prompt=prompt, n_new=n_new, n_ctx=n_ctx, **QCFG)
    assert ids == want
    seq = list(prompt)
    for s in range(n_new):
        assert bits_equal(steps[s], r.forward(np.array(seq, np.int32), last_only=True))
        seq.append(ids[s])


def test_qwen_cached_generation_equals_full_recompute(ref_qwen):
    params = qwen_params(5, scale=0.3, **QCFG)
    prompt = np.random.default_rng(6).integers(0, QCFG["V"], 11).astype(np.int32)
    n_new, n_ctx = 10, 32
    full, steps = O.qwen_generate(params, theta=1e6, prompt=prompt, n_new=n_new, n_ctx=n_ctx, **QCFG)
    cached, tops = O.qwen_generate_cached(params, theta=1e6, prompt=prompt, n_new=n_new, n_ctx=n_ctx,
                                          keep=QCFG["V"], **QCFG)
    assert cached == full
    for s in range(n_new):                         # every step's logits, bit for bit
        top_ids, top_vals = tops[s]
        assert bits_equal(top_vals, steps[s][top_ids])
    assert cached == ref_qwen(params, n_ctx, 1e6, **QCFG).generate(prompt, n_new)


@pytest.mark.parametrize("H,Kv,biases", [(4, 2, True), (4, 4, True), (4, 1, False)])
def test_ncp_forward_matches_reference(H, Kv, biases):
    n_layer, C, I, V, B, S = 2, 64, 96, 16, 3, 11
    rng = np.random.default_rng(7 + Kv)
    shapes = O.ncp_shapes(n_layer, C, H, Kv, I, V)
    params = []
    for i, s in enumerate(shapes):
        norm_gain = i == len(shapes) - 4 or (1 <= i < len(shapes) - 4 and (i - 1) % 14 in (0, 6))
        is_bias = len(s) == 1 and not norm_gain
        params.append(None if (is_bias and not biases) else (0.3 * rng.standard_normal(s)).astype(np.float32))
    ids = rng.integers(0, V, (B, S)).astype(np.int32)
    cfg = O.ncp_single_level_cfg(n_layer, C, H, Kv, V, S)
    want = O.ref_ncp_forward(cfg, O.ncp_named(params, n_layer, C), np.eye(V, dtype=np.float32)[ids])
    got = O.ncp_forward(params, n_layer, C, H, Kv, I, V, ids)
    assert bits_equal(got, want.reshape(B * S, V))


@pytest.mark.parametrize("case", sorted(MD.NCP_CASES))
def test_ncp_forward_levels_matches_reference(case):
    """The oracle's multi-level ncp_forward (levels, level embedding, block
    masks, prefix pads, qk-norm, RoPE or learned positions, every MLP and
    head kind, post-upsample convs) against the reference's ncp_forward."""
    cfg = MD.NCP_CASES[case]
    named = MD.ncp_named_weights(cfg, seed=len(case))
    rng = np.random.default_rng(3)
    B, P = 3, cfg["prefix_len"]
    first = 0 if cfg["query_level0"] else 1
    S = P + sum(cfg["levels"][first:])
    x = rng.standard_normal((B, S, cfg["vq_embed_dim"]), dtype=np.float32)
    pids = None
    if cfg["prefix_pad_token_id"] >= 0:
        pids = rng.integers(1, 9, (B, P)).astype(np.int32)
        pids[0, :2] = 0          # board 0: two pads; board 1: none; board 2: one
        pids[2, -1] = 0
    want = O.ref_ncp_forward(cfg, named, x, pids)
    got = O.ncp_forward_levels(cfg, named, x, pids)
    assert np.isfinite(want[want != -np.inf]).all()
    assert bits_equal(got, want)
