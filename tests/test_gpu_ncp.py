"""Config 1: the NCP transformer forward at its full size (4 layers, d 256,
4 query / 2 kv heads, SwiGLU 1024, vocab 16, 64 boards x 81 tokens) on the
device against the oracle's op-for-op restatement of ncp_block, which is
bit-equal to the reference's own ncp_forward (tests/test_oracle_models.py).
Bar: logits max-abs 1e-3 (north star), asserted as 1e-4."""
import ctypes

import numpy as np
import pytest

import model_data as MD
import ncmhip
import oracle as O
from conftest import bits_equal

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


def ncp_device(cfg, named, x, pids=None):
    """The library's ncp_load + ncp_forward (the reference's API) on device
    tensors; returns (logits [B][T][maxV], accessors)."""
    lib = ncmhip.load()
    fields = {k: v for k, v in cfg.items() if k not in ("levels", "vocab_size", "n_inner")}
    c = ncmhip.ncm_config(n_qlevels=len(cfg["levels"]), levels=cfg["levels"], vocab_size=cfg["vocab_size"],
                          **fields)
    store, keep = ncmhip.weight_store(named)
    m = lib.ncp_load(ctypes.byref(c), ctypes.byref(store), None)
    ncmhip.check()
    try:
        B = x.shape[0]
        T = lib.ncp_T(m)
        maxV = max(cfg["vocab_size"][:lib.ncp_ntgt(m)])
        xd = D.from_numpy(x)
        out = D.empty((B, T, maxV))
        lib.arena_reset()
        p = None if pids is None else np.ascontiguousarray(pids, np.int32)
        lib.ncp_forward(m, xd.ptr, None if p is None else p.ctypes.data, out.ptr, B)
        ncmhip.check()
        acc = dict(P=lib.ncp_P(m), T=T, ntgt=lib.ncp_ntgt(m), lvlfirst=lib.ncp_lvlfirst(m))
        return out.numpy(), acc
    finally:
        lib.ncp_free(m)


def compare_logits(got, want, tol):
    inf = np.isneginf(want)
    assert np.array_equal(np.isneginf(got), inf)
    err = float(np.max(np.abs(got[~inf] - want[~inf])))
    assert err <= tol, err
    return err


@pytest.mark.parametrize("case", sorted(MD.NCP_CASES))
def test_ncp_forward_levels(case):
    """ncp_forward on the device against the oracle's multi-level forward
    (bit-equal to the reference's ncp_forward, tests/test_oracle_models.py):
    logits max-abs 1e-3 (the north star's bar), -inf cells identical."""
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
        pids[0, :2] = 0
        pids[2, -1] = 0
    want = O.ncp_forward_levels(cfg, named, x, pids)
    got, acc = ncp_device(cfg, named, x, pids)
    assert acc == dict(P=P, T=S - P, ntgt=len(cfg["levels"]) - first, lvlfirst=first)
    err = compare_logits(got, want, 1e-3)
    print(f"[ncp] {case}: max-abs {err:.2e}")


def test_ncp_forward_levels_sudoku_scale():
    """Coarse-to-fine levels 1/9/81 over 64 boards at config-1 widths (d 256,
    4/2 heads, SwiGLU 1024, 4 layers), block-diagonal mask, RoPE."""
    cfg = MD.ncp_cfg(n_layer=4, n_embd=256, n_head=4, n_kv_heads=2, n_inner=1024, levels=[1, 9, 81],
                     vocab_size=[16, 16], vq_embed_dim=32)
    named = MD.ncp_named_weights(cfg, seed=11, scale=0.1)
    x = np.random.default_rng(12).standard_normal((64, 90, 32), dtype=np.float32)
    want = O.ncp_forward_levels(cfg, named, x)
    got, _ = ncp_device(cfg, named, x)
    err = compare_logits(got, want, 1e-3)
    print(f"[ncp] levels 1/9/81 x 64 boards: max-abs {err:.2e}")


def test_single_level_driver_equals_reference_api():
    """ncm_ncp_forward (token ids through an embedding) and ncp_forward (the
    reference API on one-hot inputs through wte = table^T, levels {1, S})
    give the same logits bit for bit."""
    n_layer, C, H, Kv, I, V, B, S = 2, 256, 4, 2, 512, 16, 8, 81
    params = ncp_weights(3, n_layer, C, H, Kv, I, V)
    ids = np.random.default_rng(4).integers(0, V, (B, S)).astype(np.int32)
    bufs = [D.from_numpy(p) for p in params]
    cfg = ncmhip.NcpConfig(n_layer, C, H, Kv, I, V, 10000)
    lib = ncmhip.load()
    lib.arena_reset()
    p = lib.ncm_ncp_forward(ctypes.byref(cfg), ncmhip.ptr_array(bufs), ids.ctypes.data, B, S)
    ncmhip.check()
    drv = np.empty((B * S, V), np.float32)
    lib.mem_d2h(drv.ctypes.data, p, drv.nbytes)
    rcfg = O.ncp_single_level_cfg(n_layer, C, H, Kv, V, S)
    got, _ = ncp_device(rcfg, O.ncp_named(params, n_layer, C), np.eye(V, dtype=np.float32)[ids])
    assert bits_equal(got.reshape(B * S, V), drv)


@pytest.mark.parametrize("n_head,n_embd", [(2, 128), (4, 96)])
def test_ncp_padded_prefix_many_boards(n_head, n_embd):
    """Padded prefix tokens on most of 40 boards: every board gets its own key
    mask and all boards run as one batch (hd 64: the MFMA attention with the
    per-board masks; hd 24: the row kernel), against the oracle, which runs
    the reference's board-by-board loop (ncp.c:571-607)."""
    cfg = MD.ncp_cfg(n_embd=n_embd, n_head=n_head, n_kv_heads=n_head // 2 or 1, n_inner=2 * n_embd,
                     prefix_len=8, prefix_pad_token_id=0, attn_pattern_block_diag=0, levels=[1, 4, 16],
                     vocab_size=[24, 32])
    named = MD.ncp_named_weights(cfg, seed=23, scale=0.2)
    rng = np.random.default_rng(24)
    B, P = 40, 8
    S = P + 4 + 16
    x = rng.standard_normal((B, S, cfg["vq_embed_dim"]), dtype=np.float32)
    pids = rng.integers(1, 9, (B, P)).astype(np.int32)
    pads = rng.random((B, P)) < 0.4
    pads[:, 0] = False                    # every board keeps a real prefix token
    pids[pads] = 0
    pids[::5] = rng.integers(1, 9, (8, P))   # some boards without pads
    want = O.ncp_forward_levels(cfg, named, x, pids)
    got, _ = ncp_device(cfg, named, x, pids)
    err = compare_logits(got, want, 1e-3)
    print(f"[ncp] padded prefix, {B} boards, hd {n_embd // n_head}: max-abs {err:.2e}")
