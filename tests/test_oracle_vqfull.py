"""Oracle pinning for the full multiscale quantizer (src/vq.c vq_load +
vq_z_to_idx + vq_idx_to_zhats with per-level lengths, Phi, the learned
level-0 cascade and refine convs): bit-equality of codes and of every
level's z_hat with the reference's own functions compiled from source, and
closed forms for the resampling (identity when a level has the full length,
constant sequences stay constant, area of a linear ramp)."""
import numpy as np
import pytest

import oracle as O
from conftest import bits_equal
from vqfull_cases import CASES, make_case, ref_inputs, ref_vq, ref_vq_ema

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference not compiled here")


@needs_ref
@pytest.mark.parametrize("name,kw", CASES, ids=[c[0] for c in CASES])
def test_oracle_matches_reference(name, kw):
    cfg, w, z = make_case(7, **kw)
    B = kw["B"]
    idx, zh, zr = O.vq_z_to_idx(cfg, w, z, B)
    ridx, rzh = ref_vq(cfg, w, z, B)
    assert np.array_equal(idx, ridx)
    zhats = O.vq_idx_to_zhats(cfg, w, idx, B)
    assert bits_equal(zhats, rzh)
    assert bits_equal(zh, zhats[-1])


@needs_ref
@pytest.mark.parametrize("name,kw", [CASES[0], CASES[2], CASES[5], CASES[8]],
                         ids=[CASES[i][0] for i in (0, 2, 5, 8)])
@pytest.mark.parametrize("soft_levels,tau", [(2, 0.5), (5, 0.05), (9, 2.0)])
def test_soft_assignment_matches_reference(name, kw, soft_levels, tau):
    """vq_z_to_idx_soft (vq.c:388-437): codes, every level's z_hat and the rng
    state after, equal to the reference's own from the same seed; the levels
    at and above soft_levels keep the argmin codes of the same residual."""
    cfg, w, z = make_case(7, **kw)
    B, seed = kw["B"], 0x9E3779B97F4A7C15
    idx, zh, zr, rng = O.vq_z_to_idx_soft(cfg, w, z, B, soft_levels, tau, seed)
    ridx, rzh, rrng = ref_vq(cfg, w, z, B, soft=(soft_levels, tau, seed))
    assert np.array_equal(idx, ridx) and rng == rrng
    assert bits_equal(O.vq_idx_to_zhats(cfg, w, idx, B), rzh)
    hard, _, _ = O.vq_z_to_idx(cfg, w, z, B)
    n_soft = sum(cfg["levels"][:min(soft_levels, cfg["n_qlevels"])])
    assert rng != seed and not np.array_equal(idx[:, :n_soft], hard[:, :n_soft])
    if soft_levels < cfg["n_qlevels"]:   # the first hard level reads a residual the draws changed
        assert idx.shape == hard.shape


@needs_ref
@pytest.mark.parametrize("name,kw", [CASES[0], CASES[1], CASES[3], CASES[5], CASES[8]],
                         ids=[CASES[i][0] for i in (0, 1, 3, 5, 8)])
def test_ema_update_matches_reference(name, kw):
    """vq_ema_init + vq_ema_update (vq.c:677-790), two calls in a row: every
    codebook after, bit for bit with the reference's own."""
    cfg, w, z = make_case(7, **kw)
    B = kw["B"]
    idx, _, _ = O.vq_z_to_idx(cfg, w, z, B)
    want = ref_vq_ema(cfg, w, z, idx, B, 0.9, 1e-5, steps=2)
    got, cs, _ = O.vq_ema_update(cfg, w, z, idx, B, 0.9, 1e-5, steps=2)
    for lv in range(cfg["n_qlevels"]):
        assert bits_equal(got[lv], want[lv]), lv
        assert not np.array_equal(got[lv], w[f"embeddings.{lv}.weight"])
    # counts: cs = 0.81 * 1 + 0.19 * count over the two decays (fp32 rounding twice)
    cnt = np.bincount(idx[:, :cfg["levels"][0]].ravel(), minlength=cs[0].size)
    c1 = np.float32(0.9 * 1.0 + 0.1 * cnt)
    assert bits_equal(cs[0], (0.9 * c1.astype(np.float64) + 0.1 * cnt).astype(np.float32))


def test_ema_update_decay_one_keeps_codebooks():
    """decay 1: the sums and counts keep their cold start (w = E, cs = 1), so
    each code becomes E / ((1 + eps) / (V + V eps) V) = E exactly."""
    cfg, w, z = make_case(5, B=3, levels=[1, 2, 4, 8, 16], V=32, D=16)
    idx, _, _ = O.vq_z_to_idx(cfg, w, z, 3)
    got, _, _ = O.vq_ema_update(cfg, w, z, idx, 3, 1.0, 1e-5)
    for lv in range(cfg["n_qlevels"]):
        assert bits_equal(got[lv], w[f"embeddings.{lv}.weight"])


def test_soft_pick_closed_forms():
    """One row's draw: the xorshift64 (13, 7, 17) step against its definition
    on a known state, the two-code case against the explicit threshold, a row
    of zeros (m = 0: no draw, rng untouched), and the empirical frequencies of
    many draws against the tempered softmax."""
    s = 0x0123456789ABCDEF
    x = s
    for sh in (13, -7, 17):
        x = (x ^ (x << sh if sh > 0 else x >> -sh)) & (2**64 - 1)
    d = np.array([1.0, 3.0], np.float32)
    j, s1 = O.soft_pick(d, 0.5, s)
    assert s1 == x
    T = 0.5 * 2.0
    p0 = 1.0 / (1.0 + np.exp(-2.0 / T))
    u = (x >> 11) * 2.0**-53
    assert j == (0 if u < p0 else 1)
    assert O.soft_pick(np.zeros(5, np.float32), 0.5, s) == (-1, s)
    rng = np.random.default_rng(3)
    d = (rng.random(6) * 4).astype(np.float32)
    T = 0.7 * float(np.mean(d.astype(np.float64)))
    p = np.exp(-(d - d.min()) / T)
    p /= p.sum()
    counts, st = np.zeros(6), 12345
    for _ in range(20000):
        j, st = O.soft_pick(d, 0.7, st)
        counts[j] += 1
    assert np.allclose(counts / 20000, p, atol=0.015)


@needs_ref
@pytest.mark.parametrize("name,kw", CASES, ids=[c[0] for c in CASES])
def test_next_input_and_ncm_input_match_reference(name, kw):
    cfg, w, z = make_case(7, **kw)
    B = kw["B"]
    idx, _, _ = O.vq_z_to_idx(cfg, w, z, B)
    rx, rsteps = ref_inputs(cfg, w, idx, B)
    assert bits_equal(O.vq_idx_to_ncm_input(cfg, w, idx, B), rx)
    zh, base = np.zeros_like(z), 0
    for lv, (rzh, rxn) in enumerate(rsteps):
        tl = cfg["levels"][lv]
        zh, xn = O.vq_next_input(cfg, w, idx[:, base:base + tl], lv, zh, B)
        assert bits_equal(zh, rzh) and bits_equal(xn, rxn)
        base += tl


def test_ncm_input_chunks_are_area_of_the_running_zhats():
    # chunk li of vq_idx_to_ncm_input = area(z_hat after level li) and the last
    # chunk, at full length, is that z_hat itself (area L -> L is the identity)
    cfg, w, z = make_case(9, B=3, levels=[1, 2, 4, 8, 16], V=32, D=16, phi=1, ratio=0.5)
    idx, _, _ = O.vq_z_to_idx(cfg, w, z, 3)
    zhats = O.vq_idx_to_zhats(cfg, w, idx, 3)
    x = O.vq_idx_to_ncm_input(cfg, w, idx, 3)
    assert x.shape == (3, 30, 16)
    assert bits_equal(x[:, 14:], zhats[3])
    # the first chunk (length 2) averages 8 rows each: a serial fp64 sum over
    # the window, divided by 8, rounded once to fp32
    want = np.empty((3, 2, 16), np.float32)
    for b in range(3):
        for t in range(2):
            for d in range(16):
                acc = 0.0
                for k in range(8 * t, 8 * t + 8):
                    acc += float(zhats[0][b, k, d])
                want[b, t, d] = np.float32(acc / 8.0)
    assert bits_equal(x[:, 0:2], want)
    # next_input threaded through the levels returns the same chunks
    zh, base, off = np.zeros_like(z), 0, 0
    for lv in range(4):
        zh, xn = O.vq_next_input(cfg, w, idx[:, base:base + cfg["levels"][lv]], lv, zh, 3)
        assert bits_equal(zh, zhats[lv]) and bits_equal(xn, x[:, off:off + cfg["levels"][lv + 1]])
        base += cfg["levels"][lv]
        off += cfg["levels"][lv + 1]


def test_full_length_levels_reduce_to_identity_resampling():
    # every level of length L: area and linear resampling are identities, so
    # the quantizer is the identity-resampling loop pinned elsewhere
    cfg, w, z = make_case(3, B=4, levels=[16, 16, 16], V=64, D=32)
    idx, zh, zr = O.vq_z_to_idx(cfg, w, z, 4)
    Es = [w[f"embeddings.{i}.weight"] for i in range(3)]
    idx2 = np.empty((4, 48), np.int32)
    zh2, zr2 = np.empty((64, 32), np.float32), np.empty((64, 32), np.float32)
    import ctypes
    Ep = (ctypes.c_void_p * 3)(*[e.ctypes.data for e in Es])
    vc = (ctypes.c_int * 3)(64, 64, 64)
    O.lib().orc_vq_multiscale(z.reshape(64, 32).ctypes.data, Ep, vc, 3, 4, 16, 32, idx2.ctypes.data,
                              zh2.ctypes.data, zr2.ctypes.data)
    assert np.array_equal(idx, idx2)
    assert bits_equal(zh.reshape(64, 32), zh2) and bits_equal(zr.reshape(64, 32), zr2)


def test_codes_of_a_planted_sequence():
    # z built from codewords held constant over each level's span: level 0
    # (length 1) sees the mean of a constant sequence = the codeword itself
    cfg, w, _ = make_case(5, B=2, levels=[1, 16], V=32, D=16)
    E0 = w["embeddings.0.weight"]
    z = np.stack([np.tile(E0[5], (16, 1)), np.tile(E0[9], (16, 1))]).astype(np.float32)
    idx, zh, zr = O.vq_z_to_idx(cfg, w, z, 2)
    assert list(idx[:, 0]) == [5, 9]
    # z_rest after level 0 is zero up to rounding of the (exact) constant mean and linear resampling
    assert np.all(idx[:, 1:] >= 0)


def _load(cfg, w):
    """The library's vq_load over a store of HOST tensors (vq_load reads shapes
    and keeps pointers; it touches no device memory)."""
    import ctypes
    import ncmhip
    from vqfull_cases import host_tensor, ncm_config, weight_store
    lib = ncmhip.load()
    arrays = {k: np.ascontiguousarray(v, np.float32) for k, v in w.items()}
    tens = [(k, host_tensor(a)) for k, a in arrays.items()]
    ws, keep = weight_store(tens)
    c = ncm_config(cfg)
    vq = lib.vq_load(ctypes.byref(c), ctypes.byref(ws), b"")
    try:
        ncmhip.check()
        return [lib.vq_total_codes(vq), lib.vq_nlevels(vq), lib.vq_level_len(vq, 1), lib.vq_level_V(vq, 0),
                lib.vq_Ltotal(vq), lib.vq_Ddim(vq)]
    finally:
        lib.vq_free(vq)


def test_library_vq_load_reads_the_reference_layout():
    cfg, w, _ = make_case(1, B=2, levels=[1, 2, 4, 8, 16], V=64, D=32, phi=4, down=[4, 4], up=[4, 4], gaps=True,
                          norm=(1, 1), refine=(1, 2, 3))
    assert _load(cfg, w) == [31, 5, 2, 64, 16, 32]
    cfg, w, _ = make_case(1, B=2, levels=[2, 16], V=8, D=16, phi=1)
    w["quant_resi.weight"], w["quant_resi.bias"] = w.pop("quant_resi.0.weight"), w.pop("quant_resi.0.bias")
    assert _load(cfg, w)[0] == 18   # the shared Phi under its unindexed name


def test_library_vq_load_refusals():
    import ncmhip
    cfg, w, _ = make_case(1, B=2, levels=[1, 4, 16], V=8, D=16, phi=0)
    del w["quant_resi.2.bias"]
    with pytest.raises(ncmhip.NcmError, match="missing weight quant_resi.2.bias"):
        _load(cfg, w)
    cfg, w, _ = make_case(1, B=2, levels=[1, 4, 16], V=8, D=16, down=[4, 2], up=[4, 4])
    with pytest.raises(ncmhip.NcmError, match="cascade maps 16 -> 2"):
        _load(cfg, w)
    cfg, w, _ = make_case(1, B=2, levels=[1, 4, 16], V=8, D=16)
    w["embeddings.1.weight"] = w["embeddings.1.weight"][:5]
    with pytest.raises(ncmhip.NcmError, match="embeddings.1.weight is not"):
        _load(cfg, w)
