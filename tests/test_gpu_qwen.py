"""Config 4: the Qwen2 decoder on the device against the oracle's restatement
of qwen_forward (every op pinned to the reference).

Bars: logits max-abs 1e-3 (north star); greedy ids exact (north star).  The
cached decode is checked against the reference's full-recompute generation,
and at the full config-4 shape (24 layers, vocab 151936, 2048-token prefill)
through a size-independent property: the cached step's logits equal the
last row of a full forward over the extended sequence."""
import ctypes

import numpy as np
import pytest

import model_data as MD
import ncmhip
import oracle as O

pytestmark = pytest.mark.gpu
D = ncmhip.DeviceBuffer


@pytest.fixture(scope="module", autouse=True)
def device():
    ncmhip.init(0)
    ncmhip.load().arena_init(8 << 30)
    ncmhip.check()
    print("[gpu] qwen tests on device 0", flush=True)


def weights(seed, n_layer, C, H, K, I, V):
    rng = np.random.default_rng(seed)
    shapes = O.qwen_shapes(n_layer, C, H, K, I, V)
    ps = []
    for i, s in enumerate(shapes):
        if len(s) == 1 and s[0] == C and (i == len(shapes) - 1 or (i - 1) % 12 in (0, 8)):
            ps.append((1.0 + 0.02 * rng.standard_normal(s)).astype(np.float32))   # RMSNorm gains
        else:
            ps.append((0.02 * rng.standard_normal(s)).astype(np.float32))
    return ps


class Model:
    def __init__(self, params, n_layer, C, H, K, I, V, n_ctx, theta):
        self.lib = ncmhip.load()
        self.bufs = [D.from_numpy(p) for p in params]
        self.cfg = ncmhip.QwenConfig(n_layer, C, H, K, I, V, n_ctx, theta)
        self.m = self.lib.ncm_qwen_new(ctypes.byref(self.cfg), ncmhip.ptr_array(self.bufs))
        ncmhip.check()
        self.V = V

    def forward(self, ids, last_only=False):
        ids = np.ascontiguousarray(ids, np.int32)
        p = self.lib.ncm_qwen_forward(self.m, ids.ctypes.data, ids.size, int(last_only))
        ncmhip.check()
        n = self.V if last_only else ids.size * self.V
        out = np.empty(n, np.float32)
        self.lib.mem_d2h(out.ctypes.data, p, out.nbytes)
        ncmhip.check()
        return out if last_only else out.reshape(ids.size, self.V)

    def decode(self, tok, pos):
        p = self.lib.ncm_qwen_decode(self.m, int(tok), pos)
        ncmhip.check()
        out = np.empty(self.V, np.float32)
        self.lib.mem_d2h(out.ctypes.data, p, out.nbytes)
        ncmhip.check()
        return out

    def generate(self, prompt, n_new, eos=-1):
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(n_new, np.int32)
        n = self.lib.ncm_qwen_generate(self.m, prompt.ctypes.data, prompt.size, n_new, eos, out.ctypes.data)
        ncmhip.check()
        return list(out[:n])

    def generate_sample(self, prompt, n_new, temp, top_k, top_p, rng, eos=-1):
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(n_new, np.int32)
        st, nf = ctypes.c_uint64(rng), ctypes.c_int(-1)
        n = self.lib.ncm_qwen_generate_sample(self.m, prompt.ctypes.data, prompt.size, n_new, eos, temp, top_k,
                                              top_p, ctypes.byref(st), out.ctypes.data, ctypes.byref(nf))
        ncmhip.check()
        return list(out[:n]), st.value, nf.value

    def close(self):
        self.lib.ncm_qwen_free(self.m)


SMALL = dict(n_layer=2, C=896, H=14, K=2, I=4864, V=151936)


def test_prefill_logits_vs_oracle():
    cfg = SMALL
    params = weights(1, **cfg)
    ids = np.random.default_rng(2).integers(0, cfg["V"], 37).astype(np.int32)
    ref = O.qwen_forward(params, theta=1e6, ids=ids, **cfg)
    m = Model(params, n_ctx=64, theta=1e6, **cfg)
    try:
        got = m.forward(ids)
        assert float(np.max(np.abs(got - ref))) <= 1e-3
        last = m.forward(ids, last_only=True)
        assert float(np.max(np.abs(last - ref[-1]))) <= 1e-3
        assert int(np.argmax(last)) == O.argmax_row(ref[-1])
    finally:
        m.close()


def test_greedy_generation_vs_full_recompute():
    cfg = SMALL
    params = weights(3, **cfg)
    prompt = np.random.default_rng(4).integers(0, cfg["V"], 21).astype(np.int32)
    n_new = 8
    ref_ids, ref_steps = O.qwen_generate(params, theta=1e6, prompt=prompt, n_new=n_new, n_ctx=64, **cfg)
    m = Model(params, n_ctx=64, theta=1e6, **cfg)
    try:
        assert m.generate(prompt, n_new) == ref_ids
        # per-step cached logits against the full-recompute logits
        m.forward(prompt, last_only=True)
        toks = list(prompt)
        for s in range(1, n_new):
            toks.append(ref_ids[s - 1])
            got = m.decode(ref_ids[s - 1], len(toks) - 1)
            assert float(np.max(np.abs(got - ref_steps[s]))) <= 1e-3
        # eos stop: the generation ends after the first occurrence of the eos id
        eos = ref_ids[2]
        assert m.generate(prompt, n_new, eos=eos) == ref_ids[:ref_ids.index(eos) + 1]
    finally:
        m.close()


def test_full_size_cached_decode_matches_full_forward():
    cfg = dict(n_layer=24, C=896, H=14, K=2, I=4864, V=151936)
    params = weights(5, **cfg)
    prompt = np.random.default_rng(6).integers(0, cfg["V"], 2048).astype(np.int32)
    m = Model(params, n_ctx=2304, theta=1e6, **cfg)
    try:
        ids = m.generate(prompt, 4)
        assert len(ids) == 4 and all(0 <= i < cfg["V"] for i in ids)
        seq = np.concatenate([prompt, np.array(ids[:3], np.int32)])
        full = m.forward(seq, last_only=True)           # recompute over 2051 tokens
        m.forward(seq[:-1], last_only=True)              # cache for positions 0..2049
        step = m.decode(seq[-1], len(seq) - 1)
        assert float(np.max(np.abs(step - full))) <= 1e-3
        assert int(np.argmax(full)) == ids[3]
    finally:
        m.close()


def test_config4_greedy_ids_256_steps_match_cpu(golden):
    """Config 4 end to end: the seeded 24-layer model, a 2048-token prompt and
    256 greedy steps give the CPU reference's ids exactly
    (tests/golden/qwen_greedy_c4.npz, written by gen_qwen_greedy.py with the
    oracle's KV-cached generation, which is bit-equal to the reference's
    qwen_generate).  Also logs the device's logit error at each step's 8
    largest CPU logits against the step's top-2 gap, the margin that keeps
    the argmax exact."""
    g = golden("qwen_greedy_c4.npz")
    params = MD.qwen_weights(MD.C4_SEED, **MD.C4)
    prompt = MD.c4_prompt()
    m = Model(params, n_ctx=MD.C4_CTX, theta=MD.C4_THETA, **MD.C4)
    try:
        ids = m.generate(prompt, MD.C4_NEW)
        first_diff = next((i for i, (a, b) in enumerate(zip(ids, g["ids"])) if a != b), None)
        # the logits of every step along the CPU's ids, from the eager cached decode
        err, gaps = [], g["top_vals"][:, 0].astype(np.float64) - g["top_vals"][:, 1]
        lg = m.forward(prompt, last_only=True)
        for s in range(MD.C4_NEW):
            err.append(float(np.max(np.abs(lg[g["top_ids"][s]] - g["top_vals"][s]))))
            if s + 1 < MD.C4_NEW:
                lg = m.decode(int(g["ids"][s]), MD.C4_PROMPT + s)
        err = np.array(err)
        print(f"[c4] 256 greedy ids: first difference at {first_diff}; max logit error {err.max():.2e}; "
              f"min top-2 gap {gaps.min():.2e} (step {int(gaps.argmin())}); min gap/error "
              f"{float(np.min(gaps / np.maximum(err, 1e-12))):.1f}", flush=True)
        assert first_diff is None and len(ids) == MD.C4_NEW
        assert err.max() <= 1e-3
    finally:
        m.close()


def test_decode_graph_replays_match_eager(monkeypatch):
    """The captured decode step, replayed over several generations with eager
    work and synchronisation in between, gives the ids of the same kernels
    launched one by one."""
    cfg = SMALL
    params = weights(7, **cfg)
    rng = np.random.default_rng(8)
    p1, p2 = rng.integers(0, cfg["V"], 19).astype(np.int32), rng.integers(0, cfg["V"], 33).astype(np.int32)
    eager = Model(params, n_ctx=64, theta=1e6, **cfg)
    graph = Model(params, n_ctx=64, theta=1e6, **cfg)
    try:
        monkeypatch.setenv("NCM_NO_GRAPH", "1")
        e1, e2 = eager.generate(p1, 12), eager.generate(p2, 12)
        monkeypatch.delenv("NCM_NO_GRAPH")
        g1 = graph.generate(p1, 12)
        graph.forward(p2[:10], last_only=True)          # eager work between replays
        ncmhip.sync()
        g2 = graph.generate(p2, 12)
        g3 = graph.generate(p1, 12)
        assert g1 == e1 and g2 == e2 and g3 == e1
    finally:
        eager.close()
        graph.close()


@pytest.mark.parametrize("temp,top_k,top_p", [(0.8, 0, 0.9), (1.3, 40, 1.0), (0.05, 0, 0.95)])
def test_sampled_generation_draws_match_oracle(temp, top_k, top_p, monkeypatch):
    """Sampling inside the replayed decode graph: every step's id and the rng
    state are the reference sampler's (oracle, pinned to kernels.c:782-825)
    on that step's logits, which the eager cached decode reproduces; graph
    and eager generation agree; the greedy setting falls back to argmax."""
    cfg = SMALL
    params = weights(5, **cfg)
    prompt = np.random.default_rng(6).integers(0, cfg["V"], 19).astype(np.int32)
    n_new, seed = 10, 0x5EED
    m = Model(params, n_ctx=64, theta=1e6, **cfg)
    try:
        ids, st, nf = m.generate_sample(prompt, n_new, temp, top_k, top_p, seed)
        assert len(ids) == n_new and nf == 0
        lg = m.forward(prompt, last_only=True)
        s = seed
        for k in range(n_new):
            want, s = O.sample_topkp(lg, temp, top_k, top_p, s)
            assert ids[k] == want, k
            if k + 1 < n_new:
                lg = m.decode(ids[k], len(prompt) + k)
        assert st == s
        ids2, st2, _ = m.generate_sample(prompt, n_new, temp, top_k, top_p, seed)   # graph replays
        monkeypatch.setenv("NCM_NO_GRAPH", "1")
        ids3, st3, _ = m.generate_sample(prompt, n_new, temp, top_k, top_p, seed)   # eager launches
        assert ids2 == ids and ids3 == ids and st2 == st3 == st
        eos = ids[3]
        ids4, _, _ = m.generate_sample(prompt, n_new, temp, top_k, top_p, seed, eos=eos)
        assert ids4 == ids[:ids.index(eos) + 1]
        assert m.generate_sample(prompt, 4, 0.0, top_k, top_p, seed)[:2] == (m.generate(prompt, 4), seed)
    finally:
        m.close()


@pytest.mark.parametrize("H,K", [(8, 2), (4, 4), (16, 1)])
def test_decode_shapes_vs_oracle(H, K):
    """The cached decode step (64-key attention chunks and their merge, the
    workgroup-per-row-pair o and down projections) at other head counts and
    GQA ratios (4, 1 and 16) and context lengths that leave a chunk partly
    filled, end one exactly and open the next, against the oracle's full
    forward over the extended sequence."""
    cfg = dict(n_layer=2, C=64 * H, H=H, K=K, I=512, V=500)
    params = weights(9, **cfg)
    rng = np.random.default_rng(10)
    m = Model(params, n_ctx=1100, theta=1e6, **cfg)
    try:
        for np_ in (70, 127, 640):
            ids = list(rng.integers(0, cfg["V"], np_ + 3))
            m.forward(np.array(ids[:np_], np.int32), last_only=True)
            for s in range(3):
                pos = np_ + s
                got = m.decode(ids[pos], pos)
                ref = O.qwen_forward(params, theta=1e6, ids=np.array(ids[:pos + 1], np.int32), last_only=True,
                                     **cfg)
                err = float(np.max(np.abs(got - ref.reshape(-1))))
                print(f"[gpu] H={H} K={K} pos={pos}: logits max-abs {err:.2e}", flush=True)
                assert err <= 1e-3, (pos, err)
    finally:
        m.close()
