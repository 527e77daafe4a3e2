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


def ncp_named_weights(cfg, seed, scale=0.3, biases=True, tied_dim=16):
    """Random NCP weights under the reference's tensor names (ncp.c:94-175,
    184-345, 406-478) for a configuration dict as oracle.ref_ncp_forward
    takes it; norm gains 1 + N(0, 0.1^2)."""
    rng = np.random.default_rng(seed)
    C, H, nkv, D = cfg["n_embd"], cfg["n_head"], cfg["n_kv_heads"], cfg["vq_embed_dim"]
    hd = C // H
    I = cfg.get("n_inner", 2 * C)
    P = cfg.get("prefix_len", 0)
    first = 0 if cfg.get("query_level0", 0) else 1
    tl = list(cfg["levels"])[first:]
    named = {}

    def w(name, shape, s=scale, mean=0.0):
        named[name] = (np.float32(mean) + np.float32(s) * rng.standard_normal(shape, dtype=np.float32)).astype(
            np.float32)

    def bias(name, shape):
        if biases:
            w(name, shape, 0.1)

    pre = "gen.transformer."
    w(pre + "wte.weight", (C, D))
    bias(pre + "wte.bias", (C,))
    w(pre + "wle.weight", (len(tl), C))
    if not cfg.get("use_rope", 0):
        w(pre + "wpe.weight", (max([P] + tl), C))
    for li in range(cfg["n_layer"]):
        b = f"{pre}blocks.{li}."
        w(b + "ln_1.weight", (C,), 0.1, 1.0)
        bias(b + "ln_1.bias", (C,))
        w(b + "attn.c_attn.weight", (C + 2 * nkv * hd, C), scale / np.sqrt(C) * 4)
        bias(b + "attn.c_attn.bias", (C + 2 * nkv * hd,))
        if cfg.get("use_qk_norm", 0):
            w(b + "attn.q_norm.weight", (hd,), 0.1, 1.0)
            w(b + "attn.k_norm.weight", (hd,), 0.1, 1.0)
        w(b + "attn.c_proj.weight", (C, C), scale / np.sqrt(C) * 4)
        bias(b + "attn.c_proj.bias", (C,))
        w(b + "ln_2.weight", (C,), 0.1, 1.0)
        bias(b + "ln_2.bias", (C,))
        if cfg.get("use_swiglu", 0) or cfg.get("use_geglu", 0):
            w(b + "mlp.w_gate.weight", (I, C), scale / np.sqrt(C) * 4)
            bias(b + "mlp.w_gate.bias", (I,))
            w(b + "mlp.w_up.weight", (I, C), scale / np.sqrt(C) * 4)
            bias(b + "mlp.w_up.bias", (I,))
        else:
            w(b + "mlp.c_fc.weight", (I, C), scale / np.sqrt(C) * 4)
            bias(b + "mlp.c_fc.bias", (I,))
        w(b + "mlp.c_proj.weight", (C, I), scale / np.sqrt(I) * 4)
        bias(b + "mlp.c_proj.bias", (C,))
    w(pre + "ln_f.weight", (C,), 0.1, 1.0)
    bias(pre + "ln_f.bias", (C,))
    if cfg.get("puc_enabled", 0):
        K = cfg["puc_kernel"]
        for k in range(len(tl)):
            w(f"gen.post_upsample_convs.{k}.weight", (D, D, K), scale / np.sqrt(D * K))
            w(f"gen.post_upsample_convs.{k}.bias", (D,), 0.1)
    vocabs = list(cfg["vocab_size"])[:len(tl)]
    if cfg.get("shared_output_head", 0):
        w("gen.lm_heads.head.weight", (max(vocabs), C))
        if cfg.get("shared_head_per_level_bias", 0):
            for k, V in enumerate(vocabs):
                w(f"gen.lm_heads.biases.{k}", (V,), 0.1)
        elif cfg.get("untied_head_bias", 0):
            w("gen.lm_heads.head.bias", (max(vocabs),), 0.1)
    elif cfg.get("tie_heads_to_codebook", 0):
        for k, V in enumerate(vocabs):
            w(f"gen.lm_heads.{k}.proj.weight", (tied_dim, C))
            bias(f"gen.lm_heads.{k}.proj.bias", (tied_dim,))
            w(f"tok.vq.embeddings.{k + first}.weight", (V, tied_dim), 1.0)
            w(f"gen.lm_heads.{k}.log_inv_T", (1,), 0.5)
            bias(f"gen.lm_heads.{k}.bias", (V,))
    else:
        for k, V in enumerate(vocabs):
            w(f"gen.lm_heads.{k}.weight", (V, C))
            bias(f"gen.lm_heads.{k}.bias", (V,))
    return named


def ncp_cfg(**kw):
    """An NCP configuration dict with the reference's defaults for the
    fields a test does not set."""
    c = dict(n_layer=2, n_head=4, n_embd=64, n_kv_heads=2, n_inner=96, prefix_len=0, query_level0=0,
             attn_pattern_block_diag=1, use_rope=1, rope_base=10000, use_qk_norm=0, puc_enabled=0, puc_kernel=3,
             shared_output_head=0, shared_head_per_level_bias=0, untied_head_bias=0, tie_heads_to_codebook=0,
             use_swiglu=1, use_geglu=0, use_relu2=0, vq_embed_dim=24, prefix_pad_token_id=-1,
             levels=[1, 2, 4, 8], vocab_size=[40, 48, 56])
    c.update(kw)
    return c


# Multi-level NCP configurations exercising every branch of ncp_forward.
NCP_CASES = {
    "block_diag_swiglu": ncp_cfg(),
    "block_causal_prefix_qknorm": ncp_cfg(attn_pattern_block_diag=0, prefix_len=5, use_qk_norm=1),
    "prefix_pads": ncp_cfg(prefix_len=6, prefix_pad_token_id=0),
    "no_rope_wpe_gelu": ncp_cfg(use_rope=0, use_swiglu=0, prefix_len=3),
    "relu2_shared_level_bias": ncp_cfg(use_swiglu=0, use_relu2=1, shared_output_head=1,
                                       shared_head_per_level_bias=1),
    "geglu_shared_bias_query0": ncp_cfg(use_swiglu=0, use_geglu=1, shared_output_head=1, untied_head_bias=1,
                                        query_level0=1, vocab_size=[32, 40, 48, 56]),
    "tied_codebook_puc_mha": ncp_cfg(tie_heads_to_codebook=1, puc_enabled=1, puc_kernel=3, n_kv_heads=4),
}


# Config 5 (BASELINE): the GPT-2-style training step, 12 layers, d 768, 12
# heads, vocab 4096, learned positions (512), batch 32 x 512 tokens.
C5 = dict(n_layer=12, C=768, H=12, V=4096, npos=512)
C5_B, C5_T = 32, 512


def gpt2_c5_weights(seed=51):
    """Parameters in oracle.gpt2_shapes order, N(0, 0.02^2) float32 draws with
    1.0 added to the LayerNorm gains (and to ln_f's last tensor), then token
    ids and shifted targets uniform in [0, V)."""
    rng = np.random.default_rng(seed)
    shapes = O.gpt2_shapes(C5["n_layer"], C5["C"], C5["V"], C5["npos"])
    ps = [(rng.standard_normal(s, dtype=np.float32) * np.float32(0.02)) for s in shapes]
    for i, s in enumerate(shapes):
        if len(s) == 1 and s[0] == C5["C"] and (i >= len(ps) - 2 or (i - 2) % 12 in (0, 6)):
            ps[i] = ps[i] + np.float32(1.0)
    ids = rng.integers(0, C5["V"], (C5_B, C5_T)).astype(np.int32)
    tgt = rng.integers(0, C5["V"], (C5_B, C5_T)).astype(np.int32)
    return ps, ids, tgt


def grad_probe_signs(n, seed):
    """A seeded +-1 vector of length n (float64): the probe direction of a
    full-tensor gradient checksum sum(g * s)."""
    rng = np.random.default_rng(seed)
    return np.where(rng.integers(0, 2, n) == 1, 1.0, -1.0)


# Config 3 (BASELINE): 65536 encoder vectors of dim 256, 4 residual scales of
# 4096 codes each.
C3 = dict(R=65536, D=256, V=4096, S=4)


def vq_c3_inputs(seed=2026):
    """z ~ N(0, 1) [R][D] and S codebooks ~ N(0, 1) / sqrt(D) [V][D], float32,
    drawn in that order from one generator."""
    rng = np.random.default_rng(seed)
    R, D, V, S = C3["R"], C3["D"], C3["V"], C3["S"]
    z = rng.standard_normal((R, D)).astype(np.float32)
    Es = [(rng.standard_normal((V, D)) / np.sqrt(D)).astype(np.float32) for _ in range(S)]
    return z, Es
