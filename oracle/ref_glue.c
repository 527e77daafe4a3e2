/* ref_glue.c -- drives the REFERENCE's own CPU functions for oracle
 * validation.  Compiled only together with the reference sources from
 * /root/reference/src into oracle/_ref/libref.so (see oracle/Makefile);
 * never part of libncmhip.so.  Test infrastructure only.
 *
 * refg_linear_bwd runs the reference tape: t_linear (train_tape.c:156-162)
 * then tape_backward_host (train_tape.c:636) with the layer output
 * registered as a parameter whose gradient buffer holds dy, so the
 * TOP_LINEAR case (train_tape.c:680-725) sees exactly that upstream
 * gradient and accumulates into the caller's dx/dW/db.
 *
 * refg_vq_multiscale runs vq_load + vq_z_to_idx (vq.c:76, vq.c:378) on a
 * zeroed NCMConfig with n levels of length L (identity resampling, no Phi)
 * and in-memory codebooks, and returns codes plus the final z_hat / z_rest,
 * which vq_z_to_idx_soft (vq.c:394-395) allocates as the first two blocks
 * of the freshly reset scratch arena. */
#include "ncm.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

void refg_linear_bwd(const float *x, const float *W, const float *b, const float *dy,
                     float *dx, float *dW, float *db, long long batch, int M, int K) {
    Tape *t = tape_new();
    float *y = (float *)malloc((size_t)(batch > 0 ? batch : 1) * M * sizeof(float));
    float *g = (float *)malloc((size_t)(batch > 0 ? batch : 1) * M * sizeof(float));
    memcpy(g, dy, (size_t)batch * M * sizeof(float));
    t_linear(t, x, W, b, y, batch, M, K);
    float *params[4] = {y, (float *)x, (float *)W, (float *)b};
    float *grads[4] = {g, dx, dW, db};
    int64_t sizes[4] = {batch * M, batch * K, (int64_t)M * K, M};
    PMap pm = {params, grads, sizes, b ? 4 : 3};
    tape_backward_host(t, &pm, 1.0f);
    tape_free(t);
    free(y);
    free(g);
}

static int g_arena_ready = 0;

int refg_vq_multiscale(const float *z, const float *E_flat, const int *vocabs, int n_levels,
                       int B, int L, int D, int *idx, float *z_hat, float *z_rest) {
    if (n_levels <= 0 || n_levels > NCM_MAX_LEVELS) return -1;
    if (!g_arena_ready) {
        arena_init_default();   /* NCM_ARENA_MB, else 2048 MB */
        g_arena_ready = 1;
    }
    NCMConfig *c = (NCMConfig *)calloc(1, sizeof(NCMConfig));
    c->n_qlevels = n_levels;
    c->vq_embed_dim = D;
    for (int i = 0; i < n_levels; i++) {
        c->levels[i] = L;
        c->vq_vocab[i] = vocabs[i];
    }
    WeightStore ws;
    ws.count = n_levels;
    ws.items = (NamedTensor *)calloc((size_t)n_levels, sizeof(NamedTensor));
    Tensor *ts = (Tensor *)calloc((size_t)n_levels, sizeof(Tensor));
    size_t off = 0;
    for (int i = 0; i < n_levels; i++) {
        snprintf(ws.items[i].name, sizeof(ws.items[i].name), "embeddings.%d.weight", i);
        ts[i].data = (float *)E_flat + off;
        ts[i].ndim = 2;
        ts[i].shape[0] = vocabs[i];
        ts[i].shape[1] = D;
        ts[i].n = (int64_t)vocabs[i] * D;
        ws.items[i].t = &ts[i];
        off += (size_t)vocabs[i] * D;
    }
    VQState *vq = vq_load(c, &ws, "");
    arena_reset();
    float *base = arena_alloc(0);
    arena_reset();
    vq_z_to_idx(vq, z, B, idx);
    size_t n = (size_t)B * L * D;
    size_t step = (n * sizeof(float) + 15) & ~(size_t)15;
    memcpy(z_rest, base, n * sizeof(float));
    memcpy(z_hat, (unsigned char *)base + step, n * sizeof(float));
    arena_reset();
    vq_free(vq);
    free(ts);
    free(ws.items);
    free(c);
    return 0;
}

/* ---- training backward: the reference tape on single records ----
 * Each helper records one op with the reference's t_* wrapper (which runs
 * the reference CPU forward), registers the op's output as a "parameter"
 * whose gradient buffer holds the upstream gradient, registers the inputs
 * with the caller's gradient buffers, and runs tape_backward_host: the op's
 * backward case then accumulates into exactly those buffers. */
static void ensure_arena(void) {
    if (!g_arena_ready) {
        arena_init_default();   /* NCM_ARENA_MB, else 2048 MB */
        g_arena_ready = 1;
    }
}

static void run_tape(Tape *t, float **params, float **grads, int64_t *sizes, int n) {
    float *p2[8], *g2[8];
    int64_t s2[8];
    int m = 0;
    for (int i = 0; i < n; i++)
        if (params[i] && grads[i]) {
            p2[m] = params[i];
            g2[m] = grads[i];
            s2[m] = sizes[i];
            m++;
        }
    PMap pm = {p2, g2, s2, m};
    tape_backward_host(t, &pm, 1.0f);
}

/* eps < 0: t_layernorm (TOP_LN, eps 1e-6); else t_layernorm_eps (TOP_LNE). */
void refg_ln_bwd(const float *x, const float *w, const float *b, const float *dy, float *y, float *dx, float *dw,
                 float *db, long long rows, int C, double eps) {
    Tape *t = tape_new();
    float *g = (float *)malloc((size_t)(rows > 0 ? rows : 1) * C * sizeof(float));
    memcpy(g, dy, (size_t)rows * C * sizeof(float));
    if (eps < 0)
        t_layernorm(t, x, w, b, y, rows, C);
    else
        t_layernorm_eps(t, x, w, b, y, rows, C, eps);
    float *params[4] = {y, (float *)x, (float *)w, (float *)b};
    float *grads[4] = {g, dx, dw, db};
    int64_t sizes[4] = {rows * C, rows * C, C, C};
    run_tape(t, params, grads, sizes, 4);
    tape_free(t);
    free(g);
}

void refg_rmsn_bwd(const float *x, const float *w, const float *dy, float *y, float *dx, float *dw, long long rows,
                   int C) {
    Tape *t = tape_new();
    float *g = (float *)malloc((size_t)(rows > 0 ? rows : 1) * C * sizeof(float));
    memcpy(g, dy, (size_t)rows * C * sizeof(float));
    t_rmsnorm(t, x, w, y, rows, C);
    float *params[3] = {y, (float *)x, (float *)w};
    float *grads[3] = {g, dx, dw};
    int64_t sizes[3] = {rows * C, rows * C, C};
    run_tape(t, params, grads, sizes, 3);
    tape_free(t);
    free(g);
}

/* t_ce (train_tape.c:442-481) + its backward into dl (accumulating). */
void refg_ce(const float *logits, const int *tgt, const float *wm, float *loss, float *probs, float *dl,
             long long rows, int V, double weight) {
    Tape *t = tape_new();
    t_ce(t, logits, tgt, wm, loss, probs, rows, V, weight);
    float *params[1] = {(float *)logits};
    float *grads[1] = {dl};
    int64_t sizes[1] = {rows * V};
    run_tape(t, params, grads, sizes, 1);
    tape_free(t);
}

/* t_sdpa (train_tape.c:277-323) + TOP_SDPA backward.  P (the probabilities
 * the tape stores) is the first block of the freshly reset scratch arena;
 * it is copied to P_out. */
void refg_sdpa_bwd(const float *q, const float *k, const float *v, const float *mask, const float *dy, float *o,
                   float *dq, float *dk, float *dv, float *P_out, int B, int H, int Hkv, int Tq, int Tkv, int hd) {
    ensure_arena();
    arena_reset();
    float *base = arena_alloc(0);
    arena_reset();
    Tape *t = tape_new();
    int64_t no = (int64_t)B * H * Tq * hd, nk = (int64_t)B * Hkv * Tkv * hd;
    float *g = (float *)malloc((size_t)(no > 0 ? no : 1) * sizeof(float));
    memcpy(g, dy, (size_t)no * sizeof(float));
    t_sdpa(t, q, k, v, mask, o, B, H, Hkv, Tq, Tkv, hd);
    memcpy(P_out, base, (size_t)B * H * Tq * Tkv * sizeof(float));
    float *params[4] = {o, (float *)q, (float *)k, (float *)v};
    float *grads[4] = {g, dq, dk, dv};
    int64_t sizes[4] = {no, no, nk, nk};
    run_tape(t, params, grads, sizes, 4);
    tape_free(t);
    free(g);
    arena_reset();
}

/* kind 0 t_gelu, 1 t_silu, 2 t_gelu_tanh (train_tape.c:209-227) */
void refg_act_bwd(int kind, const float *x, const float *dy, float *y, float *dx, long long n) {
    Tape *t = tape_new();
    float *g = (float *)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    memcpy(g, dy, (size_t)n * sizeof(float));
    if (kind == 0) t_gelu(t, x, y, n);
    else if (kind == 1) t_silu(t, x, y, n);
    else t_gelu_tanh(t, x, y, n);
    float *params[2] = {y, (float *)x};
    float *grads[2] = {g, dx};
    int64_t sizes[2] = {n, n};
    run_tape(t, params, grads, sizes, 2);
    tape_free(t);
    free(g);
}

void refg_mul_bwd(const float *a, const float *b, const float *dy, float *y, float *da, float *db, long long n) {
    Tape *t = tape_new();
    float *g = (float *)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    memcpy(g, dy, (size_t)n * sizeof(float));
    t_mul(t, a, b, y, n);
    float *params[3] = {y, (float *)a, (float *)b};
    float *grads[3] = {g, da, db};
    int64_t sizes[3] = {n, n, n};
    run_tape(t, params, grads, sizes, 3);
    tape_free(t);
    free(g);
}

/* t_rope (train_tape.c:260-275): out-of-place rope of xq, xk */
void refg_rope_bwd(const float *xq, const float *xk, const float *cos_t, const float *sin_t, const float *gq,
                   const float *gk, float *yq, float *yk, float *dxq, float *dxk, int B, int H, int Hkv, int T,
                   int hd) {
    Tape *t = tape_new();
    int64_t nq = (int64_t)B * H * T * hd, nk = (int64_t)B * Hkv * T * hd;
    float *g1 = (float *)malloc((size_t)nq * sizeof(float)), *g2 = (float *)malloc((size_t)nk * sizeof(float));
    memcpy(g1, gq, (size_t)nq * sizeof(float));
    memcpy(g2, gk, (size_t)nk * sizeof(float));
    t_rope(t, xq, xk, yq, yk, cos_t, sin_t, B, H, Hkv, T, hd);
    float *params[4] = {yq, yk, (float *)xq, (float *)xk};
    float *grads[4] = {g1, g2, dxq, dxk};
    int64_t sizes[4] = {nq, nk, nq, nk};
    run_tape(t, params, grads, sizes, 4);
    tape_free(t);
    free(g1);
    free(g2);
}

/* t_embed (train_tape.c:164-174); its index copy lives in the scratch arena */
void refg_embed_bwd(const float *W, const int *idx, int V, const float *dy, float *y, float *dW, long long n,
                    int D) {
    ensure_arena();
    arena_reset();
    Tape *t = tape_new();
    float *g = (float *)malloc((size_t)(n > 0 ? n : 1) * D * sizeof(float));
    memcpy(g, dy, (size_t)n * D * sizeof(float));
    t_embed(t, W, idx, V, y, n, D);
    float *params[2] = {y, (float *)W};
    float *grads[2] = {g, dW};
    int64_t sizes[2] = {n * D, (int64_t)V * D};
    run_tape(t, params, grads, sizes, 2);
    tape_free(t);
    free(g);
    arena_reset();
}

void refg_split_bwd(const float *in, const float *gq, const float *gk, const float *gv, float *qq, float *kk,
                    float *vv, float *dx, int B, int T, int C, int H, int hd, int K, int rep) {
    Tape *t = tape_new();
    int64_t no = (int64_t)B * H * T * hd, ni = (int64_t)B * T * (C + 2 * K * hd);
    float *g[3];
    const float *src[3] = {gq, gk, gv};
    for (int i = 0; i < 3; i++) {
        g[i] = src[i] ? (float *)malloc((size_t)no * sizeof(float)) : NULL;
        if (g[i]) memcpy(g[i], src[i], (size_t)no * sizeof(float));
    }
    t_qkvsplit(t, in, qq, kk, vv, B, T, C, H, hd, K, rep);
    float *params[4] = {qq, kk, vv, (float *)in};
    float *grads[4] = {g[0], g[1], g[2], dx};
    int64_t sizes[4] = {no, no, no, ni};
    run_tape(t, params, grads, sizes, 4);
    tape_free(t);
    for (int i = 0; i < 3; i++) free(g[i]);
}

/* kind 0 t_headmerge, 1 t_headsplit */
void refg_merge_bwd(int kind, const float *in, const float *dy, float *y, float *dx, int B, int T, int C, int H,
                    int hd) {
    Tape *t = tape_new();
    int64_t nh = (int64_t)B * H * T * hd, nc = (int64_t)B * T * C;
    int64_t ny = kind == 0 ? nc : nh, nx = kind == 0 ? nh : nc;
    float *g = (float *)malloc((size_t)ny * sizeof(float));
    memcpy(g, dy, (size_t)ny * sizeof(float));
    if (kind == 0) t_headmerge(t, in, y, B, T, C, H, hd);
    else t_headsplit(t, in, y, B, T, C, H, hd);
    float *params[2] = {y, (float *)in};
    float *grads[2] = {g, dx};
    int64_t sizes[2] = {ny, nx};
    run_tape(t, params, grads, sizes, 2);
    tape_free(t);
    free(g);
}

/* The reference's taped GPT-2 forward (train_gpt2.c:107-147) + t_ce + the
 * host tape backward on a WeightStore built from flat host arrays in the
 * order: wte, wpe, per layer the 12 h.<l>.* tensors, ln_f.weight,
 * ln_f.bias.  Returns the mean loss; grads (zeroed by the caller, same
 * order) receive dL/dparam before any clipping. */
float refg_gpt2_grads(float *const *params, float *const *grads, int n_layer, int C, int H, int V, int npos,
                      const int *ids, const int *tgt, int B, int T) {
    static const char *names[12] = {"ln_1.weight", "ln_1.bias", "attn.c_attn.weight", "attn.c_attn.bias",
                                    "attn.c_proj.weight", "attn.c_proj.bias", "ln_2.weight", "ln_2.bias",
                                    "mlp.c_fc.weight", "mlp.c_fc.bias", "mlp.c_proj.weight", "mlp.c_proj.bias"};
    const int n = 4 + 12 * n_layer;
    ensure_arena();
    arena_reset();
    NCMConfig *c = (NCMConfig *)calloc(1, sizeof(NCMConfig));
    c->n_layer = n_layer;
    c->n_head = H;
    c->n_embd = C;
    WeightStore ws;
    ws.count = n;
    ws.items = (NamedTensor *)calloc((size_t)n, sizeof(NamedTensor));
    Tensor *ts = (Tensor *)calloc((size_t)n, sizeof(Tensor));
    int64_t *sizes = (int64_t *)calloc((size_t)n, sizeof(int64_t));
    for (int i = 0; i < n; i++) {
        int64_t r = C, k = 1;
        if (i == 0) { r = V; k = C; }
        else if (i == 1) { r = npos; k = C; }
        else if (i < n - 2) {
            int j = (i - 2) % 12;
            if (j == 2) { r = 3 * C; k = C; }
            else if (j == 3) { r = 3 * C; }
            else if (j == 4) { r = C; k = C; }
            else if (j == 8) { r = 4 * C; k = C; }
            else if (j == 9) { r = 4 * C; }
            else if (j == 10) { r = C; k = 4 * C; }
        }
        if (i == 0) snprintf(ws.items[i].name, sizeof(ws.items[i].name), "wte.weight");
        else if (i == 1) snprintf(ws.items[i].name, sizeof(ws.items[i].name), "wpe.weight");
        else if (i == n - 2) snprintf(ws.items[i].name, sizeof(ws.items[i].name), "ln_f.weight");
        else if (i == n - 1) snprintf(ws.items[i].name, sizeof(ws.items[i].name), "ln_f.bias");
        else snprintf(ws.items[i].name, sizeof(ws.items[i].name), "h.%d.%s", (i - 2) / 12, names[(i - 2) % 12]);
        ts[i].data = params[i];
        ts[i].ndim = k > 1 ? 2 : 1;
        ts[i].shape[0] = r;
        ts[i].shape[1] = k;
        ts[i].n = r * k;
        ws.items[i].t = &ts[i];
        sizes[i] = r * k;
    }
    Tape *tp = tape_new();
    float *logits = train_gpt2_forward(tp, &ws, c, ids, B, T);
    float *loss = arena_alloc(1), *probs = arena_alloc((size_t)B * T * V);
    t_ce(tp, logits, tgt, NULL, loss, probs, (int64_t)B * T, V, 1.0);
    PMap pm = {(float **)params, (float **)grads, sizes, n};
    tape_backward_host(tp, &pm, 0);
    float lh = *loss;
    tape_free(tp);
    arena_reset();
    free(sizes);
    free(ts);
    free(ws.items);
    free(c);
    return lh;
}

/* ---- the NCP transformer forward (ncp.c:94-175, 480-640) ----
 * refg_ncp_forward fills an NCMConfig from cfg[] (indices below) and the
 * level / vocabulary lists, a WeightStore from (names, data, shapes), and
 * runs the reference's own ncp_load + ncp_forward: x [B][P+T][D] -> logits
 * [B][T][maxV] (entries past a level's vocabulary are -inf, ncp.c:604).
 * prefix_ids may be NULL (no pad bias). */
enum {
    NCPC_N_LAYER, NCPC_N_HEAD, NCPC_N_EMBD, NCPC_N_KV, NCPC_PREFIX_LEN, NCPC_QUERY_LEVEL0, NCPC_BLOCK_DIAG,
    NCPC_USE_ROPE, NCPC_ROPE_BASE, NCPC_QK_NORM, NCPC_PUC, NCPC_PUC_KERNEL, NCPC_SHARED_HEAD,
    NCPC_SHARED_HEAD_LEVEL_BIAS, NCPC_UNTIED_HEAD_BIAS, NCPC_TIE_CODEBOOK, NCPC_SWIGLU, NCPC_GEGLU, NCPC_RELU2,
    NCPC_VQ_DIM, NCPC_PAD_ID, NCPC_COUNT
};

void refg_parena_once(void) {
    /* the persistent arena is sized by its first user and never reset, so
     * reserve room for every model a test process opens (malloc'd lazily) */
    static int ready = 0;
    if (!ready) {
        parena_init((size_t)1 << 30);
        ready = 1;
    }
}

int refg_ncp_forward(const int *cfg, int n_qlevels, const int *levels, const int *vocabs, int n_vocabs,
                     const char *const *names, float *const *data, const long long *shapes, const int *ndims,
                     int n_tensors, const float *x, const int *prefix_ids, int B, float *logits) {
    if (n_qlevels <= 0 || n_qlevels > NCM_MAX_LEVELS || n_vocabs > NCM_MAX_VOCAB_LIST) return -1;
    refg_parena_once();
    ensure_arena();
    arena_reset();
    NCMConfig *c = (NCMConfig *)calloc(1, sizeof(NCMConfig));
    c->n_layer = cfg[NCPC_N_LAYER];
    c->n_head = cfg[NCPC_N_HEAD];
    c->n_embd = cfg[NCPC_N_EMBD];
    c->n_kv_heads = cfg[NCPC_N_KV];
    c->prefix_len = cfg[NCPC_PREFIX_LEN];
    c->query_level0 = cfg[NCPC_QUERY_LEVEL0];
    c->attn_pattern_block_diag = cfg[NCPC_BLOCK_DIAG];
    c->use_rope = cfg[NCPC_USE_ROPE];
    c->rope_base = cfg[NCPC_ROPE_BASE];
    c->use_qk_norm = cfg[NCPC_QK_NORM];
    c->puc_enabled = cfg[NCPC_PUC];
    c->puc_kernel = cfg[NCPC_PUC_KERNEL];
    c->shared_output_head = cfg[NCPC_SHARED_HEAD];
    c->shared_head_per_level_bias = cfg[NCPC_SHARED_HEAD_LEVEL_BIAS];
    c->untied_head_bias = cfg[NCPC_UNTIED_HEAD_BIAS];
    c->tie_heads_to_codebook = cfg[NCPC_TIE_CODEBOOK];
    c->use_swiglu = cfg[NCPC_SWIGLU];
    c->use_geglu = cfg[NCPC_GEGLU];
    c->use_relu2 = cfg[NCPC_RELU2];
    c->vq_embed_dim = cfg[NCPC_VQ_DIM];
    c->prefix_pad_token_id = cfg[NCPC_PAD_ID];
    c->n_qlevels = n_qlevels;
    for (int i = 0; i < n_qlevels; i++) c->levels[i] = levels[i];
    for (int i = 0; i < n_vocabs; i++) c->vocab_size[i] = vocabs[i];
    WeightStore ws;
    ws.count = n_tensors;
    ws.items = (NamedTensor *)calloc((size_t)n_tensors, sizeof(NamedTensor));
    Tensor *ts = (Tensor *)calloc((size_t)n_tensors, sizeof(Tensor));
    for (int i = 0; i < n_tensors; i++) {
        snprintf(ws.items[i].name, sizeof(ws.items[i].name), "%s", names[i]);
        ts[i].data = data[i];
        ts[i].ndim = ndims[i];
        int64_t n = 1;
        for (int d = 0; d < ndims[i]; d++) {
            ts[i].shape[d] = shapes[4 * i + d];
            n *= shapes[4 * i + d];
        }
        ts[i].n = n;
        ws.items[i].t = &ts[i];
    }
    NCPState *m = ncp_load(c, &ws, NULL);
    arena_reset();
    ncp_forward(m, x, prefix_ids, logits, B);
    arena_reset();
    ncp_free(m);
    free(ts);
    free(ws.items);
    free(c);
    return 0;
}
