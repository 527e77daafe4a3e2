/* qwen.c -- the Qwen2 decoder of qwen.c (reference) on the device: the
 * full forward of qwen_forward (qwen.c:121-190) for prefill, and a KV-cached
 * decode step for greedy generation (qwen_generate, qwen.c:204-228, which
 * recomputes the whole sequence per token; every row it keeps depends only
 * on its prefix, so the cached step computes the same values).
 *
 * Parameters: one flat array of device pointers -- 0 embed_tokens [V][C]
 * (also the tied lm head); per layer l at 1 + 12 l: input_layernorm [C],
 * q_proj.weight [C][C], q_proj.bias [C], k_proj.weight [K*hd][C],
 * k_proj.bias, v_proj.weight [K*hd][C], v_proj.bias, o_proj.weight [C][C],
 * post_attention_layernorm [C], gate_proj [I][C], up_proj [I][C],
 * down_proj [C][I]; last: norm.weight [C] (the order of qwen.c:60-75). */
#include "internal.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define QW_PER_LAYER 12

#define HIP_TRY_NULL(call)                                                                \
    do {                                                                                  \
        hipError_t e_ = (call);                                                           \
        if (e_ != hipSuccess) {                                                           \
            ncm_fail(NCM_E_HIP, "%s:%d %s: %s", __FILE__, __LINE__, #call, hipGetErrorString(e_)); \
            return NULL;                                                                  \
        }                                                                                 \
    } while (0)

struct NcmQwen {
    NcmQwenConfig c;
    float **P;
    float *cos_t, *sin_t;   /* [n_ctx][hd] */
    float *kcache, *vcache; /* [n_layer][K][n_ctx][hd] */
    /* decode scratch */
    float *x, *h1, *q, *k, *v, *qr, *ctx, *x1, *h2, *gate, *up, *logits, *part_o, *part_ml;
    int *ids_dev;           /* token ids, one slot per position */
    int *pos_dev;           /* position of the current decode step (device) */
    float *amax_v;          /* greedy-argmax block partials */
    int *amax_i, amax_blocks;
    int head_grid;          /* dec_head_stream workgroups (0: the LM head runs as dec_gemv) */
    int nchunk_max;
    hipGraphExec_t step_graph; /* one decode step + argmax, replayed per token */
    int graph_state;        /* 0 not built, 1 built, -1 capture failed (eager) */
    /* sampling (temp > 0): the xorshift64* state, per-position certification
     * flags, a sampler workspace owned by the model (graph-stable), and the
     * decode + sample graph with the settings it was captured for */
    unsigned long long *rng_dev;
    int *flags_dev;
    void *samp_ws;
    hipGraphExec_t samp_graph;
    int samp_state, samp_top_k;
    float samp_temp, samp_top_p;
};

int ncm_qwen_param_count(const NcmQwenConfig *c) { return c ? 2 + QW_PER_LAYER * c->n_layer : 0; }

int64_t ncm_qwen_param_shape(const NcmQwenConfig *c, int i, int64_t *rows, int64_t *cols) {
    const int n = ncm_qwen_param_count(c);
    if (!c || i < 0 || i >= n) return -1;
    const int64_t C = c->n_embd, KH = (int64_t)c->n_kv * (c->n_embd / c->n_head), I = c->n_inner;
    int64_t r = C, k = 1;
    if (i == 0) { r = c->vocab; k = C; }
    else if (i < n - 1) {
        switch ((i - 1) % QW_PER_LAYER) {
        case 1: case 7: k = C; break;
        case 3: case 5: r = KH; k = C; break;
        case 4: case 6: r = KH; break;
        case 9: case 10: r = I; k = C; break;
        case 11: k = I; break;
        default: break;
        }
    }
    if (rows) *rows = r;
    if (cols) *cols = k;
    return r * k;
}

static int cfg_ok(const NcmQwenConfig *c) {
    if (!c || c->n_layer < 0 || c->n_embd <= 0 || c->n_head <= 0 || c->n_embd % c->n_head || c->n_kv <= 0 ||
        c->n_head % c->n_kv || c->n_inner <= 0 || c->vocab <= 0 || c->n_ctx <= 0 || (c->n_embd / c->n_head) % 2)
        return ncm_fail(NCM_E_ARG, "qwen: bad configuration");
    return 0;
}

void ncm_qwen_free(NcmQwen *m) {
    if (!m) return;
    if (!ncm_ready()) ncm_hip_sync();
    float *bufs[] = {m->cos_t, m->sin_t, m->kcache, m->vcache, m->x, m->h1, m->q, m->k, m->v, m->qr, m->ctx,
                     m->x1, m->h2, m->gate, m->up, m->logits, m->part_o, m->part_ml};
    for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++) ncm_hip_free(bufs[i]);
    ncm_hip_free(m->ids_dev);
    ncm_hip_free(m->pos_dev);
    ncm_hip_free(m->amax_v);
    ncm_hip_free(m->amax_i);
    if (m->graph_state == 1) hipGraphExecDestroy(m->step_graph);
    if (m->samp_state == 1) hipGraphExecDestroy(m->samp_graph);
    ncm_hip_free(m->rng_dev);
    ncm_hip_free(m->flags_dev);
    ncm_hip_free(m->samp_ws);
    free(m->P);
    free(m);
}

/* RoPE tables of qwen.c:85-101: angle t * theta^(-2d/hd) in fp64, cos/sin
 * rounded to float, duplicated over the two halves. */
static int build_rope(NcmQwen *m) {
    const int hd = m->c.n_embd / m->c.n_head, T = m->c.n_ctx, h = hd / 2;
    float *hc = (float *)malloc((size_t)T * hd * sizeof(float)), *hs = (float *)malloc((size_t)T * hd * sizeof(float));
    if (!hc || !hs) {
        free(hc);
        free(hs);
        return ncm_fail(NCM_E_OOM, "qwen: rope tables");
    }
    for (int t = 0; t < T; t++)
        for (int d = 0; d < h; d++) {
            double a = (double)t * pow(m->c.rope_theta, -(double)(2 * d) / (double)hd);
            float co = (float)cos(a), si = (float)sin(a);
            hc[(size_t)t * hd + d] = hc[(size_t)t * hd + d + h] = co;
            hs[(size_t)t * hd + d] = hs[(size_t)t * hd + d + h] = si;
        }
    mem_h2d(m->cos_t, hc, (size_t)T * hd * sizeof(float));
    mem_h2d(m->sin_t, hs, (size_t)T * hd * sizeof(float));
    free(hc);
    free(hs);
    return 0;
}

NcmQwen *ncm_qwen_new(const NcmQwenConfig *c, float *const *params) {
    if (cfg_ok(c) || !params || ncm_ready()) return NULL;
    NcmQwen *m = (NcmQwen *)calloc(1, sizeof(NcmQwen));
    if (!m) { ncm_fail(NCM_E_OOM, "qwen: state"); return NULL; }
    m->c = *c;
    const int n = ncm_qwen_param_count(c);
    m->P = (float **)malloc((size_t)n * sizeof(float *));
    if (!m->P) { free(m); ncm_fail(NCM_E_OOM, "qwen: params"); return NULL; }
    memcpy(m->P, params, (size_t)n * sizeof(float *));
    const int C = c->n_embd, hd = C / c->n_head, KH = c->n_kv * hd, I = c->n_inner;
    const size_t cache = (size_t)c->n_layer * c->n_kv * c->n_ctx * hd * sizeof(float);
    m->nchunk_max = (c->n_ctx + 63) / 64;    /* decode attention chunks of 64 keys */
#define ALLOC(f, bytes) if (!(m->f = (float *)ncm_hip_malloc(bytes))) goto fail
    ALLOC(cos_t, (size_t)c->n_ctx * hd * 4);
    ALLOC(sin_t, (size_t)c->n_ctx * hd * 4);
    ALLOC(kcache, cache ? cache : 4);
    ALLOC(vcache, cache ? cache : 4);
    ALLOC(x, (size_t)C * 4);
    ALLOC(h1, (size_t)C * 4);
    ALLOC(q, (size_t)C * 4);
    ALLOC(k, (size_t)KH * 4);
    ALLOC(v, (size_t)KH * 4);
    ALLOC(qr, (size_t)C * 4);
    ALLOC(ctx, (size_t)C * 4);
    ALLOC(x1, (size_t)C * 4);
    ALLOC(h2, (size_t)C * 4);
    ALLOC(gate, (size_t)I * 4);
    ALLOC(up, (size_t)I * 4);
    ALLOC(logits, (size_t)c->vocab * 4);
    ALLOC(part_o, (size_t)c->n_head * m->nchunk_max * 64 * 4);
    ALLOC(part_ml, (size_t)c->n_head * m->nchunk_max * 2 * 4);
#undef ALLOC
    if (!(m->ids_dev = (int *)ncm_hip_malloc((size_t)(c->n_ctx + 1) * sizeof(int)))) goto fail;
    if (!(m->pos_dev = (int *)ncm_hip_malloc(sizeof(int)))) goto fail;
    if (!(m->rng_dev = (unsigned long long *)ncm_hip_malloc(sizeof(unsigned long long)))) goto fail;
    if (!(m->flags_dev = (int *)ncm_hip_malloc((size_t)(c->n_ctx + 1) * sizeof(int)))) goto fail;
    m->amax_blocks = (c->vocab + 4095) / 4096;
    /* decode LM head: two streaming workgroups per CU when a row fits one
     * float4 prefetch per lane (K <= 1024) */
    m->head_grid = (C <= 1024 && C % 4 == 0) ? 2 * ncm_cu_count() : 0;
    {
        const int na = m->amax_blocks > 4 * m->head_grid ? m->amax_blocks : 4 * m->head_grid;
        if (!(m->amax_v = (float *)ncm_hip_malloc((size_t)na * sizeof(float)))) goto fail;
        if (!(m->amax_i = (int *)ncm_hip_malloc((size_t)na * sizeof(int)))) goto fail;
    }
    if (build_rope(m)) goto fail;
    return m;
fail:
    ncm_qwen_free(m);
    return NULL;
}

static float *A(int64_t n) {
    float *p = arena_alloc((size_t)n);
    if (!p) ncm_fail(NCM_E_OOM, "qwen: arena");
    return p;
}

/* qwen_forward (qwen.c:121-190) with the causal mask generated in the
 * attention kernel (the reference's -1e9 entries contribute exactly 0), and
 * the post-RoPE keys/values of positions 0..T-1 stored in the KV cache.
 * ids HOST [T]; returns logits [T][V] or [V] (last_only) in the arena. */
float *ncm_qwen_forward(NcmQwen *m, const int *ids, int T, int last_only) {
    if (!m || !ids || T <= 0 || T > m->c.n_ctx) { ncm_fail(NCM_E_ARG, "ncm_qwen_forward: bad arguments"); return NULL; }
    if (ncm_ready()) return NULL;
    arena_reset();
    const NcmQwenConfig *c = &m->c;
    const int C = c->n_embd, H = c->n_head, K = c->n_kv, hd = C / H, I = c->n_inner, V = c->vocab;
    float *const *P = m->P;
    int *bids = (int *)A(T);
    float *h = A((int64_t)T * C);
    if (!h) return NULL;
    if (ncm_h2d_async(bids, ids, (size_t)T * sizeof(int))) return NULL;
    embedding_fwd_v(P[0], V, bids, h, T, C);
    for (int li = 0; li < c->n_layer; li++) {
        float *const *w = P + 1 + QW_PER_LAYER * li;
        float *h1 = A((int64_t)T * C), *ql = A((int64_t)T * C), *kl = A((int64_t)T * K * hd),
              *vl = A((int64_t)T * K * hd), *qq = A((int64_t)T * C), *kk = A((int64_t)T * K * hd),
              *vv = A((int64_t)T * K * hd), *mo = A((int64_t)T * C),
              *x1 = A((int64_t)T * C), *h2 = A((int64_t)T * C),
              *gu = A((int64_t)T * I), *out = A((int64_t)T * C);
        if (!out) return NULL;
        rmsnorm_fwd(h, w[0], h1, T, C);
        {   /* q | k | v in one launch */
            const float *const W3[3] = {w[1], w[3], w[5]}, *const b3[3] = {w[2], w[4], w[6]};
            float *const y3[3] = {ql, kl, vl};
            const int n3[3] = {C, K * hd, K * hd};
            ncm_linear_fwd3(h1, W3, b3, y3, n3, T, C);
        }
        /* heads to [H][T][hd] with RoPE, and k, v also into the KV cache for
         * the cached decode: [K][T][hd] at rows 0..T-1 of [K][n_ctx][hd] */
        float *kc = m->kcache + (size_t)li * K * c->n_ctx * hd, *vc = m->vcache + (size_t)li * K * c->n_ctx * hd;
        {
            int ld = c->n_ctx;
            void *a[] = {&ql, &kl, &vl, &qq, &kk, &vv, &kc, &vc, &m->cos_t, &m->sin_t, &T, (void *)&H, (void *)&K,
                         (void *)&hd, &ld};
            if (ncm_launch_named("qkv_rope_cache_k", (unsigned)T, 1, 1, 256, a)) return NULL;
        }
        ncm_sdpa_fwd_causal_merged(qq, kk, vv, mo, 1, H, K, T, T, hd);   /* heads merged: mo [T][C] */
        linear_fwd_ep(mo, w[7], NULL, h, x1, T, C, C, NCM_ACT_NONE);   /* x1 = h + mo W^T */
        rmsnorm_fwd(x1, w[8], h2, T, C);
        linear_fwd_gated(h2, w[9], NULL, w[10], NULL, gu, T, I, C, NCM_ACT_SILU);   /* silu(gate) * up */
        linear_fwd_ep(gu, w[11], NULL, x1, out, T, C, I, NCM_ACT_NONE);
        h = out;
    }
    const int n = ncm_qwen_param_count(c);
    float *lnf = A((int64_t)T * C);
    if (!lnf) return NULL;
    rmsnorm_fwd(h, P[n - 1], lnf, T, C);
    float *logits;
    if (last_only) {
        logits = A(V);
        if (logits) linear_fwd(lnf + (size_t)(T - 1) * C, P[0], NULL, logits, 1, V, C);
    } else {
        logits = A((int64_t)T * V);
        if (logits) linear_fwd(lnf, P[0], NULL, logits, T, V, C);
    }
    return logits;
}

/* Decode GEMV launch (dec_gemv_r*): rows of up to three matrices, optional
 * fused RMSNorm of x, mode 1 = SwiGLU pair, res added in mode 0. */
typedef struct {
    const float *x, *nw, *res;
    const float *W[3];
    const float *b[3];
    float *y[3];
    int N[3];
    int K, mode;
    const float *cos_t, *sin_t;
    const int *posp;
    float *kc, *vc;
    int ld;
} DecGemvArgs;

/* Mode 0/1 launch (mode 2 sets the RoPE fields in dec_qkv). */
static int dec_launch(DecGemvArgs *a) {
    int units, dots = a->mode == 0 ? 1 : 2;
    if (a->mode == 0) units = a->N[0] + a->N[1] + a->N[2];
    else if (a->mode == 1) units = a->N[0];
    else units = (a->N[0] + a->N[1] + a->N[2]) / 2;
    const char *k;
    int rw = 1;
    if (dots == 1) {
        if (a->K <= 1024) {
            if (units >= 16 * 1024) { k = "dec_gemv_d1_r4_p4_x1"; rw = 4; }
            else k = "dec_gemv_d1_r1_p4_x1";
        } else {
            k = a->K <= 5120 ? "dec_gemv_d1_r1_p20_x5" : "dec_gemv_d1_r1_p8_x8";
        }
    } else if (a->K <= 1024) {
        k = "dec_gemv_d2_r1_p4_x1";
    } else {
        k = "dec_gemv_d2_r1_p8_x8";
    }
    void *args[] = {a};
    return ncm_launch_named(k, (unsigned)((units + 4 * rw - 1) / (4 * rw)), 1, 1, 256, args);
}

static int dec_gemv(const float *x, const float *nw, const float *res, int nmat, const float *const *W,
                    const float *const *b, float *const *y, const int *N, int K, int mode) {
    DecGemvArgs a;
    memset(&a, 0, sizeof(a));
    a.x = x; a.nw = nw; a.res = res; a.K = K; a.mode = mode;
    for (int i = 0; i < nmat; i++) {
        a.W[i] = W[i]; a.b[i] = b[i]; a.y[i] = y[i]; a.N[i] = N[i];
    }
    return dec_launch(&a);
}

/* One cached decode step at position *pos_dev for the token ids_dev[*pos_dev]
 * (the cache holds positions 0..pos-1): logits [V] into m->logits.  Every
 * launch has the same arguments at every position. */
static int decode_core(NcmQwen *m) {
    const NcmQwenConfig *c = &m->c;
    const int C = c->n_embd, H = c->n_head, K = c->n_kv, hd = C / H, I = c->n_inner, V = c->vocab, KH = K * hd;
    float *const *P = m->P;
    {
        void *a[] = {(void *)&P[0], &m->ids_dev, &m->pos_dev, &m->x, (void *)&C, (void *)&V};
        if (ncm_launch_named("dec_embed_k", (unsigned)((C + 255) / 256), 1, 1, 256, a)) return -1;
    }
    for (int li = 0; li < c->n_layer; li++) {
        float *const *w = P + 1 + QW_PER_LAYER * li;
        float *kc = m->kcache + (size_t)li * K * c->n_ctx * hd, *vc = m->vcache + (size_t)li * K * c->n_ctx * hd;
        {   /* rmsnorm + q | k | v + RoPE + cache append */
            DecGemvArgs a;
            memset(&a, 0, sizeof(a));
            a.x = m->x; a.nw = w[0]; a.K = C; a.mode = 2;
            a.W[0] = w[1]; a.W[1] = w[3]; a.W[2] = w[5];
            a.b[0] = w[2]; a.b[1] = w[4]; a.b[2] = w[6];
            a.y[0] = m->qr;
            a.N[0] = C; a.N[1] = KH; a.N[2] = KH;
            a.cos_t = m->cos_t; a.sin_t = m->sin_t; a.posp = m->pos_dev;
            a.kc = kc; a.vc = vc; a.ld = c->n_ctx;
            if (dec_launch(&a)) return -1;
        }
        {
            int ld = c->n_ctx, stride = m->nchunk_max;
            float scale = 1.0f / sqrtf((float)hd);
            void *a[] = {&m->qr, &kc, &vc, &m->part_o, &m->part_ml, (void *)&H, (void *)&K, &m->pos_dev, &ld, &scale};
            if (ncm_launch_named("sdpa_decode_partial", (unsigned)m->nchunk_max, (unsigned)K, 1, 256, a)) return -1;
            void *a2[] = {&m->part_o, &m->part_ml, &m->ctx, &stride, &m->pos_dev};
            if (ncm_launch_named("sdpa_decode_combine", (unsigned)H, 1, 1, 64, a2)) return -1;
        }
        if (C <= 1024) {   /* x1 = x + o_proj(ctx) (ctx [H][hd] is the merged row): a workgroup per
                            * two rows, K split over its threads */
            DecGemvArgs a;
            memset(&a, 0, sizeof(a));
            a.x = m->ctx; a.res = m->x; a.K = C; a.mode = 0;
            a.W[0] = w[7]; a.y[0] = m->x1; a.N[0] = C;
            void *args[] = {&a};
            if (ncm_launch_named("dec_wg_plain_r2_x1", (unsigned)((C + 1) / 2), 1, 1, 256, args)) return -1;
        } else {
            const float *W[1] = {w[7]}, *b[1] = {NULL};
            float *y[1] = {m->x1};
            int N[1] = {C};
            if (dec_gemv(m->ctx, NULL, m->x, 1, W, b, y, N, C, 0)) return -1;
        }
        {   /* gu = silu(gate(rmsnorm(x1))) * up(rmsnorm(x1)) */
            const float *W[2] = {w[9], w[10]}, *b[2] = {NULL, NULL};
            float *y[2] = {m->up, NULL};
            int N[2] = {I, I};
            if (dec_gemv(m->x1, w[8], NULL, 2, W, b, y, N, C, 1)) return -1;
        }
        if (I <= 5120) {   /* x = x1 + down(gu): a workgroup per two rows, K split over its threads */
            DecGemvArgs a;
            memset(&a, 0, sizeof(a));
            a.x = m->up; a.res = m->x1; a.K = I; a.mode = 0;
            a.W[0] = w[11]; a.y[0] = m->x; a.N[0] = C;
            void *args[] = {&a};
            if (ncm_launch_named("dec_wg_plain_r2_x5", (unsigned)((C + 1) / 2), 1, 1, 256, args)) return -1;
        } else {
            const float *W[1] = {w[11]}, *b[1] = {NULL};
            float *y[1] = {m->x};
            int N[1] = {C};
            if (dec_gemv(m->up, NULL, m->x1, 1, W, b, y, N, I, 0)) return -1;
        }
    }
    const int n = ncm_qwen_param_count(c);
    if (m->head_grid) {
        void *a[] = {&m->x, (void *)&P[n - 1], (void *)&P[0], &m->logits, (void *)&V, (void *)&C, &m->amax_v,
                     &m->amax_i};
        return ncm_launch_named("dec_head_stream", (unsigned)m->head_grid, 1, 1, 256, a);
    }
    const float *W[1] = {P[0]}, *b[1] = {NULL};
    float *y[1] = {m->logits};
    int N[1] = {V};
    return dec_gemv(m->x, P[n - 1], NULL, 1, W, b, y, N, C, 0);
}

/* greedy id of logits -> ids[*pos + 1], *pos += 1 (two launches) */
static int greedy_next(NcmQwen *m, const float *logits) {
    int V = m->c.vocab;
    void *a[] = {(void *)&logits, &V, &m->amax_v, &m->amax_i};
    if (ncm_launch_named("dec_argmax_part_k", (unsigned)m->amax_blocks, 1, 1, 256, a)) return -1;
    void *a2[] = {(void *)&logits, &m->amax_v, &m->amax_i, &m->amax_blocks, &m->ids_dev, &m->pos_dev};
    return ncm_launch_named("dec_argmax_final_k", 1, 1, 1, 64, a2);
}

/* After decode_core: with the streamed head its workgroups' maxima are already in
 * amax_v / amax_i, so only the merge runs. */
static int decode_argmax(NcmQwen *m) {
    if (!m->head_grid) return greedy_next(m, m->logits);
    int nblk = m->head_grid;
    void *a2[] = {&m->logits, &m->amax_v, &m->amax_i, &nblk, &m->ids_dev, &m->pos_dev};
    return ncm_launch_named("dec_argmax_final_k", 1, 1, 1, 64, a2);
}

static int decode_ok(const NcmQwen *m, const char *fn) {
    const int hd = m->c.n_embd / m->c.n_head;
    if (hd != 64 || m->c.n_head / m->c.n_kv > 16 || m->c.n_embd % 4 || m->c.n_inner % 4 || m->c.n_embd > 8192 ||
        m->c.n_inner > 8192)
        return ncm_fail(NCM_E_ARG, "%s: decode needs hd = 64, <= 16 query heads per kv head, C and I "
                                   "multiples of 4 and at most 8192", fn);
    return 0;
}

float *ncm_qwen_decode(NcmQwen *m, int id, int pos) {
    if (!m || pos < 1 || pos >= m->c.n_ctx) { ncm_fail(NCM_E_ARG, "ncm_qwen_decode: bad position"); return NULL; }
    if (ncm_ready() || decode_ok(m, "ncm_qwen_decode")) return NULL;
    mem_h2d(m->ids_dev + pos, &id, sizeof(int));
    mem_h2d(m->pos_dev, &pos, sizeof(int));
    return decode_core(m) ? NULL : m->logits;
}

/* Captures decode_core + decode_argmax once; later steps replay it. */
static int step_graph(NcmQwen *m) {
    if (m->graph_state != 0 || getenv("NCM_NO_GRAPH")) return m->graph_state == 1;
    hipStream_t s = ncm_stream();
    hipGraph_t g = NULL;
    m->graph_state = -1;
    if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) return 0;
    int rc = decode_core(m) || decode_argmax(m);
    hipError_t e = hipStreamEndCapture(s, &g);
    if (rc || e != hipSuccess || !g) {
        if (g) hipGraphDestroy(g);
        ncm_fail(NCM_E_HIP, "qwen: decode graph capture failed");
        return 0;
    }
    e = hipGraphInstantiate(&m->step_graph, g, NULL, NULL, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) return ncm_fail(NCM_E_HIP, "qwen: graph instantiate: %s", hipGetErrorString(e)), 0;
    m->graph_state = 1;
    return 1;
}

static int decode_token(NcmQwen *m) {
    if (step_graph(m)) {
        hipError_t e = hipGraphLaunch(m->step_graph, ncm_stream());
        if (e != hipSuccess) return ncm_fail(NCM_E_HIP, "qwen: graph launch: %s", hipGetErrorString(e));
        return 0;
    }
    return decode_core(m) || decode_argmax(m);
}

/* Greedy generation (qwen_generate with temp 0, qwen.c:204-228): prefill of
 * the prompt, then n_new steps of argmax + cached decode.  The ids and the
 * position stay on the device (each step's argmax writes the next id where
 * the next step reads it and advances the position), so one captured graph
 * per model replays every step (NCM_NO_GRAPH=1 launches the same kernels
 * one by one instead).  With eos >= 0 each step is synchronised to stop at
 * eos as the reference does; with eos < 0 all steps run without a host
 * round trip.  Returns the number of ids written to out. */
int ncm_qwen_generate(NcmQwen *m, const int *prompt, int np, int n_new, int eos, int *out) {
    if (!m || !prompt || np <= 0 || n_new < 0 || !out) { ncm_fail(NCM_E_ARG, "ncm_qwen_generate: bad arguments"); return -1; }
    if (np + n_new > m->c.n_ctx) { ncm_fail(NCM_E_ARG, "ncm_qwen_generate: context overflow"); return -1; }
    if (ncm_ready() || decode_ok(m, "ncm_qwen_generate")) return -1;
    if (n_new == 0) return 0;
    float *lg = ncm_qwen_forward(m, prompt, np, 1);
    if (!lg) return -1;
    /* the prefill's greedy id goes to ids[np]; *pos becomes np */
    int p0 = np - 1;
    mem_h2d(m->pos_dev, &p0, sizeof(int));
    if (greedy_next(m, lg)) return -1;
    int made = 1;
    if (eos >= 0) {
        mem_d2h(out, m->ids_dev + np, sizeof(int));
        if (out[0] == eos) return 1;
    }
    for (int s = 1; s < n_new; s++) {
        if (decode_token(m)) return -1;
        made++;
        if (eos >= 0) {
            mem_d2h(out + s, m->ids_dev + np + s, sizeof(int));
            if (out[s] == eos) return made;
        }
    }
    mem_d2h(out, m->ids_dev + np, (size_t)made * sizeof(int));
    return made;
}

/* Decode step + device sampling, captured once per sampling setting. */
static int samp_graph(NcmQwen *m, float temp, int top_k, float top_p) {
    if (m->samp_state == 1 && (m->samp_temp != temp || m->samp_top_k != top_k || m->samp_top_p != top_p)) {
        hipGraphExecDestroy(m->samp_graph);
        m->samp_state = 0;
    }
    if (m->samp_state != 0 || getenv("NCM_NO_GRAPH")) return m->samp_state == 1;
    hipStream_t s = ncm_stream();
    hipGraph_t g = NULL;
    if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) return 0;
    int rc = decode_core(m) || ncm_sample_launch(m->logits, m->c.vocab, temp, top_k, top_p, m->rng_dev, NULL,
                                                 m->ids_dev, m->pos_dev, m->flags_dev, m->samp_ws);
    hipError_t e = hipStreamEndCapture(s, &g);
    if (rc || e != hipSuccess || !g) {
        if (g) hipGraphDestroy(g);
        m->samp_state = -1;
        ncm_fail(NCM_E_HIP, "qwen: sampling graph capture failed");
        return 0;
    }
    e = hipGraphInstantiate(&m->samp_graph, g, NULL, NULL, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) {
        m->samp_state = -1;
        return ncm_fail(NCM_E_HIP, "qwen: graph instantiate: %s", hipGetErrorString(e)), 0;
    }
    m->samp_state = 1;
    m->samp_temp = temp;
    m->samp_top_k = top_k;
    m->samp_top_p = top_p;
    return 1;
}

/* qwen_generate (qwen.c:204-228) with sampling: the same loop as
 * ncm_qwen_generate, the greedy id replaced by sample_topkp's draw on the
 * device (csrc/sample.hip) from the xorshift64* state *rng, which is
 * advanced once per generated token, as the reference's host loop does.
 * temp <= 0 is the greedy path (rng untouched).  n_flagged (may be NULL)
 * receives the number of draws not certified equal to the reference's
 * arithmetic on these logits (flag 1 or 2 of sample_topkp_dev). */
int ncm_qwen_generate_sample(NcmQwen *m, const int *prompt, int np, int n_new, int eos, float temp, int top_k,
                             float top_p, unsigned long long *rng, int *out, int *n_flagged) {
    if (n_flagged) *n_flagged = 0;
    if (!(temp > 0.0f)) return ncm_qwen_generate(m, prompt, np, n_new, eos, out);
    if (!m || !prompt || np <= 0 || n_new < 0 || !out || !rng) {
        ncm_fail(NCM_E_ARG, "ncm_qwen_generate_sample: bad arguments");
        return -1;
    }
    if (np + n_new > m->c.n_ctx) { ncm_fail(NCM_E_ARG, "ncm_qwen_generate_sample: context overflow"); return -1; }
    if (top_p < 0.0f) { ncm_fail(NCM_E_ARG, "ncm_qwen_generate_sample: top_p must be >= 0"); return -1; }
    if (ncm_ready() || decode_ok(m, "ncm_qwen_generate_sample")) return -1;
    if (n_new == 0) return 0;
    if (!m->samp_ws) {
        size_t b = ncm_sample_ws_bytes(m->c.vocab);
        if (!b) { ncm_fail(NCM_E_ARG, "ncm_qwen_generate_sample: vocab %d exceeds the sampler's 262144", m->c.vocab); return -1; }
        if (!(m->samp_ws = ncm_hip_malloc(b))) return -1;
    }
    mem_h2d(m->rng_dev, rng, sizeof *rng);
    float *lg = ncm_qwen_forward(m, prompt, np, 1);
    if (!lg) return -1;
    int p0 = np - 1;
    mem_h2d(m->pos_dev, &p0, sizeof(int));
    if (ncm_sample_launch(lg, m->c.vocab, temp, top_k, top_p, m->rng_dev, NULL, m->ids_dev, m->pos_dev,
                          m->flags_dev, m->samp_ws))
        return -1;
    int made = 1, stop = 0;
    if (eos >= 0) {
        mem_d2h(out, m->ids_dev + np, sizeof(int));
        stop = out[0] == eos;
    }
    for (int s = 1; s < n_new && !stop; s++) {
        if (samp_graph(m, temp, top_k, top_p)) {
            hipError_t e = hipGraphLaunch(m->samp_graph, ncm_stream());
            if (e != hipSuccess) { ncm_fail(NCM_E_HIP, "qwen: graph launch: %s", hipGetErrorString(e)); return -1; }
        } else if (m->samp_state == -1 || getenv("NCM_NO_GRAPH")) {
            if (decode_core(m) || ncm_sample_launch(m->logits, m->c.vocab, temp, top_k, top_p, m->rng_dev, NULL,
                                                    m->ids_dev, m->pos_dev, m->flags_dev, m->samp_ws))
                return -1;
        } else {
            return -1;
        }
        made++;
        if (eos >= 0) {
            mem_d2h(out + s, m->ids_dev + np + s, sizeof(int));
            stop = out[s] == eos;
        }
    }
    mem_d2h(out, m->ids_dev + np, (size_t)made * sizeof(int));
    mem_d2h(rng, m->rng_dev, sizeof *rng);
    if (n_flagged) {
        int *fl = (int *)malloc((size_t)made * sizeof(int));
        if (!fl) { ncm_fail(NCM_E_OOM, "ncm_qwen_generate_sample: flags"); return -1; }
        mem_d2h(fl, m->flags_dev + np, (size_t)made * sizeof(int));
        for (int i = 0; i < made; i++) *n_flagged += fl[i] != 0;
        free(fl);
    }
    return made;
}
