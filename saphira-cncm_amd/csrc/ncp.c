/* ncp.c -- the NCP transformer forward of ncp.c (reference) on the device:
 * token embedding, n_layer blocks of ncp_block (ncp.c:184-338), ln_f and an
 * output head, for a single level of S tokens per board with RoPE positions
 * 0..S-1 and no attention mask.
 *
 * Block: norm -> c_attn (fused q | k | v, GQA) -> split with the kv heads
 * replicated to all query heads -> RoPE -> SDPA -> merge -> c_proj ->
 * x += . -> norm -> SwiGLU (w_gate, w_up, silu, gate*up, c_proj) -> x += .
 * The norm is LayerNorm (eps 1e-6) as ncp.c:195-199 calls it.
 *
 * Parameters: one flat array of device pointers (biases may be NULL):
 * 0 wte [V][C]; per layer l at 1 + 14 l: ln_1.weight, ln_1.bias,
 * attn.c_attn.weight [C + 2 Kv hd][C], attn.c_attn.bias, attn.c_proj.weight
 * [C][C], attn.c_proj.bias, ln_2.weight, ln_2.bias, mlp.w_gate.weight [I][C],
 * mlp.w_gate.bias, mlp.w_up.weight [I][C], mlp.w_up.bias, mlp.c_proj.weight
 * [C][I], mlp.c_proj.bias; then ln_f.weight, ln_f.bias, head.weight [V][C],
 * head.bias. */
#include "internal.h"

#include <math.h>
#include <stdlib.h>

#define NCP_PER_LAYER 14

int ncm_ncp_param_count(const NcmNcpConfig *c) { return c ? 5 + NCP_PER_LAYER * c->n_layer : 0; }

int64_t ncm_ncp_param_shape(const NcmNcpConfig *c, int i, int64_t *rows, int64_t *cols) {
    const int n = ncm_ncp_param_count(c);
    if (!c || i < 0 || i >= n) return -1;
    const int64_t C = c->n_embd, hd = c->n_embd / c->n_head, QKV = C + 2 * (int64_t)c->n_kv * hd, I = c->n_inner;
    int64_t r = C, k = 1;
    if (i == 0 || i == n - 2) { r = c->vocab; k = C; }
    else if (i == n - 1) { r = c->vocab; }
    else if (i < n - 4) {
        switch ((i - 1) % NCP_PER_LAYER) {
        case 2: r = QKV; k = C; break;
        case 3: r = QKV; break;
        case 4: k = C; break;
        case 8: case 10: r = I; k = C; break;
        case 9: case 11: r = I; break;
        case 12: k = I; break;
        default: break;
        }
    }
    if (rows) *rows = r;
    if (cols) *cols = k;
    return r * k;
}

/* build_rope (ncp.c:80-92): inv = 1 / base^(d / half), angle = pos * inv in
 * fp64, cos/sin rounded to float, duplicated over the halves. */
int ncm_ncp_rope_tables(int S, int hd, int base, float *cos_host, float *sin_host) {
    if (S <= 0 || hd <= 0 || (hd & 1) || !cos_host || !sin_host) return ncm_fail(NCM_E_ARG, "ncp: rope tables");
    const int half = hd / 2;
    for (int t = 0; t < S; t++)
        for (int d = 0; d < half; d++) {
            double inv = 1.0 / pow((double)base, (double)d / half);
            double f = t * inv;
            float co = (float)cos(f), si = (float)sin(f);
            cos_host[t * hd + d] = cos_host[t * hd + half + d] = co;
            sin_host[t * hd + d] = sin_host[t * hd + half + d] = si;
        }
    return 0;
}

static int rope_upload(const int *pos, int n, int hd, int base, float **cd, float **sd);

/* q [B][H][S][hd], k and v [B][nkv][S][hd] from qkv rows (ncp.c:206-244: split,
 * optional qk-norm, optional RoPE); one wave per row when hd = 64 and a row
 * holds at most 16 heads, else one wave per head. */
static int ncp_qkv_launch(const float *qkv, float *q, float *k, float *v, const float *qn, const float *kn,
                          const float *cs, const float *sn, int B, int S, int H, int nkv, int hd) {
    if (hd == 64 && H + 2 * nkv <= 16 && (int64_t)B * S <= INT32_MAX - 3) {
        void *a[] = {&qkv, &q, &k, &v, &qn, &kn, &cs, &sn, &B, &S, &H, &nkv};
        return ncm_launch_named("ncp_qkv_rows_k", (unsigned)(((int64_t)B * S + 3) / 4), 1, 1, 256, a);
    }
    void *a[] = {&qkv, &q, &k, &v, &qn, &kn, &cs, &sn, &B, &S, &H, &nkv, &hd};
    return ncm_launch_named("ncp_qkv_k", (unsigned)(((int64_t)B * (H + 2 * nkv) * S + 3) / 4), 1, 1, 256, a);
}

static float *A(int64_t n) {
    float *p = arena_alloc((size_t)n);
    if (!p) ncm_fail(NCM_E_OOM, "ncp: arena");
    return p;
}

static void norm(const NcmNcpConfig *c, const float *x, const float *w, const float *b, float *y, int64_t rows) {
    layernorm_fwd(x, w, b, y, rows, c->n_embd);
}

/* ids HOST [B][S] -> logits [B*S][V] in the arena (arena_reset first, as
 * the reference's forward owns its scratch arena). */
float *ncm_ncp_forward(const NcmNcpConfig *c, float *const *P, const int *ids, int B, int S) {
    if (!c || !P || !ids || B <= 0 || S <= 0 || c->n_layer < 0 || c->n_embd <= 0 || c->n_head <= 0 ||
        c->n_embd % c->n_head || c->n_kv <= 0 || c->n_head % c->n_kv || c->n_inner <= 0 || c->vocab <= 0 ||
        ((c->n_embd / c->n_head) & 1)) {
        ncm_fail(NCM_E_ARG, "ncm_ncp_forward: bad arguments");
        return NULL;
    }
    if (ncm_ready()) return NULL;
    arena_reset();
    const int C = c->n_embd, H = c->n_head, Kv = c->n_kv, hd = C / H, I = c->n_inner, V = c->vocab;
    const int QKV = C + 2 * Kv * hd, rep = H / Kv;
    const int64_t R = (int64_t)B * S;
    float *x = A(R * C);
    int *bids = (int *)A(R);
    if (!bids) return NULL;
    /* RoPE tables for positions 0..S-1 (ncp.c:80-92): built once per (S, hd,
     * base) and kept on the device */
    static float *tab_cos = NULL, *tab_sin = NULL;
    static int tab_S = 0, tab_hd = 0, tab_base = 0;
    if (!tab_cos || tab_S != S || tab_hd != hd || tab_base != c->rope_base) {
        ncm_hip_free(tab_cos);
        ncm_hip_free(tab_sin);
        tab_cos = tab_sin = NULL;
        int *pos = (int *)malloc((size_t)S * sizeof(int));
        if (!pos) {
            ncm_fail(NCM_E_OOM, "ncp: positions");
            return NULL;
        }
        for (int t = 0; t < S; t++) pos[t] = t;
        int rc = rope_upload(pos, S, hd, c->rope_base, &tab_cos, &tab_sin);
        free(pos);
        if (rc) return NULL;
        tab_S = S;
        tab_hd = hd;
        tab_base = c->rope_base;
    }
    const float *cosd = tab_cos, *sind = tab_sin;
    if (ncm_h2d_async(bids, ids, (size_t)R * sizeof(int))) return NULL;
    embedding_fwd_v(P[0], V, bids, x, R, C);
    /* K and V at their kv-head count when the fused split applies (hd <= 64),
     * else replicated to every query head as ncp.c:213-236 does */
    const int fused = hd <= 64, hk = fused ? Kv : H;
    float *ln = A(R * C), *qkv = A(R * QKV), *qq = A(R * C), *kk = A((int64_t)B * hk * S * hd),
          *vv = A((int64_t)B * hk * S * hd), *mo = A(R * C), *g = A(R * I);
    if (!g) return NULL;
    for (int li = 0; li < c->n_layer; li++) {
        float *const *w = P + 1 + NCP_PER_LAYER * li;
        norm(c, x, w[0], w[1], ln, R);
        linear_fwd(ln, w[2], w[3], qkv, R, QKV, C);
        if (fused) {   /* split + RoPE, kv heads kept */
            if (ncp_qkv_launch(qkv, qq, kk, vv, NULL, NULL, cosd, sind, B, S, H, Kv, hd)) return NULL;
        } else {
            qkv_split_rope_fwd(qkv, qq, kk, vv, cosd, sind, B, S, C, H, hd, Kv, rep);   /* split, then RoPE */
        }
        sdpa_fwd_gqa_merged(qq, kk, vv, NULL, mo, B, H, hk, S, S, hd);              /* heads merged on output */
        linear_fwd_ep(mo, w[4], w[5], x, x, R, C, C, NCM_ACT_NONE);      /* x += c_proj(.) */
        norm(c, x, w[6], w[7], ln, R);
        linear_fwd_gated(ln, w[8], w[9], w[10], w[11], g, R, I, C, NCM_ACT_SILU);   /* silu(w_gate(.)) * w_up(.) */
        linear_fwd_ep(g, w[12], w[13], x, x, R, C, I, NCM_ACT_NONE);     /* x += c_proj(.) */
    }
    const int n = ncm_ncp_param_count(c);
    norm(c, x, P[n - 4], P[n - 3], ln, R);
    float *logits = A(R * V);
    if (!logits) return NULL;
    linear_fwd(ln, P[n - 2], P[n - 1], logits, R, V, C);
    return logits;
}

/* ==================================================================== */
/* The reference's NCP model API (ncm.h:249-268): ncp_load / ncp_forward */
/* on a WeightStore of device tensors, every level layout and block      */
/* variant of ncp.c, all steps on the device.                            */
/* ==================================================================== */

typedef struct {
    const float *ln1w, *ln1b, *attw, *attb, *qn, *kn, *projw, *projb, *ln2w, *ln2b;
    const float *gw, *gb, *uw, *ub; /* gated MLP (w_gate, w_up) */
    const float *fcw, *fcb;         /* plain MLP (c_fc) */
    const float *mpw, *mpb;         /* mlp.c_proj */
    int inner;
} NcpLayer;

typedef struct {
    const float *w, *b;          /* linear head, or the tied head's proj */
    const float *E;              /* tied: codebook [V][Dd] */
    double *esq, *ds;            /* tied: |E_v|^2 and the mean of them (device) */
    float invT;                  /* tied: expf(log_inv_T) */
    const float *tb;             /* tied: optional logits bias */
    int Dd;
} NcpHead;

struct NCPState {
    NCMConfig cfg;
    WeightStore *ws;
    VQVAEState *vqvae;
    int P, T, S, lvl_first, n_tgt, C, H, nkv, hd, D, maxV;
    int tl[NCM_MAX_LEVELS], toff[NCM_MAX_LEVELS];
    const float *wte, *wteb, *wpe, *lnfw, *lnfb;
    float *rope_cos, *rope_sin; /* [S][hd], level positions */
    float *gcos[NCM_MAX_LEVELS], *gsin[NCM_MAX_LEVELS]; /* [P + l_k][hd] */
    float *lvl_pos;             /* [T][C] */
    float *mask;                /* [S][S] without pads */
    int *lvl;                   /* [T] level of each target row */
    NcpLayer *layer;
    NcpHead head[NCM_MAX_LEVELS];
};

static unsigned blocks256(int64_t n) { return (unsigned)((n + 255) / 256); }

static const float *wget(WeightStore *ws, const char *name, int required, int64_t n, int *err) {
    Tensor *t = weights_get(ws, name);
    if (!t) {
        if (required && !*err) *err = ncm_fail(NCM_E_ARG, "ncp_load: missing weight %s", name);
        return NULL;
    }
    if (n >= 0 && t->n != n && !*err)
        *err = ncm_fail(NCM_E_ARG, "ncp_load: %s has %lld elements, expected %lld", name, (long long)t->n,
                        (long long)n);
    return t->data;
}

/* build_rope (ncp.c:80-92) for the positions pos[0..n) into new device tables */
static int rope_upload(const int *pos, int n, int hd, int base, float **cd, float **sd) {
    float *hc = (float *)malloc((size_t)n * hd * sizeof(float)), *hs = (float *)malloc((size_t)n * hd * sizeof(float));
    int rc = 0;
    if (!hc || !hs) {
        rc = ncm_fail(NCM_E_OOM, "ncp_load: rope tables");
    } else {
        const int half = hd / 2;
        for (int t = 0; t < n; t++)
            for (int d = 0; d < half; d++) {
                double inv = 1.0 / pow((double)base, (double)d / half);
                double f = pos[t] * inv;
                float co = (float)cos(f), si = (float)sin(f);
                hc[t * hd + d] = hc[t * hd + half + d] = co;
                hs[t * hd + d] = hs[t * hd + half + d] = si;
            }
        *cd = (float *)ncm_hip_malloc((size_t)n * hd * sizeof(float));
        *sd = (float *)ncm_hip_malloc((size_t)n * hd * sizeof(float));
        if (!*cd || !*sd) rc = NCM_E_OOM;
        else {
            mem_h2d(*cd, hc, (size_t)n * hd * sizeof(float));
            mem_h2d(*sd, hs, (size_t)n * hd * sizeof(float));
        }
    }
    free(hc);
    free(hs);
    return rc;
}

void ncp_free(NCPState *m) {
    if (!m) return;
    ncm_hip_free(m->rope_cos);
    ncm_hip_free(m->rope_sin);
    for (int k = 0; k < NCM_MAX_LEVELS; k++) {
        ncm_hip_free(m->gcos[k]);
        ncm_hip_free(m->gsin[k]);
        ncm_hip_free(m->head[k].esq);
        ncm_hip_free(m->head[k].ds);
    }
    ncm_hip_free(m->lvl_pos);
    ncm_hip_free(m->mask);
    ncm_hip_free(m->lvl);
    free(m->layer);
    free(m);
}

static int ncp_load_heads(NCPState *m, int *err) {
    const NCMConfig *c = &m->cfg;
    WeightStore *ws = m->ws;
    char kw[160];
    for (int k = 0; k < m->n_tgt; k++) {
        NcpHead *h = &m->head[k];
        const int V = c->vocab_size[k];
        if (c->shared_output_head) {
            h->w = wget(ws, "gen.lm_heads.head.weight", 1, -1, err);
            Tensor *t = weights_get(ws, "gen.lm_heads.head.weight");
            if (t && (t->shape[0] < V || t->n != t->shape[0] * m->C) && !*err)
                *err = ncm_fail(NCM_E_ARG, "ncp_load: gen.lm_heads.head.weight is too small for vocabulary %d", V);
            if (c->shared_head_per_level_bias) {
                snprintf(kw, sizeof kw, "gen.lm_heads.biases.%d", k);
                h->b = wget(ws, kw, 1, V, err);
            } else if (c->untied_head_bias) {
                h->b = wget(ws, "gen.lm_heads.head.bias", 1, -1, err);
            }
        } else if (c->tie_heads_to_codebook) {
            snprintf(kw, sizeof kw, "gen.lm_heads.%d.proj.weight", k);
            Tensor *tp = weights_get(ws, kw);
            h->w = wget(ws, kw, 1, -1, err);
            if (!tp || *err) return *err;
            h->Dd = (int)tp->shape[0];
            if (tp->n != (int64_t)h->Dd * m->C)
                return *err = ncm_fail(NCM_E_ARG, "ncp_load: %s is not [Dd][%d]", kw, m->C);
            snprintf(kw, sizeof kw, "gen.lm_heads.%d.proj.bias", k);
            h->b = wget(ws, kw, 0, h->Dd, err);
            snprintf(kw, sizeof kw, "tok.vq.embeddings.%d.weight", k + m->lvl_first);
            h->E = wget(ws, kw, 1, (int64_t)V * h->Dd, err);
            snprintf(kw, sizeof kw, "gen.lm_heads.%d.log_inv_T", k);
            const float *lit = wget(ws, kw, 1, -1, err);
            snprintf(kw, sizeof kw, "gen.lm_heads.%d.bias", k);
            h->tb = wget(ws, kw, 0, V, err);
            if (*err) return *err;
            /* invT = expf(log_inv_T) as the reference evaluates it on the host
             * (ncp.c:459-460); E_sq and the mean of them on the device, in its
             * serial fp64 order (ncp.c:448-453) */
            float l = 0.f;
            mem_d2h(&l, lit, sizeof(float));
            h->invT = expf(l);
            h->esq = (double *)ncm_hip_malloc((size_t)V * sizeof(double));
            h->ds = (double *)ncm_hip_malloc(sizeof(double));
            if (!h->esq || !h->ds) return *err = NCM_E_OOM;
            int Dd = h->Dd, Vv = V;
            void *a1[] = {&h->E, &h->esq, &Vv, &Dd};
            void *a2[] = {&h->esq, &h->ds, &Vv};
            if ((*err = ncm_launch_named("ncp_esq_k", blocks256(V), 1, 1, 256, a1)) ||
                (*err = ncm_launch_named("ncp_dscale_k", 1, 1, 1, 64, a2)))
                return *err;
        } else {
            snprintf(kw, sizeof kw, "gen.lm_heads.%d.weight", k);
            h->w = wget(ws, kw, 1, (int64_t)V * m->C, err);
            snprintf(kw, sizeof kw, "gen.lm_heads.%d.bias", k);
            h->b = wget(ws, kw, 0, V, err);
        }
    }
    return *err;
}

NCPState *ncp_load(const NCMConfig *c, WeightStore *ws, VQVAEState *vqvae) {
    if (!c || !ws) {
        ncm_fail(NCM_E_ARG, "ncp_load: null config or weights");
        return NULL;
    }
    if (ncm_ready()) return NULL;
    const int C = c->n_embd, H = c->n_head, nkv = c->n_kv_heads;
    if (C <= 0 || H <= 0 || C % H || nkv <= 0 || H % nkv || c->n_layer < 0 || c->n_qlevels <= 0 ||
        c->n_qlevels > NCM_MAX_LEVELS || c->vq_embed_dim <= 0 || c->prefix_len < 0) {
        ncm_fail(NCM_E_ARG, "ncp_load: bad configuration (n_embd %d, n_head %d, n_kv_heads %d, levels %d)", C, H,
                 nkv, c->n_qlevels);
        return NULL;
    }
    NCPState *m = (NCPState *)calloc(1, sizeof(NCPState));
    if (!m) {
        ncm_fail(NCM_E_OOM, "ncp_load");
        return NULL;
    }
    m->cfg = *c;
    m->ws = ws;
    m->vqvae = vqvae;
    m->C = C;
    m->H = H;
    m->nkv = nkv;
    m->hd = C / H;
    m->D = c->vq_embed_dim;
    m->P = c->prefix_len;
    m->lvl_first = c->query_level0 ? 0 : 1;
    m->n_tgt = c->n_qlevels - m->lvl_first;
    int err = 0;
    if (m->n_tgt <= 0 || m->n_tgt > NCM_MAX_VOCAB_LIST)
        err = ncm_fail(NCM_E_ARG, "ncp_load: no target level");
    if (!err && (m->hd & 1) && c->use_rope) err = ncm_fail(NCM_E_ARG, "ncp_load: odd head size %d with RoPE", m->hd);
    for (int k = 0; !err && k < m->n_tgt; k++) {
        m->tl[k] = c->levels[k + m->lvl_first];
        m->toff[k] = m->T;
        if (m->tl[k] <= 0 || c->vocab_size[k] <= 0)
            err = ncm_fail(NCM_E_ARG, "ncp_load: target level %d has length %d, vocabulary %d", k, m->tl[k],
                           c->vocab_size[k]);
        m->T += m->tl[k];
        if (c->vocab_size[k] > m->maxV) m->maxV = c->vocab_size[k];
    }
    m->S = m->P + m->T;
    if (err) {
        ncp_free(m);
        return NULL;
    }
    const int S = m->S, T = m->T, P = m->P, hd = m->hd;
    /* RoPE tables of the level positions (ncp.c:102-142) */
    int *pos = (int *)malloc((size_t)S * sizeof(int));
    int *lvl = (int *)malloc((size_t)(T > 0 ? T : 1) * sizeof(int)), *tpos = (int *)malloc((size_t)(T > 0 ? T : 1) * sizeof(int));
    if (!pos || !lvl || !tpos) err = ncm_fail(NCM_E_OOM, "ncp_load: positions");
    if (!err) {
        for (int i = 0; i < P; i++) pos[i] = i;
        for (int k = 0, o = P; k < m->n_tgt; k++)
            for (int t = 0; t < m->tl[k]; t++, o++) {
                pos[o] = t;
                lvl[o - P] = k + m->lvl_first;
                tpos[o - P] = t;
            }
        err = rope_upload(pos, S, hd, c->rope_base, &m->rope_cos, &m->rope_sin);
        for (int k = 0; !err && k < m->n_tgt; k++) {
            int *pk = (int *)malloc((size_t)(P + m->tl[k]) * sizeof(int));
            if (!pk) {
                err = ncm_fail(NCM_E_OOM, "ncp_load: positions");
                break;
            }
            for (int i = 0; i < P; i++) pk[i] = i;
            for (int t = 0; t < m->tl[k]; t++) pk[P + t] = t;
            err = rope_upload(pk, P + m->tl[k], hd, c->rope_base, &m->gcos[k], &m->gsin[k]);
            free(pk);
        }
    }
    /* weights (ncp.c:189-345, 349-357, 520-560) */
    const int64_t QKV = (int64_t)C + 2 * (int64_t)nkv * hd;
    char kk[192], pre[128];
    if (!err) {
        m->wte = wget(ws, "gen.transformer.wte.weight", 1, (int64_t)C * m->D, &err);
        m->wteb = wget(ws, "gen.transformer.wte.bias", 0, C, &err);
        m->lnfw = wget(ws, "gen.transformer.ln_f.weight", 1, C, &err);
        m->lnfb = wget(ws, "gen.transformer.ln_f.bias", 0, C, &err);
        if (!c->use_rope) m->wpe = wget(ws, "gen.transformer.wpe.weight", 1, -1, &err);
        m->layer = (NcpLayer *)calloc((size_t)(c->n_layer > 0 ? c->n_layer : 1), sizeof(NcpLayer));
        if (!m->layer && !err) err = ncm_fail(NCM_E_OOM, "ncp_load: layers");
    }
    const int gated = c->use_swiglu || c->use_geglu;
    for (int li = 0; !err && li < c->n_layer; li++) {
        NcpLayer *L = &m->layer[li];
        snprintf(pre, sizeof pre, "gen.transformer.blocks.%d.", li);
#define NCPW(field, name, req, n) (snprintf(kk, sizeof kk, "%s%s", pre, name), L->field = wget(ws, kk, req, n, &err))
        NCPW(ln1w, "ln_1.weight", 1, C);
        NCPW(ln1b, "ln_1.bias", 0, C);
        NCPW(attw, "attn.c_attn.weight", 1, QKV * C);
        NCPW(attb, "attn.c_attn.bias", 0, QKV);
        if (c->use_qk_norm) {
            NCPW(qn, "attn.q_norm.weight", 1, hd);
            NCPW(kn, "attn.k_norm.weight", 1, hd);
        }
        NCPW(projw, "attn.c_proj.weight", 1, (int64_t)C * C);
        NCPW(projb, "attn.c_proj.bias", 0, C);
        NCPW(ln2w, "ln_2.weight", 1, C);
        NCPW(ln2b, "ln_2.bias", 0, C);
        Tensor *t = NULL;
        snprintf(kk, sizeof kk, "%s%s", pre, gated ? "mlp.w_gate.weight" : "mlp.c_fc.weight");
        t = weights_get(ws, kk);
        L->inner = t ? (int)t->shape[0] : 0;
        if (!t || L->inner <= 0 || t->n != (int64_t)L->inner * C) {
            if (!err) err = ncm_fail(NCM_E_ARG, "ncp_load: missing or mis-shaped %s", kk);
            break;
        }
        const int I = L->inner;
        if (gated) {
            NCPW(gw, "mlp.w_gate.weight", 1, (int64_t)I * C);
            NCPW(gb, "mlp.w_gate.bias", 0, I);
            NCPW(uw, "mlp.w_up.weight", 1, (int64_t)I * C);
            NCPW(ub, "mlp.w_up.bias", 0, I);
        } else {
            NCPW(fcw, "mlp.c_fc.weight", 1, (int64_t)I * C);
            NCPW(fcb, "mlp.c_fc.bias", 0, I);
        }
        NCPW(mpw, "mlp.c_proj.weight", 1, (int64_t)C * I);
        NCPW(mpb, "mlp.c_proj.bias", 0, C);
#undef NCPW
    }
    if (!err && c->puc_enabled)
        for (int k = 0; !err && k < m->n_tgt; k++) {
            /* the device convolution takes kernels up to 16 taps, as vq_load */
            if (c->puc_kernel <= 0 || c->puc_kernel > 16)
                err = ncm_fail(NCM_E_ARG, "ncp_load: puc_kernel %d outside 1..16", c->puc_kernel);
            snprintf(kk, sizeof kk, "gen.post_upsample_convs.%d.weight", k);
            wget(ws, kk, 1, (int64_t)m->D * m->D * c->puc_kernel, &err);
            snprintf(kk, sizeof kk, "gen.post_upsample_convs.%d.bias", k);
            wget(ws, kk, 1, m->D, &err);
        }
    if (!err) ncp_load_heads(m, &err);
    /* level embedding rows wle[level] (+ wpe[t] without RoPE) (ncp.c:144-172),
     * the level of each target row and the pad-free mask (ncp.c:361-386) */
    if (!err) {
        const float *wle = wget(ws, "gen.transformer.wle.weight", 1, (int64_t)m->n_tgt * C, &err);
        Tensor *twpe = m->wpe ? weights_get(ws, "gen.transformer.wpe.weight") : NULL;
        int Tmax = P;
        for (int k = 0; k < m->n_tgt; k++)
            if (m->tl[k] > Tmax) Tmax = m->tl[k];
        if (twpe && twpe->n < (int64_t)Tmax * C && !err)
            err = ncm_fail(NCM_E_ARG, "ncp_load: gen.transformer.wpe.weight has fewer than %d rows", Tmax);
        m->lvl_pos = (float *)ncm_hip_malloc((size_t)(T > 0 ? T : 1) * C * sizeof(float));
        m->lvl = (int *)ncm_hip_malloc((size_t)(T > 0 ? T : 1) * sizeof(int));
        m->mask = (float *)ncm_hip_malloc((size_t)S * S * sizeof(float));
        int *ldev = (int *)ncm_hip_malloc((size_t)(T > 0 ? T : 1) * sizeof(int));
        if (!m->lvl_pos || !m->lvl || !m->mask || !ldev) err = err ? err : NCM_E_OOM;
        if (!err) {
            int *rel = (int *)malloc((size_t)(T > 0 ? T : 1) * sizeof(int));
            for (int t = 0; rel && t < T; t++) rel[t] = lvl[t] - m->lvl_first;
            if (!rel) err = ncm_fail(NCM_E_OOM, "ncp_load");
            else {
                mem_h2d(m->lvl, lvl, (size_t)T * sizeof(int));
                mem_h2d(ldev, rel, (size_t)T * sizeof(int));
                embedding_fwd(wle, ldev, m->lvl_pos, T, C);
                if (m->wpe) {
                    float *tmp = (float *)ncm_hip_malloc((size_t)(T > 0 ? T : 1) * C * sizeof(float));
                    mem_h2d(ldev, tpos, (size_t)T * sizeof(int));
                    if (!tmp) err = NCM_E_OOM;
                    else {
                        embedding_fwd(m->wpe, ldev, tmp, T, C);
                        add_fwd(m->lvl_pos, tmp, m->lvl_pos, (int64_t)T * C);
                        ncm_hip_free(tmp);
                    }
                }
                free(rel);
            }
        }
        if (!err) {
            const int *nopad = NULL;
            int bd = c->attn_pattern_block_diag, Pi = P, Ti = T, one = 1;
            void *a[] = {&m->mask, &m->lvl, &nopad, &Pi, &Ti, &bd, &one};
            err = ncm_launch_named("ncp_mask_k", blocks256((int64_t)S * S), 1, 1, 256, a);
        }
        ncm_hip_free(ldev);
    }
    free(pos);
    free(lvl);
    free(tpos);
    if (err) {
        ncp_free(m);
        return NULL;
    }
    return m;
}

int ncp_P(NCPState *m) { return m ? m->P : 0; }
int ncp_T(NCPState *m) { return m ? m->T : 0; }
int ncp_ntgt(NCPState *m) { return m ? m->n_tgt : 0; }
int ncp_lvlfirst(NCPState *m) { return m ? m->lvl_first : 0; }
float *ncp_rope_cos(NCPState *m) { return m ? m->rope_cos : NULL; }
float *ncp_rope_sin(NCPState *m) { return m ? m->rope_sin : NULL; }
float *ncp_rope_gen_cos(NCPState *m, int k) { return m && k >= 0 && k < m->n_tgt ? m->gcos[k] : NULL; }
float *ncp_rope_gen_sin(NCPState *m, int k) { return m && k >= 0 && k < m->n_tgt ? m->gsin[k] : NULL; }

/* ncp_block (ncp.c:184-345) on x [nb*S][C] in place; per_board: mask holds
 * one [S][S] mask per board */
static int ncp_block_dev(NCPState *m, const NcpLayer *L, float *x, int nb, const float *mask, int per_board) {
    const NCMConfig *c = &m->cfg;
    const int C = m->C, H = m->H, nkv = m->nkv, hd = m->hd, S = m->S, I = L->inner;
    const int64_t R = (int64_t)nb * S, QKV = (int64_t)C + 2 * (int64_t)nkv * hd;
    const int fused = hd <= 64;
    const int hk = fused ? nkv : H;   /* kv heads as the attention sees them */
    float *ln = A(R * C), *qkv = A(R * QKV), *q = A(R * C), *k = A((int64_t)nb * hk * S * hd),
          *v = A((int64_t)nb * hk * S * hd), *mo = A(R * C), *g = A(R * I);
    if (!g) return NCM_E_OOM;
    layernorm_fwd(x, L->ln1w, L->ln1b, ln, R, C);
    linear_fwd(ln, L->attw, L->attb, qkv, R, (int)QKV, C);
    const float *cs = c->use_rope ? m->rope_cos : NULL, *sn = c->use_rope ? m->rope_sin : NULL;
    if (fused) {
        int rc = ncp_qkv_launch(qkv, q, k, v, L->qn, L->kn, cs, sn, nb, S, H, nkv, hd);
        if (rc) return rc;
    } else {
        /* the reference's own sequence: split with the kv heads replicated,
         * qk-norm, RoPE (ncp.c:213-243) */
        qkv_split_fwd(qkv, q, k, v, nb, S, C, H, hd, nkv, H / nkv);
        if (L->qn) {
            rmsnorm_fwd(q, L->qn, q, (int64_t)nb * H * S, hd);
            rmsnorm_fwd(k, L->kn, k, (int64_t)nb * H * S, hd);
        }
        if (cs) rope_apply(q, k, cs, sn, nb, H, S, hd);
    }
    if (per_board)
        ncm_sdpa_fwd_gqa_merged_bmask(q, k, v, mask, mo, nb, H, hk, S, S, hd);
    else
        sdpa_fwd_gqa_merged(q, k, v, mask, mo, nb, H, hk, S, S, hd);
    linear_fwd_ep(mo, L->projw, L->projb, x, x, R, C, C, NCM_ACT_NONE);            /* x += c_proj(.) */
    layernorm_fwd(x, L->ln2w, L->ln2b, ln, R, C);
    if (L->gw)
        linear_fwd_gated(ln, L->gw, L->gb, L->uw, L->ub, g, R, I, C, c->use_swiglu ? NCM_ACT_SILU : NCM_ACT_GELU);
    else
        linear_fwd_ep(ln, L->fcw, L->fcb, NULL, g, R, I, C, c->use_relu2 ? NCM_ACT_RELU2 : NCM_ACT_GELU);
    linear_fwd_ep(g, L->mpw, L->mpb, x, x, R, C, I, NCM_ACT_NONE);                  /* x += c_proj(.) */
    return 0;
}

/* run_stack (ncp.c:347-358): the blocks, then ln_f into out */
static int ncp_stack_dev(NCPState *m, float *h, float *out, int nb, const float *mask, int per_board) {
    for (int li = 0; li < m->cfg.n_layer; li++) {
        int rc = ncp_block_dev(m, &m->layer[li], h, nb, mask, per_board);
        if (rc) return rc;
    }
    layernorm_fwd(h, m->lnfw, m->lnfb, out, (int64_t)nb * m->S, m->C);
    return 0;
}

void ncp_forward(NCPState *m, const float *x, const int *prefix_ids, float *logits, int B) {
    if (!m || !x || !logits || B <= 0) {
        ncm_fail(NCM_E_ARG, "ncp_forward: null model/x/logits or B <= 0");
        return;
    }
    if (ncm_ready()) return;
    const NCMConfig *c = &m->cfg;
    const int C = m->C, S = m->S, P = m->P, T = m->T, D = m->D;
    const int64_t R = (int64_t)B * S;
    float *h = A(R * C), *hf = A(R * C);
    if (!hf) return;
    /* post-upsample convs on each target level's rows of x (ncp.c:503-534) */
    const float *xin = x;
    if (c->puc_enabled) {
        float *xw = A(R * D);
        int Kc = c->puc_kernel, To = m->tl[0];
        for (int k = 1; k < m->n_tgt; k++)
            if (m->tl[k] > To) To = m->tl[k];
        To += 2 * (Kc / 2) + 1;
        float *chunk = A((int64_t)B * To * D), *co = A((int64_t)B * To * D);
        if (!co) return;
        if (ncm_copy_async(xw, x, (size_t)R * D * sizeof(float))) return;
        char kw[96], kb[96];
        for (int k = 0; k < m->n_tgt; k++) {
            int Bi = B, Si = S, off = P + m->toff[k], lk = m->tl[k], Di = D;
            void *a[] = {&xw, &chunk, &Bi, &Si, &off, &lk, &Di};
            if (ncm_launch_named("ncp_gather_rows_k", blocks256((int64_t)B * lk * D), 1, 1, 256, a)) return;
            snprintf(kw, sizeof kw, "gen.post_upsample_convs.%d.weight", k);
            snprintf(kb, sizeof kb, "gen.post_upsample_convs.%d.bias", k);
            const float *W = weights_get(m->ws, kw)->data, *bb = weights_get(m->ws, kb)->data;
            if (ncm_conv1d_btd(chunk, W, bb, co, B, lk, D, Kc, 1, Kc / 2)) return;
            int64_t tb = (int64_t)(lk + 2 * (Kc / 2) - Kc + 1) * D;   /* rows of one board's conv output */
            void *a2[] = {&xw, &co, &Bi, &Si, &off, &lk, &Di, &tb};
            if (ncm_launch_named("ncp_add_rows_k", blocks256((int64_t)B * lk * D), 1, 1, 256, a2)) return;
        }
        xin = xw;
    }
    /* wte over every row (prefix and target share it, ncp.c:536-546), the
     * level embedding on the target rows, wpe on the prefix without RoPE */
    linear_fwd(xin, m->wte, m->wteb, h, R, C, D);
    {
        int Bi = B, Si = S, off = P, Ti = T, Ci = C;
        int64_t tb = 0;
        void *a[] = {&h, &m->lvl_pos, &Bi, &Si, &off, &Ti, &Ci, &tb};
        if (T > 0 && ncm_launch_named("ncp_add_rows_k", blocks256((int64_t)B * T * C), 1, 1, 256, a)) return;
        if (!c->use_rope && P > 0) {
            int z = 0, Pi = P;
            void *a2[] = {&h, &m->wpe, &Bi, &Si, &z, &Pi, &Ci, &tb};
            if (ncm_launch_named("ncp_add_rows_k", blocks256((int64_t)B * P * C), 1, 1, 256, a2)) return;
        }
    }
    /* with padded prefix tokens every board gets its own mask, its pad keys
     * masked out (ncp.c:571-607 runs such boards one at a time): the pad
     * flags of all boards go up in one stream-ordered copy, one launch
     * builds the B masks, and the stack runs over every board at once */
    int any_pad = 0;
    if (c->prefix_pad_token_id >= 0 && prefix_ids)
        for (int64_t i = 0; i < (int64_t)B * P; i++)
            if (prefix_ids[i] == c->prefix_pad_token_id) any_pad = 1;
    if (!any_pad) {
        if (ncp_stack_dev(m, h, hf, B, m->mask, 0)) return;
    } else {
        float *bm = A((int64_t)B * S * S);
        int *pad = (int *)A((int64_t)B * P);
        int *flags = (int *)malloc((size_t)B * P * sizeof(int));
        if (!bm || !pad || !flags) {
            free(flags);
            if (bm && pad) ncm_fail(NCM_E_OOM, "ncp_forward: pad flags");
            return;
        }
        for (int64_t i = 0; i < (int64_t)B * P; i++) flags[i] = prefix_ids[i] == c->prefix_pad_token_id;
        int rc = ncm_h2d_async(pad, flags, (size_t)B * P * sizeof(int));
        free(flags);
        if (rc) return;
        int bd = c->attn_pattern_block_diag, Pi = P, Ti = T, nb = B;
        void *a[] = {&bm, &m->lvl, &pad, &Pi, &Ti, &bd, &nb};
        if (ncm_launch_named("ncp_mask_k", blocks256((int64_t)B * S * S), 1, 1, 256, a) ||
            ncp_stack_dev(m, h, hf, B, bm, 1))
            return;
    }
    /* heads per target level (ncp.c:601-637) */
    for (int k = 0; k < m->n_tgt; k++) {
        const NcpHead *hp = &m->head[k];
        int lk = m->tl[k], V = c->vocab_size[k];
        const int64_t rows = (int64_t)B * lk;
        float *sl = A(rows * C), *lg = A(rows * V);
        if (!lg) return;
        int Bi = B, Si = S, off = P + m->toff[k], Ci = C;
        void *a[] = {&hf, &sl, &Bi, &Si, &off, &lk, &Ci};
        if (ncm_launch_named("ncp_gather_rows_k", blocks256(rows * C), 1, 1, 256, a)) return;
        if (c->tie_heads_to_codebook && !c->shared_output_head) {
            float *z = A(rows * hp->Dd);
            if (!z) return;
            linear_fwd(sl, hp->w, hp->b, z, rows, hp->Dd, C);
            int ri = (int)rows, Vi = V, Dd = hp->Dd;
            float invT = hp->invT;
            const float *E = hp->E, *tb = hp->tb;
            const double *esq = hp->esq, *ds = hp->ds;
            void *a2[] = {&z, &E, &esq, &ds, &invT, &tb, &lg, &ri, &Vi, &Dd};
            if (ncm_launch_named("ncp_tied_head_k", blocks256(rows * V), 1, 1, 256, a2)) return;
        } else {
            linear_fwd(sl, hp->w, hp->b, lg, rows, V, C);
        }
        int Ti = T, offt = m->toff[k], maxV = m->maxV;
        void *a3[] = {&lg, &logits, &Bi, &Ti, &offt, &lk, &V, &maxV};
        if (ncm_launch_named("ncp_logits_k", blocks256(rows * maxV), 1, 1, 256, a3)) return;
    }
}
