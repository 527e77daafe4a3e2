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
    int *ids_dev;           /* generated ids, one slot per position */
    int nchunk_max;
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
    m->nchunk_max = (c->n_ctx + 255) / 256;
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
    mem_h2d(bids, ids, (size_t)T * sizeof(int));
    embedding_fwd_v(P[0], V, bids, h, T, C);
    for (int li = 0; li < c->n_layer; li++) {
        float *const *w = P + 1 + QW_PER_LAYER * li;
        float *h1 = A((int64_t)T * C), *ql = A((int64_t)T * C), *kl = A((int64_t)T * K * hd),
              *vl = A((int64_t)T * K * hd), *qq = A((int64_t)T * C), *kk = A((int64_t)T * K * hd),
              *vv = A((int64_t)T * K * hd), *ctx = A((int64_t)T * C), *mo = A((int64_t)T * C),
              *x1 = A((int64_t)T * C), *h2 = A((int64_t)T * C), *gt = A((int64_t)T * I), *up = A((int64_t)T * I),
              *gu = A((int64_t)T * I), *out = A((int64_t)T * C);
        if (!out) return NULL;
        rmsnorm_fwd(h, w[0], h1, T, C);
        linear_fwd(h1, w[1], w[2], ql, T, C, C);
        linear_fwd(h1, w[3], w[4], kl, T, K * hd, C);
        linear_fwd(h1, w[5], w[6], vl, T, K * hd, C);
        heads_transpose_fwd(ql, qq, T, H, hd);
        heads_transpose_fwd(kl, kk, T, K, hd);
        heads_transpose_fwd(vl, vv, T, K, hd);
        rope_apply_gqa(qq, kk, m->cos_t, m->sin_t, 1, H, K, T, hd);
        sdpa_fwd_gqa_causal(qq, kk, vv, ctx, 1, H, K, T, T, hd);
        /* keep k, v for the cached decode: [K][T][hd] -> cache [K][n_ctx][hd] */
        const size_t pitch = (size_t)c->n_ctx * hd * sizeof(float), row = (size_t)T * hd * sizeof(float);
        float *kc = m->kcache + (size_t)li * K * c->n_ctx * hd, *vc = m->vcache + (size_t)li * K * c->n_ctx * hd;
        HIP_TRY_NULL(hipMemcpy2DAsync(kc, pitch, kk, row, row, K, hipMemcpyDeviceToDevice, ncm_stream()));
        HIP_TRY_NULL(hipMemcpy2DAsync(vc, pitch, vv, row, row, K, hipMemcpyDeviceToDevice, ncm_stream()));
        head_merge_fwd(ctx, mo, 1, T, C, H, hd);
        linear_fwd_ep(mo, w[7], NULL, h, x1, T, C, C, NCM_ACT_NONE);   /* x1 = h + mo W^T */
        rmsnorm_fwd(x1, w[8], h2, T, C);
        linear_fwd_ep(h2, w[9], NULL, NULL, gt, T, I, C, NCM_ACT_SILU);
        linear_fwd(h2, w[10], NULL, up, T, I, C);
        mul_fwd(gt, up, gu, (int64_t)T * I);
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

/* One cached decode step: the token id at ids_dev[pos] (device) at position
 * pos (the cache holds positions 0..pos-1).  Logits [V] in the model's
 * buffer; returns it. */
static float *decode_step(NcmQwen *m, int pos) {
    const NcmQwenConfig *c = &m->c;
    const int C = c->n_embd, H = c->n_head, K = c->n_kv, hd = C / H, I = c->n_inner, V = c->vocab;
    float *const *P = m->P;
    embedding_fwd_v(P[0], V, m->ids_dev + pos, m->x, 1, C);
    float *h = m->x;
    const int nchunk = (pos + 1 + 255) / 256;
    for (int li = 0; li < c->n_layer; li++) {
        float *const *w = P + 1 + QW_PER_LAYER * li;
        float *kc = m->kcache + (size_t)li * K * c->n_ctx * hd, *vc = m->vcache + (size_t)li * K * c->n_ctx * hd;
        rmsnorm_fwd(h, w[0], m->h1, 1, C);
        linear_fwd(m->h1, w[1], w[2], m->q, 1, C, C);
        linear_fwd(m->h1, w[3], w[4], m->k, 1, K * hd, C);
        linear_fwd(m->h1, w[5], w[6], m->v, 1, K * hd, C);
        {
            int n_thr = (H + K) * (hd / 2) + K * hd, ld = c->n_ctx;
            void *a[] = {&m->q, &m->k, &m->v, &m->cos_t, &m->sin_t, &m->qr, &kc, &vc, (void *)&H, (void *)&K,
                         (void *)&hd, &ld, &pos};
            if (ncm_launch_named("rope_append_k", (unsigned)((n_thr + 255) / 256), 1, 1, 256, a)) return NULL;
        }
        {
            int tkv = pos + 1, ld = c->n_ctx;
            float scale = 1.0f / sqrtf((float)hd);
            void *a[] = {&m->qr, &kc, &vc, &m->part_o, &m->part_ml, (void *)&H, (void *)&K, &tkv, &ld, &scale};
            if (ncm_launch_named("sdpa_decode_partial", (unsigned)nchunk, (unsigned)K, 1, 256, a)) return NULL;
            int nc = nchunk;
            void *a2[] = {&m->part_o, &m->part_ml, &m->ctx, &nc};
            if (ncm_launch_named("sdpa_decode_combine", (unsigned)H, 1, 1, 64, a2)) return NULL;
        }
        /* ctx [H][1][hd] is already the merged row [C] */
        linear_fwd_ep(m->ctx, w[7], NULL, h, m->x1, 1, C, C, NCM_ACT_NONE);
        rmsnorm_fwd(m->x1, w[8], m->h2, 1, C);
        linear_fwd_ep(m->h2, w[9], NULL, NULL, m->gate, 1, I, C, NCM_ACT_SILU);
        linear_fwd(m->h2, w[10], NULL, m->up, 1, I, C);
        mul_fwd(m->gate, m->up, m->up, I);
        linear_fwd_ep(m->up, w[11], NULL, m->x1, m->x, 1, C, I, NCM_ACT_NONE);   /* h = x1 + down */
    }
    const int n = ncm_qwen_param_count(c);
    rmsnorm_fwd(h, P[n - 1], m->h1, 1, C);
    linear_fwd(m->h1, P[0], NULL, m->logits, 1, V, C);
    return m->logits;
}

float *ncm_qwen_decode(NcmQwen *m, int id, int pos) {
    if (!m || pos < 1 || pos >= m->c.n_ctx) { ncm_fail(NCM_E_ARG, "ncm_qwen_decode: bad position"); return NULL; }
    if (ncm_ready()) return NULL;
    if (m->c.n_embd / m->c.n_head != 64 || m->c.n_head / m->c.n_kv > 16) {
        ncm_fail(NCM_E_ARG, "ncm_qwen_decode: needs hd = 64 and at most 16 query heads per kv head");
        return NULL;
    }
    mem_h2d(m->ids_dev + pos, &id, sizeof(int));
    return decode_step(m, pos);
}

/* Greedy generation (qwen_generate with temp 0, qwen.c:204-228): prefill of
 * the prompt, then n_new steps of argmax + cached decode.  The ids stay on
 * the device (argmax_rows writes the next id where the next step reads it);
 * with eos >= 0 each step is synchronised to stop at eos as the reference
 * does, with eos < 0 all steps run without a host round trip.  Returns the
 * number of ids written to out. */
int ncm_qwen_generate(NcmQwen *m, const int *prompt, int np, int n_new, int eos, int *out) {
    if (!m || !prompt || np <= 0 || n_new < 0 || !out) { ncm_fail(NCM_E_ARG, "ncm_qwen_generate: bad arguments"); return -1; }
    if (np + n_new > m->c.n_ctx) { ncm_fail(NCM_E_ARG, "ncm_qwen_generate: context overflow"); return -1; }
    if (m->c.n_embd / m->c.n_head != 64 || m->c.n_head / m->c.n_kv > 16) {
        ncm_fail(NCM_E_ARG, "ncm_qwen_generate: needs hd = 64 and at most 16 query heads per kv head");
        return -1;
    }
    if (n_new == 0) return 0;
    float *lg = ncm_qwen_forward(m, prompt, np, 1);
    if (!lg) return -1;
    argmax_rows(lg, m->ids_dev + np, 1, m->c.vocab);
    int made = 1;
    if (eos >= 0) {
        mem_d2h(out, m->ids_dev + np, sizeof(int));
        if (out[0] == eos) return 1;
    }
    for (int s = 1; s < n_new; s++) {
        const int pos = np + s - 1;   /* position of the id generated last */
        float *l = decode_step(m, pos);
        if (!l || ncm_ready()) return -1;
        argmax_rows(l, m->ids_dev + pos + 1, 1, m->c.vocab);
        made++;
        if (eos >= 0) {
            mem_d2h(out + s, m->ids_dev + pos + 1, sizeof(int));
            if (out[s] == eos) return made;
        }
    }
    mem_d2h(out, m->ids_dev + np, (size_t)made * sizeof(int));
    return made;
}
