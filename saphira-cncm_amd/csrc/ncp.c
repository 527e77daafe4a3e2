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
    float *cosd = A((int64_t)S * hd), *sind = A((int64_t)S * hd), *x = A(R * C);
    int *bids = (int *)A(R);
    float *hc = (float *)malloc((size_t)S * hd * sizeof(float)), *hs = (float *)malloc((size_t)S * hd * sizeof(float));
    if (!bids || !hc || !hs) {
        free(hc);
        free(hs);
        if (bids) ncm_fail(NCM_E_OOM, "ncp: host tables");
        return NULL;
    }
    ncm_ncp_rope_tables(S, hd, c->rope_base, hc, hs);
    mem_h2d(cosd, hc, (size_t)S * hd * sizeof(float));
    mem_h2d(sind, hs, (size_t)S * hd * sizeof(float));
    free(hc);
    free(hs);
    mem_h2d(bids, ids, (size_t)R * sizeof(int));
    embedding_fwd_v(P[0], V, bids, x, R, C);
    float *ln = A(R * C), *qkv = A(R * QKV), *qq = A(R * C), *kk = A(R * C), *vv = A(R * C),
          *mo = A(R * C), *g = A(R * I);
    if (!g) return NULL;
    for (int li = 0; li < c->n_layer; li++) {
        float *const *w = P + 1 + NCP_PER_LAYER * li;
        norm(c, x, w[0], w[1], ln, R);
        linear_fwd(ln, w[2], w[3], qkv, R, QKV, C);
        qkv_split_rope_fwd(qkv, qq, kk, vv, cosd, sind, B, S, C, H, hd, Kv, rep);   /* split, then RoPE */
        sdpa_fwd_gqa_merged(qq, kk, vv, NULL, mo, B, H, H, S, S, hd);               /* heads merged on output */
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
