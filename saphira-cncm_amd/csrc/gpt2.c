/* gpt2.c -- the taped GPT-2 forward and training step of train_gpt2.c:42-180
 * on the device tape: wte + wpe embed; per block LayerNorm (eps 1e-5) ->
 * c_attn -> qkv split -> causal SDPA -> merge -> c_proj -> residual ->
 * LayerNorm -> c_fc -> gelu_new -> c_proj -> residual; final LayerNorm and
 * the tied head (a linear on wte).  Then mean cross-entropy, tape backward,
 * global-norm clip at 1.0 and AdamW with the cosine warm-up schedule.
 *
 * Parameters are addressed as one flat array of device pointers in the
 * order ncm_gpt2_param_shape documents (the order of the reference's
 * WeightStore names: wte, wpe, h.<l>.{ln_1.weight, ln_1.bias,
 * attn.c_attn.weight, attn.c_attn.bias, attn.c_proj.weight,
 * attn.c_proj.bias, ln_2.weight, ln_2.bias, mlp.c_fc.weight, mlp.c_fc.bias,
 * mlp.c_proj.weight, mlp.c_proj.bias}, ln_f.weight, ln_f.bias).
 * Activations come from the library arena (arena_alloc), as the reference
 * takes them from its scratch arena. */
#include "internal.h"

#include <math.h>
#include <stdlib.h>

#define GPT2_LN_EPS 1e-5
#define PER_LAYER 12

int ncm_gpt2_param_count(const NcmGpt2Config *c) { return c ? 4 + PER_LAYER * c->n_layer : 0; }

int64_t ncm_gpt2_param_shape(const NcmGpt2Config *c, int i, int64_t *rows, int64_t *cols) {
    int64_t r = 0, k = 0;
    const int C = c->n_embd;
    const int n = ncm_gpt2_param_count(c);
    if (i < 0 || i >= n) return -1;
    if (i == 0) { r = c->vocab; k = C; }
    else if (i == 1) { r = c->n_pos; k = C; }
    else if (i >= n - 2) { r = C; k = 1; }
    else {
        switch ((i - 2) % PER_LAYER) {
        case 0: case 1: case 5: case 6: case 7: case 11: r = C; k = 1; break;
        case 2: r = 3 * (int64_t)C; k = C; break;
        case 3: r = 3 * (int64_t)C; k = 1; break;
        case 4: r = C; k = C; break;
        case 8: r = 4 * (int64_t)C; k = C; break;
        case 9: r = 4 * (int64_t)C; k = 1; break;
        case 10: r = C; k = 4 * (int64_t)C; break;
        }
    }
    if (rows) *rows = r;
    if (cols) *cols = k;
    return r * k;
}

static int cfg_ok(const NcmGpt2Config *c, int B, int T) {
    if (!c || c->n_layer < 0 || c->n_embd <= 0 || c->n_head <= 0 || c->n_embd % c->n_head || c->vocab <= 0 ||
        c->n_pos <= 0 || B <= 0 || T <= 0 || T > c->n_pos)
        return ncm_fail(NCM_E_ARG, "gpt2: bad configuration or batch (B=%d T=%d)", B, T);
    return 0;
}

static float *A(int64_t n) {
    float *p = arena_alloc((size_t)n);
    if (!p) ncm_fail(NCM_E_OOM, "gpt2: arena");
    return p;
}

/* train_gpt2.c:42-103 */
static float *gpt2_block(NcmTape *tp, const NcmGpt2Config *c, float *const *P, int li, float *x, int B, int T) {
    const int C = c->n_embd, H = c->n_head, hd = C / H, I = 4 * C;
    const int64_t R = (int64_t)B * T;
    float *const *w = P + 2 + PER_LAYER * li;
    float *ln = A(R * C), *qkv = A(R * 3 * C);
    float *qq = A(R * C), *kk = A(R * C), *vv = A(R * C), *ctx = A(R * C);
    float *mo = A(R * C), *x1 = A(R * C), *mn = A(R * C);
    float *mm = A(R * I), *m2 = A(R * I), *out = A(R * C);
    if (!out) return NULL;
    ncm_t_layernorm_eps(tp, x, w[0], w[1], ln, R, C, GPT2_LN_EPS);
    ncm_t_linear_qkvsplit(tp, ln, w[2], w[3], qkv, qq, kk, vv, B, T, C, H, hd, H, 1);   /* GEMM to heads */
    ncm_t_sdpa_causal_merge(tp, qq, kk, vv, ctx, mo, B, H, H, T, hd);   /* causal mask generated, heads merged */
    ncm_t_linear_res(tp, mo, w[4], w[5], x, x1, R, C, C);   /* x1 = x + attn proj */
    ncm_t_layernorm_eps(tp, x1, w[6], w[7], mn, R, C, GPT2_LN_EPS);
    ncm_t_linear_act(tp, mn, w[8], w[9], mm, m2, R, I, C, 2);   /* m2 = gelu_tanh(mm) */
    ncm_t_linear_res(tp, m2, w[10], w[11], x1, out, R, C, I);  /* out = x1 + mlp proj */
    return out;
}

/* train_gpt2.c:107-147: ids [B][T] host ints -> logits [B*T][vocab] (arena) */
float *ncm_gpt2_forward(NcmTape *tp, const NcmGpt2Config *c, float *const *P, const int *ids, int B, int T) {
    if (cfg_ok(c, B, T) || !tp || !P || !ids) return NULL;
    if (ncm_ready()) return NULL;
    const int C = c->n_embd, V = c->vocab;
    const int64_t R = (int64_t)B * T;
    float *h = A(R * C), *xe = A(R * C), *pe = A(R * C);
    int *ph = (int *)malloc((size_t)R * sizeof(int));
    if (!pe || !ph) {
        free(ph);
        if (pe) ncm_fail(NCM_E_OOM, "gpt2: host buffers");
        return NULL;
    }
    ncm_t_embed(tp, P[0], ids, V, xe, R, C);
    for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++) ph[(size_t)b * T + t] = t;
    ncm_t_embed(tp, P[1], ph, c->n_pos, pe, R, C);
    free(ph);
    ncm_t_add(tp, xe, pe, h, R * C);
    /* the causal -1e9 mask of train_gpt2.c:112-121 is generated in the SDPA
     * kernels (exactly zero probability for every later key, as -1e9 gives) */
    for (int li = 0; li < c->n_layer && h; li++) h = gpt2_block(tp, c, P, li, h, B, T);
    if (!h) return NULL;
    const int n = ncm_gpt2_param_count(c);
    float *lnf = A(R * C), *logits = A(R * V);
    if (!logits) return NULL;
    ncm_t_layernorm_eps(tp, h, P[n - 2], P[n - 1], lnf, R, C, GPT2_LN_EPS);
    ncm_t_linear(tp, lnf, P[0], NULL, logits, R, V, C);
    return logits;
}

/* train_gpt2.c:149-180 with the optimizer of train.c:102-145: one step on
 * the device.  grads must hold zeros on entry and are zeroed again on exit
 * (adamw_zero_grad); m, v are the AdamW moments; step is the optimizer step
 * number after this update (the reference increments first).  Returns the
 * mean loss; *gnorm_out gets the pre-clip gradient norm. */
float ncm_gpt2_train_step(NcmTape *tp, const NcmGpt2Config *c, float *const *P, float *const *G, float *const *M,
                          float *const *Vm, const int *xin, const int *xout, int B, int T, long step, double base_lr,
                          double warmup, double total, double wd, double *gnorm_out) {
    if (cfg_ok(c, B, T) || !P || !G || !M || !Vm || !xin || !xout || step < 1) {
        ncm_fail(NCM_E_ARG, "ncm_gpt2_train_step: bad arguments");
        return -1.0f;
    }
    const int n = ncm_gpt2_param_count(c);
    int64_t *sizes = (int64_t *)malloc((size_t)n * sizeof(int64_t));
    if (!sizes) { ncm_fail(NCM_E_OOM, "gpt2: sizes"); return -1.0f; }
    for (int i = 0; i < n; i++) sizes[i] = ncm_gpt2_param_shape(c, i, NULL, NULL);
    ncm_tape_clear(tp);
    arena_reset();
    float *logits = ncm_gpt2_forward(tp, c, P, xin, B, T);
    float *loss = A(1);
    float lh = -1.0f;
    if (logits && loss) {
        const int64_t R = (int64_t)B * T;
        ncm_t_ce(tp, logits, xout, NULL, loss, NULL, R, c->vocab, 1.0);
        NcmPMap pm = {(float **)P, (float **)G, sizes, n};
        ncm_tape_backward(tp, &pm);
        const double b1 = 0.9, b2 = 0.95, eps = 1e-8;
        const double lr = base_lr * sched_cosine_warmup(step, warmup, total);
        const double b1t = 1.0 - pow(b1, (double)step), b2t = 1.0 - pow(b2, (double)step);
        const double *g2_dev = NULL;
        if (ncm_clip_adamw_multi(P, G, M, Vm, sizes, n, 1.0, lr, b1, b2, b1t, b2t, eps, wd, 1, &g2_dev) == 0) {
            /* clip + update in three launches; loss and norm read back once, at the end */
            double g2 = 0.0;
            mem_d2h(&lh, loss, sizeof(float));
            mem_d2h(&g2, g2_dev, sizeof(double));
            if (gnorm_out) *gnorm_out = sqrt(g2);
        } else if (!ncm_ready()) {
            double gnorm = grad_clip_global(G, sizes, n, 1.0);
            if (gnorm_out) *gnorm_out = gnorm;
            mem_d2h(&lh, loss, sizeof(float));
            for (int i = 0; i < n; i++) {
                /* the update also clears the gradient for the next step */
                ncm_adamw_update_clear(P[i], G[i], M[i], Vm[i], sizes[i], lr, b1, b2, b1t, b2t, eps, wd);
            }
        }
    }
    free(sizes);
    return lh;
}
