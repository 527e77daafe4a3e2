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
        arena_init((size_t)2 << 30);
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
        arena_init((size_t)2 << 30);
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
