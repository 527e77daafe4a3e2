/* train.c -- host side of the training-step kernels: norm backward,
 * softmax cross-entropy, stored attention probabilities, SDPA backward,
 * AdamW, learning-rate schedule and global-norm clipping.
 *
 * Every gradient output accumulates (+=) into the caller's buffer, the
 * contract of the reference's tape backward (train_tape.c:636-1051); a NULL
 * gradient pointer skips that gradient. */
#include "internal.h"

#include <limits.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define NORM_ROWS 128
#define NBF_ROWS 32   /* rows per workgroup of the fused norm backward */

static unsigned blocks_of(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

static int shape_ok(const char *fn, int64_t rows, int C) {
    if (rows < 0 || C <= 0 || (rows + 3) / 4 > UINT_MAX)
        return ncm_fail(NCM_E_ARG, "%s: bad shape rows=%lld C=%d", fn, (long long)rows, C);
    return 0;
}

/* ---- LayerNorm / RMSNorm backward (train_tape.c:569-634, 748-792) ---- */
/* beta 0: dx is written (0.0f + the gradient) instead of accumulated. */
/* base (with dx): dx = (0.0f + base) + the gradient, written (a residual
 * gradient passed through, then the norm's own accumulated onto it) */
static void norm_bwd(const char *fn, int kind, const float *x, const float *w, const float *dy, float *dx,
                     float *dw, float *db, int64_t rows, int C, double eps, int beta, const float *base) {
    if (shape_ok(fn, rows, C)) return;
    if (rows == 0) return;
    if (!x || !dy) { ncm_fail(NCM_E_ARG, "%s: null input", fn); return; }
    if (ncm_ready()) return;
    if (!dx) base = NULL;
    const int want_param = dw || db;
    if (C % 4 == 0 && C <= 1024 && is_aligned16(x) && is_aligned16(dy) && (!dx || is_aligned16(dx)) &&
        (!w || is_aligned16(w)) && (!base || is_aligned16(base)) && (rows + NBF_ROWS - 1) / NBF_ROWS <= INT_MAX) {
        /* one pass: rows in registers, dx and the parameter partials together */
        static const char *const names[2][4] = {{"ln_bwd_fused_1", "ln_bwd_fused_2", "ln_bwd_fused_3", "ln_bwd_fused_4"},
                                                {"rmsn_bwd_fused_1", "rmsn_bwd_fused_2", "rmsn_bwd_fused_3",
                                                 "rmsn_bwd_fused_4"}};
        const int chunks = (int)((rows + NBF_ROWS - 1) / NBF_ROWS);
        double *part = NULL;
        if (want_param) {
            part = (double *)ncm_workspace(WS_TRAIN, (size_t)chunks * C * 2 * sizeof(double));
            if (!part) return;
        }
        void *a[] = {&x, &w, &dy, &dx, &part, &rows, &C, &eps, &beta, &base};
        if (ncm_launch_named(names[kind][(C + 255) / 256 - 1], (unsigned)chunks, 1, 1, 256, a)) return;
        if (!want_param) return;
        float *dbk = kind == 0 ? db : NULL;
        void *a2[] = {&part, &dw, &dbk, (void *)&chunks, &C};
        ncm_launch_named("norm_param_sum", blocks_of(C, 64), 1, 1, 1024, a2);
        return;
    }
    const int chunks = (int)((rows + NORM_ROWS - 1) / NORM_ROWS);
    if (chunks > 65535 && want_param) { ncm_fail(NCM_E_ARG, "%s: too many rows", fn); return; }
    if (base) {   /* dx = 0.0f + base, then the norm's gradient accumulated */
        ncm_add_inplace_ex(dx, base, rows * C, 0);
        beta = 1;
    }
    if (dx && !beta && ncm_zero_async(dx, (size_t)rows * C * sizeof(float))) return;
    size_t stats_bytes = (size_t)rows * 2 * sizeof(double);
    size_t part_bytes = want_param ? (size_t)chunks * C * 2 * sizeof(double) : 0;
    char *ws = (char *)ncm_workspace(WS_TRAIN, stats_bytes + part_bytes);
    if (!ws) return;
    double *stats = (double *)ws, *part = (double *)(ws + stats_bytes);
    if (kind == 0) {
        void *a[] = {&x, &w, &dy, &dx, &stats, &rows, &C, &eps};
        if (ncm_launch_named("ln_bwd_rows", blocks_of(rows, 4), 1, 1, 256, a)) return;
    } else {
        void *a[] = {&x, &w, &dy, &dx, &stats, &rows, &C};
        if (ncm_launch_named("rmsn_bwd_rows", blocks_of(rows, 4), 1, 1, 256, a)) return;
    }
    if (!want_param) return;
    void *a2[] = {&x, &dy, &stats, &part, &rows, &C, &kind};
    if (ncm_launch_named("norm_param_partial", blocks_of(C, 256), (unsigned)chunks, 1, 256, a2)) return;
    float *dbk = kind == 0 ? db : NULL;
    void *a3[] = {&part, &dw, &dbk, (void *)&chunks, &C};
    ncm_launch_named("norm_param_final", blocks_of(C, 256), 1, 1, 256, a3);
}

void layernorm_bwd(const float *x, const float *w, const float *dy, float *dx, float *dw, float *db, int64_t rows,
                   int C, double eps) {
    norm_bwd("layernorm_bwd", 0, x, w, dy, dx, dw, db, rows, C, eps, 1, NULL);
}

void rmsnorm_bwd(const float *x, const float *w, const float *dy, float *dx, float *dw, int64_t rows, int C) {
    norm_bwd("rmsnorm_bwd", 1, x, w, dy, dx, dw, NULL, rows, C, 1e-6, 1, NULL);
}

void ncm_layernorm_bwd_ex(const float *x, const float *w, const float *dy, float *dx, float *dw, float *db,
                          int64_t rows, int C, double eps, int beta) {
    norm_bwd("layernorm_bwd", 0, x, w, dy, dx, dw, db, rows, C, eps, beta, NULL);
}

void ncm_layernorm_bwd_base(const float *x, const float *w, const float *dy, float *dx, float *dw, float *db,
                            int64_t rows, int C, double eps, const float *base) {
    norm_bwd("layernorm_bwd", 0, x, w, dy, dx, dw, db, rows, C, eps, 0, base);
}

void ncm_rmsnorm_bwd_ex(const float *x, const float *w, const float *dy, float *dx, float *dw, int64_t rows, int C,
                        int beta) {
    norm_bwd("rmsnorm_bwd", 1, x, w, dy, dx, dw, NULL, rows, C, 1e-6, beta, NULL);
}

void ncm_rmsnorm_bwd_base(const float *x, const float *w, const float *dy, float *dx, float *dw, int64_t rows, int C,
                          const float *base) {
    norm_bwd("rmsnorm_bwd", 1, x, w, dy, dx, dw, NULL, rows, C, 1e-6, 0, base);
}

/* ---- softmax cross-entropy (train_tape.c:442-481, 657-679, 1801-1810) ---- */
static int ce_check(const char *fn, const float *in, const int *tgt, const float *loss, int64_t rows, int V) {
    if (rows <= 0 || V <= 0 || (rows + 3) / 4 > UINT_MAX)
        return ncm_fail(NCM_E_ARG, "%s: bad shape rows=%lld V=%d", fn, (long long)rows, V);
    if (!in || !tgt || !loss) return ncm_fail(NCM_E_ARG, "%s: null pointer", fn);
    return ncm_ready();
}

static void ce_run(const char *fn, const float *logits, const int *tgt, const float *wm, float *loss, float *out,
                   int64_t rows, int V, double weight, int mode) {
    if (ce_check(fn, logits, tgt, loss, rows, V)) return;
    if (!out) { ncm_fail(NCM_E_ARG, "%s: null output", fn); return; }
    double *ws = (double *)ncm_workspace(WS_TRAIN, ((size_t)rows * 2 + 1) * sizeof(double));
    if (!ws) return;
    double *rowstat = ws, *cnt = ws + 2 * rows;
    const double *cnt_in = NULL;
    double cnt_val = (double)rows;
    if (mode == 1 && wm) {
        void *a[] = {&wm, &cnt, &rows};
        if (ncm_launch_named("ce_count", 1, 1, 1, 256, a)) return;
        cnt_in = cnt;
    }
    void *a[] = {&logits, &tgt, &wm, &out, &rowstat, &cnt_in, &cnt_val, &weight, &rows, &V, &mode};
    if (ncm_launch_named("ce_rows", blocks_of(rows, 4), 1, 1, 256, a)) return;
    void *a2[] = {&rowstat, &loss, &rows};
    ncm_launch_named("ce_loss_final", 1, 1, 1, 256, a2);
}

void ce_fwd(const float *logits, const int *tgt, const float *wmask, float *loss, float *probs, int64_t rows,
            int V) {
    ce_run("ce_fwd", logits, tgt, wmask, loss, probs, rows, V, 1.0, 0);
}

void ce_fwd_bwd(const float *logits, const int *tgt, const float *wmask, float *loss, float *dlogits,
                int64_t rows, int V, double weight) {
    ce_run("ce_fwd_bwd", logits, tgt, wmask, loss, dlogits, rows, V, weight, 1);
}

void ce_bwd(const float *probs, const int *tgt, const float *wmask, float *dlogits, int64_t rows, int V,
            double inv) {
    if (rows < 0 || V <= 0 || (rows * V + 255) / 256 > UINT_MAX) {
        ncm_fail(NCM_E_ARG, "ce_bwd: bad shape");
        return;
    }
    if (rows == 0) return;
    if (!probs || !tgt || !dlogits) { ncm_fail(NCM_E_ARG, "ce_bwd: null pointer"); return; }
    if (ncm_ready()) return;
    void *a[] = {&probs, &tgt, &wmask, &dlogits, &rows, &V, &inv};
    ncm_launch_named("ce_bwd_k", blocks_of(rows * V, 256), 1, 1, 256, a);
}

/* ---- attention: stored probabilities and backward ---- */
static int attn_check(const char *fn, int B, int H, int Hkv, int Tq, int Tkv, int hd) {
    if (B < 0 || H <= 0 || Hkv <= 0 || H % Hkv || Tq < 0 || Tkv <= 0 || hd <= 0 || hd > 256)
        return ncm_fail(NCM_E_ARG, "%s: bad shape B=%d H=%d Hkv=%d Tq=%d Tkv=%d hd=%d", fn, B, H, Hkv, Tq, Tkv,
                        hd);
    if (B > 65535 || H > 65535) return ncm_fail(NCM_E_ARG, "%s: grid too large", fn);
    return 0;
}

static int mfma_path(int hd, int Tkv, const void *a, const void *b, const void *c, const void *d, const void *e) {
    return hd == 64 && Tkv % 4 == 0 && is_aligned16(a) && is_aligned16(b) && is_aligned16(c) && is_aligned16(d) &&
           is_aligned16(e);
}

void sdpa_probs_gqa(const float *q, const float *k, const float *mask, float *P, int B, int H, int Hkv, int Tq,
                    int Tkv, int hd) {
    if (attn_check("sdpa_probs_gqa", B, H, Hkv, Tq, Tkv, hd)) return;
    if ((int64_t)B * Tq == 0) return;
    if (!q || !k || !P) { ncm_fail(NCM_E_ARG, "sdpa_probs_gqa: null pointer"); return; }
    if (ncm_ready()) return;
    float scale = 1.0f / sqrtf((float)hd);
    if (mfma_path(hd, Tkv, q, k, P, P, P)) {
        void *a[] = {&q, &k, &mask, &P, &H, &Hkv, &Tq, &Tkv, &scale};
        ncm_launch_named("sdpa_probs_hd64", blocks_of(Tq, 64), (unsigned)H, (unsigned)B, 256, a);
    } else {
        void *a[] = {&q, &k, &mask, &P, &B, &H, &Hkv, &Tq, &Tkv, &hd, &scale};
        ncm_launch_named("sdpa_probs_rows", blocks_of((int64_t)B * H * Tq, 4), 1, 1, 256, a);
    }
}

void sdpa_bwd_gqa(const float *q, const float *k, const float *v, const float *P, const float *dO, float *dq,
                  float *dk, float *dv, int B, int H, int Hkv, int Tq, int Tkv, int hd) {
    if (attn_check("sdpa_bwd_gqa", B, H, Hkv, Tq, Tkv, hd)) return;
    if ((int64_t)B * Tq == 0 || (!dq && !dk && !dv)) return;
    if (!q || !k || !v || !P || !dO) { ncm_fail(NCM_E_ARG, "sdpa_bwd_gqa: null input"); return; }
    if (ncm_ready()) return;
    const int64_t rows = (int64_t)B * H * Tq;
    float *D = (float *)ncm_workspace(WS_TRAIN, (size_t)rows * sizeof(float));
    if (!D) return;
    float scale = 1.0f / sqrtf((float)hd);
    const int want_kv = dk || dv;
    float *Dout = want_kv ? D : NULL;
    if (mfma_path(hd, Tkv, q, k, v, P, dO) && (!dq || is_aligned16(dq)) && (!dk || is_aligned16(dk)) &&
        (!dv || is_aligned16(dv))) {
        void *a[] = {&k, &v, &P, &dO, &dq, &Dout, &H, &Hkv, &Tq, &Tkv, &scale};
        if (ncm_launch_named("sdpa_bwd_dq_hd64", blocks_of(Tq, 64), (unsigned)H, (unsigned)B, 256, a)) return;
        if (!want_kv) return;
        void *a2[] = {&q, &v, &P, &dO, &D, &dk, &dv, &H, &Hkv, &Tq, &Tkv, &scale};
        ncm_launch_named("sdpa_bwd_dkdv_hd64", blocks_of(Tkv, 64), (unsigned)Hkv, (unsigned)B, 256, a2);
    } else {
        void *a[] = {&k, &v, &P, &dO, &dq, &Dout, &B, &H, &Hkv, &Tq, &Tkv, &hd, &scale};
        if (ncm_launch_named("sdpa_bwd_dq_rows", blocks_of(rows, 4), 1, 1, 256, a)) return;
        if (!want_kv) return;
        void *a2[] = {&q, &v, &P, &dO, &D, &dk, &dv, &B, &H, &Hkv, &Tq, &Tkv, &hd, &scale};
        ncm_launch_named("sdpa_bwd_dkdv_rows", blocks_of((int64_t)B * Hkv * Tkv, 4), 1, 1, 256, a2);
    }
}

/* The recomputing backward of the tape's SDPA records (hd 64, aligned): D =
 * rowsum(dO o O), then the dq and dk/dv kernels rebuild P tile by tile from
 * the forward's row statistics.  Gradients accumulate. */
/* ldo 0: dq, dk, dv as [B][heads][T][hd]; ldo > 0: rows (b, t) of stride ldo
 * floats with head h at column h hd (the layout of the q | k | v rows).
 * o_ld 0: o as [B][H][Tq][hd]; o_ld > 0: o with the heads merged, rows of
 * stride o_ld. */
static void sdpa_bwd_flash_any(const float *q, const float *k, const float *v, const float *o, const float *stats,
                               const float *mask, int causal, const float *dO, float *dq, float *dk, float *dv, int B,
                               int H, int Hkv, int Tq, int Tkv, int hd, int beta, int ldo, int o_ld) {
    if (attn_check("ncm_sdpa_bwd_flash", B, H, Hkv, Tq, Tkv, hd)) return;
    if ((int64_t)B * Tq == 0 || (!dq && !dk && !dv)) return;
    if (hd != 64 || !q || !k || !v || !o || !stats || !dO) {
        ncm_fail(NCM_E_ARG, "ncm_sdpa_bwd_flash: hd %d (64 only) or null input", hd);
        return;
    }
    if (causal && Tq > Tkv) {
        ncm_fail(NCM_E_ARG, "ncm_sdpa_bwd_flash: causal attention needs Tq <= Tkv");
        return;
    }
    if ((Tq + 63) / 64 > 65535 || (Tkv + 63) / 64 > 65535) {   /* tiles are the grid's z dimension */
        ncm_fail(NCM_E_ARG, "ncm_sdpa_bwd_flash: grid too large");
        return;
    }
    if (ncm_ready()) return;
    const int64_t rows = (int64_t)B * H * Tq;
    float *D = (float *)ncm_workspace(WS_TRAIN, (size_t)rows * sizeof(float));
    if (!D) return;
    float scale = 1.0f / sqrtf((float)hd);
    void *a0[] = {&dO, &o, &D, (void *)&rows, &hd, &H, &Tq, &o_ld};
    if (ncm_launch_named("sdpa_bwd_rowdot", blocks_of(rows, 4), 1, 1, 256, a0)) return;
    if (dq) {
        void *a[] = {&q, &k, &v, &mask, &stats, &D, &dO, &dq, &H, &Hkv, &Tq, &Tkv, &scale, &causal, &beta, &ldo};
        if (ncm_launch_named("sdpa_fbwd_dq_hd64", (unsigned)H, (unsigned)B, blocks_of(Tq, 64), 256, a)) return;
    }
    if (dk || dv) {
        void *a[] = {&q, &k, &v, &mask, &stats, &D, &dO, &dk, &dv, &H, &Hkv, &Tq, &Tkv, &scale, &causal, &beta,
                     &ldo};
        ncm_launch_named("sdpa_fbwd_dkdv_hd64", (unsigned)Hkv, (unsigned)B, blocks_of(Tkv, 64), 256, a);
    }
}

void ncm_sdpa_bwd_flash(const float *q, const float *k, const float *v, const float *o, const float *stats,
                        const float *mask, int causal, const float *dO, float *dq, float *dk, float *dv, int B, int H,
                        int Hkv, int Tq, int Tkv, int hd) {
    sdpa_bwd_flash_any(q, k, v, o, stats, mask, causal, dO, dq, dk, dv, B, H, Hkv, Tq, Tkv, hd, 1, 0, 0);
}

/* beta 0: dq, dk and dv are written (every element has one writer in the
 * kernels) instead of accumulated. */
void ncm_sdpa_bwd_flash_ex(const float *q, const float *k, const float *v, const float *o, const float *stats,
                           const float *mask, int causal, const float *dO, float *dq, float *dk, float *dv, int B,
                           int H, int Hkv, int Tq, int Tkv, int hd, int beta, int o_ld) {
    sdpa_bwd_flash_any(q, k, v, o, stats, mask, causal, dO, dq, dk, dv, B, H, Hkv, Tq, Tkv, hd, beta, 0, o_ld);
}

void ncm_sdpa_bwd_flash_rows(const float *q, const float *k, const float *v, const float *o, const float *stats,
                             const float *mask, int causal, const float *dO, float *dqkv, int B, int H, int Hkv,
                             int Tq, int Tkv, int hd, int beta, int o_ld) {
    const int64_t ld = (int64_t)(H + 2 * Hkv) * hd;
    if (Tq != Tkv || ld > INT_MAX || !dqkv) {
        ncm_fail(NCM_E_ARG, "ncm_sdpa_bwd_flash_rows: needs Tq == Tkv and a gradient buffer");
        return;
    }
    float *dq = dqkv, *dk = dqkv + (int64_t)H * hd, *dv = dk + (int64_t)Hkv * hd;
    sdpa_bwd_flash_any(q, k, v, o, stats, mask, causal, dO, dq, dk, dv, B, H, Hkv, Tq, Tkv, hd, beta, (int)ld, o_ld);
}

/* ---- optimizer (train.c:51-64, 102-145, 172-178; train_gpt2.c:160-173) ---- */
static void adamw_any(float *p, float *g, float *m, float *v, int64_t n, double lr, double b1, double b2,
                      double b1t, double b2t, double eps, double wd, int clear_g) {
    if (n < 0 || (n + 255) / 256 > UINT_MAX) { ncm_fail(NCM_E_ARG, "adamw_update: bad size"); return; }
    if (n == 0) return;
    if (!p || !g || !m || !v) { ncm_fail(NCM_E_ARG, "adamw_update: null pointer"); return; }
    if (ncm_ready()) return;
    void *a[] = {&p, &g, &m, &v, &n, &lr, &b1, &b2, &b1t, &b2t, &eps, &wd, &clear_g};
    ncm_launch_named("adamw_k", blocks_of(n, 256), 1, 1, 256, a);
}

void adamw_update(float *p, const float *g, float *m, float *v, int64_t n, double lr, double b1, double b2,
                  double b1t, double b2t, double eps, double wd) {
    adamw_any(p, (float *)g, m, v, n, lr, b1, b2, b1t, b2t, eps, wd, 0);   /* g is only read */
}

void ncm_adamw_update_clear(float *p, float *g, float *m, float *v, int64_t n, double lr, double b1, double b2,
                            double b1t, double b2t, double eps, double wd) {
    adamw_any(p, g, m, v, n, lr, b1, b2, b1t, b2t, eps, wd, 1);
}

double sched_cosine_warmup(long step, double warmup, double total) {
    double w = warmup, T = total;
    if (step < w) return step / (w > 0 ? w : 1);
    if (step >= T) return 0.0;
    double x = (step - w) / (T - w);
    return 0.5 * (1 + cos(3.141592653589793 * x));
}

/* ---------------------------------------------------------------- AdamW object
 * train.c:15-159 of the reference with the moments and gradient accumulators
 * on the device (so adamw_step launches adamw_update per tensor and nothing
 * crosses PCIe).  Every buffer of one tensor is allocated before the next. */
void adamw_free(AdamW *o) {
    if (!o) return;
    for (int i = 0; i < o->n; i++) {
        ncm_hip_free(o->m[i]);
        ncm_hip_free(o->v[i]);
        ncm_hip_free(o->g[i]);
    }
    free(o->params);
    free(o->m);
    free(o->v);
    free(o->g);
    free(o->sizes);
    free(o->lr);
    free(o);
}

AdamW *adamw_new(WeightStore *ws, const int *frozen) {
    if (!ws || ws->count < 0) return ncm_fail(NCM_E_ARG, "adamw_new: bad store"), NULL;
    if (ncm_ready()) return NULL;
    AdamW *o = (AdamW *)calloc(1, sizeof *o);
    size_t cap = (size_t)ws->count + 1;
    if (o) {
        o->params = (float **)calloc(cap, sizeof(float *));
        o->m = (float **)calloc(cap, sizeof(float *));
        o->v = (float **)calloc(cap, sizeof(float *));
        o->g = (float **)calloc(cap, sizeof(float *));
        o->sizes = (int64_t *)calloc(cap, sizeof(int64_t));
        o->lr = (double *)calloc(cap, sizeof(double));
    }
    if (!o || !o->params || !o->m || !o->v || !o->g || !o->sizes || !o->lr) {
        adamw_free(o);
        return ncm_fail(NCM_E_OOM, "adamw_new: out of memory"), NULL;
    }
    o->b1 = 0.9;
    o->b2 = 0.95;
    o->eps = 1e-8;
    o->wd = 0.01;
    for (int i = 0; i < ws->count; i++) {
        if (frozen && frozen[i]) continue;
        const Tensor *t = ws->items[i].t;
        size_t bytes = (size_t)t->n * sizeof(float);
        int k = o->n;
        o->params[k] = t->data;
        o->sizes[k] = t->n;
        o->lr[k] = 1.0;
        o->m[k] = (float *)ncm_hip_malloc(bytes);
        o->v[k] = (float *)ncm_hip_malloc(bytes);
        o->g[k] = (float *)ncm_hip_malloc(bytes);
        o->n++; /* counted before the check, so adamw_free releases a partial tensor */
        if (!o->m[k] || !o->v[k] || !o->g[k]) {
            adamw_free(o);
            return NULL;
        }
        if (ncm_zero_async(o->m[k], bytes) || ncm_zero_async(o->v[k], bytes) || ncm_zero_async(o->g[k], bytes)) {
            adamw_free(o);
            return NULL;
        }
    }
    return o;
}

void adamw_zero_grad(AdamW *o) {
    if (!o || ncm_ready()) return;
    for (int i = 0; i < o->n; i++)
        if (ncm_zero_async(o->g[i], (size_t)o->sizes[i] * sizeof(float))) return;
}

void adamw_step(AdamW *o, double base_lr, double warmup, double total) {
    if (!o) return;
    o->step++;
    const double lr_t = base_lr * sched_cosine_warmup(o->step, warmup, total);
    const double b1t = 1.0 - pow(o->b1, (double)o->step), b2t = 1.0 - pow(o->b2, (double)o->step);
    for (int i = 0; i < o->n; i++)
        adamw_update(o->params[i], o->g[i], o->m[i], o->v[i], o->sizes[i], lr_t * o->lr[i], o->b1, o->b2, b1t, b2t,
                     o->eps, o->wd);
}

void adamw_sync_to_host(AdamW *o) { (void)o; }

#define CLIP_MAX_BLOCKS 1024

double grad_clip_global(float *const *grads, const int64_t *sizes, int count, double max_norm) {
    if (count < 0 || (count > 0 && (!grads || !sizes))) {
        ncm_fail(NCM_E_ARG, "grad_clip_global: bad arguments");
        return -1.0;
    }
    if (ncm_ready()) return -1.0;
    int64_t nparts = 0;
    for (int i = 0; i < count; i++) {
        if (sizes[i] < 0 || (sizes[i] > 0 && !grads[i])) {
            ncm_fail(NCM_E_ARG, "grad_clip_global: tensor %d", i);
            return -1.0;
        }
        int64_t b = (sizes[i] + 255) / 256;
        nparts += b < CLIP_MAX_BLOCKS ? b : CLIP_MAX_BLOCKS;
    }
    if (nparts > INT_MAX - 1) { ncm_fail(NCM_E_ARG, "grad_clip_global: too many tensors"); return -1.0; }
    double *ws = (double *)ncm_workspace(WS_TRAIN, (size_t)(nparts + 1) * sizeof(double));
    if (!ws) return -1.0;
    double *part = ws, *total = ws + nparts;
    int64_t off = 0;
    for (int i = 0; i < count; i++) {
        if (sizes[i] == 0) continue;
        int64_t b = (sizes[i] + 255) / 256;
        unsigned nb = (unsigned)(b < CLIP_MAX_BLOCKS ? b : CLIP_MAX_BLOCKS);
        double *pp = part + off;
        const float *g = grads[i];
        int64_t n = sizes[i];
        void *a[] = {&g, &n, &pp};
        if (ncm_launch_named("sumsq_partial", nb, 1, 1, 256, a)) return -1.0;
        off += nb;
    }
    int np = (int)off;
    void *a2[] = {&part, &np, &total};
    if (ncm_launch_named("sumsq_final", 1, 1, 1, 64, a2)) return -1.0;
    double g2 = 0.0;
    mem_d2h(&g2, total, sizeof(double));
    double gnorm = sqrt(g2);
    if (gnorm > max_norm) {
        float s = (float)(1.0 / gnorm);
        for (int i = 0; i < count; i++) {
            if (sizes[i] == 0) continue;
            float *g = grads[i];
            int64_t n = sizes[i];
            void *a[] = {&g, &n, &s};
            if (ncm_launch_named("scale_inplace_k", blocks_of(n, 256), 1, 1, 256, a)) return -1.0;
        }
    }
    return gnorm;
}

/* ---- clip + AdamW over a tensor list in three launches (multi-tensor) ----
 * grad_clip_global followed by ncm_adamw_update_clear on every tensor, with
 * no host synchronisation in between: sumsq_multi (the same per-tensor
 * partials as sumsq_partial), clip_final (the norm and the clip scale on the
 * device) and adamw_multi (the gradient times the scale, the adamw_k update,
 * the gradient cleared).  The tensor tables live on the device and are
 * rebuilt only when the list (pointers, sizes, multipliers) changes. */
typedef struct {   /* must match struct MtTensor in train.hip */
    float *p, *g, *m, *v;
    int64_t n;
    double lr_mul;
} MtTensor;
#define MT_MAX 2048       /* tensors per list (the kernels' LDS table) */
#define MT_CHUNK 16384    /* elements per adamw_multi workgroup */

static struct {
    int count, nparts, nchunks;
    MtTensor *tt;         /* host copy of the device table */
    char *dev;            /* tt | boff | chunks | partials | g2 | scale */
    size_t bytes;
} g_mt;

static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

/* Device tables for the list; returns 0, or -1 when the list does not fit
 * (the caller then takes the per-tensor path). */
static int mt_prepare(float *const *P, float *const *G, float *const *M, float *const *V, const int64_t *sizes,
                      const double *lr_mul, int count) {
    if (count < 1 || count > MT_MAX) return -1;
    MtTensor *tt = (MtTensor *)malloc((size_t)count * sizeof(MtTensor));
    int *boff = (int *)malloc((size_t)(count + 1) * sizeof(int));
    if (!tt || !boff) { free(tt); free(boff); return -1; }
    int64_t nparts = 0, nchunks = 0;
    for (int i = 0; i < count; i++) {
        tt[i].p = P[i]; tt[i].g = G[i]; tt[i].m = M[i]; tt[i].v = V[i];
        tt[i].n = sizes[i];
        tt[i].lr_mul = lr_mul ? lr_mul[i] : 1.0;
        boff[i] = (int)nparts;
        if (sizes[i] > 0) {
            const int64_t b = (sizes[i] + 255) / 256;
            nparts += b < CLIP_MAX_BLOCKS ? b : CLIP_MAX_BLOCKS;
            nchunks += (sizes[i] + MT_CHUNK - 1) / MT_CHUNK;
        }
    }
    boff[count] = (int)nparts;
    if (nparts == 0 || nparts > INT_MAX / 2 || nchunks > INT_MAX / 2) { free(tt); free(boff); return -1; }
    if (g_mt.dev && g_mt.count == count && memcmp(g_mt.tt, tt, (size_t)count * sizeof(MtTensor)) == 0) {
        free(tt);
        free(boff);
        return 0;
    }
    const size_t b_tt = al256((size_t)count * sizeof(MtTensor)), b_bo = al256((size_t)(count + 1) * sizeof(int)),
                 b_ch = al256((size_t)nchunks * 2 * sizeof(int)), b_pa = al256((size_t)nparts * sizeof(double));
    const size_t bytes = b_tt + b_bo + b_ch + b_pa + 256 + 256;
    int *ch = (int *)malloc((size_t)nchunks * 2 * sizeof(int));
    if (!ch) { free(tt); free(boff); return -1; }
    int64_t c = 0;
    for (int i = 0; i < count; i++)
        for (int64_t k = 0; sizes[i] > 0 && k < (sizes[i] + MT_CHUNK - 1) / MT_CHUNK; k++) {
            ch[2 * c] = i;
            ch[2 * c + 1] = (int)k;
            c++;
        }
    if (g_mt.bytes < bytes) {
        if (g_mt.dev) { ncm_hip_sync(); ncm_hip_free(g_mt.dev); }
        g_mt.dev = (char *)ncm_hip_malloc(bytes);
        g_mt.bytes = g_mt.dev ? bytes : 0;
    }
    int rc = -1;
    if (g_mt.dev) {
        mem_h2d(g_mt.dev, tt, (size_t)count * sizeof(MtTensor));
        mem_h2d(g_mt.dev + b_tt, boff, (size_t)(count + 1) * sizeof(int));
        mem_h2d(g_mt.dev + b_tt + b_bo, ch, (size_t)nchunks * 2 * sizeof(int));
        free(g_mt.tt);
        g_mt.tt = tt;
        tt = NULL;
        g_mt.count = count;
        g_mt.nparts = (int)nparts;
        g_mt.nchunks = (int)nchunks;
        rc = ncm_ready() ? -1 : 0;
    }
    free(tt);
    free(boff);
    free(ch);
    return rc;
}

/* Launches the clip and the update; *g2_dev gets the device address of the
 * sum of squares of the gradients (before clipping). */
static int mt_clip_adamw(double max_norm, double lr, double b1, double b2, double b1t, double b2t, double eps,
                         double wd, int clear_g, const double **g2_dev) {
    const int count = g_mt.count;
    const size_t b_tt = al256((size_t)count * sizeof(MtTensor)), b_bo = al256((size_t)(count + 1) * sizeof(int)),
                 b_ch = al256((size_t)g_mt.nchunks * 2 * sizeof(int)), b_pa = al256((size_t)g_mt.nparts * sizeof(double));
    const MtTensor *tt = (const MtTensor *)g_mt.dev;
    const int *boff = (const int *)(g_mt.dev + b_tt), *chs = (const int *)(g_mt.dev + b_tt + b_bo);
    double *part = (double *)(g_mt.dev + b_tt + b_bo + b_ch), *g2 = (double *)(g_mt.dev + b_tt + b_bo + b_ch + b_pa);
    float *scale = (float *)(g_mt.dev + b_tt + b_bo + b_ch + b_pa + 256);
    int np = g_mt.nparts, len = MT_CHUNK;
    void *a1[] = {&tt, &boff, (void *)&count, &part};
    if (ncm_launch_named("sumsq_multi", (unsigned)np, 1, 1, 256, a1)) return -1;
    void *a2[] = {&part, &np, &g2, &scale, &max_norm};
    if (ncm_launch_named("clip_final", 1, 1, 1, 64, a2)) return -1;
    void *a3[] = {&tt, &chs, &len, &scale, &lr, &b1, &b2, &b1t, &b2t, &eps, &wd, &clear_g};
    if (ncm_launch_named("adamw_multi", (unsigned)g_mt.nchunks, 1, 1, 256, a3)) return -1;
    *g2_dev = g2;
    return 0;
}

int ncm_clip_adamw_multi(float *const *P, float *const *G, float *const *M, float *const *V, const int64_t *sizes,
                         int count, double max_norm, double lr, double b1, double b2, double b1t, double b2t,
                         double eps, double wd, int clear_g, const double **g2_dev) {
    if (ncm_ready()) return -1;
    if (mt_prepare(P, G, M, V, sizes, NULL, count)) return -1;
    return mt_clip_adamw(max_norm, lr, b1, b2, b1t, b2t, eps, wd, clear_g, g2_dev);
}

/* ---- remaining tape backward cases ---- */
static int elt_check(const char *fn, int64_t n, const void *a, const void *b) {
    if (n < 0 || (n + 255) / 256 > UINT_MAX) return ncm_fail(NCM_E_ARG, "%s: bad size", fn);
    if (n == 0) return 1;
    if (!a || !b) return ncm_fail(NCM_E_ARG, "%s: null pointer", fn);
    return ncm_ready();
}

static void act_bwd(const char *fn, const float *x, const float *dy, float *dx, int64_t n, int kind, int beta) {
    if (elt_check(fn, n, x, dy) || !dx) return;
    if (n % 4 == 0 && (((uintptr_t)x | (uintptr_t)dy | (uintptr_t)dx) & 15) == 0) {
        int64_t n4 = n / 4;
        void *a[] = {&x, &dy, &dx, &n4, &kind, &beta};
        ncm_launch_named("act_bwd4_k", blocks_of(n4, 256), 1, 1, 256, a);
        return;
    }
    if (!beta && ncm_zero_async(dx, (size_t)n * sizeof(float))) return;
    void *a[] = {&x, &dy, &dx, &n, &kind};
    ncm_launch_named("act_bwd_k", blocks_of(n, 256), 1, 1, 256, a);
}
void gelu_bwd(const float *x, const float *dy, float *dx, int64_t n) { act_bwd("gelu_bwd", x, dy, dx, n, 0, 1); }
void silu_bwd(const float *x, const float *dy, float *dx, int64_t n) { act_bwd("silu_bwd", x, dy, dx, n, 1, 1); }
void gelu_tanh_bwd(const float *x, const float *dy, float *dx, int64_t n) {
    act_bwd("gelu_tanh_bwd", x, dy, dx, n, 2, 1);
}
void ncm_act_bwd_ex(int kind, const float *x, const float *dy, float *dx, int64_t n, int beta) {
    static const char *const fn[3] = {"gelu_bwd", "silu_bwd", "gelu_tanh_bwd"};
    const int k = kind == 0 || kind == 1 ? kind : 2;   /* the tape's act codes: 0 gelu, 1 silu, else gelu_tanh */
    act_bwd(fn[k], x, dy, dx, n, k, beta);
}

void mul_bwd(const float *a, const float *b, const float *dy, float *da, float *db, int64_t n) {
    if (elt_check("mul_bwd", n, a, b) || (!da && !db)) return;
    if (!dy) { ncm_fail(NCM_E_ARG, "mul_bwd: null dy"); return; }
    void *args[] = {&a, &b, &dy, &da, &db, &n};
    ncm_launch_named("mul_bwd_k", blocks_of(n, 256), 1, 1, 256, args);
}

void rope_bwd_gqa(const float *gq, const float *gk, const float *cos_t, const float *sin_t, float *dxq, float *dxk,
                  int B, int H, int Hkv, int T, int hd) {
    if (B < 0 || H < 0 || Hkv < 0 || T <= 0 || hd <= 0 || (hd & 1)) {
        ncm_fail(NCM_E_ARG, "rope_bwd_gqa: bad shape");
        return;
    }
    if (!cos_t || !sin_t) { ncm_fail(NCM_E_ARG, "rope_bwd_gqa: null tables"); return; }
    if (ncm_ready()) return;
    const float *g[2] = {gq, gk};
    float *d[2] = {dxq, dxk};
    int64_t rows[2] = {(int64_t)B * H * T, (int64_t)B * Hkv * T};
    for (int i = 0; i < 2; i++) {
        if (!g[i] || !d[i] || rows[i] == 0) continue;
        int64_t n = rows[i] * (hd / 2);
        void *a[] = {&d[i], &g[i], &cos_t, &sin_t, &rows[i], &T, &hd};
        if (ncm_launch_named("rope_bwd_k", blocks_of(n, 256), 1, 1, 256, a)) return;
    }
}

void embedding_bwd(const float *dy, const int *idx, int64_t n, int D, float *dW, int V) {
    if (n < 0 || D <= 0 || V <= 0 || n > INT_MAX) { ncm_fail(NCM_E_ARG, "embedding_bwd: bad shape"); return; }
    if (n == 0) return;
    if (!dy || !idx || !dW) { ncm_fail(NCM_E_ARG, "embedding_bwd: null pointer"); return; }
    if (ncm_ready()) return;
    /* group the rows by id (counting sort, rows ascending within an id) */
    int *cnt = (int *)calloc((size_t)V + 1, sizeof(int));
    int *host = (int *)malloc(((size_t)n * 2 + (size_t)V + 2) * sizeof(int));
    if (!cnt || !host) {
        free(cnt);
        free(host);
        ncm_fail(NCM_E_OOM, "embedding_bwd: host allocation");
        return;
    }
    for (int64_t i = 0; i < n; i++)
        if (idx[i] >= 0 && idx[i] < V) cnt[idx[i]]++;
    int *uid = host, nu = 0;
    for (int v = 0; v < V; v++)
        if (cnt[v]) uid[nu++] = v;
    int *off = uid + nu, *rowlist = off + nu + 1;
    int *pos = (int *)malloc((size_t)V * sizeof(int));
    if (!pos) {
        free(cnt);
        free(host);
        ncm_fail(NCM_E_OOM, "embedding_bwd: host allocation");
        return;
    }
    off[0] = 0;
    for (int u = 0; u < nu; u++) {
        pos[uid[u]] = off[u];
        off[u + 1] = off[u] + cnt[uid[u]];
    }
    for (int64_t i = 0; i < n; i++)
        if (idx[i] >= 0 && idx[i] < V) rowlist[pos[idx[i]]++] = (int)i;
    int total = nu + (nu + 1) + off[nu];
    free(pos);
    free(cnt);
    if (nu == 0 || nu > 65535 * 64) {
        free(host);
        if (nu) ncm_fail(NCM_E_ARG, "embedding_bwd: too many distinct ids");
        return;
    }
    int *dev = (int *)ncm_workspace(WS_TRAIN, (size_t)total * sizeof(int));
    if (!dev) { free(host); return; }
    mem_h2d(dev, host, (size_t)total * sizeof(int));
    free(host);
    const int *duid = dev, *doff = dev + nu, *drow = dev + nu + nu + 1;
    for (int u0 = 0; u0 < nu; u0 += 65535) {
        int cntu = nu - u0 < 65535 ? nu - u0 : 65535;
        const int *pu = duid + u0, *po = doff + u0;
        void *a[] = {&dy, &pu, &po, &drow, &dW, &D};
        if (ncm_launch_named("emb_bwd_k", blocks_of(D, 256), (unsigned)cntu, 1, 256, a)) return;
    }
}

/* beta 0: dx is fresh (not cleared): the row kernel writes it when every
 * element has a source (q, k and v gradients, C == H hd); otherwise it is
 * cleared first and accumulated. */
static void qkv_split_bwd_any(const float *gq, const float *gk, const float *gv, float *dx, int B, int T, int C,
                              int H, int hd, int K, int rep, int beta) {
    if (B < 0 || T < 0 || C < 0 || H <= 0 || hd <= 0 || K <= 0 || rep <= 0 || (H - 1) / rep >= K ||
        (int64_t)H * hd > C) {
        ncm_fail(NCM_E_ARG, "qkv_split_bwd: bad shape");
        return;
    }
    int64_t n = (int64_t)B * T * ((int64_t)C + 2 * K * hd);
    if (elt_check("qkv_split_bwd", n, dx, dx)) return;
    const int rows_path = hd % 4 == 0 && C % 4 == 0 && (int64_t)B * T <= INT_MAX &&
                          (int64_t)C + 2 * K * hd <= INT_MAX && is_aligned16(gq) && is_aligned16(gk) &&
                          is_aligned16(gv) && is_aligned16(dx);
    if (!beta && !(rows_path && gq && gk && gv && C == H * hd)) {
        if (ncm_zero_async(dx, (size_t)n * sizeof(float))) return;
        beta = 1;
    }
    if (!gq && !gk && !gv) return;
    if (rows_path) {
        void *a[] = {&gq, &gk, &gv, &dx, &T, &C, &H, &hd, &K, &rep, &beta};
        ncm_launch_named("qkv_split_bwd_rows_k", (unsigned)((int64_t)B * T), 1, 1, 256, a);
        return;
    }
    void *a[] = {&gq, &gk, &gv, &dx, &B, &T, &C, &H, &hd, &K, &rep};
    ncm_launch_named("qkv_split_bwd_k", blocks_of(n, 256), 1, 1, 256, a);
}

void qkv_split_bwd(const float *gq, const float *gk, const float *gv, float *dx, int B, int T, int C, int H, int hd,
                   int K, int rep) {
    qkv_split_bwd_any(gq, gk, gv, dx, B, T, C, H, hd, K, rep, 1);
}

void ncm_qkv_split_bwd_ex(const float *gq, const float *gk, const float *gv, float *dx, int B, int T, int C, int H,
                          int hd, int K, int rep, int beta) {
    qkv_split_bwd_any(gq, gk, gv, dx, B, T, C, H, hd, K, rep, beta);
}

/* beta 0: dx is fresh; the row kernel writes every element when the rows are
 * whole heads (C == H hd), otherwise dx is cleared first. */
static void heads_bwd(const char *fn, const float *dy, float *dx, int B, int T, int C, int H, int hd, int dir,
                      int beta) {
    if (B < 0 || T < 0 || C < 0 || H <= 0 || hd <= 0 || C > (int64_t)H * hd) {
        ncm_fail(NCM_E_ARG, "%s: bad shape", fn);
        return;
    }
    int64_t n = dir == 0 ? (int64_t)B * H * T * hd : (int64_t)B * T * C;
    if (elt_check(fn, n, dy, dx)) return;
    const int rows_path = hd % 4 == 0 && C % 4 == 0 && (int64_t)B * T <= INT_MAX && is_aligned16(dy) &&
                          is_aligned16(dx);
    if (!beta && !(rows_path && (dir == 1 || C == H * hd))) {
        if (ncm_zero_async(dx, (size_t)n * sizeof(float))) return;
        beta = 1;
    }
    if (rows_path) {
        void *a[] = {&dy, &dx, &T, &C, &H, &hd, &dir, &beta};
        ncm_launch_named("heads_bwd_rows_k", (unsigned)((int64_t)B * T), 1, 1, 256, a);
        return;
    }
    void *a[] = {&dy, &dx, &B, &T, &C, &H, &hd, &dir};
    ncm_launch_named("heads_bwd_k", blocks_of(n, 256), 1, 1, 256, a);
}

void head_merge_bwd(const float *dy, float *dctx, int B, int T, int C, int H, int hd) {
    heads_bwd("head_merge_bwd", dy, dctx, B, T, C, H, hd, 0, 1);
}

void heads_transpose_bwd(const float *dy, float *dx, int B, int T, int C, int H, int hd) {
    heads_bwd("heads_transpose_bwd", dy, dx, B, T, C, H, hd, 1, 1);
}

void ncm_heads_bwd_ex(const float *dy, float *dx, int B, int T, int C, int H, int hd, int dir, int beta) {
    heads_bwd(dir == 0 ? "head_merge_bwd" : "heads_transpose_bwd", dy, dx, B, T, C, H, hd, dir, beta);
}
