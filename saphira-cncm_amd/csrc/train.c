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

#define NORM_ROWS 128

static unsigned blocks_of(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

static int shape_ok(const char *fn, int64_t rows, int C) {
    if (rows < 0 || C <= 0 || (rows + 3) / 4 > UINT_MAX)
        return ncm_fail(NCM_E_ARG, "%s: bad shape rows=%lld C=%d", fn, (long long)rows, C);
    return 0;
}

/* ---- LayerNorm / RMSNorm backward (train_tape.c:569-634, 748-792) ---- */
static void norm_bwd(const char *fn, int kind, const float *x, const float *w, const float *dy, float *dx,
                     float *dw, float *db, int64_t rows, int C, double eps) {
    if (shape_ok(fn, rows, C)) return;
    if (rows == 0) return;
    if (!x || !dy) { ncm_fail(NCM_E_ARG, "%s: null input", fn); return; }
    if (ncm_ready()) return;
    const int chunks = (int)((rows + NORM_ROWS - 1) / NORM_ROWS);
    const int want_param = dw || db;
    if (chunks > 65535 && want_param) { ncm_fail(NCM_E_ARG, "%s: too many rows", fn); return; }
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
    norm_bwd("layernorm_bwd", 0, x, w, dy, dx, dw, db, rows, C, eps);
}

void rmsnorm_bwd(const float *x, const float *w, const float *dy, float *dx, float *dw, int64_t rows, int C) {
    norm_bwd("rmsnorm_bwd", 1, x, w, dy, dx, dw, NULL, rows, C, 1e-6);
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

/* ---- optimizer (train.c:51-64, 102-145, 172-178; train_gpt2.c:160-173) ---- */
void adamw_update(float *p, const float *g, float *m, float *v, int64_t n, double lr, double b1, double b2,
                  double b1t, double b2t, double eps, double wd) {
    if (n < 0 || (n + 255) / 256 > UINT_MAX) { ncm_fail(NCM_E_ARG, "adamw_update: bad size"); return; }
    if (n == 0) return;
    if (!p || !g || !m || !v) { ncm_fail(NCM_E_ARG, "adamw_update: null pointer"); return; }
    if (ncm_ready()) return;
    void *a[] = {&p, &g, &m, &v, &n, &lr, &b1, &b2, &b1t, &b2t, &eps, &wd};
    ncm_launch_named("adamw_k", blocks_of(n, 256), 1, 1, 256, a);
}

double sched_cosine_warmup(long step, double warmup, double total) {
    double w = warmup, T = total;
    if (step < w) return step / (w > 0 ? w : 1);
    if (step >= T) return 0.0;
    double x = (step - w) / (T - w);
    return 0.5 * (1 + cos(3.141592653589793 * x));
}

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
