/* tape.c -- a device-resident autodiff tape for the hot-path ops.
 *
 * Mirrors the reference's Tape (train_tape.c:19-162, 277-481, 636-1051):
 * every recorder runs the forward on the device and appends a record with
 * the same fields as TopRec (op kind, input/output pointers, dims, scalar);
 * ncm_tape_backward walks the records in reverse, looks the upstream
 * gradient up by output pointer and accumulates input gradients, creating
 * zeroed buffers on first use (the reference's GMap) and writing parameter
 * gradients straight into the caller's buffers (PMap aliases).
 *
 * Differences that keep everything on the device: the SDPA record stores P
 * computed by a kernel (the reference computes it on the host); the CE
 * record computes loss and dlogits together at record time (its backward
 * only depends on the logits and targets), so the probabilities are never
 * stored; no host staging anywhere except the embedding ids, which the
 * reference also keeps on the host.
 *
 * Memory: records and gradients live in two device pools of 256 MiB chunks
 * that grow on demand and are reused after ncm_tape_clear. */
#include "internal.h"

#include <stdlib.h>
#include <string.h>

#define POOL_CHUNK ((size_t)256 << 20)

typedef struct {
    char **chunk;
    size_t *size;
    int n, cap, cur;
    size_t off;
    /* zeroing pools (the gradient pool): per chunk, the extent cleared since
     * the last reset and the largest extent used by an earlier cycle.  The
     * first allocation in a chunk clears that earlier extent with one memset,
     * so a step's gradient buffers cost one clear per chunk, not one each. */
    int zeroing;
    size_t *zeroed, *high;
} Pool;

/* Zeroing pools: makes [0, p->off) of the current chunk zero.  This
 * cycle's allocations are contiguous from 0 and [0, zeroed) was cleared after
 * the last reset and, past p->off before this allocation, not handed out
 * since, so clearing [zeroed, max(off, high)) suffices. */
static int pool_zero(Pool *p) {
    const int c = p->cur;
    if (p->off <= p->zeroed[c]) return 0;
    const size_t to = p->off > p->high[c] ? p->off : p->high[c];
    if (ncm_zero_async(p->chunk[c] + p->zeroed[c], to - p->zeroed[c])) return -1;
    p->zeroed[c] = to;
    return 0;
}

static void *pool_alloc(Pool *p, size_t bytes) {
    bytes = (bytes + 255) & ~(size_t)255;
    if (bytes == 0) bytes = 256;
    while (p->cur < p->n) {
        if (p->off + bytes <= p->size[p->cur]) {
            void *r = p->chunk[p->cur] + p->off;
            p->off += bytes;
            if (p->zeroing && pool_zero(p)) return NULL;
            return r;
        }
        p->cur++;
        p->off = 0;
    }
    if (p->n == p->cap) {
        int cap = p->cap ? 2 * p->cap : 8;
        char **c = (char **)realloc(p->chunk, (size_t)cap * sizeof(char *));
        if (!c) return NULL;
        p->chunk = c;
        size_t *s = (size_t *)realloc(p->size, (size_t)cap * sizeof(size_t));
        if (!s) return NULL;
        p->size = s;
        size_t *z = (size_t *)realloc(p->zeroed, (size_t)cap * sizeof(size_t));
        if (!z) return NULL;
        p->zeroed = z;
        size_t *h = (size_t *)realloc(p->high, (size_t)cap * sizeof(size_t));
        if (!h) return NULL;
        p->high = h;
        p->cap = cap;
    }
    size_t sz = bytes > POOL_CHUNK ? bytes : POOL_CHUNK;
    void *m = ncm_hip_malloc(sz);
    if (!m) return NULL;
    p->chunk[p->n] = (char *)m;
    p->size[p->n] = sz;
    p->zeroed[p->n] = 0;
    p->high[p->n] = 0;
    p->cur = p->n++;
    p->off = bytes;
    if (p->zeroing && pool_zero(p)) return NULL;
    return m;
}

static void pool_reset(Pool *p) {
    for (int i = 0; i < p->n; i++) {
        if (p->zeroed[i] > p->high[i]) p->high[i] = p->zeroed[i];
        p->zeroed[i] = 0;
    }
    p->cur = 0;
    p->off = 0;
}

static void pool_free(Pool *p) {
    for (int i = 0; i < p->n; i++) ncm_hip_free(p->chunk[i]);
    free(p->chunk);
    free(p->size);
    free(p->zeroed);
    free(p->high);
    memset(p, 0, sizeof(*p));
}

typedef enum {
    NT_LINEAR, NT_EMBED, NT_LN, NT_RMSN, NT_ACT, NT_MUL, NT_ADD, NT_SCALE,
    NT_ROPE, NT_SDPA, NT_SPLIT, NT_MERGE, NT_HEADSPLIT, NT_CE
} NtKind;

typedef struct {
    NtKind op;
    const float *a, *b, *c;
    float *y;
    float *aux;                 /* SDPA: P, or the row statistics (p6 & 1); CE: dlogits */
    const float *mask;          /* SDPA: the additive mask (may be NULL) */
    int *ids;                   /* EMBED: host copy of the ids */
    const float *cos_t, *sin_t; /* ROPE tables */
    const float *orow;          /* SDPA: the output's values with the heads merged (y only keys the gradient) */
    int o_ld;                   /* SDPA: orow's row stride */
    int64_t n;
    int p1, p2, p3, p4, p5, p6;
    double s;
} NtRec;

typedef struct {
    const float *key;
    float *g;
} GEnt;

#define PEND_MAX 8
struct NcmTape {
    NtRec *r;
    int n, cap;
    Pool rec, grad, gradw;   /* gradw: gradients whose first writer overwrites (not cleared) */
    GEnt *gm;
    int gn, gcap;
    /* residual gradients passed through (backward): the gradient of key, not
     * yet written, is 0.0f + base, to be written by the norm that reads key */
    const float *pend_key[PEND_MAX];
    const float *pend_base[PEND_MAX];
    int64_t pend_n[PEND_MAX];
    int npend;
};

/* The first record at or before index j (the backward visits them in that
 * order) that names key as an operand or output, or NULL. */
static const NtRec *next_use(const NcmTape *t, int j, const float *key) {
    for (; j >= 0; j--) {
        const NtRec *q = &t->r[j];
        if (q->a == key || q->b == key || q->c == key || q->y == key) return q;
    }
    return NULL;
}

static const float *pend_take(NcmTape *t, const float *key) {
    for (int k = 0; k < t->npend; k++)
        if (t->pend_key[k] == key) {
            const float *b = t->pend_base[k];
            t->pend_key[k] = t->pend_key[t->npend - 1];
            t->pend_base[k] = t->pend_base[t->npend - 1];
            t->pend_n[k] = t->pend_n[t->npend - 1];
            t->npend--;
            return b;
        }
    return NULL;
}

NcmTape *ncm_tape_new(void) {
    NcmTape *t = (NcmTape *)calloc(1, sizeof(NcmTape));
    if (t) t->grad.zeroing = 1;   /* gradient buffers start at zero */
    return t;
}

static void free_recs(NcmTape *t) {
    for (int i = 0; i < t->n; i++) free(t->r[i].ids);
    t->n = 0;
}

void ncm_tape_clear(NcmTape *t) {
    if (!t) return;
    free_recs(t);
    pool_reset(&t->rec);
    pool_reset(&t->grad);
    pool_reset(&t->gradw);
    t->gn = 0;
}

void ncm_tape_free(NcmTape *t) {
    if (!t) return;
    if (!ncm_ready()) ncm_hip_sync();
    free_recs(t);
    pool_free(&t->rec);
    pool_free(&t->grad);
    pool_free(&t->gradw);
    free(t->r);
    free(t->gm);
    free(t);
}

int ncm_tape_size(const NcmTape *t) { return t ? t->n : 0; }

static NtRec *emit(NcmTape *t, NtKind op) {
    if (t->n == t->cap) {
        int cap = t->cap ? 2 * t->cap : 64;
        NtRec *r = (NtRec *)realloc(t->r, (size_t)cap * sizeof(NtRec));
        if (!r) {
            ncm_fail(NCM_E_OOM, "tape: record allocation");
            return NULL;
        }
        t->r = r;
        t->cap = cap;
    }
    NtRec *r = &t->r[t->n++];
    memset(r, 0, sizeof(*r));
    r->op = op;
    return r;
}

/* ---------------- gradient map ---------------- */
static float *gmap_find(NcmTape *t, const float *key) {
    if (!key) return NULL;
    for (int i = 0; i < t->gn; i++)
        if (t->gm[i].key == key) return t->gm[i].g;
    return NULL;
}

static int gmap_put(NcmTape *t, const float *key, float *g) {
    if (t->gn == t->gcap) {
        int cap = t->gcap ? 2 * t->gcap : 64;
        GEnt *e = (GEnt *)realloc(t->gm, (size_t)cap * sizeof(GEnt));
        if (!e) return ncm_fail(NCM_E_OOM, "tape: gradient map");
        t->gm = e;
        t->gcap = cap;
    }
    t->gm[t->gn].key = key;
    t->gm[t->gn].g = g;
    t->gn++;
    return 0;
}

/* The gradient buffer of `key` (n floats), zeroed on first use. */
static float *gmap_get(NcmTape *t, const float *key, int64_t n) {
    if (!key) return NULL;
    float *g = gmap_find(t, key);
    if (g) return g;
    g = (float *)pool_alloc(&t->grad, (size_t)n * sizeof(float));   /* zeroed by the pool */
    if (!g) {
        ncm_fail(NCM_E_OOM, "tape: gradient buffer of %lld floats", (long long)n);
        return NULL;
    }
    if (gmap_put(t, key, g)) return NULL;
    return g;
}

/* The gradient buffer of `key` for an op that can write its first gradient
 * instead of accumulating it: an existing buffer is returned with *beta = 1
 * (accumulate); a new one comes from the pool that is not cleared, with
 * *beta = 0, and the op must write every element of it. */
static float *gmap_get_fresh(NcmTape *t, const float *key, int64_t n, int *beta) {
    *beta = 1;
    if (!key) return NULL;
    float *g = gmap_find(t, key);
    if (g) return g;
    g = (float *)pool_alloc(&t->gradw, (size_t)n * sizeof(float));
    if (!g) {
        ncm_fail(NCM_E_OOM, "tape: gradient buffer of %lld floats", (long long)n);
        return NULL;
    }
    if (gmap_put(t, key, g)) return NULL;
    *beta = 0;
    return g;
}

/* ---------------- recorders (forward on the device + record) ---------------- */
#define REC_OR_RETURN(r, t, op) \
    NtRec *r = emit(t, op);     \
    if (!r) return

void ncm_t_linear(NcmTape *t, const float *x, const float *W, const float *b, float *y, int64_t batch, int M,
                  int K) {
    linear_fwd(x, W, b, y, batch, M, K);
    REC_OR_RETURN(r, t, NT_LINEAR);
    r->a = x; r->b = W; r->c = b; r->y = y;
    r->n = batch; r->p1 = M; r->p2 = K;
}

void ncm_t_embed(NcmTape *t, const float *W, const int *idx, int V, float *y, int64_t n, int D) {
    if (n < 0 || !idx) { ncm_fail(NCM_E_ARG, "ncm_t_embed: bad ids"); return; }
    int *hcopy = (int *)malloc((size_t)(n > 0 ? n : 1) * sizeof(int));
    int *dcopy = (int *)pool_alloc(&t->rec, (size_t)(n > 0 ? n : 1) * sizeof(int));
    if (!hcopy || !dcopy) {
        free(hcopy);
        ncm_fail(NCM_E_OOM, "ncm_t_embed: id copies");
        return;
    }
    memcpy(hcopy, idx, (size_t)n * sizeof(int));
    if (ncm_h2d_async(dcopy, idx, (size_t)n * sizeof(int))) {
        free(hcopy);
        return;
    }
    embedding_fwd_v(W, V, dcopy, y, n, D);
    NtRec *r = emit(t, NT_EMBED);
    if (!r) { free(hcopy); return; }
    r->a = W; r->y = y; r->ids = hcopy;
    r->n = n; r->p1 = D; r->p2 = V;
}

static void rec_ln(NcmTape *t, const float *x, const float *w, const float *b, float *y, int64_t rows, int C,
                   double eps) {
    REC_OR_RETURN(r, t, NT_LN);
    r->a = x; r->b = w; r->c = b; r->y = y;
    r->n = rows; r->p1 = C; r->s = eps;
}

void ncm_t_layernorm(NcmTape *t, const float *x, const float *w, const float *b, float *y, int64_t rows, int C) {
    layernorm_fwd(x, w, b, y, rows, C);
    rec_ln(t, x, w, b, y, rows, C, 1e-6);
}

void ncm_t_layernorm_eps(NcmTape *t, const float *x, const float *w, const float *b, float *y, int64_t rows, int C,
                         double eps) {
    layernorm_eps_fwd(x, w, b, y, rows, C, (float)eps);
    rec_ln(t, x, w, b, y, rows, C, eps);
}

void ncm_t_rmsnorm(NcmTape *t, const float *x, const float *w, float *y, int64_t rows, int C) {
    rmsnorm_fwd(x, w, y, rows, C);
    REC_OR_RETURN(r, t, NT_RMSN);
    r->a = x; r->b = w; r->y = y;
    r->n = rows; r->p1 = C;
}

static void rec_act(NcmTape *t, const float *x, float *y, int64_t n, int kind) {
    REC_OR_RETURN(r, t, NT_ACT);
    r->a = x; r->y = y; r->n = n; r->p1 = kind;
}

void ncm_t_gelu(NcmTape *t, const float *x, float *y, int64_t n) { gelu_fwd(x, y, n); rec_act(t, x, y, n, 0); }
void ncm_t_silu(NcmTape *t, const float *x, float *y, int64_t n) { silu_fwd(x, y, n); rec_act(t, x, y, n, 1); }
void ncm_t_gelu_tanh(NcmTape *t, const float *x, float *y, int64_t n) {
    gelu_tanh_fwd(x, y, n);
    rec_act(t, x, y, n, 2);
}

/* ncm_t_linear (x -> pre) then the activation (pre -> y), the GEMM writing
 * both outputs; the same two records. */
void ncm_t_linear_act(NcmTape *t, const float *x, const float *W, const float *b, float *pre, float *y,
                      int64_t batch, int M, int K, int kind) {
    static const int acts[3] = {NCM_ACT_GELU, NCM_ACT_SILU, NCM_ACT_GELU_TANH};
    if (kind < 0 || kind > 2) { ncm_fail(NCM_E_ARG, "ncm_t_linear_act: unknown activation %d", kind); return; }
    ncm_linear_fwd_pre(x, W, b, pre, y, batch, M, K, acts[kind]);
    REC_OR_RETURN(r, t, NT_LINEAR);
    r->a = x; r->b = W; r->c = b; r->y = pre;
    r->n = batch; r->p1 = M; r->p2 = K;
    rec_act(t, pre, y, batch * M, kind);
}

/* y = res + (x W^T + b) in one GEMM launch: the records of ncm_t_linear and
 * ncm_t_add without the linear output in between -- the linear record's
 * output is y itself (the add passes y's gradient through unchanged) and
 * the add record carries only res. */
void ncm_t_linear_res(NcmTape *t, const float *x, const float *W, const float *b, const float *res, float *y,
                      int64_t batch, int M, int K) {
    if (!res || res == y) { ncm_fail(NCM_E_ARG, "ncm_t_linear_res: res must be a buffer other than y"); return; }
    linear_fwd_ep(x, W, b, res, y, batch, M, K, NCM_ACT_NONE);
    NtRec *r = emit(t, NT_LINEAR);
    if (!r) return;
    r->a = x; r->b = W; r->c = b; r->y = y;
    r->n = batch; r->p1 = M; r->p2 = K;
    REC_OR_RETURN(ra, t, NT_ADD);
    ra->a = res; ra->b = NULL; ra->y = y; ra->n = batch * M;
}

void ncm_t_mul(NcmTape *t, const float *a, const float *b, float *y, int64_t n) {
    mul_fwd(a, b, y, n);
    REC_OR_RETURN(r, t, NT_MUL);
    r->a = a; r->b = b; r->y = y; r->n = n;
}

void ncm_t_add(NcmTape *t, const float *a, const float *b, float *y, int64_t n) {
    add_fwd(a, b, y, n);
    REC_OR_RETURN(r, t, NT_ADD);
    r->a = a; r->b = b; r->y = y; r->n = n;
}

void ncm_t_scale(NcmTape *t, const float *x, float s, float *y, int64_t n) {
    scale_fwd(x, s, y, n);
    REC_OR_RETURN(r, t, NT_SCALE);
    r->a = x; r->y = y; r->n = n; r->s = s;
}

void ncm_t_rope(NcmTape *t, const float *xq, const float *xk, float *yq, float *yk, const float *cos_t,
                const float *sin_t, int B, int H, int Hkv, int T, int hd) {
    if (B < 0 || H < 0 || Hkv < 1 || T < 0 || hd < 0) { ncm_fail(NCM_E_ARG, "ncm_t_rope: bad shape"); return; }
    if (ncm_ready()) return;
    if (ncm_copy_async(yq, xq, (size_t)B * H * T * hd * sizeof(float)) ||
        ncm_copy_async(yk, xk, (size_t)B * Hkv * T * hd * sizeof(float)))
        return;
    rope_apply_gqa(yq, yk, cos_t, sin_t, B, H, Hkv, T, hd);
    REC_OR_RETURN(r, t, NT_ROPE);
    r->a = xq; r->b = xk; r->c = yq; r->y = yk;
    r->cos_t = cos_t; r->sin_t = sin_t;
    r->n = B; r->p1 = H; r->p2 = T; r->p3 = hd; r->p4 = Hkv;
}

/* The forward of an SDPA record.  hd = 64 with aligned operands (the MFMA
 * path): the forward also keeps each query row's softmax (max, sum), and the
 * backward rebuilds P from them (p6 bit 0; bit 1 = causal); otherwise P is
 * stored, as the reference's t_sdpa keeps it (train_tape.c:289-313). */
static void t_sdpa_any(NcmTape *t, const float *q, const float *k, const float *v, const float *mask, int causal,
                       float *o, int B, int H, int Hkv, int Tq, int Tkv, int hd) {
    if (Hkv < 1 || H % Hkv) { ncm_fail(NCM_E_ARG, "ncm_t_sdpa: H=%d Hkv=%d", H, Hkv); return; }
    const int flash = hd == 64 && Tkv % 4 == 0 && is_aligned16(q) && is_aligned16(k) && is_aligned16(v) &&
                      is_aligned16(o);
    float *aux;
    if (flash) {
        aux = (float *)pool_alloc(&t->rec, (size_t)B * H * Tq * 2 * sizeof(float));
        if (!aux) { ncm_fail(NCM_E_OOM, "ncm_t_sdpa: row statistics"); return; }
        ncm_sdpa_fwd_stats(q, k, v, mask, o, aux, B, H, Hkv, Tq, Tkv, hd, causal);
    } else {
        float *m = NULL;
        if (causal) {   /* the -1e9 causal mask of the reference's callers */
            m = (float *)pool_alloc(&t->rec, (size_t)Tq * Tkv * sizeof(float));
            float *hm = (float *)malloc((size_t)Tq * Tkv * sizeof(float));
            if (!m || !hm) { free(hm); ncm_fail(NCM_E_OOM, "ncm_t_sdpa: mask"); return; }
            for (int i = 0; i < Tq; i++)
                for (int j = 0; j < Tkv; j++) hm[(size_t)i * Tkv + j] = j <= i + (Tkv - Tq) ? 0.0f : -1e9f;
            mem_h2d(m, hm, (size_t)Tq * Tkv * sizeof(float));
            free(hm);
            mask = m;
        }
        sdpa_fwd_gqa(q, k, v, mask, o, B, H, Hkv, Tq, Tkv, hd);
        aux = (float *)pool_alloc(&t->rec, (size_t)B * H * Tq * Tkv * sizeof(float));
        if (!aux) { ncm_fail(NCM_E_OOM, "ncm_t_sdpa: probabilities"); return; }
        sdpa_probs_gqa(q, k, mask, aux, B, H, Hkv, Tq, Tkv, hd);
    }
    REC_OR_RETURN(r, t, NT_SDPA);
    r->a = q; r->b = k; r->c = v; r->y = o; r->aux = aux; r->mask = mask;
    r->n = B; r->p1 = H; r->p2 = Hkv; r->p3 = Tq; r->p4 = Tkv; r->p5 = hd; r->p6 = flash | (causal ? 2 : 0);
}

void ncm_t_sdpa(NcmTape *t, const float *q, const float *k, const float *v, const float *mask, float *o, int B,
                int H, int Hkv, int Tq, int Tkv, int hd) {
    t_sdpa_any(t, q, k, v, mask, 0, o, B, H, Hkv, Tq, Tkv, hd);
}

void ncm_t_sdpa_causal(NcmTape *t, const float *q, const float *k, const float *v, float *o, int B, int H, int Hkv,
                       int Tq, int Tkv, int hd) {
    if (Tq > Tkv) { ncm_fail(NCM_E_ARG, "ncm_t_sdpa_causal: Tq %d > Tkv %d", Tq, Tkv); return; }
    t_sdpa_any(t, q, k, v, NULL, 1, o, B, H, Hkv, Tq, Tkv, hd);
}

/* ncm_t_sdpa_causal (q, k, v -> ctx) then ncm_t_headmerge (ctx -> out) with
 * the attention writing the merged rows itself: the same records, ctx keying
 * its gradient while the attention record reads its output values from out
 * (flash path; otherwise the two calls). */
void ncm_t_sdpa_causal_merge(NcmTape *t, const float *q, const float *k, const float *v, float *ctx, float *out,
                             int B, int H, int Hkv, int T, int hd) {
    const int C = H * hd;
    const int flash = hd == 64 && T % 4 == 0 && Hkv >= 1 && H % Hkv == 0 && is_aligned16(q) && is_aligned16(k) &&
                      is_aligned16(v) && is_aligned16(out);
    if (!flash) {
        ncm_t_sdpa_causal(t, q, k, v, ctx, B, H, Hkv, T, T, hd);
        ncm_t_headmerge(t, ctx, out, B, T, C, H, hd);
        return;
    }
    float *aux = (float *)pool_alloc(&t->rec, (size_t)B * H * T * 2 * sizeof(float));
    if (!aux) { ncm_fail(NCM_E_OOM, "ncm_t_sdpa_causal_merge: row statistics"); return; }
    ncm_sdpa_fwd_stats_merged(q, k, v, NULL, out, aux, B, H, Hkv, T, T, hd, 1);
    NtRec *r = emit(t, NT_SDPA);
    if (!r) return;
    r->a = q; r->b = k; r->c = v; r->y = ctx; r->aux = aux; r->mask = NULL;
    r->orow = out; r->o_ld = C;
    r->n = B; r->p1 = H; r->p2 = Hkv; r->p3 = T; r->p4 = T; r->p5 = hd; r->p6 = 1 | 2;
    REC_OR_RETURN(rm, t, NT_MERGE);
    rm->a = ctx; rm->y = out;
    rm->n = B; rm->p1 = T; rm->p2 = C; rm->p3 = H; rm->p4 = hd;
}

void ncm_t_qkvsplit(NcmTape *t, const float *in, float *qq, float *kk, float *vv, int B, int T, int C, int H, int hd,
                    int K, int rep) {
    qkv_split_fwd(in, qq, kk, vv, B, T, C, H, hd, K, rep);
    REC_OR_RETURN(r, t, NT_SPLIT);
    r->a = in; r->b = qq; r->c = kk; r->y = vv;
    r->n = B; r->p1 = T; r->p2 = C; r->p3 = H; r->p4 = hd; r->p5 = K; r->p6 = rep;
}

/* ncm_t_linear (x -> qkv) then ncm_t_qkvsplit (qkv -> qq, kk, vv) with the
 * split done by the GEMM's epilogue: the same two records, qkv serving as
 * the key of its gradient (its values are never read by the backward). */
void ncm_t_linear_qkvsplit(NcmTape *t, const float *x, const float *W, const float *b, float *qkv, float *qq,
                           float *kk, float *vv, int B, int T, int C, int H, int hd, int K, int rep) {
    ncm_linear_fwd_qkv_heads(x, W, b, qkv, qq, kk, vv, B, T, C, H, hd, K, rep);
    NtRec *r = emit(t, NT_LINEAR);
    if (!r) return;
    r->a = x; r->b = W; r->c = b; r->y = qkv;
    r->n = (int64_t)B * T; r->p1 = C + 2 * K * hd; r->p2 = C;
    REC_OR_RETURN(rs, t, NT_SPLIT);
    rs->a = qkv; rs->b = qq; rs->c = kk; rs->y = vv;
    rs->n = B; rs->p1 = T; rs->p2 = C; rs->p3 = H; rs->p4 = hd; rs->p5 = K; rs->p6 = rep;
}

void ncm_t_headmerge(NcmTape *t, const float *ctx, float *out, int B, int T, int C, int H, int hd) {
    head_merge_fwd(ctx, out, B, T, C, H, hd);
    REC_OR_RETURN(r, t, NT_MERGE);
    r->a = ctx; r->y = out;
    r->n = B; r->p1 = T; r->p2 = C; r->p3 = H; r->p4 = hd;
}

void ncm_t_headsplit(NcmTape *t, const float *in, float *out, int B, int T, int C, int H, int hd) {
    heads_transpose_fwd_b(in, out, B, T, H, hd);
    REC_OR_RETURN(r, t, NT_HEADSPLIT);
    r->a = in; r->y = out;
    r->n = B; r->p1 = T; r->p2 = C; r->p3 = H; r->p4 = hd;
}

void ncm_t_ce(NcmTape *t, const float *logits, const int *tgt, const float *wmask, float *loss, float *probs,
              int64_t rows, int V, double weight) {
    if (rows <= 0 || V <= 0 || !tgt) { ncm_fail(NCM_E_ARG, "ncm_t_ce: bad arguments"); return; }
    if (ncm_ready()) return;
    int *dt = (int *)pool_alloc(&t->rec, (size_t)rows * sizeof(int));
    float *dw = wmask ? (float *)pool_alloc(&t->rec, (size_t)rows * sizeof(float)) : NULL;
    float *dl = (float *)pool_alloc(&t->rec, (size_t)rows * V * sizeof(float));
    if (!dt || (wmask && !dw) || !dl) { ncm_fail(NCM_E_OOM, "ncm_t_ce: buffers"); return; }
    if (ncm_h2d_async(dt, tgt, (size_t)rows * sizeof(int))) return;
    if (wmask && ncm_h2d_async(dw, wmask, (size_t)rows * sizeof(float))) return;
    if (ncm_zero_async(dl, (size_t)rows * V * sizeof(float))) return;
    if (probs) ce_fwd(logits, dt, dw, loss, probs, rows, V);
    ce_fwd_bwd(logits, dt, dw, loss, dl, rows, V, weight);
    REC_OR_RETURN(r, t, NT_CE);
    r->a = logits; r->y = loss; r->aux = dl;
    r->n = rows; r->p1 = V; r->s = weight;
}

/* ---------------- backward ---------------- */
void ncm_tape_backward(NcmTape *t, const NcmPMap *pm) {
    if (!t || ncm_ready()) return;
    t->gn = 0;
    t->npend = 0;
    pool_reset(&t->grad);
    pool_reset(&t->gradw);
    if (pm)
        for (int i = 0; i < pm->n; i++)
            if (pm->params[i] && pm->grads[i] && gmap_put(t, pm->params[i], pm->grads[i])) return;
    for (int i = t->n - 1; i >= 0; i--) {
        NtRec *r = &t->r[i];
        if (r->op == NT_CE) {
            float *g = gmap_find(t, r->a);
            if (g)
                add_inplace_fwd(g, r->aux, r->n * r->p1);
            else if (gmap_put(t, r->a, r->aux))
                return;
            continue;
        }
        float *dy = gmap_find(t, r->y);
        if (!dy) {
            if (r->op == NT_ROPE && gmap_find(t, r->c)) {
                /* only the q output carries a gradient */
            } else if (r->op == NT_SPLIT && (gmap_find(t, r->b) || gmap_find(t, r->c))) {
            } else {
                /* a norm left with nothing to add still owes the pending first
                 * write of its input's gradient */
                const float *base = t->npend && (r->op == NT_LN || r->op == NT_RMSN) ? pend_take(t, r->a) : NULL;
                if (base) ncm_add_inplace_ex(gmap_find(t, r->a), base, r->n * r->p1, 0);
                continue;
            }
        }
        switch (r->op) {
        case NT_LINEAR: {
            int64_t batch = r->n;
            int M = r->p1, K = r->p2, bx;
            const NtRec *ra = i > 0 ? &t->r[i - 1] : NULL;
            if (ra && ra->op == NT_ACT && ra->y == r->a && ra->n == batch * K && !gmap_find(t, r->a) &&
                ncm_linear_dx_fusable(batch, M, K, dy, r->b)) {
                /* the record right before is the activation that produced this
                 * linear's input, and nothing else reads that input: its
                 * backward runs in the dX GEMM's epilogue, the input's gradient
                 * is never stored, and the activation record is done too */
                float *dxa = gmap_get_fresh(t, ra->a, ra->n, &bx);
                if (!dxa) return;
                ncm_linear_bwd_act(r->a, r->b, dy, dxa, ra->a, ra->p1, bx, gmap_get(t, r->b, (int64_t)M * K),
                                   r->c ? gmap_get(t, r->c, M) : NULL, batch, M, K);
                i--;
                break;
            }
            if (ra && ra->op == NT_MERGE && ra->y == r->a && ra->p4 == 64 && ra->p2 == ra->p3 * 64 && K == ra->p2 &&
                (int64_t)ra->n * ra->p1 == batch && ra->p1 % 64 == 0 && !gmap_find(t, r->a) &&
                ncm_linear_dx_fusable(batch, M, K, dy, r->b)) {
                /* the record right before merged the attention heads into this
                 * linear's input, and nothing else reads it: the dX GEMM writes
                 * the heads' gradient directly (the merged rows' gradient is
                 * never stored), and the merge record is done too */
                float *dctx = gmap_get_fresh(t, ra->a, batch * K, &bx);
                if (!dctx) return;
                ncm_linear_bwd_heads(r->a, r->b, dy, dctx, bx, gmap_get(t, r->b, (int64_t)M * K),
                                     r->c ? gmap_get(t, r->c, M) : NULL, (int)ra->n, ra->p1, M, ra->p3);
                i--;
                break;
            }
            float *dx = gmap_get_fresh(t, r->a, batch * K, &bx);
            ncm_linear_bwd_ex(r->a, r->b, dy, dx, gmap_get(t, r->b, (int64_t)M * K),
                              r->c ? gmap_get(t, r->c, M) : NULL, batch, M, K, bx);
            break;
        }
        case NT_EMBED:
            embedding_bwd(dy, r->ids, r->n, r->p1, gmap_get(t, r->a, (int64_t)r->p2 * r->p1), r->p2);
            break;
        case NT_LN: {
            int bx;
            float *dx = gmap_get_fresh(t, r->a, r->n * r->p1, &bx);
            const float *base = pend_take(t, r->a);
            if (base)
                ncm_layernorm_bwd_base(r->a, r->b, dy, dx, r->b ? gmap_get(t, r->b, r->p1) : NULL,
                                       r->c ? gmap_get(t, r->c, r->p1) : NULL, r->n, r->p1, r->s, base);
            else
                ncm_layernorm_bwd_ex(r->a, r->b, dy, dx, r->b ? gmap_get(t, r->b, r->p1) : NULL,
                                     r->c ? gmap_get(t, r->c, r->p1) : NULL, r->n, r->p1, r->s, bx);
            break;
        }
        case NT_RMSN: {
            int bx;
            float *dx = gmap_get_fresh(t, r->a, r->n * r->p1, &bx);
            const float *base = pend_take(t, r->a);
            if (base)
                ncm_rmsnorm_bwd_base(r->a, r->b, dy, dx, r->b ? gmap_get(t, r->b, r->p1) : NULL, r->n, r->p1, base);
            else
                ncm_rmsnorm_bwd_ex(r->a, r->b, dy, dx, r->b ? gmap_get(t, r->b, r->p1) : NULL, r->n, r->p1, bx);
            break;
        }
        case NT_ACT: {
            int bx;
            float *dx = gmap_get_fresh(t, r->a, r->n, &bx);
            ncm_act_bwd_ex(r->p1, r->a, dy, dx, r->n, bx);
            break;
        }
        case NT_MUL:
            mul_bwd(r->a, r->b, dy, gmap_get(t, r->a, r->n), gmap_get(t, r->b, r->n), r->n);
            break;
        case NT_ADD: {
            int ba, bb;
            float *ga = gmap_get_fresh(t, r->a, r->n, &ba);
            const NtRec *nu = ga && !ba && !r->b && t->npend < PEND_MAX ? next_use(t, i - 1, r->a) : NULL;
            if (nu && (nu->op == NT_LN || nu->op == NT_RMSN) && nu->a == r->a && nu->n * nu->p1 == r->n) {
                /* a residual input whose gradient is new and whose next use
                 * (in backward order) is the norm that reads it: its first
                 * write, 0.0f + dy, is left to that norm's backward, which
                 * writes (0.0f + dy) + its own gradient in one pass; dy is not
                 * written again before then (its writers ran before this
                 * record) */
                t->pend_key[t->npend] = r->a;
                t->pend_base[t->npend] = dy;
                t->pend_n[t->npend] = r->n;
                t->npend++;
            } else if (ga) {
                ncm_add_inplace_ex(ga, dy, r->n, ba);
            }
            float *gb = r->b ? gmap_get_fresh(t, r->b, r->n, &bb) : NULL;   /* after a's write: b may be a */
            if (gb) ncm_add_inplace_ex(gb, dy, r->n, bb);
            break;
        }
        case NT_SCALE: {
            float *dx = gmap_get(t, r->a, r->n);
            float s = (float)r->s;
            int64_t n = r->n;
            if (dx && n > 0) {
                void *a[] = {&dx, &dy, &s, &n};
                ncm_launch_named("axpy_k", (unsigned)((n + 255) / 256), 1, 1, 256, a);
            }
            break;
        }
        case NT_ROPE: {
            int B = (int)r->n, H = r->p1, T = r->p2, hd = r->p3, Hkv = r->p4;
            float *gq = gmap_find(t, r->c), *gk = gmap_find(t, r->y);
            float *dxq = gq ? gmap_get(t, r->a, (int64_t)B * H * T * hd) : NULL;
            float *dxk = gk ? gmap_get(t, r->b, (int64_t)B * Hkv * T * hd) : NULL;
            rope_bwd_gqa(gq, gk, r->cos_t, r->sin_t, dxq, dxk, B, H, Hkv, T, hd);
            break;
        }
        case NT_SDPA: {
            int B = (int)r->n, H = r->p1, Hkv = r->p2, Tq = r->p3, Tkv = r->p4, hd = r->p5;
            const int64_t nq = (int64_t)B * H * Tq * hd, nk = (int64_t)B * Hkv * Tkv * hd;
            const NtRec *rs = i > 0 ? &t->r[i - 1] : NULL;
            if ((r->p6 & 1) && rs && rs->op == NT_SPLIT && rs->b == r->a && rs->c == r->b && rs->y == r->c &&
                rs->n == B && rs->p1 == Tq && Tq == Tkv && rs->p3 == H && rs->p4 == hd && rs->p5 == Hkv &&
                Hkv == H && rs->p6 == 1 && rs->p2 == H * hd && !gmap_find(t, r->a) && !gmap_find(t, r->b) &&
                !gmap_find(t, r->c)) {
                /* the record right before is the split that produced q, k and v
                 * from rows [B*T][3 C], one kv head per query head, and only
                 * the attention reads them: its gradients go straight into the
                 * rows' gradient (what the split's backward would form), and
                 * the split record is done too */
                int bx;
                float *gx = gmap_get_fresh(t, rs->a, (int64_t)B * Tq * 3 * H * hd, &bx);
                if (!gx) return;
                ncm_sdpa_bwd_flash_rows(r->a, r->b, r->c, r->orow ? r->orow : r->y, r->aux, r->mask, (r->p6 >> 1) & 1,
                                        dy, gx, B, H, Hkv, Tq, Tkv, hd, bx, r->orow ? r->o_ld : 0);
                i--;
                break;
            }
            int fq, fk, fv;
            float *gq = gmap_get_fresh(t, r->a, nq, &fq);
            float *gk = gmap_get_fresh(t, r->b, nk, &fk), *gv = gmap_get_fresh(t, r->c, nk, &fv);
            /* one flag for the three outputs: written only when all three are
             * new and distinct (the flash kernels give every element one
             * writer); otherwise the new ones are cleared and accumulated */
            int beta = 1;
            if ((r->p6 & 1) && !fq && !fk && !fv && gq != gk && gq != gv && gk != gv) {
                beta = 0;
            } else {
                if (!fq && gq && ncm_zero_async(gq, (size_t)nq * sizeof(float))) return;
                if (!fk && gk && gk != gq && ncm_zero_async(gk, (size_t)nk * sizeof(float))) return;
                if (!fv && gv && gv != gq && gv != gk && ncm_zero_async(gv, (size_t)nk * sizeof(float))) return;
            }
            if (r->p6 & 1)
                ncm_sdpa_bwd_flash_ex(r->a, r->b, r->c, r->orow ? r->orow : r->y, r->aux, r->mask, (r->p6 >> 1) & 1,
                                      dy, gq, gk, gv, B, H, Hkv, Tq, Tkv, hd, beta, r->orow ? r->o_ld : 0);
            else
                sdpa_bwd_gqa(r->a, r->b, r->c, r->aux, dy, gq, gk, gv, B, H, Hkv, Tq, Tkv, hd);
            break;
        }
        case NT_SPLIT: {
            int B = (int)r->n, T = r->p1, C = r->p2, H = r->p3, hd = r->p4, K = r->p5, rep = r->p6, bx;
            float *dx = gmap_get_fresh(t, r->a, (int64_t)B * T * ((int64_t)C + 2 * K * hd), &bx);
            ncm_qkv_split_bwd_ex(gmap_find(t, r->b), gmap_find(t, r->c), gmap_find(t, r->y), dx, B, T, C, H, hd, K,
                                 rep, bx);
            break;
        }
        case NT_MERGE: {
            int B = (int)r->n, T = r->p1, C = r->p2, H = r->p3, hd = r->p4, bx;
            float *dx = gmap_get_fresh(t, r->a, (int64_t)B * H * T * hd, &bx);
            ncm_heads_bwd_ex(dy, dx, B, T, C, H, hd, 0, bx);
            break;
        }
        case NT_HEADSPLIT: {
            int B = (int)r->n, T = r->p1, C = r->p2, H = r->p3, hd = r->p4, bx;
            float *dx = gmap_get_fresh(t, r->a, (int64_t)B * T * C, &bx);
            ncm_heads_bwd_ex(dy, dx, B, T, C, H, hd, 1, bx);
            break;
        }
        case NT_CE:
            break;
        }
        if (ncm_ready()) return;
    }
    /* (every pending write is taken by its norm record; none is left unless
     * that record was never visited) */
    while (t->npend > 0) {
        const int k = t->npend - 1;
        ncm_add_inplace_ex(gmap_find(t, t->pend_key[k]), t->pend_base[k], t->pend_n[k], 0);
        t->npend--;
    }
}

/* The gradient the last backward accumulated for `key` (NULL if none). */
float *ncm_tape_grad(NcmTape *t, const float *key) { return t ? gmap_find(t, key) : NULL; }
