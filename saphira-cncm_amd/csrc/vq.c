/* vq.c -- host side of the VQ nearest-codeword search and the multiscale
 * residual loop (reference: kernels.c:753-770, vq.c:378-500). */
#include "internal.h"

#include <limits.h>

#include "noalloc.h"

/* Must match struct VqArgs in vq.hip. */
typedef struct {
    const float *X;
    const float *E;
    const float *cn;
    const float *xn;
    const unsigned *cmax_bits;
    int *idx;
    int *flag_list;
    int *flag_count;
    int *pair_list;
    int *pair_count;
    unsigned long long *keys;
    unsigned *done;
    int rows, V, D;
    int L, total, off;
} VqArgs;

#define VQ_MAXD 4096
#define RESCORE_GRID 1024

/* Device scratch of one search: counters | cn[V] | xn[rows] | flags[rows] |
 * pairs[3*rows] | keys[rows] (u64) | done[rows]. */
typedef struct {
    unsigned *counters;
    float *cn;
    float *xn;
    int *flags;
    int *pairs;
    unsigned long long *keys;
    unsigned *done;
} VqScratch;

static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

/* Byte offsets of the scratch parts for (rows, V); returns the total. */
static size_t vq_scratch_layout(int rows, int V, size_t off[6]) {
    off[0] = 256;                                  /* cn */
    off[1] = off[0] + al256((size_t)V * 4);        /* xn */
    off[2] = off[1] + al256((size_t)rows * 4);     /* flags */
    off[3] = off[2] + al256((size_t)rows * 4);     /* pairs */
    off[4] = off[3] + al256((size_t)rows * 12);    /* keys */
    off[5] = off[4] + al256((size_t)rows * 8);     /* done */
    return off[5] + (size_t)rows * 4;
}

/* Carves the scratch from base (at least vq_scratch_layout bytes) or, when
 * base is NULL, from the library's workspace. */
static int vq_scratch(VqScratch *s, int rows, int V, unsigned char *base) {
    size_t off[6];
    size_t total = vq_scratch_layout(rows, V, off);
    if (!base) base = (unsigned char *)ncm_workspace(WS_VQ, total);
    if (!base) return NCM_E_OOM;
    s->counters = (unsigned *)base;
    s->cn = (float *)(base + off[0]);
    s->xn = (float *)(base + off[1]);
    s->flags = (int *)(base + off[2]);
    s->pairs = (int *)(base + off[3]);
    s->keys = (unsigned long long *)(base + off[4]);
    s->done = (unsigned *)(base + off[5]);
    return 0;
}

/* Rescore counting for the tests: when on, every search waits for its
 * rescore and adds the rows that took the pair rescore and the full rescore. */
static int g_count_rescores = 0;
static long long g_rescore_pairs = 0, g_rescore_full = 0;

void ncm_vq_count_rescores(int on) {
    g_count_rescores = on;
    g_rescore_pairs = g_rescore_full = 0;
}

void ncm_vq_rescore_counts(long long *pairs, long long *full) {
    if (pairs) *pairs = g_rescore_pairs;
    if (full) *full = g_rescore_full;
}

/* codes of `rows` rows of X against E, written at idx[(row/L)*total + off + row%L] */
static int vq_search(const float *X, const float *E, int *idx, int rows, int V, int D, int L,
                     int total, int off, unsigned char *scratch) {
    VqScratch s;
    if (vq_scratch(&s, rows, V, scratch)) return NCM_E_OOM;
    int rc;
    void *a0[] = {&s.counters};
    if ((rc = ncm_launch_named("vq_init", 1, 1, 1, 64, a0))) return rc;
    unsigned *cmax = s.counters + 1;
    int vec = (D % 4 == 0) && is_aligned16(X) && is_aligned16(E);
    void *a1[] = {&E, &V, &D, &vec, &s.cn, &cmax};
    unsigned pgrid = (unsigned)((V + 3) / 4) < 256u ? (unsigned)((V + 3) / 4) : 256u;
    if ((rc = ncm_launch_named("vq_prep_codebook_w", pgrid, 1, 1, 256, a1))) return rc;
    void *a2[] = {&X, &rows, &D, &s.xn};
    if ((rc = ncm_launch_named("vq_rownorm", (unsigned)((rows + 3) / 4), 1, 1, 256, a2))) return rc;

    VqArgs p = {X, E, s.cn, s.xn, cmax, idx, s.flags, (int *)s.counters,
                s.pairs, (int *)s.counters + 2, s.keys, s.done, rows, V, D, L, total, off};
    void *a3[] = {&p};
    if ((rc = ncm_launch_named(vec ? "vq_argmin_main_v" : "vq_argmin_main_s", (unsigned)((rows + 63) / 64), 1,
                               1, 256, a3)))
        return rc;
    const unsigned *cnt = s.counters;
    void *a4[] = {&X, &E, &V, &D, &vec, &s.flags, &s.pairs, &cnt, &s.keys, &s.done, &idx, &L, &total, &off};
    if ((rc = ncm_launch_named("vq_rescore", RESCORE_GRID, 1, 1, 256, a4)) || !g_count_rescores) return rc;
    unsigned c[3];
    mem_d2h(c, s.counters, sizeof c);
    g_rescore_full += c[0];
    g_rescore_pairs += c[2];
    return ncm_ready();
}

static int vq_check(const char *fn, int64_t rows, int V, int D) {
    if (rows < 0 || rows > INT_MAX / 2 || V <= 0 || D <= 0)
        return ncm_fail(NCM_E_ARG, "%s: bad shape rows=%lld V=%d D=%d", fn, (long long)rows, V, D);
    if (D > VQ_MAXD) return ncm_fail(NCM_E_ARG, "%s: D=%d exceeds %d", fn, D, VQ_MAXD);
    return 0;
}

void vq_argmin(const float *a, const float *E, int *idx, int64_t rows, int V, int D) {
    if (vq_check("vq_argmin", rows, V, D) || rows == 0) return;
    if (!a || !E || !idx) {
        ncm_fail(NCM_E_ARG, "vq_argmin: null pointer");
        return;
    }
    if (ncm_ready()) return;
    vq_search(a, E, idx, (int)rows, V, D, (int)rows, (int)rows, 0, NULL);
}

/* vq_argmin with its scratch in the library's fixed device array instead of
 * a workspace: no allocation on any call (see noalloc.h for the limits).
 * Every kernel of the search clears or overwrites the scratch it reads
 * (vq_init zeroes the counters; each flagged row's key and counter are set
 * when the row is flagged), so nothing carries over from the last call. */
int vq_argmin_noalloc(const float *a, const float *E, int *idx, int64_t rows, int V, int D) {
    int rc;
    if ((rc = vq_check("vq_argmin_noalloc", rows, V, D))) return rc;
    if (rows > NCM_NOALLOC_MAX_ROWS || V > NCM_NOALLOC_MAX_V)
        return ncm_fail(NCM_E_ARG, "vq_argmin_noalloc: rows=%lld V=%d exceed the fixed scratch's limits rows <= %d, V <= %d",
                        (long long)rows, V, NCM_NOALLOC_MAX_ROWS, NCM_NOALLOC_MAX_V);
    if (rows == 0) return 0;
    if (!a || !E || !idx) return ncm_fail(NCM_E_ARG, "vq_argmin_noalloc: null pointer");
    if ((rc = ncm_ready())) return rc;
    size_t off[6];
    if (vq_scratch_layout((int)rows, V, off) > NCM_NOALLOC_SCRATCH_BYTES)
        return ncm_fail(NCM_E_ARG, "vq_argmin_noalloc: scratch for rows=%lld V=%d exceeds %u bytes", (long long)rows,
                        V, NCM_NOALLOC_SCRATCH_BYTES);
    int err = 0;
    unsigned char *base = (unsigned char *)ncm_noalloc_scratch(ncm_device(), &err);
    if (!base)
        return ncm_fail(NCM_E_INIT, "vq_argmin_noalloc: no fixed scratch on device %d (%s)", ncm_device(),
                        err ? ncm_noalloc_error_string(err) : "lookup never ran");
    return vq_search(a, E, idx, (int)rows, V, D, (int)rows, (int)rows, 0, base);
}

void vq_quantize_multiscale(const float *z, const float *const *E, const int *vocabs, int n_levels,
                            int B, int L, int D, int *idx, float *z_hat, float *z_rest) {
    if (n_levels <= 0 || B < 0 || L <= 0 || !E || !vocabs) {
        ncm_fail(NCM_E_ARG, "vq_quantize_multiscale: bad levels/shape");
        return;
    }
    int64_t rows64 = (int64_t)B * L;
    if ((int64_t)n_levels * L > INT_MAX) {
        ncm_fail(NCM_E_ARG, "vq_quantize_multiscale: n_levels*L too large");
        return;
    }
    for (int lv = 0; lv < n_levels; lv++)
        if (vq_check("vq_quantize_multiscale", rows64, vocabs[lv], D) || !E[lv]) {
            if (!E[lv]) ncm_fail(NCM_E_ARG, "vq_quantize_multiscale: null codebook %d", lv);
            return;
        }
    if (rows64 == 0) return;
    if (!z || !idx || !z_hat || !z_rest) {
        ncm_fail(NCM_E_ARG, "vq_quantize_multiscale: null pointer");
        return;
    }
    if (ncm_ready()) return;
    int rows = (int)rows64;
    int total = n_levels * L;
    /* z_rest = z (vq.c:396-403); z_hat starts at +0.0 (first level adds into 0.0f) */
    hipError_t e = hipMemcpyAsync(z_rest, z, (size_t)rows * D * sizeof(float),
                                  hipMemcpyDeviceToDevice, ncm_stream());
    if (e != hipSuccess) {
        ncm_fail(NCM_E_HIP, "vq_quantize_multiscale copy: %s", hipGetErrorString(e));
        return;
    }
    for (int lv = 0; lv < n_levels; lv++) {
        int off = lv * L;
        if (vq_search(z_rest, E[lv], idx, rows, vocabs[lv], D, L, total, off, NULL)) return;
        const float *El = E[lv];
        int V = vocabs[lv];
        int first = lv == 0;
        int64_t n = (int64_t)rows * D;
        void *args[] = {&El, &idx, &rows, &V, &D, &L, &total, &off, &first, &z_hat, &z_rest};
        if (D % 4 == 0 && n / 4 <= UINT32_MAX - 256 && is_aligned16(El) && is_aligned16(z_hat) &&
            is_aligned16(z_rest)) {
            if (ncm_launch_named("vq_residual4", (unsigned)((n / 4 + 255) / 256), 1, 1, 256, args)) return;
        } else if (ncm_launch_named("vq_residual", (unsigned)((n + 255) / 256), 1, 1, 256, args)) {
            return;
        }
    }
}

void rowwise_l2sq(const float *a, const float *b, float *d2, int64_t rows, int64_t colsA, int C) {
    if (rows < 0 || colsA < 0 || C <= 0) {
        ncm_fail(NCM_E_ARG, "rowwise_l2sq: bad shape");
        return;
    }
    int64_t n = rows * colsA;
    if (n == 0) return;
    if (!a || !b || !d2) {
        ncm_fail(NCM_E_ARG, "rowwise_l2sq: null pointer");
        return;
    }
    if ((n + 255) / 256 > UINT_MAX) {
        ncm_fail(NCM_E_ARG, "rowwise_l2sq: too many outputs");
        return;
    }
    if (ncm_ready()) return;
    void *args[] = {&a, &b, &d2, &rows, &colsA, &C};
    ncm_launch_named("l2sq_exact", (unsigned)((n + 255) / 256), 1, 1, 256, args);
}

/* ------------------------------------------------------------------ */
/* The full multiscale quantizer: vq_load / vq_z_to_idx / vq_idx_to_zhats  */
/* (vq.c:76-197, 378-552) on device tensors.                              */
/* ------------------------------------------------------------------ */

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define VQ_MAX_STAGES 16
#define VQF_KMAX 16

struct VQState {
    int n_levels, D, L, total;
    int levels[NCM_MAX_LEVELS], vocabs[NCM_MAX_LEVELS];
    const float *E[NCM_MAX_LEVELS];
    int n_phi;                       /* 0: Phi off */
    float resi_ratio;
    const float *phiW[NCM_MAX_LEVELS], *phib[NCM_MAX_LEVELS];
    int n_down, n_up;                /* 0: no learned level-0 sampling */
    const float *downW[VQ_MAX_STAGES], *downB[VQ_MAX_STAGES], *upW[VQ_MAX_STAGES], *upB[VQ_MAX_STAGES];
    int downK[VQ_MAX_STAGES], upK[VQ_MAX_STAGES];
    int l1_norm, l1_norm_final;
    int has_all;
    const float *drefW[NCM_MAX_LEVELS], *drefB[NCM_MAX_LEVELS], *urefW[NCM_MAX_LEVELS], *urefB[NCM_MAX_LEVELS];
    float *ema_cs[NCM_MAX_LEVELS];   /* host [V]: EMA code counts (vq_ema_init) */
    float *ema_w[NCM_MAX_LEVELS];    /* device [V][D]: EMA code sums */
};

static Tensor *vq_weight(WeightStore *ws, const char *prefix, const char *name) {
    char key[320];
    snprintf(key, sizeof key, "%s%s", prefix ? prefix : "", name);
    return weights_get(ws, key);
}

/* A conv weight [D][D][k] with its bias [D]; k (out) is the last dimension. */
static int vq_conv_w(WeightStore *ws, const char *prefix, const char *wn, const char *bn, int D,
                     const float **W, const float **b, int *k) {
    Tensor *tw = vq_weight(ws, prefix, wn), *tb = vq_weight(ws, prefix, bn);
    if (!tw || !tb) return ncm_fail(NCM_E_ARG, "vq_load: missing weight %s%s", prefix ? prefix : "", !tw ? wn : bn);
    if (tw->ndim != 3 || tw->shape[0] != D || tw->shape[1] != D || tw->shape[2] < 1 || tw->shape[2] > VQF_KMAX ||
        tb->n != D)
        return ncm_fail(NCM_E_ARG, "vq_load: %s%s must be [%d][%d][k <= %d] with a [%d] bias", prefix ? prefix : "",
                        wn, D, D, VQF_KMAX, D);
    *W = tw->data;
    *b = tb->data;
    if (k) *k = (int)tw->shape[2];
    return 0;
}

VQState *vq_load(const NCMConfig *c, WeightStore *ws, const char *prefix) {
    if (!c || !ws) {
        ncm_fail(NCM_E_ARG, "vq_load: null config or store");
        return NULL;
    }
    const int n = c->n_qlevels, D = c->vq_embed_dim;
    if (n < 1 || n > NCM_MAX_LEVELS || D < 1 || D > VQ_MAXD) {
        ncm_fail(NCM_E_ARG, "vq_load: n_qlevels=%d, vq_embed_dim=%d out of range", n, D);
        return NULL;
    }
    VQState *v = (VQState *)calloc(1, sizeof *v);
    if (!v) {
        ncm_fail(NCM_E_OOM, "vq_load: state");
        return NULL;
    }
    v->n_levels = n;
    v->D = D;
    v->L = c->levels[n - 1];
    for (int i = 0; i < n; i++) {
        v->levels[i] = c->levels[i];
        v->vocabs[i] = c->vq_vocab[i];
        if (v->levels[i] < 1 || v->levels[i] > v->L || v->vocabs[i] < 1) {
            ncm_fail(NCM_E_ARG, "vq_load: level %d has length %d (L = %d) and vocab %d", i, v->levels[i], v->L,
                     v->vocabs[i]);
            goto fail;
        }
        v->total += v->levels[i];
        char nm[64];
        snprintf(nm, sizeof nm, "embeddings.%d.weight", i);
        Tensor *t = vq_weight(ws, prefix, nm);
        if (!t || t->n != (int64_t)v->vocabs[i] * D) {
            ncm_fail(NCM_E_ARG, "vq_load: %s%s %s", prefix ? prefix : "", nm, t ? "is not [vocab][D]" : "missing");
            goto fail;
        }
        v->E[i] = t->data;
    }
    /* Phi (vq.c:93-126): per level (share mode 0), shared (1) or k partially shared */
    if (c->quant_resi_enabled && fabsf(c->quant_resi_ratio) > 1e-6f) {
        const int sm = c->quant_resi_share_mode;
        v->n_phi = sm == 0 ? n : (sm == 1 ? 1 : sm);
        if (v->n_phi < 1 || v->n_phi > NCM_MAX_LEVELS) {
            ncm_fail(NCM_E_ARG, "vq_load: quant_resi_share_mode %d", sm);
            goto fail;
        }
        v->resi_ratio = c->quant_resi_ratio;
        for (int i = 0; i < v->n_phi; i++) {
            char wn[64], bn[64];
            snprintf(wn, sizeof wn, "quant_resi.%d.weight", i);
            if (!vq_weight(ws, prefix, wn) && v->n_phi == 1) snprintf(wn, sizeof wn, "quant_resi.weight");
            snprintf(bn, sizeof bn, "quant_resi.%d.bias", i);
            if (!vq_weight(ws, prefix, bn) && v->n_phi == 1) snprintf(bn, sizeof bn, "quant_resi.bias");
            int k = 0;
            if (vq_conv_w(ws, prefix, wn, bn, D, &v->phiW[i], &v->phib[i], &k)) goto fail;
            if (k != 3) {
                ncm_fail(NCM_E_ARG, "vq_load: %s has kernel %d, not 3", wn, k);
                goto fail;
            }
        }
    }
    /* learned level-0 cascade (vq.c:127-165): convs in module-index order */
    if (c->learned_l1_sampling) {
        v->l1_norm = c->learned_l1_norm;
        v->l1_norm_final = c->learned_l1_norm_final;
        for (int s = 0; s < VQ_MAX_STAGES; s++) {
            char wn[64], bn[64];
            snprintf(wn, sizeof wn, "learned_down_l1.%d.weight", s);
            snprintf(bn, sizeof bn, "learned_down_l1.%d.bias", s);
            if (vq_weight(ws, prefix, wn)) {
                if (vq_conv_w(ws, prefix, wn, bn, D, &v->downW[v->n_down], &v->downB[v->n_down], &v->downK[v->n_down]))
                    goto fail;
                v->n_down++;
            }
            snprintf(wn, sizeof wn, "learned_up_l1.%d.weight", s);
            snprintf(bn, sizeof bn, "learned_up_l1.%d.bias", s);
            if (vq_weight(ws, prefix, wn)) {
                if (vq_conv_w(ws, prefix, wn, bn, D, &v->upW[v->n_up], &v->upB[v->n_up], &v->upK[v->n_up])) goto fail;
                v->n_up++;
            }
        }
        if (!v->n_down) {
            ncm_fail(NCM_E_ARG, "vq_load: learned_l1 weights missing");
            goto fail;
        }
        /* the cascade must map L to levels[0] and back (the reference's buffers assume it) */
        int Td = v->L, Tu = v->levels[0];
        for (int i = 0; i < v->n_down; i++) Td /= v->downK[i];
        for (int i = 0; i < v->n_up; i++) Tu *= v->upK[i];
        if (Td != v->levels[0] || Tu != v->L || ((c->learned_l1_norm || c->learned_l1_norm_final) && D % 8)) {
            ncm_fail(NCM_E_ARG, "vq_load: learned level-0 cascade maps %d -> %d -> %d, not L=%d -> %d -> L "
                                "(or GroupNorm with D %% 8 != 0)", v->L, Td, Tu, v->L, v->levels[0]);
            goto fail;
        }
    }
    /* refine convs of the middle levels (vq.c:167-185) */
    if (c->learned_all_sampling) {
        v->has_all = 1;
        for (int i = 1; i <= n - 2; i++) {
            char wn[64], bn[64];
            int k = 3;
            snprintf(wn, sizeof wn, "learned_down_refine.%d.weight", i);
            snprintf(bn, sizeof bn, "learned_down_refine.%d.bias", i);
            if (vq_weight(ws, prefix, wn) && (vq_conv_w(ws, prefix, wn, bn, D, &v->drefW[i], &v->drefB[i], &k) || k != 3))
                goto fail_k;
            snprintf(wn, sizeof wn, "learned_up_refine.%d.weight", i);
            snprintf(bn, sizeof bn, "learned_up_refine.%d.bias", i);
            if (vq_weight(ws, prefix, wn) && (vq_conv_w(ws, prefix, wn, bn, D, &v->urefW[i], &v->urefB[i], &k) || k != 3))
                goto fail_k;
        }
    }
    return v;
fail_k:
    ncm_fail(NCM_E_ARG, "vq_load: refine conv of level with a kernel other than 3");
fail:
    free(v);
    return NULL;
}

static void vq_ema_release(VQState *vq);

void vq_free(VQState *vq) {
    if (!vq) return;
    vq_ema_release(vq);
    free(vq);
}
int vq_total_codes(const VQState *vq) { return vq ? vq->total : 0; }
int vq_nlevels(const VQState *vq) { return vq ? vq->n_levels : 0; }
int vq_level_len(const VQState *vq, int k) { return vq && k >= 0 && k < vq->n_levels ? vq->levels[k] : 0; }
int vq_level_V(const VQState *vq, int k) { return vq && k >= 0 && k < vq->n_levels ? vq->vocabs[k] : 0; }
int vq_Ltotal(const VQState *vq) { return vq ? vq->L : 0; }
int vq_Ddim(const VQState *vq) { return vq ? vq->D : 0; }

/* ---- device steps ---- */

static unsigned grid256(int64_t n) { return (unsigned)((n + 255) / 256); }

static int vqf_conv(const float *x, const float *W, const float *b, float *y, int B, int T, int D, int K, int stride,
                    int pad, int transposed, int *To_out) {
    int To = transposed ? (T - 1) * stride + K : (T + 2 * pad - K) / stride + 1;
    if (To_out) *To_out = To;
    void *a[] = {&x, &W, &b, &y, &T, &D, &D, &K, &stride, &pad, &To};
    const char *name = transposed ? "vqf_convT1d"
                       : (K == 3 && stride == 1 && pad == 1 && D % 32 == 0) ? "vqf_conv3" : "vqf_conv1d";
    return ncm_launch_named(name, (unsigned)((D + 63) / 64), (unsigned)((To + 15) / 16), (unsigned)B, 256, a);
}

int ncm_conv1d_btd(const float *x, const float *W, const float *b, float *y, int B, int T, int D, int K, int stride,
                   int pad) {
    return vqf_conv(x, W, b, y, B, T, D, K, stride, pad, 0, NULL);
}

static int vqf_gn(const float *x, float *y, int B, int T, int D) {
    void *a[] = {&x, &y, &T, &D};
    return ncm_launch_named("vqf_groupnorm", (unsigned)B * 8u, 1, 1, 64, a);
}

/* y rows b * ystride + yoff + t = area(x [B][Tin][D] -> Tout) */
static int vqf_area(const float *x, float *y, int B, int Tin, int Tout, int D, int ystride, int yoff) {
    void *a[] = {&x, &y, &B, &Tin, &Tout, &D, &ystride, &yoff};
    return ncm_launch_named("vqf_area", grid256((int64_t)B * Tout * D), 1, 1, 256, a);
}

static int vqf_mix(float *h, const float *c, int64_t n, float r, int add) {
    void *a[] = {&h, &c, &n, &r, &add};
    return ncm_launch_named("vqf_blend", grid256(n), 1, 1, 256, a);
}

/* Work buffers of one call: z_rest, z_hat, down, up, two cascade/conv
 * buffers (all [B][L][D]) and the device codes [B][total]. */
typedef struct {
    float *zr, *zh, *down, *up, *t1, *t2;
    int *idx;
} VqfWs;

static int vqf_ws(const VQState *v, int B, VqfWs *w) {
    const size_t n = (size_t)B * v->L * v->D * sizeof(float);
    const size_t a = (n + 255) & ~(size_t)255;
    char *base = (char *)ncm_workspace(WS_VQF, 6 * a + (size_t)B * v->total * sizeof(int));
    if (!base) return NCM_E_OOM;
    w->zr = (float *)base;
    w->zh = (float *)(base + a);
    w->down = (float *)(base + 2 * a);
    w->up = (float *)(base + 3 * a);
    w->t1 = (float *)(base + 4 * a);
    w->t2 = (float *)(base + 5 * a);
    w->idx = (int *)(base + 6 * a);
    return 0;
}

/* the learned cascade of level 0 from src [B][T][D] into dst (vq.c:285-309, 336-355) */
static int vqf_cascade(const VQState *v, const float *src, float *dst, VqfWs *w, int B, int T, int up) {
    const int D = v->D, n = up ? v->n_up : v->n_down;
    const float *cur = src;
    int Tc = T;
    for (int i = 0; i < n; i++) {
        const int s = up ? v->upK[i] : v->downK[i];
        if (v->l1_norm && i > 0) {
            float *g = cur == w->t1 ? w->t2 : w->t1;
            if (vqf_gn(cur, g, B, Tc, D)) return -1;
            cur = g;
        }
        float *nx = (i == n - 1 && !v->l1_norm_final) ? dst : (cur == w->t1 ? w->t2 : w->t1);
        int To;
        if (vqf_conv(cur, up ? v->upW[i] : v->downW[i], up ? v->upB[i] : v->downB[i], nx, B, Tc, D, s, s, 0, up, &To))
            return -1;
        cur = nx;
        Tc = To;
    }
    if (v->l1_norm_final) return vqf_gn(cur, dst, B, Tc, D) ? -1 : 0;
    if (n == 0) return ncm_copy_async(dst, src, (size_t)B * Tc * D * sizeof(float)) ? -1 : 0;
    return 0;
}

/* out += conv3(out) (the refine step) */
static int vqf_refine(const VQState *v, float *out, const float *W, const float *b, float *tmp, int B, int T) {
    if (vqf_conv(out, W, b, tmp, B, T, v->D, 3, 1, 1, 0, NULL)) return -1;
    return vqf_mix(out, tmp, (int64_t)B * T * v->D, 0.0f, 1);
}

static int phi_slot(const VQState *v, int lv) {
    if (v->n_phi == 1) return 0;
    const double at = (double)lv / (v->n_levels - 1);
    int best = 0;
    double bd = 1e300;
    for (int j = 0; j < v->n_phi; j++) {
        const double tick = v->n_phi == 4 ? (j + 1.0 / 3.0) / v->n_phi : (j + 0.5) / v->n_phi;
        const double d = fabs(tick - at);
        if (d < bd) {
            bd = d;
            best = j;
        }
    }
    return best;
}

/* up [B][L][D] <- level lv's codes up-sampled, refined and Phi-blended; the
 * codes of sequence b are idx[b * total + off + t] (device) */
static int vqf_level_up_at(const VQState *v, const int *idx, int total, int B, int lv, int off, VqfWs *w) {
    const int D = v->D, L = v->L, tl = v->levels[lv], V = v->vocabs[lv];
    const int64_t nq = (int64_t)B * tl * D, nL = (int64_t)B * L * D;
    const float *E = v->E[lv];
    float *q = w->down;   /* free at this point of a level */
    void *ga[] = {&E, &idx, (void *)&V, &total, &off, &B, (void *)&tl, (void *)&D, &q};
    if (ncm_launch_named("vqf_gather", grid256(nq), 1, 1, 256, ga)) return -1;
    if (lv == 0 && v->n_down > 0) {
        if (vqf_cascade(v, q, w->up, w, B, tl, 1)) return -1;
    } else {
        void *la[] = {&q, &w->up, &B, (void *)&tl, (void *)&L, (void *)&D};
        if (ncm_launch_named("vqf_linear", grid256(nL), 1, 1, 256, la)) return -1;
    }
    if (v->has_all && lv >= 1 && lv <= v->n_levels - 2 && v->urefW[lv] &&
        vqf_refine(v, w->up, v->urefW[lv], v->urefB[lv], w->t1, B, L))
        return -1;
    if (v->n_phi > 0) {
        const int j = phi_slot(v, lv);
        if (vqf_conv(w->up, v->phiW[j], v->phib[j], w->t1, B, L, D, 3, 1, 1, 0, NULL)) return -1;
        if (vqf_mix(w->up, w->t1, nL, v->resi_ratio, 0)) return -1;
    }
    return 0;
}

static int vqf_level_up(const VQState *v, const int *idx, int B, int lv, int off, VqfWs *w) {
    return vqf_level_up_at(v, idx, v->total, B, lv, off, w);
}

static int vqf_check(const VQState *vq, const float *z, int B, const char *fn) {
    if (!vq || !z || B < 0) return ncm_fail(NCM_E_ARG, "%s: bad arguments", fn);
    if ((int64_t)B * vq->L > INT_MAX / 2 || (int64_t)B * vq->total > INT_MAX)
        return ncm_fail(NCM_E_ARG, "%s: B=%d too large", fn, B);
    return ncm_ready();
}

static int g_soft_host_rows = 0;

int ncm_vq_soft_host_rows(void) { return g_soft_host_rows; }

/* vq.c:400-431: the soft draws of one level's rows (B * tl of them, codes
 * into idx [B][total] at column off + t).  The distances are the reference's
 * rowwise_l2sq values; a kernel takes each row's mean, minimum and weight sum
 * (fp64, in index order, as the reference's serial loops), the host steps the
 * xorshift64 state once per row whose mean is positive, in row order, and a
 * second kernel draws (or takes the argmin where the mean is not positive).
 * A draw the device's exp could have decided differently from glibc's (the
 * pick kernel marks it) is decided again here with the reference's loop and
 * libm exp, from the row's distances and the device's row statistics (the
 * same fp64 operations as the reference's, so the same values). */
static int vqf_soft(const float *down, const float *E, int *idx, int rows, int V, int D, int tl, int total, int off,
                    double tau, unsigned long long *rng) {
    const size_t dd_b = al256((size_t)rows * V * sizeof(float)), st_b = al256((size_t)rows * 3 * sizeof(double));
    const size_t u_b = al256((size_t)rows * sizeof(double)), f_b = al256((size_t)rows);
    char *base = (char *)ncm_workspace(WS_VQSOFT, dd_b + st_b + u_b + 2 * f_b);
    if (!base) return NCM_E_OOM;
    float *dd = (float *)base;
    double *st = (double *)(base + dd_b), *u = (double *)(base + dd_b + st_b);
    unsigned char *flag = (unsigned char *)(base + dd_b + st_b + u_b), *near = flag + f_b;
    rowwise_l2sq(down, E, dd, rows, V, D);
    void *a[] = {&dd, &rows, &V, &tau, &st, &flag};
    if (ncm_ready() || ncm_launch_named("vq_soft_stats", grid256(rows), 1, 1, 256, a)) return ncm_ready();
    unsigned char *fh = (unsigned char *)malloc((size_t)rows);
    double *uh = (double *)malloc((size_t)rows * sizeof(double));
    float *row = (float *)malloc((size_t)V * sizeof(float));
    int rc = 0;
    if (!fh || !uh || !row) {
        rc = ncm_fail(NCM_E_OOM, "vq_z_to_idx_soft: host draws of %d rows", rows);
        goto done;
    }
    mem_d2h(fh, flag, (size_t)rows);
    unsigned long long x = *rng;
    for (int r = 0; r < rows; r++) {
        if (!fh[r]) {
            uh[r] = -1.0;
            continue;
        }
        x ^= x << 13;
        x ^= x >> 7;
        x ^= x << 17;
        uh[r] = (double)(x >> 11) * (1.0 / 9007199254740992.0);
    }
    if (!ncm_ready()) *rng = x;
    mem_h2d(u, uh, (size_t)rows * sizeof(double));
    void *b[] = {&dd, &rows, &V, &st, &u, &idx, &tl, &total, &off, &near};
    if ((rc = ncm_ready()) || (rc = ncm_launch_named("vq_soft_pick", grid256(rows), 1, 1, 256, b))) goto done;
    mem_d2h(fh, near, (size_t)rows);
    for (int r = 0; r < rows && !(rc = ncm_ready()); r++) {
        if (!fh[r]) continue;
        double s3[3];
        mem_d2h(s3, st + 3 * (size_t)r, sizeof s3);
        mem_d2h(row, dd + (size_t)r * V, (size_t)V * sizeof(float));
        const double T = s3[0], bv = s3[1];
        double acc = 0, csum = 0;
        for (int j = 0; j < V; j++) acc += exp(-(row[j] - bv) / T);
        const double draw = uh[r] * acc;
        int bi = V - 1;
        for (int j = 0; j < V; j++) {
            csum += exp(-(row[j] - bv) / T);
            if (draw < csum) {
                bi = j;
                break;
            }
        }
        mem_h2d(idx + (size_t)(r / tl) * total + off + r % tl, &bi, sizeof bi);
        g_soft_host_rows++;
    }
done:
    free(fh);
    free(uh);
    free(row);
    return rc;
}

/* z_rest down-sampled to level lv's length into w->down (vq.c:280-330) */
static int vqf_down(const VQState *vq, VqfWs *w, int B, int lv) {
    const int tl = vq->levels[lv];
    if (lv == 0 && vq->n_down > 0) {
        if (vqf_cascade(vq, w->zr, w->down, w, B, vq->L, 0)) return 1;
    } else {
        if (vqf_area(w->zr, w->down, B, vq->L, tl, vq->D, tl, 0)) return 1;
    }
    if (vq->has_all && lv >= 1 && lv <= vq->n_levels - 2 && vq->drefW[lv] &&
        vqf_refine(vq, w->down, vq->drefW[lv], vq->drefB[lv], w->t1, B, tl))
        return 1;
    return 0;
}

static void vqf_run(VQState *vq, const float *z, int B, int *idx, float *z_hat, float *z_rest, int soft_levels,
                    double tau, unsigned long long *rng, const char *fn) {
    if (vqf_check(vq, z, B, fn) || B == 0) return;
    if (!idx) {
        ncm_fail(NCM_E_ARG, "%s: null idx", fn);
        return;
    }
    VqfWs w;
    if (vqf_ws(vq, B, &w)) return;
    const int D = vq->D, L = vq->L;
    const int64_t nL = (int64_t)B * L * D;
    if (ncm_copy_async(w.zr, z, (size_t)nL * sizeof(float))) return;
    int off = 0;
    for (int lv = 0; lv < vq->n_levels; lv++) {
        const int tl = vq->levels[lv];
        if (vqf_down(vq, &w, B, lv)) return;
        if (rng && lv < soft_levels && tau > 0) {
            if (vqf_soft(w.down, vq->E[lv], idx, B * tl, vq->vocabs[lv], D, tl, vq->total, off, tau, rng)) return;
        } else if (vq_search(w.down, vq->E[lv], idx, B * tl, vq->vocabs[lv], D, tl, vq->total, off, NULL)) {
            return;
        }
        if (vqf_level_up(vq, idx, B, lv, off, &w)) return;
        int init = lv == 0;
        void *ua[] = {&w.zh, &w.zr, &w.up, (void *)&nL, &init};
        if (ncm_launch_named("vqf_update", grid256(nL), 1, 1, 256, ua)) return;
        off += tl;
    }
    if (z_hat && ncm_copy_async(z_hat, w.zh, (size_t)nL * sizeof(float))) return;
    if (z_rest) ncm_copy_async(z_rest, w.zr, (size_t)nL * sizeof(float));
}

void vq_z_to_idx_dev(VQState *vq, const float *z, int B, int *idx, float *z_hat, float *z_rest) {
    vqf_run(vq, z, B, idx, z_hat, z_rest, 0, 0.0, NULL, "vq_z_to_idx_dev");
}

void vq_z_to_idx_soft(VQState *vq, const float *z, int B, int *idx, int soft_levels, double soft_tau,
                      unsigned long long *rng) {
    g_soft_host_rows = 0;
    if (vqf_check(vq, z, B, "vq_z_to_idx_soft") || B == 0) return;
    if (!idx) {
        ncm_fail(NCM_E_ARG, "vq_z_to_idx_soft: null idx");
        return;
    }
    VqfWs w;
    if (vqf_ws(vq, B, &w)) return;
    vqf_run(vq, z, B, w.idx, NULL, NULL, soft_levels, soft_tau, rng, "vq_z_to_idx_soft");
    mem_d2h(idx, w.idx, (size_t)B * vq->total * sizeof(int));
}

/* Frees the EMA state of every level and clears the pointers. */
static void vq_ema_release(VQState *vq) {
    for (int i = 0; i < NCM_MAX_LEVELS; i++) {
        free(vq->ema_cs[i]);
        vq->ema_cs[i] = NULL;
        if (vq->ema_w[i]) ncm_hip_free(vq->ema_w[i]);
        vq->ema_w[i] = NULL;
    }
}

/* Non-zero unless every level holds its EMA counts and sums. */
static int vq_ema_missing(const VQState *vq) {
    for (int i = 0; i < vq->n_levels; i++)
        if (!vq->ema_cs[i] || !vq->ema_w[i]) return 1;
    return 0;
}

/* vq.c:677-695: EMA counts 1 (host), EMA sums = the codebooks (device), once.
 * All or nothing: a failure at any level (allocation or copy) releases every
 * level, so the state is either whole or absent and a later call starts
 * again. */
static int vq_ema_prepare(VQState *vq) {
    int rc;
    if ((rc = ncm_ready())) return rc;
    if (!vq_ema_missing(vq)) return 0;
    vq_ema_release(vq);
    for (int i = 0; i < vq->n_levels; i++) {
        const int V = vq->vocabs[i];
        vq->ema_cs[i] = (float *)malloc((size_t)V * sizeof(float));
        vq->ema_w[i] = (float *)ncm_hip_malloc((size_t)V * vq->D * sizeof(float));
        if (!vq->ema_cs[i] || !vq->ema_w[i]) {
            rc = ncm_fail(NCM_E_OOM, "vq_ema_init: level %d", i);
            vq_ema_release(vq);
            return rc;
        }
        for (int v = 0; v < V; v++) vq->ema_cs[i][v] = 1.0f;
        if ((rc = ncm_copy_async(vq->ema_w[i], vq->E[i], (size_t)V * vq->D * sizeof(float)))) {
            vq_ema_release(vq);
            return rc;
        }
    }
    return 0;
}

void vq_ema_init(VQState *vq) {
    if (vq) vq_ema_prepare(vq);
}

/* vq.c:697-790.  codes: host [B][total] level-major, as the reference's.  Per
 * level the host does the counts (serial, fp64), the EMA counts and the
 * smoothing divisor per code, and lists each code's rows in row order; a
 * kernel per (code, d) sums the code's rows in that order (fp64, the
 * reference's order) into the EMA sums and rewrites the codebook the state
 * was loaded with; the residual then advances with the new codebook as in
 * vq_z_to_idx. */
void vq_ema_update(VQState *vq, const float *z, const int *codes, int B, double decay, double eps) {
    if (vqf_check(vq, z, B, "vq_ema_update") || B == 0) return;
    if (!codes) {
        ncm_fail(NCM_E_ARG, "vq_ema_update: null codes");
        return;
    }
    const int total = vq->total, D = vq->D;
    for (int lv = 0, off = 0; lv < vq->n_levels; off += vq->levels[lv], lv++)
        for (int b = 0; b < B; b++)
            for (int t = 0; t < vq->levels[lv]; t++) {
                const int c = codes[(size_t)b * total + off + t];
                if (c < 0 || c >= vq->vocabs[lv]) {
                    ncm_fail(NCM_E_ARG, "vq_ema_update: code %d outside [0, %d) at level %d", c, vq->vocabs[lv], lv);
                    return;
                }
            }
    VqfWs w;
    if (vq_ema_prepare(vq) || vq_ema_missing(vq) || vqf_ws(vq, B, &w)) return;
    const int64_t nL = (int64_t)B * vq->L * D;
    mem_h2d(w.idx, codes, (size_t)B * total * sizeof(int));
    if (ncm_ready() || ncm_copy_async(w.zr, z, (size_t)nL * sizeof(float))) return;
    int maxV = 0;
    for (int lv = 0; lv < vq->n_levels; lv++) maxV = vq->vocabs[lv] > maxV ? vq->vocabs[lv] : maxV;
    const int maxrows = B * vq->L;
    const size_t sm_b = al256((size_t)maxV * sizeof(double)), st_b = al256((size_t)(maxV + 1) * sizeof(int));
    char *base = (char *)ncm_workspace(WS_VQSOFT, sm_b + st_b + (size_t)maxrows * sizeof(int));
    double *smh = (double *)malloc(sm_b);
    int *sth = (int *)malloc(st_b), *lsh = (int *)malloc((size_t)maxrows * sizeof(int));
    double *cnt = (double *)malloc((size_t)maxV * sizeof(double));
    if (!base || !smh || !sth || !lsh || !cnt) {
        ncm_fail(NCM_E_OOM, "vq_ema_update: staging");
        goto done;
    }
    double *smd = (double *)base;
    int *std_ = (int *)(base + sm_b), *lsd = (int *)(base + sm_b + st_b);
    for (int lv = 0, off = 0; lv < vq->n_levels; off += vq->levels[lv], lv++) {
        const int tl = vq->levels[lv], V = vq->vocabs[lv], rows = B * tl;
        if (vqf_down(vq, &w, B, lv)) goto done;
        for (int v = 0; v < V; v++) cnt[v] = 0;
        for (int r = 0; r < rows; r++) cnt[codes[(size_t)(r / tl) * total + off + r % tl]] += 1.0;
        sth[0] = 0;
        for (int v = 0; v < V; v++) sth[v + 1] = sth[v] + (int)cnt[v];
        for (int v = 0; v < V; v++) smh[v] = sth[v];   /* fill cursors */
        for (int r = 0; r < rows; r++) {
            const int c = codes[(size_t)(r / tl) * total + off + r % tl];
            lsh[(int)smh[c]] = r;
            smh[c] += 1;
        }
        float *cs = vq->ema_cs[lv];
        double nsum = 0;
        for (int v = 0; v < V; v++) {
            const double keep = decay * cs[v], add = (1 - decay) * cnt[v];
            cs[v] = (float)(keep + add);
            nsum += cs[v];
        }
        for (int v = 0; v < V; v++) {
            const double a = cs[v] + eps, den = nsum + V * eps;
            smh[v] = a / den * nsum;
        }
        mem_h2d(smd, smh, (size_t)V * sizeof(double));
        mem_h2d(std_, sth, (size_t)(V + 1) * sizeof(int));
        mem_h2d(lsd, lsh, (size_t)rows * sizeof(int));
        float *E = (float *)vq->E[lv], *ew = vq->ema_w[lv];
        const int64_t n = (int64_t)V * D;
        void *a[] = {&w.down, &std_, &lsd, &smd, &ew, &E, (void *)&V, (void *)&D, &decay};
        if (ncm_ready() || ncm_launch_named("vq_ema_codebook", grid256(n), 1, 1, 256, a)) goto done;
        if (vqf_level_up(vq, w.idx, B, lv, off, &w)) goto done;
        int init = lv == 0;
        void *ua[] = {&w.zh, &w.zr, &w.up, (void *)&nL, &init};
        if (ncm_launch_named("vqf_update", grid256(nL), 1, 1, 256, ua)) goto done;
    }
done:   /* (every upload above is synchronous: the host staging is free to go) */
    free(smh);
    free(sth);
    free(lsh);
    free(cnt);
}

void vq_z_to_idx(VQState *vq, const float *z, int B, int *idx) {
    if (vqf_check(vq, z, B, "vq_z_to_idx") || B == 0) return;
    if (!idx) {
        ncm_fail(NCM_E_ARG, "vq_z_to_idx: null idx");
        return;
    }
    VqfWs w;
    if (vqf_ws(vq, B, &w)) return;
    vq_z_to_idx_dev(vq, z, B, w.idx, NULL, NULL);
    mem_d2h(idx, w.idx, (size_t)B * vq->total * sizeof(int));
}

void vq_idx_to_zhats(VQState *vq, const int *idx, int B, float **zhats) {
    if (!vq || !idx || !zhats || B < 0) {
        ncm_fail(NCM_E_ARG, "vq_idx_to_zhats: bad arguments");
        return;
    }
    if (B == 0 || vqf_check(vq, zhats[0], B, "vq_idx_to_zhats")) return;
    VqfWs w;
    if (vqf_ws(vq, B, &w)) return;
    mem_h2d(w.idx, idx, (size_t)B * vq->total * sizeof(int));
    const int64_t nL = (int64_t)B * vq->L * vq->D;
    float *none = NULL;
    int base = 0;
    for (int lv = 0; lv < vq->n_levels; lv++) {
        if (vqf_level_up(vq, w.idx, B, lv, base, &w)) return;
        int init = lv == 0;
        void *ua[] = {&w.zh, &none, &w.up, (void *)&nL, &init};
        if (ncm_launch_named("vqf_update", grid256(nL), 1, 1, 256, ua)) return;
        if (zhats[lv] && ncm_copy_async(zhats[lv], w.zh, (size_t)nL * sizeof(float))) return;
        base += vq->levels[lv];
    }
}

void vq_next_input(VQState *vq, const int *codes, int level_idx, float *z_hat, float *x_out, int B) {
    if (!vq || !codes || !z_hat || !x_out || B < 0 || level_idx < 0 || level_idx + 1 >= vq->n_levels) {
        ncm_fail(NCM_E_ARG, "vq_next_input: bad arguments (level %d of %d)", level_idx, vq ? vq->n_levels : 0);
        return;
    }
    if (B == 0 || vqf_check(vq, z_hat, B, "vq_next_input")) return;
    VqfWs w;
    if (vqf_ws(vq, B, &w)) return;
    const int tl = vq->levels[level_idx], nlen = vq->levels[level_idx + 1];
    mem_h2d(w.idx, codes, (size_t)B * tl * sizeof(int));
    if (vqf_level_up_at(vq, w.idx, tl, B, level_idx, 0, &w)) return;
    const int64_t nL = (int64_t)B * vq->L * vq->D;
    float *none = NULL;
    int init = 0;
    void *ua[] = {&z_hat, &none, &w.up, (void *)&nL, &init};
    if (ncm_launch_named("vqf_update", grid256(nL), 1, 1, 256, ua)) return;
    vqf_area(z_hat, x_out, B, vq->L, nlen, vq->D, nlen, 0);
}

void vq_idx_to_ncm_input(VQState *vq, const int *idx, int B, float *x_out) {
    if (!vq || !idx || !x_out || B < 0) {
        ncm_fail(NCM_E_ARG, "vq_idx_to_ncm_input: bad arguments");
        return;
    }
    if (B == 0 || vqf_check(vq, x_out, B, "vq_idx_to_ncm_input")) return;
    VqfWs w;
    if (vqf_ws(vq, B, &w)) return;
    mem_h2d(w.idx, idx, (size_t)B * vq->total * sizeof(int));
    const int T = vq->total - vq->levels[0];
    const int64_t nL = (int64_t)B * vq->L * vq->D;
    float *none = NULL;
    int base = 0, off = 0;
    for (int li = 0; li < vq->n_levels - 1; li++) {
        if (vqf_level_up(vq, w.idx, B, li, base, &w)) return;
        int init = li == 0;
        void *ua[] = {&w.zh, &none, &w.up, (void *)&nL, &init};
        if (ncm_launch_named("vqf_update", grid256(nL), 1, 1, 256, ua)) return;
        const int nlen = vq->levels[li + 1];
        if (vqf_area(w.zh, x_out, B, vq->L, nlen, vq->D, T, off)) return;
        base += vq->levels[li];
        off += nlen;
    }
}
