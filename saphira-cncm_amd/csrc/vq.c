/* vq.c -- host side of the VQ nearest-codeword search and the multiscale
 * residual loop (reference: kernels.c:753-770, vq.c:378-500). */
#include "internal.h"

#include <limits.h>

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

static int vq_scratch(VqScratch *s, int rows, int V) {
    size_t off_cn = 256;
    size_t off_xn = off_cn + al256((size_t)V * 4);
    size_t off_fl = off_xn + al256((size_t)rows * 4);
    size_t off_pr = off_fl + al256((size_t)rows * 4);
    size_t off_ky = off_pr + al256((size_t)rows * 12);
    size_t off_dn = off_ky + al256((size_t)rows * 8);
    size_t total = off_dn + (size_t)rows * 4;
    unsigned char *base = (unsigned char *)ncm_workspace(WS_VQ, total);
    if (!base) return NCM_E_OOM;
    s->counters = (unsigned *)base;
    s->cn = (float *)(base + off_cn);
    s->xn = (float *)(base + off_xn);
    s->flags = (int *)(base + off_fl);
    s->pairs = (int *)(base + off_pr);
    s->keys = (unsigned long long *)(base + off_ky);
    s->done = (unsigned *)(base + off_dn);
    return 0;
}

/* codes of `rows` rows of X against E, written at idx[(row/L)*total + off + row%L] */
static int vq_search(const float *X, const float *E, int *idx, int rows, int V, int D, int L,
                     int total, int off) {
    VqScratch s;
    if (vq_scratch(&s, rows, V)) return NCM_E_OOM;
    int rc;
    void *a0[] = {&s.counters};
    if ((rc = ncm_launch_named("vq_init", 1, 1, 1, 64, a0))) return rc;
    unsigned *cmax = s.counters + 1;
    void *a1[] = {&E, &V, &D, &s.cn, &cmax};
    if ((rc = ncm_launch_named("vq_prep_codebook", (unsigned)((V + 255) / 256), 1, 1, 256, a1))) return rc;
    void *a2[] = {&X, &rows, &D, &s.xn};
    if ((rc = ncm_launch_named("vq_rownorm", (unsigned)((rows + 3) / 4), 1, 1, 256, a2))) return rc;

    int vec = (D % 4 == 0) && is_aligned16(X) && is_aligned16(E);
    VqArgs p = {X, E, s.cn, s.xn, cmax, idx, s.flags, (int *)s.counters,
                s.pairs, (int *)s.counters + 2, s.keys, s.done, rows, V, D, L, total, off};
    void *a3[] = {&p};
    if ((rc = ncm_launch_named(vec ? "vq_argmin_main_v" : "vq_argmin_main_s", (unsigned)((rows + 63) / 64), 1,
                               1, 256, a3)))
        return rc;
    const unsigned *cnt = s.counters;
    void *a4[] = {&X, &E, &V, &D, &vec, &s.flags, &s.pairs, &cnt, &s.keys, &s.done, &idx, &L, &total, &off};
    return ncm_launch_named("vq_rescore", RESCORE_GRID, 1, 1, 256, a4);
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
    vq_search(a, E, idx, (int)rows, V, D, (int)rows, (int)rows, 0);
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
        if (vq_search(z_rest, E[lv], idx, rows, vocabs[lv], D, L, total, off)) return;
        const float *El = E[lv];
        int V = vocabs[lv];
        int first = lv == 0;
        int64_t n = (int64_t)rows * D;
        void *args[] = {&El, &idx, &rows, &V, &D, &L, &total, &off, &first, &z_hat, &z_rest};
        if (ncm_launch_named("vq_residual", (unsigned)((n + 255) / 256), 1, 1, 256, args)) return;
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
