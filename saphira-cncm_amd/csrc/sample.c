/* sample.c -- host side of the device sampler (csrc/sample.hip): the
 * reference's sample_topkp (src/kernels.c:782-825) with the row on the
 * device.  Launch sequence per row: 4 radix passes (a digit histogram, then
 * a scatter that forms its own offsets from it), the probabilities, and the
 * one-workgroup finish: 10 launches. */
#define _GNU_SOURCE /* qsort_r */
#include "internal.h"

#include <limits.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define SMP_NT 1024
#define SMP_SB 8192
#define SMP_MAXB 32
#define SMP_PB 1024
#define SMP_VMAX (SMP_SB * SMP_MAXB)

/* Must match struct SmpFinishArgs in sample.hip. */
typedef struct {
    const float *x;
    float temp;
    int keep;
    float top_p;
    const int *idx;
    const double *p;
    const double *bsum;
    int nbp;
    const int *bad;
    int nblk;
    unsigned long long *rng;
    int *out;
    int *ids;
    int *pos;
    int *flag;
    int n;
} SmpFinishArgs;

/* Workspace: sort keys and indices (two buffers each), the histogram, the
 * per-block non-finite flags, probabilities and block sums, and the staging
 * of the host entry point (row, rng, id, flag). */
typedef struct {
    unsigned *k[2];
    int *i[2];
    int *hist, *bad;
    double *p, *bsum;
    float *row;
    unsigned long long *rng;
    int *out, *flag;
} SmpWs;

static size_t up8(size_t n) { return (n + 7) & ~(size_t)7; }

/* Byte offsets of the workspace parts for a row of V; returns the total. */
static size_t smp_layout(int V, size_t off[12]) {
    const int nblk = (V + SMP_SB - 1) / SMP_SB, nbp = (V + SMP_PB - 1) / SMP_PB;
    const size_t v4 = up8((size_t)V * 4);
    size_t total = 0;
    const size_t sz[12] = {v4, v4, v4, v4, up8((size_t)4 * 256 * nblk * 4), up8((size_t)nblk * 4),
                           (size_t)V * 8, (size_t)nbp * 8, v4, 8, 8, 8};
    for (int j = 0; j < 12; j++) {
        off[j] = total;
        total += sz[j];
    }
    return total;
}

size_t ncm_sample_ws_bytes(int V) {
    size_t off[12];
    return V >= 1 && V <= SMP_VMAX ? smp_layout(V, off) : 0;
}

/* Carves the workspace from own (a caller-owned buffer of
 * ncm_sample_ws_bytes(V)) or, when own is null, from the library's. */
static int smp_ws_at(int V, void *own, SmpWs *w) {
    size_t off[12];
    const size_t total = smp_layout(V, off);
    char *b = own ? (char *)own : (char *)ncm_workspace(WS_SAMPLE, total);
    if (!b) return NCM_E_OOM;
    w->k[0] = (unsigned *)(b + off[0]);
    w->k[1] = (unsigned *)(b + off[1]);
    w->i[0] = (int *)(b + off[2]);
    w->i[1] = (int *)(b + off[3]);
    w->hist = (int *)(b + off[4]);
    w->bad = (int *)(b + off[5]);
    w->p = (double *)(b + off[6]);
    w->bsum = (double *)(b + off[7]);
    w->row = (float *)(b + off[8]);
    w->rng = (unsigned long long *)(b + off[9]);
    w->out = (int *)(b + off[10]);
    w->flag = (int *)(b + off[11]);
    return 0;
}

static int smp_ws(int V, SmpWs *w) { return smp_ws_at(V, NULL, w); }

static int smp_check(const char *fn, const float *x, int V, float top_p) {
    if (!x || V < 1 || V > SMP_VMAX)
        return ncm_fail(NCM_E_ARG, "%s: need logits and 1 <= V <= %d (V = %d)", fn, SMP_VMAX, V);
    if (top_p < 0.0f)
        /* the reference then keeps no rank and reads ord[-1] (kernels.c:812-819) */
        return ncm_fail(NCM_E_ARG, "%s: top_p must be >= 0 (got %g)", fn, (double)top_p);
    return 0;
}

/* The device sampler for temp > 0: sorts the row, then the finish kernel
 * writes the id to *out and the flag to *flag, or, when pos is set, to
 * ids[*pos + 1] and flag[*pos + 1] and advances *pos.  All pointers are
 * device memory; launches only (no copies, no fills), so the sequence can
 * be captured in a graph (with ws, a caller-owned workspace, whose address
 * then stays valid). */
int ncm_sample_launch(const float *x, int V, float temp, int top_k, float top_p, unsigned long long *rng,
                      int *out, int *ids, int *pos, int *flag, void *ws) {
    int rc = smp_check("sample", x, V, top_p);
    if (rc) return rc;
    if (!(temp > 0.0f)) return ncm_fail(NCM_E_ARG, "sample: temp must be > 0 on the sampling path");
    if (!rng || !flag || (!out && !(ids && pos))) return ncm_fail(NCM_E_ARG, "sample: null pointer");
    if ((rc = ncm_ready())) return rc;
    SmpWs w;
    if ((rc = smp_ws_at(V, ws, &w))) return rc;
    const int nblk = (V + SMP_SB - 1) / SMP_SB;
    const int keep = top_k > 0 && top_k < V ? top_k : V, nbp = (keep + SMP_PB - 1) / SMP_PB;
    const unsigned *kin = NULL;
    const int *iin = NULL;
    for (int pass = 0; pass < 4; pass++) {
        unsigned *kout = w.k[pass & 1];
        int *iout = w.i[pass & 1];
        void *ha[] = {&x, &temp, &kin, &V, &pass, &w.hist, (void *)&nblk, &w.bad};
        if ((rc = ncm_launch_named("smp_hist", (unsigned)nblk, 1, 1, SMP_NT, ha))) return rc;
        void *ca[] = {&x, &temp, &kin, &iin, &V, &pass, &w.hist, (void *)&nblk, &kout, &iout};
        if ((rc = ncm_launch_named("smp_scatter", (unsigned)nblk, 1, 1, SMP_NT, ca))) return rc;
        kin = kout;
        iin = iout;
    }
    const int *idx = iin;
    void *pa[] = {&x, &temp, &idx, &V, (void *)&keep, &w.p, &w.bsum};
    if ((rc = ncm_launch_named("smp_probs", (unsigned)nbp, 1, 1, 256, pa))) return rc;
    SmpFinishArgs f = {x, temp, keep, top_p, idx, w.p, w.bsum, nbp, w.bad, nblk, rng, out, ids, pos, flag, V};
    void *fa[] = {&f};
    return ncm_launch_named("smp_finish", 1, 1, 1, 1024, fa);
}

void sample_topkp_dev(const float *logits, int V, float temp, int top_k, float top_p,
                      unsigned long long *rng, int *out, int *flag) {
    if (smp_check("sample_topkp_dev", logits, V, top_p)) return;
    if (!out || !rng) {
        ncm_fail(NCM_E_ARG, "sample_topkp_dev: null pointer");
        return;
    }
    if (ncm_ready()) return;
    if (!(temp > 0.0f)) {
        /* kernels.c:796: greedy, the rng untouched */
        int n = V;
        void *args[] = {&logits, &n, &out};
        if (ncm_launch_named("argmax_rows_k", 1, 1, 1, 256, args)) return;
        if (flag) ncm_zero_async(flag, sizeof(int));
        return;
    }
    int *fl = flag;
    if (!fl) {
        SmpWs w;
        if (smp_ws(V, &w)) return;
        fl = w.flag;
    }
    ncm_sample_launch(logits, V, temp, top_k, top_p, rng, out, NULL, NULL, fl, NULL);
}

unsigned long long rng_next(unsigned long long *state) {
    unsigned long long v = *state;
    v ^= v >> 12;
    v ^= v << 25;
    v ^= v >> 27;
    *state = v;
    return v * 0x2545F4914F6CDD1DULL;
}

static int g_last_flag = 0;

int ncm_hip_sample_flag(void) { return g_last_flag; }

/* Descending order of the scaled logits, comparing values only: equal values
 * (and any pair involving a NaN) compare equal, as the reference's comparator
 * does (kernels.c:784-789); glibc's qsort is a stable merge sort, so equal
 * values keep their index order. */
static int smp_cmp_desc(const void *a, const void *b, void *ctx) {
    const float *w = (const float *)ctx;
    const float va = w[*(const int *)a], vb = w[*(const int *)b];
    return (va < vb) - (va > vb);
}

/* The reference's draw, recomputed on the host from the caller's row and the
 * rng state before the device draw (kernels.c:794-825): the row divided by
 * temp in float, the index order sorted by glibc's qsort with the comparator
 * above, fp64 exponentials relative to the maximum over the first keep ranks
 * and their serial sum, the nucleus cut at the first rank whose preceding
 * mass minus its own exceeds top_p, then u = U * (the kept mass, summed
 * again) against the running sum, U from one xorshift64* step.  Used when
 * the device cannot certify its draw equal to this one.  Returns the id, or
 * -1 (error recorded) when host memory runs out. */
static int smp_host_draw(const float *logits, int V, float temp, int top_k, float top_p,
                         unsigned long long *rng) {
    float *w = (float *)malloc((size_t)V * sizeof *w);
    int *ord = (int *)malloc((size_t)V * sizeof *ord);
    double *q = (double *)malloc((size_t)V * sizeof *q);
    if (!w || !ord || !q) {
        free(w);
        free(ord);
        free(q);
        ncm_fail(NCM_E_OOM, "sample_topkp: no host memory for the exact draw (V = %d)", V);
        return -1;
    }
    for (int i = 0; i < V; i++) {
        w[i] = logits[i] / temp;
        ord[i] = i;
    }
    qsort_r(ord, (size_t)V, sizeof *ord, smp_cmp_desc, w);
    const int keep = top_k > 0 && top_k < V ? top_k : V;
    const double top = w[ord[0]];
    double total = 0.0;
    for (int r = 0; r < keep; r++) {
        q[r] = exp((double)w[ord[r]] - top);
        total += q[r];
    }
    for (int r = 0; r < keep; r++) q[r] /= total;
    int cut = keep;
    double before = 0.0;
    for (int r = 0; r < keep; r++) {
        if (before - q[r] > top_p) {
            cut = r;
            break;
        }
        before += q[r];
    }
    /* top_p >= 0 (checked by the caller), so rank 0 is always kept */
    double mass = 0.0;
    for (int r = 0; r < cut; r++) mass += q[r];
    const double u = (double)(rng_next(rng) >> 11) * (1.0 / 9007199254740992.0) * mass;
    int pick = ord[cut - 1];
    double run = 0.0;
    for (int r = 0; r < cut; r++) {
        run += q[r];
        if (u <= run) {
            pick = ord[r];
            break;
        }
    }
    free(w);
    free(ord);
    free(q);
    return pick;
}

int sample_topkp(const float *logits, int V, float temp, int top_k, float top_p, unsigned long long *rng) {
    g_last_flag = 0;
    if (!logits || V < 1) {
        ncm_fail(NCM_E_ARG, "sample_topkp: need logits and V >= 1");
        return 0;
    }
    if (!(temp > 0.0f)) return argmax_row(logits, V);   /* host row, as the reference */
    if (!rng) {
        ncm_fail(NCM_E_ARG, "sample_topkp: null rng");
        return 0;
    }
    if (smp_check("sample_topkp", logits, V, top_p) || ncm_ready()) return 0;
    SmpWs w;
    if (smp_ws(V, &w)) return 0;
    hipStream_t s = ncm_stream();
    const unsigned long long rng0 = *rng;
    int res[2] = {0, 0};
    if (hipMemcpyAsync(w.row, logits, (size_t)V * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(w.rng, rng, 8, hipMemcpyHostToDevice, s) != hipSuccess) {
        ncm_fail(NCM_E_HIP, "sample_topkp: copy of the row failed");
        return 0;
    }
    if (ncm_sample_launch(w.row, V, temp, top_k, top_p, w.rng, w.out, NULL, NULL, w.flag, NULL)) return 0;
    if (hipMemcpyAsync(&res[0], w.out, 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipMemcpyAsync(&res[1], w.flag, 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipMemcpyAsync(rng, w.rng, 8, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        ncm_fail(NCM_E_HIP, "sample_topkp: copy of the result failed");
        return 0;
    }
    g_last_flag = res[1];
    if (res[1] != 0) {
        /* the device draw is not certified equal to the reference's (u within
         * the rounding bound of a cumulative sum, or non-finite logits): the
         * row is host memory here, so draw again exactly as the reference
         * does from the state the call started with (one rng step either
         * way); the flag stays readable through ncm_hip_sample_flag */
        unsigned long long st = rng0;
        const int pick = smp_host_draw(logits, V, temp, top_k, top_p, &st);
        if (pick < 0) return 0;
        *rng = st;
        return pick;
    }
    return res[0];
}
