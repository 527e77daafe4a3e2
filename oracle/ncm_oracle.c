/* ncm_oracle.c -- CPU restatement of the reference arithmetic (test
 * infrastructure only; see ncm_oracle.h).
 *
 * Parallel loops partition outputs only and keep each output's serial
 * reduction order, so results do not depend on the thread count (the same
 * property the reference states in ARCHITECTURE.md:50-54). */
#include "ncm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* kernels.c:38-54: per output, acc starts at the bias (double), adds
 * (double)x*W over k ascending, and is rounded to float once. */
void orc_linear_fwd(const float *x, const float *W, const float *b, float *y,
                    int64_t batch, int M, int K) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < batch; r++) {
        const float *xr = x + r * K;
        for (int m = 0; m < M; m++) {
            const float *wr = W + (int64_t)m * K;
            double acc = b ? (double)b[m] : 0.0;
            for (int k = 0; k < K; k++) acc += (double)xr[k] * (double)wr[k];
            y[r * M + m] = (float)acc;
        }
    }
}

/* train_tape.c:680-725.  dx: per (r,k) an fp64 sum over m ascending, rounded
 * to float, then added into dx.  dW and db: per output an fp64 sum over r
 * ascending, rounded to float and added into a zeroed temporary, which is
 * then added into the gradient (hadd_into, train_tape.c:535-537); the
 * temporary turns a -0.0 sum into +0.0 before it reaches the gradient. */
void orc_linear_bwd(const float *x, const float *W, const float *dy,
                    float *dx, float *dW, float *db, int64_t batch, int M, int K) {
    if (dx) {
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < batch; r++)
            for (int k = 0; k < K; k++) {
                double s = 0.0;
                for (int m = 0; m < M; m++) s += (double)dy[r * M + m] * (double)W[(int64_t)m * K + k];
                dx[r * K + k] += (float)s;
            }
    }
    if (dW || db) {
#pragma omp parallel for schedule(static)
        for (int m = 0; m < M; m++) {
            if (db) {
                double bs = 0.0;
                for (int64_t r = 0; r < batch; r++) bs += dy[r * M + m];
                float t = 0.0f;
                t += (float)bs;
                db[m] += t;
            }
            if (dW)
                for (int k = 0; k < K; k++) {
                    double s = 0.0;
                    for (int64_t r = 0; r < batch; r++) s += (double)dy[r * M + m] * (double)x[r * K + k];
                    float t = 0.0f;
                    t += (float)s;
                    dW[(int64_t)m * K + k] += t;
                }
        }
    }
}

/* kernels.c:753-770: diff in double, square and add as separate roundings
 * (no contraction under -std=c11), serial over c, rounded to float. */
static float l2sq_one(const float *a, const float *b, int C) {
    double s = 0.0;
    for (int c = 0; c < C; c++) {
        double d = (double)a[c] - (double)b[c];
        s += d * d;
    }
    return (float)s;
}

void orc_l2sq(const float *a, const float *b, float *d2, int64_t rows, int64_t cols, int C) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < rows; i++)
        for (int64_t j = 0; j < cols; j++) d2[i * cols + j] = l2sq_one(a + i * C, b + j * C, C);
}

/* vq.c:440-443: start at index 0 with its float distance, replace only on a
 * strictly smaller float value. */
void orc_vq_argmin(const float *a, const float *E, int *idx, int64_t rows, int V, int D) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < rows; i++) {
        const float *x = a + i * D;
        float bv = l2sq_one(x, E, D);
        int bi = 0;
        for (int j = 1; j < V; j++) {
            float d = l2sq_one(x, E + (int64_t)j * D, D);
            if (d < bv) {
                bv = d;
                bi = j;
            }
        }
        idx[i] = bi;
    }
}

/* vq.c:388-500 with identity resampling and no Phi: z_rest = z, z_hat = 0;
 * per level: codes by argmin over E[lv]; q = E[code];
 * z_hat += q; z_rest -= q (float).  Codes are stored level-major per batch
 * row: idx[b*total + lv*L + t] (vq.c:444-445). */
void orc_vq_multiscale(const float *z, const float *const *E, const int *vocabs,
                       int n_levels, int B, int L, int D,
                       int *idx, float *z_hat, float *z_rest) {
    int64_t rows = (int64_t)B * L;
    int64_t n = rows * D;
    int total = n_levels * L;
    memcpy(z_rest, z, (size_t)n * sizeof(float));
    memset(z_hat, 0, (size_t)n * sizeof(float));
    int *codes = (int *)malloc((size_t)(rows ? rows : 1) * sizeof(int));
    for (int lv = 0; lv < n_levels; lv++) {
        orc_vq_argmin(z_rest, E[lv], codes, rows, vocabs[lv], D);
        for (int64_t r = 0; r < rows; r++)
            idx[(r / L) * total + (int64_t)lv * L + r % L] = codes[r];
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            const float *q = E[lv] + (int64_t)codes[r] * D;
            for (int c = 0; c < D; c++) {
                z_hat[r * D + c] += q[c];
                z_rest[r * D + c] -= q[c];
            }
        }
    }
    free(codes);
}

/* kernels.c:731-735 */
int orc_argmax_row(const float *x, int n) {
    int bi = 0;
    float bv = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > bv) {
            bv = x[i];
            bi = i;
        }
    return bi;
}

/* kernels.c:185-194 */
void orc_gelu(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float v = x[i];
        y[i] = 0.5f * v * (1.0f + erff(v * 0.7071067811865475f));
    }
}

/* kernels.c:207-218 (CPU branch evaluates in double) */
void orc_gelu_tanh(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        double v = x[i];
        double t = 0.7978845608028654 * (v + 0.044715 * v * v * v);
        y[i] = (float)(0.5 * v * (1.0 + tanh(t)));
    }
}

/* kernels.c:220-226 */
void orc_silu(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float v = x[i];
        y[i] = v / (1.0f + expf(-v));
    }
}

/* kernels.c:843-849 */
void orc_add(const float *a, const float *b, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = a[i] + b[i];
}

/* kernels.c:774-780 xorshift64* */
uint64_t orc_rng_next(uint64_t *state) {
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return x * 0x2545F4914F6CDD1DULL;
}

/* kernels.c:782-825 sample_topkp.  The reference sorts the indices with
 * glibc's qsort under a (value desc) comparator; glibc 2.35 sorts with a
 * stable merge sort, so equal values keep ascending index order.  Here the
 * order is the total order (value desc, index asc), which any sort yields
 * identically -- the same permutation for finite inputs (NaN, on which the
 * reference's comparator is inconsistent, is outside this restatement). */
typedef struct { float v; int i; } OrcVI;

static int orc_vi_desc(const void *a, const void *b) {
    const OrcVI *x = (const OrcVI *)a, *y = (const OrcVI *)b;
    if (x->v != y->v) return x->v > y->v ? -1 : 1;
    return (x->i > y->i) - (x->i < y->i);
}

int orc_sample_topkp(const float *logits, int V, float temp, int top_k, float top_p, uint64_t *rng) {
    if (!(temp > 0)) return orc_argmax_row(logits, V);
    OrcVI *s = (OrcVI *)malloc((size_t)V * sizeof *s);
    double *q = (double *)malloc((size_t)V * sizeof *q);
    for (int i = 0; i < V; i++) {
        s[i].v = logits[i] / temp;
        s[i].i = i;
    }
    qsort(s, (size_t)V, sizeof *s, orc_vi_desc);
    const int keep = top_k > 0 && top_k < V ? top_k : V;
    /* unnormalised probabilities relative to the maximum, fp64 serial sum */
    const double mx = s[0].v;
    double den = 0.0;
    for (int r = 0; r < keep; r++) {
        q[r] = exp((double)s[r].v - mx);
        den += q[r];
    }
    for (int r = 0; r < keep; r++) q[r] /= den;
    /* nucleus: the first rank whose preceding mass minus its own exceeds top_p */
    int nkeep = keep;
    double before = 0.0;
    for (int r = 0; r < keep; r++) {
        if (before - q[r] > top_p) {
            nkeep = r;
            break;
        }
        before += q[r];
    }
    if (nkeep == 0) { /* top_p < -q[0]: the reference then reads ord[-1] */
        free(s);
        free(q);
        return -1;
    }
    double mass = 0.0;
    for (int r = 0; r < nkeep; r++) mass += q[r];
    const double u = (double)(orc_rng_next(rng) >> 11) * (1.0 / 9007199254740992.0) * mass;
    int pick = s[nkeep - 1].i;
    double run = 0.0;
    for (int r = 0; r < nkeep; r++) {
        run += q[r];
        if (u <= run) {
            pick = s[r].i;
            break;
        }
    }
    free(s);
    free(q);
    return pick;
}

/* ---- the full multiscale quantizer (src/vq.c), [B][T][D] layout ---- */

/* kernels.c:681-700 interpolate_area_fwd per (b, d) column: output t
 * averages inputs [floor(t Tin / Tout), ceil((t + 1) Tin / Tout)) in fp64. */
static void orc_area(const float *x, float *y, int B, int Tin, int Tout, int D) {
    for (int b = 0; b < B; b++)
        for (int d = 0; d < D; d++)
            for (int t = 0; t < Tout; t++) {
                int64_t s = (int64_t)((double)t * Tin / Tout);
                int64_t e = (int64_t)ceil((double)(t + 1) * Tin / Tout);
                if (e <= s) e = s + 1;
                if (s < 0) s = 0;
                if (e > Tin) e = Tin;
                double acc = 0;
                for (int64_t k = s; k < e; k++) acc += x[((int64_t)b * Tin + k) * D + d];
                y[((int64_t)b * Tout + t) * D + d] = (float)(acc / (double)(e - s));
            }
}

/* kernels.c:702-727 interpolate_linear_fwd (align_corners = False; a
 * length-1 side averages) */
static void orc_lin(const float *x, float *y, int B, int Tin, int Tout, int D) {
    for (int b = 0; b < B; b++)
        for (int d = 0; d < D; d++) {
            const float *xc = x + (int64_t)b * Tin * D + d;
            float *yc = y + (int64_t)b * Tout * D + d;
            if (Tout == 1 || Tin == 1) {
                double acc = 0;
                for (int k = 0; k < Tin; k++) acc += xc[(int64_t)k * D];
                for (int t = 0; t < Tout; t++) yc[(int64_t)t * D] = (float)(acc / Tin);
                continue;
            }
            const double scale = (double)Tin / Tout;
            for (int t = 0; t < Tout; t++) {
                const double src = (t + 0.5) * scale - 0.5;
                const int64_t s0 = (int64_t)floor(src), s1 = s0 + 1;
                const double w1 = src - s0, w0 = 1.0 - w1;
                const double v0 = xc[(s0 < 0 ? 0 : (s0 >= Tin ? Tin - 1 : s0)) * (int64_t)D];
                const double v1 = xc[(s1 < 0 ? 0 : (s1 >= Tin ? Tin - 1 : s1)) * (int64_t)D];
                yc[(int64_t)t * D] = (float)(w0 * v0 + w1 * v1);
            }
        }
}

/* kernels.c:546-566 conv1d_fwd: fp64 over ci (outer) and k (inner), W [Cout][Cin][K] */
static void orc_conv1d(const float *x, const float *W, const float *bias, float *y, int B, int T, int Cin,
                       int Cout, int K, int stride, int pad) {
    const int64_t To = (T + 2 * pad - K) / stride + 1;
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; b++)
        for (int64_t t = 0; t < To; t++)
            for (int co = 0; co < Cout; co++) {
                double acc = bias ? bias[co] : 0.0;
                for (int ci = 0; ci < Cin; ci++)
                    for (int k = 0; k < K; k++) {
                        const int ti = (int)(t * stride + k - pad);
                        if (ti < 0 || ti >= T) continue;
                        acc += (double)x[((int64_t)b * T + ti) * Cin + ci] * W[((int64_t)co * Cin + ci) * K + k];
                    }
                y[((int64_t)b * To + t) * Cout + co] = (float)acc;
            }
}

/* kernels.c:568-590 convtranspose1d_fwd: W [Cin][Cout][K], output length (T - 1) s + K */
static void orc_convT1d(const float *x, const float *W, const float *bias, float *y, int B, int T, int Cin,
                        int Cout, int K, int stride) {
    const int64_t To = (int64_t)(T - 1) * stride + K;
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; b++)
        for (int64_t t = 0; t < To; t++)
            for (int co = 0; co < Cout; co++) {
                double acc = bias ? bias[co] : 0.0;
                for (int ci = 0; ci < Cin; ci++)
                    for (int k = 0; k < K; k++) {
                        const int num = (int)(t - k);
                        if (num < 0 || num % stride != 0) continue;
                        const int ti = num / stride;
                        if (ti >= T) continue;
                        acc += (double)x[((int64_t)b * T + ti) * Cin + ci] * W[((int64_t)ci * Cout + co) * K + k];
                    }
                y[((int64_t)b * To + t) * Cout + co] = (float)acc;
            }
}

/* kernels.c:618-640 groupnorm_fwd (8 groups, no affine, eps 1e-5): fp64
 * mean then variance over channel (outer) and position (inner) */
static void orc_groupnorm(const float *x, float *y, int B, int T, int C) {
    const int G = 8, Cg = C / G;
    for (int b = 0; b < B; b++)
        for (int g = 0; g < G; g++) {
            const int64_t cnt = (int64_t)Cg * T;
            double mean = 0;
            for (int c = 0; c < Cg; c++)
                for (int t = 0; t < T; t++) mean += x[((int64_t)b * T + t) * C + g * Cg + c];
            mean /= cnt;
            double var = 0;
            for (int c = 0; c < Cg; c++)
                for (int t = 0; t < T; t++) {
                    const double d = x[((int64_t)b * T + t) * C + g * Cg + c] - mean;
                    var += d * d;
                }
            var /= cnt;
            const double inv = 1.0 / sqrt(var + 1e-5);
            for (int c = 0; c < Cg; c++)
                for (int t = 0; t < T; t++) {
                    const int64_t i = ((int64_t)b * T + t) * C + g * Cg + c;
                    y[i] = (float)((x[i] - mean) * inv);
                }
        }
}

/* vq.c:206-215 phi_index with the ticks of vq.c:118-125 */
static int orc_phi_index(const OrcVq *q, int level) {
    if (q->n_phi == 1) return 0;
    const double at = (double)level / (q->n_levels - 1);
    int best = 0;
    double bd = 1e300;
    for (int j = 0; j < q->n_phi; j++) {
        const double tick = q->n_phi == 4 ? (j + 1.0 / 3.0) / q->n_phi : (j + 0.5) / q->n_phi;
        const double d = fabs(tick - at);
        if (d < bd) {
            bd = d;
            best = j;
        }
    }
    return best;
}

/* y += conv1d(y, W, b) with kernel 3, padding 1 (the refine step of vq.c:310-330, 356-375) */
static void orc_refine(float *y, const float *W, const float *bias, int B, int T, int D) {
    float *r = (float *)malloc((size_t)B * T * D * sizeof(float));
    orc_conv1d(y, W, bias, r, B, T, D, D, 3, 1, 1);
    for (size_t i = 0; i < (size_t)B * T * D; i++) y[i] += r[i];
    free(r);
}

/* the learned level-0 cascade: optional GroupNorm before every stage but the
 * first, optional final GroupNorm (vq.c:285-309 down, 336-355 up) */
static float *orc_cascade(const OrcVq *q, const float *x, int B, int T, int up, int *Tout) {
    const int D = q->D, n = up ? q->n_up : q->n_down;
    float *cur = (float *)malloc((size_t)B * T * D * sizeof(float));
    memcpy(cur, x, (size_t)B * T * D * sizeof(float));
    int Tc = T;
    for (int i = 0; i < n; i++) {
        const int s = up ? q->upK[i] : q->downK[i];
        if (q->l1_norm && i > 0) {
            float *g = (float *)malloc((size_t)B * Tc * D * sizeof(float));
            orc_groupnorm(cur, g, B, Tc, D);
            free(cur);
            cur = g;
        }
        const int To = up ? (Tc - 1) * s + s : Tc / s;
        float *nx = (float *)malloc((size_t)B * To * D * sizeof(float));
        if (up)
            orc_convT1d(cur, q->upW[i], q->upB[i], nx, B, Tc, D, D, s, s);
        else
            orc_conv1d(cur, q->downW[i], q->downB[i], nx, B, Tc, D, D, s, s, 0);
        free(cur);
        cur = nx;
        Tc = To;
    }
    if (q->l1_norm_final) {
        float *g = (float *)malloc((size_t)B * Tc * D * sizeof(float));
        orc_groupnorm(cur, g, B, Tc, D);
        free(cur);
        cur = g;
    }
    *Tout = Tc;
    return cur;
}

/* vq.c:280-330 down_for_quant: z_rest [B][L][D] -> out [B][levels[lv]][D] */
static void orc_down(const OrcVq *q, const float *z, int B, int lv, float *out) {
    const int D = q->D, L = q->levels[q->n_levels - 1], tl = q->levels[lv];
    if (lv == 0 && q->n_down > 0) {
        int Tc;
        float *c = orc_cascade(q, z, B, L, 0, &Tc);
        memcpy(out, c, (size_t)B * tl * D * sizeof(float));
        free(c);
    } else {
        orc_area(z, out, B, L, tl, D);
    }
    if (q->has_all && lv >= 1 && lv <= q->n_levels - 2 && q->drefW[lv]) orc_refine(out, q->drefW[lv], q->drefB[lv], B, tl, D);
}

/* vq.c:332-376 up_to_full: q [B][levels[lv]][D] -> out [B][L][D] */
static void orc_up(const OrcVq *q, const float *x, int B, int lv, float *out) {
    const int D = q->D, L = q->levels[q->n_levels - 1], tl = q->levels[lv];
    if (lv == 0 && q->n_down > 0) {
        int Tc;
        float *c = orc_cascade(q, x, B, tl, 1, &Tc);
        memcpy(out, c, (size_t)B * L * D * sizeof(float));
        free(c);
    } else {
        orc_lin(x, out, B, tl, L, D);
    }
    if (q->has_all && lv >= 1 && lv <= q->n_levels - 2 && q->urefW[lv]) orc_refine(out, q->urefW[lv], q->urefB[lv], B, L, D);
}

/* vq.c:243-277 apply_resi: h = (1 - r) h + r Phi(h) in float */
static void orc_resi(const OrcVq *q, float *h, int B, int lv) {
    if (q->n_phi <= 0) return;
    const int D = q->D, L = q->levels[q->n_levels - 1], j = orc_phi_index(q, lv);
    const size_t n = (size_t)B * L * D;
    float *c = (float *)malloc(n * sizeof(float));
    orc_conv1d(h, q->phiW[j], q->phib[j], c, B, L, D, D, 3, 1, 1);
    const float r = q->resi_ratio;
    for (size_t i = 0; i < n; i++) h[i] = (1 - r) * h[i] + r * c[i];
    free(c);
}

/* q = E[lv][codes of level lv] ([B][tl][D], sequence b's codes at
 * idx[b * total + base + t]), then up-sampled and Phi-blended into up */
static void orc_level_up_at(const OrcVq *q, const int *idx, int total, int B, int lv, int base, float *up) {
    const int D = q->D, tl = q->levels[lv];
    float *qq = (float *)malloc((size_t)B * tl * D * sizeof(float));
    for (int b = 0; b < B; b++)
        for (int t = 0; t < tl; t++)
            memcpy(qq + ((size_t)b * tl + t) * D, q->E[lv] + (size_t)idx[(int64_t)b * total + base + t] * D,
                   (size_t)D * sizeof(float));
    orc_up(q, qq, B, lv, up);
    free(qq);
    orc_resi(q, up, B, lv);
}

static void orc_level_up(const OrcVq *q, const int *idx, int B, int lv, int base, float *up) {
    int total = 0;
    for (int k = 0; k < q->n_levels; k++) total += q->levels[k];
    orc_level_up_at(q, idx, total, B, lv, base, up);
}

/* vq.c:402-431: one row's soft draw.  m = mean of the row's distances (double,
 * in index order); m <= 0 returns -1 (the caller takes the argmin, the rng is
 * not advanced).  Else T = tau * m, bv = the row minimum, w_j = exp(-(d_j -
 * bv) / T), one xorshift64 (13, 7, 17) step, draw = (rng >> 11) * 2^-53 *
 * sum w, and the first j whose running sum of w exceeds the draw (V - 1 if
 * none). */
int orc_soft_pick(const float *d, int V, double tau, unsigned long long *rng) {
    double m = 0;
    for (int j = 0; j < V; j++) m += d[j];
    m /= V;
    if (!(m > 0)) return -1;
    const double T = tau * m;
    double bv = d[0];
    for (int j = 1; j < V; j++)
        if (d[j] < bv) bv = d[j];
    double acc = 0;
    for (int j = 0; j < V; j++) acc += exp(-(d[j] - bv) / T);
    unsigned long long x = *rng;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *rng = x;
    const double draw = ((double)(x >> 11) * (1.0 / 9007199254740992.0)) * acc;
    double csum = 0;
    for (int j = 0; j < V; j++) {
        csum += exp(-(d[j] - bv) / T);
        if (draw < csum) return j;
    }
    return V - 1;
}

/* vq.c:388-500 vq_z_to_idx_soft: levels below soft_levels draw from the
 * tempered softmax over the row's distances (orc_soft_pick, rows in order,
 * one rng state), the rest take the argmin; soft_levels <= 0, tau <= 0 or no
 * rng is vq_z_to_idx. */
void orc_vq_z_to_idx_soft(const OrcVq *q, const float *z, int B, int *idx, float *z_hat, float *z_rest,
                          int soft_levels, double tau, unsigned long long *rng) {
    const int D = q->D, L = q->levels[q->n_levels - 1];
    const size_t n = (size_t)B * L * D;
    int total = 0;
    for (int k = 0; k < q->n_levels; k++) total += q->levels[k];
    float *zr = (float *)malloc(n * sizeof(float)), *zh = (float *)calloc(n, sizeof(float));
    float *down = (float *)malloc(n * sizeof(float)), *up = (float *)malloc(n * sizeof(float));
    memcpy(zr, z, n * sizeof(float));
    int off = 0;
    for (int lv = 0; lv < q->n_levels; lv++) {
        const int tl = q->levels[lv], V = q->vocabs[lv];
        orc_down(q, zr, B, lv, down);
        int *codes = (int *)malloc((size_t)B * tl * sizeof(int));
        orc_vq_argmin(down, q->E[lv], codes, (int64_t)B * tl, V, D);
        if (rng && lv < soft_levels && tau > 0) {
            float *dd = (float *)malloc((size_t)V * sizeof(float));
            for (int r = 0; r < B * tl; r++) {
                orc_l2sq(down + (size_t)r * D, q->E[lv], dd, 1, V, D);
                const int j = orc_soft_pick(dd, V, tau, rng);
                if (j >= 0) codes[r] = j;
            }
            free(dd);
        }
        for (int r = 0; r < B * tl; r++) idx[(int64_t)(r / tl) * total + off + r % tl] = codes[r];
        free(codes);
        orc_level_up(q, idx, B, lv, off, up);
        off += tl;
        for (size_t i = 0; i < n; i++) zh[i] += up[i];
        for (size_t i = 0; i < n; i++) zr[i] -= up[i];
    }
    if (z_hat) memcpy(z_hat, zh, n * sizeof(float));
    if (z_rest) memcpy(z_rest, zr, n * sizeof(float));
    free(zr);
    free(zh);
    free(down);
    free(up);
}

/* vq.c:697-790 vq_ema_update with the EMA state passed in (vq_ema_init,
 * vq.c:677-695: cs[lv] = 1, w[lv] = E[lv]); codes [B][total] level-major.  Per
 * level: the level's input rows (down-sampled z_rest), count[v] and the fp64
 * sum over the rows holding code v, in row order; cs = (float)(decay cs + (1 -
 * decay) count), w = (float)(decay w + (1 - decay) sum); the codebook E
 * (rewritten in place) = (float)(w / ((cs + eps) / (n + V eps) n)), n = the
 * sum of cs; then the residual advances with the new codebook as in
 * vq_z_to_idx. */
void orc_vq_ema_update(const OrcVq *q, float *const *cs, float *const *w, const float *z, const int *codes, int B,
                       double decay, double eps) {
    const int D = q->D, L = q->levels[q->n_levels - 1];
    const size_t n = (size_t)B * L * D;
    int total = 0;
    for (int k = 0; k < q->n_levels; k++) total += q->levels[k];
    float *zr = (float *)malloc(n * sizeof(float)), *zh = (float *)calloc(n, sizeof(float));
    float *down = (float *)malloc(n * sizeof(float)), *up = (float *)malloc(n * sizeof(float));
    memcpy(zr, z, n * sizeof(float));
    int off = 0;
    for (int lv = 0; lv < q->n_levels; lv++) {
        const int tl = q->levels[lv], V = q->vocabs[lv], rows = B * tl;
        orc_down(q, zr, B, lv, down);
        double *cnt = (double *)calloc((size_t)V, sizeof(double));
        for (int r = 0; r < rows; r++) cnt[codes[(size_t)(r / tl) * total + off + r % tl]] += 1.0;
        for (int v = 0; v < V; v++) {
            cs[lv][v] = (float)(decay * cs[lv][v] + (1 - decay) * cnt[v]);
            for (int d = 0; d < D; d++) {
                double sum = 0;
                for (int r = 0; r < rows; r++)
                    if (codes[(size_t)(r / tl) * total + off + r % tl] == v) sum += down[(size_t)r * D + d];
                w[lv][(size_t)v * D + d] = (float)(decay * w[lv][(size_t)v * D + d] + (1 - decay) * sum);
            }
        }
        free(cnt);
        double nsum = 0;
        for (int v = 0; v < V; v++) nsum += cs[lv][v];
        float *E = (float *)q->E[lv];
        for (int v = 0; v < V; v++) {
            const double sm = (cs[lv][v] + eps) / (nsum + V * eps) * nsum;
            for (int d = 0; d < D; d++) E[(size_t)v * D + d] = (float)(w[lv][(size_t)v * D + d] / sm);
        }
        orc_level_up(q, codes, B, lv, off, up);
        off += tl;
        for (size_t i = 0; i < n; i++) zh[i] += up[i];
        for (size_t i = 0; i < n; i++) zr[i] -= up[i];
    }
    free(zr);
    free(zh);
    free(down);
    free(up);
}

/* vq.c:378-500 vq_z_to_idx (argmin at every level) */
void orc_vq_z_to_idx(const OrcVq *q, const float *z, int B, int *idx, float *z_hat, float *z_rest) {
    const int D = q->D, L = q->levels[q->n_levels - 1];
    const size_t n = (size_t)B * L * D;
    int total = 0;
    for (int k = 0; k < q->n_levels; k++) total += q->levels[k];
    float *zr = (float *)malloc(n * sizeof(float)), *zh = (float *)calloc(n, sizeof(float));
    float *down = (float *)malloc(n * sizeof(float)), *up = (float *)malloc(n * sizeof(float));
    memcpy(zr, z, n * sizeof(float));
    int off = 0;
    for (int lv = 0; lv < q->n_levels; lv++) {
        const int tl = q->levels[lv], V = q->vocabs[lv];
        orc_down(q, zr, B, lv, down);
        int *codes = (int *)malloc((size_t)B * tl * sizeof(int));
        orc_vq_argmin(down, q->E[lv], codes, (int64_t)B * tl, V, D);
        for (int r = 0; r < B * tl; r++) idx[(int64_t)(r / tl) * total + off + r % tl] = codes[r];
        free(codes);
        orc_level_up(q, idx, B, lv, off, up);
        off += tl;
        for (size_t i = 0; i < n; i++) zh[i] += up[i];
        for (size_t i = 0; i < n; i++) zr[i] -= up[i];
    }
    if (z_hat) memcpy(z_hat, zh, n * sizeof(float));
    if (z_rest) memcpy(z_rest, zr, n * sizeof(float));
    free(zr);
    free(zh);
    free(down);
    free(up);
}

/* vq.c:502-552 vq_idx_to_zhats */
void orc_vq_idx_to_zhats(const OrcVq *q, const int *idx, int B, float *zhats) {
    const int D = q->D, L = q->levels[q->n_levels - 1];
    const size_t n = (size_t)B * L * D;
    float *zh = (float *)calloc(n, sizeof(float)), *up = (float *)malloc(n * sizeof(float));
    int base = 0;
    for (int lv = 0; lv < q->n_levels; lv++) {
        orc_level_up(q, idx, B, lv, base, up);
        for (size_t i = 0; i < n; i++) zh[i] += up[i];
        memcpy(zhats + (size_t)lv * n, zh, n * sizeof(float));
        base += q->levels[lv];
    }
    free(zh);
    free(up);
}

/* vq.c:554-597 vq_next_input: codes [B][levels[lv]]; z_hat [B][L][D] += the
 * level's up-sampled, Phi-blended codewords; x_out [B][levels[lv + 1]][D] =
 * area(z_hat) */
void orc_vq_next_input(const OrcVq *q, const int *codes, int lv, float *z_hat, float *x_out, int B) {
    const int D = q->D, L = q->levels[q->n_levels - 1];
    const size_t n = (size_t)B * L * D;
    float *up = (float *)malloc(n * sizeof(float));
    orc_level_up_at(q, codes, q->levels[lv], B, lv, 0, up);
    for (size_t i = 0; i < n; i++) z_hat[i] += up[i];
    orc_area(z_hat, x_out, B, L, q->levels[lv + 1], D);
    free(up);
}

/* vq.c:601-670 vq_idx_to_ncm_input: idx [B][total] level-major; x_out
 * [B][total - levels[0]][D] holds, for li < n_levels - 1 in turn, area(z_hat
 * after level li -> levels[li + 1]) */
void orc_vq_idx_to_ncm_input(const OrcVq *q, const int *idx, int B, float *x_out) {
    const int D = q->D, L = q->levels[q->n_levels - 1];
    const size_t n = (size_t)B * L * D;
    int total = 0;
    for (int k = 0; k < q->n_levels; k++) total += q->levels[k];
    const int T = total - q->levels[0];
    float *zh = (float *)calloc(n, sizeof(float)), *up = (float *)malloc(n * sizeof(float));
    int base = 0, off = 0;
    for (int li = 0; li + 1 < q->n_levels; li++) {
        const int nlen = q->levels[li + 1];
        orc_level_up(q, idx, B, li, base, up);
        for (size_t i = 0; i < n; i++) zh[i] += up[i];
        float *cv = (float *)malloc((size_t)B * nlen * D * sizeof(float));
        orc_area(zh, cv, B, L, nlen, D);
        for (int b = 0; b < B; b++)
            memcpy(x_out + ((size_t)b * T + off) * D, cv + (size_t)b * nlen * D, (size_t)nlen * D * sizeof(float));
        free(cv);
        base += q->levels[li];
        off += nlen;
    }
    free(zh);
    free(up);
}

/* tests/ktest_kernels.c:8-12: xorshift (13, 7, 17) mapped to [-2, 2) */
void orc_fill_ktest(uint64_t *state, float *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        uint64_t r = *state;
        r ^= r << 13;
        r ^= r >> 7;
        r ^= r << 17;
        *state = r;
        out[i] = (float)((r >> 11) * (1.0 / 9007199254740992.0) * 4.0 - 2.0);
    }
}

/* kernels.c:150-162 rmsnorm_fwd: ms in fp64 over c ascending, s rounded to
 * float, y = (x * s) * w in float. */
void orc_rmsnorm(const float *x, const float *w, float *y, int64_t rows, int C) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * C;
        float *yr = y + r * C;
        double ms = 0;
        for (int c = 0; c < C; c++) ms += (double)xr[c] * xr[c];
        ms /= C;
        float s = (float)(1.0 / sqrt(ms + 1e-6));
        for (int c = 0; c < C; c++) yr[c] = xr[c] * s * (w ? w[c] : 1.0f);
    }
}

/* kernels.c:101-148 layernorm_fwd (eps = 1e-6, a double literal) and
 * layernorm_eps_fwd (float eps widened to double): mean and var in fp64,
 * y = (float)((x - mean) * inv) * w + b in float. */
static void ln_rows(const float *x, const float *w, const float *b, float *y, int64_t rows, int C,
                    double eps) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * C;
        float *yr = y + r * C;
        double mean = 0;
        for (int c = 0; c < C; c++) mean += xr[c];
        mean /= C;
        double var = 0;
        for (int c = 0; c < C; c++) {
            double d = xr[c] - mean;
            var += d * d;
        }
        var /= C;
        double inv = 1.0 / sqrt(var + eps);
        for (int c = 0; c < C; c++) yr[c] = (float)((xr[c] - mean) * inv) * (w ? w[c] : 1.0f) + (b ? b[c] : 0.0f);
    }
}
void orc_layernorm(const float *x, const float *w, const float *b, float *y, int64_t rows, int C) {
    ln_rows(x, w, b, y, rows, C, 1e-6);
}
void orc_layernorm_eps(const float *x, const float *w, const float *b, float *y, int64_t rows, int C, float eps) {
    ln_rows(x, w, b, y, rows, C, (double)eps);
}

/* kernels.c:249-264 rope_one_exact, in place over rows of hd (position = row % T):
 * y[d] = a*c[d] + (-b)*s[d], y[d+h] = b*c[d+h] + a*s[d+h], float. */
void orc_rope(float *x, const float *cos_t, const float *sin_t, int64_t rows, int T, int hd) {
    int h = hd / 2;
    for (int64_t r = 0; r < rows; r++) {
        int t = (int)(r % T);
        float *xr = x + r * hd;
        const float *co = cos_t + (int64_t)t * hd;
        const float *si = sin_t + (int64_t)t * hd;
        for (int d = 0; d < h; d++) {
            float a = xr[d], b = xr[d + h];
            xr[d] = a * co[d] + (-b) * si[d];
            xr[d + h] = b * co[d + h] + a * si[d + h];
        }
    }
}

/* qwen.c:85-101 RoPE tables: angle t * theta^(-2d/hd) in double with libm,
 * cos/sin rounded to float, pair-duplicated. */
void orc_rope_tables_qwen(int T, int hd, double theta, float *cos_t, float *sin_t) {
    int h = hd / 2;
    for (int t = 0; t < T; t++)
        for (int d = 0; d < h; d++) {
            double a = (double)t * pow(theta, -(double)(2 * d) / (double)hd);
            float co = (float)cos(a), si = (float)sin(a);
            cos_t[(int64_t)t * hd + d] = co;
            cos_t[(int64_t)t * hd + d + h] = co;
            sin_t[(int64_t)t * hd + d] = si;
            sin_t[(int64_t)t * hd + d + h] = si;
        }
}

/* kernels.c:423-464 sdpa_fwd_gqa, CPU branch: pass 1 finds the row max of
 * s = (sum_d q*k in fp64) * scale + mask; pass 2 recomputes s, p = exp(s - mx)
 * in double, accumulates (float)p * v into the float output and the fp64
 * denominator, then scales by 1/den.  scale = 1/sqrtf(hd) in float. */
void orc_sdpa_gqa(const float *q, const float *k, const float *v, const float *mask, float *out,
                  int B, int Hq, int Hkv, int Tq, int Tkv, int hd) {
    float scale = 1.0f / sqrtf((float)hd);
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; b++)
        for (int h = 0; h < Hq; h++) {
            int kvh = h / (Hq / Hkv);
            for (int tq = 0; tq < Tq; tq++) {
                const float *qr = q + ((int64_t)b * Hq + h) * Tq * hd + (int64_t)tq * hd;
                double mx = -1e300, den = 0;
                for (int tk = 0; tk < Tkv; tk++) {
                    const float *kr = k + ((int64_t)b * Hkv + kvh) * Tkv * hd + (int64_t)tk * hd;
                    double s = 0;
                    for (int d = 0; d < hd; d++) s += (double)qr[d] * kr[d];
                    s *= scale;
                    if (mask) s += mask[(int64_t)tq * Tkv + tk];
                    if (s > mx) mx = s;
                }
                float *o = out + ((int64_t)b * Hq + h) * Tq * hd + (int64_t)tq * hd;
                for (int d = 0; d < hd; d++) o[d] = 0;
                for (int tk = 0; tk < Tkv; tk++) {
                    const float *kr = k + ((int64_t)b * Hkv + kvh) * Tkv * hd + (int64_t)tk * hd;
                    double s = 0;
                    for (int d = 0; d < hd; d++) s += (double)qr[d] * kr[d];
                    s *= scale;
                    if (mask) s += mask[(int64_t)tq * Tkv + tk];
                    double p = exp(s - mx);
                    den += p;
                    const float *vr = v + ((int64_t)b * Hkv + kvh) * Tkv * hd + (int64_t)tk * hd;
                    for (int d = 0; d < hd; d++) o[d] += (float)p * vr[d];
                }
                double inv = 1.0 / den;
                for (int d = 0; d < hd; d++) o[d] = (float)(o[d] * inv);
            }
        }
}

/* kernels.c:67-74 embedding_fwd */
void orc_embedding(const float *W, const int *idx, float *y, int64_t n, int D) {
    for (int64_t i = 0; i < n; i++) memcpy(y + i * D, W + (int64_t)idx[i] * D, (size_t)D * sizeof(float));
}

/* kernels.c:345-357 heads_transpose_fwd_b: [B][T][H*hd] -> [B][H][T][hd] */
void orc_heads_transpose(const float *in, float *out, int B, int64_t T, int H, int hd) {
    for (int b = 0; b < B; b++)
        for (int64_t t = 0; t < T; t++)
            for (int h = 0; h < H; h++)
                for (int d = 0; d < hd; d++)
                    out[(((int64_t)b * H + h) * T + t) * hd + d] = in[(((int64_t)b * T + t) * H + h) * hd + d];
}

/* kernels.c:913-926 qkv_split_fwd (GQA replication: kv head = h / rep) */
void orc_qkv_split(const float *in, float *qq, float *kk, float *vv, int B, int T, int C, int H, int hd,
                   int K, int rep) {
    int64_t W = (int64_t)C + 2 * K * hd;
    for (int b = 0; b < B; b++)
        for (int h = 0; h < H; h++)
            for (int t = 0; t < T; t++)
                for (int d = 0; d < hd; d++) {
                    int kvh = h / rep;
                    int64_t o = (((int64_t)b * H + h) * T + t) * hd + d;
                    const float *row = in + ((int64_t)b * T + t) * W;
                    qq[o] = row[h * hd + d];
                    kk[o] = row[C + kvh * hd + d];
                    vv[o] = row[C + K * hd + kvh * hd + d];
                }
}

/* kernels.c:928-936 head_merge_fwd: [B][H][T][hd] -> [B][T][C] */
void orc_head_merge(const float *ctx, float *out, int B, int T, int C, int H, int hd) {
    for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++)
            for (int h = 0; h < H; h++)
                for (int d = 0; d < hd; d++)
                    out[((int64_t)b * T + t) * C + h * hd + d] = ctx[(((int64_t)b * H + h) * T + t) * hd + d];
}

/* kernels.c:859-866 mul_fwd, :868-874 scale_fwd */
void orc_mul(const float *a, const float *b, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = a[i] * b[i];
}
void orc_scale(const float *x, float s, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = x[i] * s;
}

/* ------------------------------------------------------------------ */
/* training backward and optimizer                                     */
/* ------------------------------------------------------------------ */

/* train_tape.c:569-634 host_ln_bwd: fp64 row statistics; dw/db are the
 * fp64 rr-ascending column sums rounded to float and then float-added into
 * the existing gradients; dx += (float)(...) per element. */
void orc_layernorm_bwd(const float *x, const float *w, const float *dy, float *dx, float *dw, float *db,
                       int64_t rows, int C, double eps) {
    double *pmean = (double *)malloc((size_t)(rows > 0 ? rows : 1) * sizeof(double));
    double *pinv = (double *)malloc((size_t)(rows > 0 ? rows : 1) * sizeof(double));
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * C;
        double mean = 0;
        for (int c = 0; c < C; c++) mean += xr[c];
        mean /= C;
        double var = 0;
        for (int c = 0; c < C; c++) {
            double d = xr[c] - mean;
            var += d * d;
        }
        var /= C;
        pmean[r] = mean;
        pinv[r] = 1.0 / sqrt(var + eps);
    }
    if (dw || db) {
#pragma omp parallel for schedule(static)
        for (int c = 0; c < C; c++) {
            double sw = 0, sb = 0;
            for (int64_t r = 0; r < rows; r++) {
                double yh = (x[r * C + c] - pmean[r]) * pinv[r];
                sw += dy[r * C + c] * yh;
                sb += dy[r * C + c];
            }
            if (dw) dw[c] += (float)sw;
            if (db) db[c] += (float)sb;
        }
    }
    if (dx) {
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            const float *xr = x + r * C, *gr = dy + r * C;
            double mean = pmean[r], inv = pinv[r];
            double dmean = 0, dvar = 0;
            for (int c = 0; c < C; c++) {
                double wc = w ? w[c] : 1.0;
                double d = gr[c] * wc;
                dmean += d;
                dvar += d * (xr[c] - mean);
            }
            dmean /= C;
            dvar *= -0.5 * inv * inv * inv / C;
            for (int c = 0; c < C; c++) {
                double wc = w ? w[c] : 1.0;
                double d = gr[c] * wc;
                dx[r * C + c] += (float)((d - dmean) * inv + 2 * (xr[c] - mean) * dvar);
            }
        }
    }
    free(pmean);
    free(pinv);
}

/* train_tape.c:748-792 TOP_RMSN: dw is a FLOAT rr-ascending sum of
 * (float)((dy*x as a float product) * inv); dx in fp64. */
void orc_rmsnorm_bwd(const float *x, const float *w, const float *dy, float *dx, float *dw, int64_t rows, int C) {
    double *pinv = (double *)malloc((size_t)(rows > 0 ? rows : 1) * sizeof(double));
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        double ms = 0;
        for (int c = 0; c < C; c++) ms += (double)x[r * C + c] * x[r * C + c];
        ms /= C;
        pinv[r] = 1.0 / sqrt(ms + 1e-6);
    }
    if (dw) {
#pragma omp parallel for schedule(static)
        for (int c = 0; c < C; c++) {
            float sw = 0;
            for (int64_t r = 0; r < rows; r++) {
                float g = dy[r * C + c] * x[r * C + c];
                sw += (float)(g * pinv[r]);
            }
            dw[c] += sw;
        }
    }
    if (dx) {
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            const float *xr = x + r * C, *gr = dy + r * C;
            double inv = pinv[r], dot = 0;
            for (int c = 0; c < C; c++) {
                double wc = w ? w[c] : 1.0;
                dot += gr[c] * wc * xr[c];
            }
            dot /= C;
            for (int c = 0; c < C; c++) {
                double wc = w ? w[c] : 1.0;
                dx[r * C + c] += (float)((gr[c] * wc - dot * xr[c] * inv * inv) * inv);
            }
        }
    }
    free(pinv);
}

/* train_tape.c:442-481 t_ce: per row float max (strict '>'), fp64
 * exp/denominator, probs = (float)e / (float)den; loss = (float)(sum_r
 * w_r * -log(p[tgt] + 1e-30) / sum_r w_r) over rows with w_r != 0.
 * Returns the count sum_r w_r. */
double orc_ce_fwd(const float *logits, const int *tgt, const float *wm, float *loss, float *probs, int64_t rows,
                  int V) {
    double nll = 0, cnt = 0;
    for (int64_t r = 0; r < rows; r++) {
        const float *l = logits + r * V;
        float *p = probs + r * V;
        float m = l[0];
        for (int v = 1; v < V; v++)
            if (l[v] > m) m = l[v];
        double den = 0;
        for (int v = 0; v < V; v++) {
            double e = exp((double)l[v] - m);
            p[v] = (float)e;
            den += e;
        }
        for (int v = 0; v < V; v++) p[v] /= (float)den;
        float w = wm ? wm[r] : 1.0f;
        if (w != 0) {
            nll += w * -log(p[tgt[r]] + 1e-30);
            cnt += w;
        }
    }
    *loss = cnt > 0 ? (float)(nll / cnt) : 0.0f;
    return cnt;
}

/* train_tape.c:657-679 TOP_CE backward: dl += (float)((p - onehot) * w * inv),
 * inv = weight / cnt; rows with w == 0 untouched. */
void orc_ce_bwd(const float *probs, const int *tgt, const float *wm, float *dl, int64_t rows, int V, double inv) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        float w = wm ? wm[r] : 1.0f;
        if (w == 0) continue;
        for (int v = 0; v < V; v++)
            dl[r * V + v] += (float)((probs[r * V + v] - (v == tgt[r] ? 1.0 : 0.0)) * w * inv);
    }
}

/* train.c:131-141 (host loop) = train.c:51-64 (k_adamw): decoupled decay,
 * moments in fp64 rounded to float, bias-corrected step in fp64. */
void orc_adamw(float *p, const float *g, float *m, float *v, int64_t n, double lr, double b1, double b2,
               double b1t, double b2t, double eps, double wd) {
    for (int64_t k = 0; k < n; k++) {
        float gk = g[k];
        p[k] -= (float)(lr * wd * p[k]);
        m[k] = (float)(b1 * m[k] + (1 - b1) * gk);
        v[k] = (float)(b2 * v[k] + (1 - b2) * gk * gk);
        double mh = m[k] / b1t, vh = v[k] / b2t;
        p[k] -= (float)(lr * mh / (sqrt(vh) + eps));
    }
}

/* train.c:172-178 */
double orc_sched_cosine_warmup(long step, double warmup, double total) {
    double w = warmup, T = total;
    if (step < w) return step / (w > 0 ? w : 1);
    if (step >= T) return 0.0;
    double x = (step - w) / (T - w);
    return 0.5 * (1 + cos(3.141592653589793 * x));
}

/* train_gpt2.c:160-173: global L2 norm over every gradient (fp64, serial),
 * scale by (float)(1/gnorm) when the norm exceeds max_norm (1.0 there). */
double orc_grad_clip(float *const *g, const int64_t *n, int count, double max_norm) {
    double g2 = 0;
    for (int i = 0; i < count; i++)
        for (int64_t k = 0; k < n[i]; k++) g2 += (double)g[i][k] * g[i][k];
    double gnorm = sqrt(g2);
    if (gnorm > max_norm) {
        float s = (float)(1.0 / gnorm);
        for (int i = 0; i < count; i++)
            for (int64_t k = 0; k < n[i]; k++) g[i][k] *= s;
    }
    return gnorm;
}

/* train_tape.c:289-313 (t_sdpa): the probabilities the tape stores for the
 * backward.  Scores in fp64 rounded to float, max over the fp64 scores,
 * (float)exp(float score - max), float division by (float)den. */
void orc_sdpa_probs(const float *q, const float *k, const float *mask, float *P, int B, int H, int Hkv, int Tq,
                    int Tkv, int hd) {
    float scale = 1.0f / sqrtf((float)hd);
    int rep = H / Hkv;
    int64_t rows = (int64_t)B * H * Tq;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        int bh = (int)(r / Tq), tq = (int)(r % Tq);
        int h = bh % H, b = bh / H, kvh = h / rep;
        const float *qr = q + r * hd;
        float *pr = P + r * Tkv;
        double mx = -1e300;
        for (int tk = 0; tk < Tkv; tk++) {
            const float *kr = k + (((int64_t)b * Hkv + kvh) * Tkv + tk) * hd;
            double s = 0;
            for (int d = 0; d < hd; d++) s += (double)qr[d] * kr[d];
            s *= scale;
            if (mask) s += mask[(int64_t)tq * Tkv + tk];
            pr[tk] = (float)s;
            if (s > mx) mx = s;
        }
        double den = 0;
        for (int tk = 0; tk < Tkv; tk++) {
            pr[tk] = (float)exp(pr[tk] - mx);
            den += pr[tk];
        }
        for (int tk = 0; tk < Tkv; tk++) pr[tk] /= (float)den;
    }
}

/* train_tape.c:936-1051 TOP_SDPA backward (the GQA path; with Hkv == H it
 * is the MHA path): ds = P (dP - sum_tk P dP) in fp64 with dP = dO . v;
 * dq += (float)(ds*scale*k) tk-ascending; dk, dv are float sums over the
 * h-group then tq (ascending) of (float)(ds*scale*q) and (float)(P*dO),
 * float-added into the existing gradients.  Any of dq/dk/dv may be NULL. */
void orc_sdpa_bwd(const float *q, const float *k, const float *v, const float *P, const float *dy, float *dq,
                  float *dk, float *dv, int B, int H, int Hkv, int Tq, int Tkv, int hd) {
    float scale = 1.0f / sqrtf((float)hd);
    int rep = H / Hkv;
    int64_t rows = (int64_t)B * H * Tq;
    double *ds = (double *)malloc((size_t)(rows > 0 ? rows : 1) * (size_t)(Tkv > 0 ? Tkv : 1) * sizeof(double));
#pragma omp parallel for schedule(static)
    for (int64_t rr = 0; rr < rows; rr++) {
        int b = (int)(rr / ((int64_t)H * Tq)), h = (int)((rr / Tq) % H), tq = (int)(rr % Tq);
        int kvh = h / rep;
        double tot = 0;
        for (int tk = 0; tk < Tkv; tk++) {
            const float *vr = v + ((int64_t)b * Hkv + kvh) * Tkv * hd + (int64_t)tk * hd;
            double s = 0;
            for (int d = 0; d < hd; d++) s += (double)dy[rr * hd + d] * vr[d];
            s *= P[rr * Tkv + tk];
            ds[rr * Tkv + tk] = s;
            tot += s;
        }
        for (int tk = 0; tk < Tkv; tk++) ds[rr * Tkv + tk] -= P[rr * Tkv + tk] * tot;
        if (dq)
            for (int tk = 0; tk < Tkv; tk++) {
                const float *kr = k + ((int64_t)b * Hkv + kvh) * Tkv * hd + (int64_t)tk * hd;
                for (int d = 0; d < hd; d++)
                    dq[((int64_t)b * H + h) * Tq * hd + (int64_t)tq * hd + d] +=
                        (float)(ds[rr * Tkv + tk] * scale * kr[d]);
            }
    }
    if (dk || dv) {
#pragma omp parallel for collapse(3) schedule(static)
        for (int b = 0; b < B; b++)
            for (int kvh = 0; kvh < Hkv; kvh++)
                for (int tk = 0; tk < Tkv; tk++)
                    for (int d = 0; d < hd; d++) {
                        float sk = 0, sv = 0;
                        for (int h = kvh * rep; h < (kvh + 1) * rep && h < H; h++)
                            for (int tq = 0; tq < Tq; tq++) {
                                int64_t rr = ((int64_t)b * H + h) * Tq + tq;
                                const float *qr = q + ((int64_t)b * H + h) * Tq * hd + (int64_t)tq * hd;
                                sk += (float)(ds[rr * Tkv + tk] * scale * qr[d]);
                                sv += (float)(P[rr * Tkv + tk] * dy[rr * hd + d]);
                            }
                        int64_t o = ((int64_t)b * Hkv + kvh) * Tkv * hd + (int64_t)tk * hd + d;
                        if (dk) dk[o] += sk;
                        if (dv) dv[o] += sv;
                    }
    }
    free(ds);
}

/* train_tape.c:830-873 TOP_GELU / TOP_SILU / TOP_GELU_TANH backward:
 * dx += (float)(dy * g(x)) with g in fp64.  kind: 0 gelu (erf), 1 silu,
 * 2 gelu_tanh. */
void orc_act_bwd(const float *x, const float *dy, float *dx, int64_t n, int kind) {
    const double s2 = 1.4142135623730951, ip = 0.3989422804014327;
    const double c0 = 0.7978845608028654, c1 = 0.044715;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        double g;
        if (kind == 0) {
            double e = erf(x[i] / s2);
            g = 0.5 * (1 + e) + x[i] * exp(-0.5 * x[i] * x[i]) * ip;
        } else if (kind == 1) {
            double s = 1.0 / (1.0 + exp(-x[i]));
            g = s * (1 + x[i] * (1 - s));
        } else {
            double xv = x[i];
            double u = c0 * (xv + c1 * xv * xv * xv);
            double th = tanh(u);
            g = 0.5 * (1.0 + th) + 0.5 * xv * (1.0 - th * th) * c0 * (1.0 + 3.0 * c1 * xv * xv);
        }
        dx[i] += (float)(dy[i] * g);
    }
}

/* train_tape.c:1254-1268 TOP_MUL: da += dy*b, db += dy*a in float */
void orc_mul_bwd(const float *a, const float *b, const float *dy, float *da, float *db, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        if (da) da[i] += dy[i] * b[i];
        if (db) db[i] += dy[i] * a[i];
    }
}

/* train_tape.c:890-930 TOP_ROPE: the transposed rotation in fp64, per row of
 * hd (position row % T). */
void orc_rope_bwd(const float *g, const float *cos_t, const float *sin_t, float *dx, int64_t rows, int T, int hd) {
    int h = hd / 2;
#pragma omp parallel for schedule(static)
    for (int64_t rr = 0; rr < rows; rr++) {
        int t = (int)(rr % T);
        for (int d = 0; d < h; d++) {
            double g0 = g[rr * hd + d], g1 = g[rr * hd + h + d];
            double c0 = cos_t[t * hd + d], s0 = sin_t[t * hd + d];
            double c1 = cos_t[t * hd + h + d], s1 = sin_t[t * hd + h + d];
            dx[rr * hd + d] += (float)(g0 * c0 + g1 * s1);
            dx[rr * hd + h + d] += (float)(-g0 * s0 + g1 * c1);
        }
    }
}

/* train_tape.c:726-741 TOP_EMBED: per id a float sum of dy rows in
 * ascending row order, then float-added into dW; ids outside [0, V) skipped. */
void orc_embedding_bwd(const float *dy, const int *idx, int64_t n, int D, float *dW, int V) {
    float *acc = (float *)calloc((size_t)V * D, sizeof(float));
    for (int64_t i = 0; i < n; i++) {
        int id = idx[i];
        if (id < 0 || id >= V) continue;
        for (int d = 0; d < D; d++) acc[(size_t)id * D + d] += dy[i * D + d];
    }
    for (int64_t j = 0; j < (int64_t)V * D; j++) dW[j] += acc[j];
    free(acc);
}

/* train_tape.c:1293-1328 TOP_SPLIT: q grads copied back into the fused row;
 * k/v grads summed over the query heads of each kv head (float, ascending h). */
void orc_qkv_split_bwd(const float *gq, const float *gk, const float *gv, float *dx, int B, int T, int C, int H,
                       int hd, int K, int rep) {
    int64_t row = (int64_t)C + 2 * K * hd;
    for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++) {
            float *dr = dx + ((int64_t)b * T + t) * row;
            if (gq)
                for (int h = 0; h < H; h++)
                    for (int d = 0; d < hd; d++) dr[h * hd + d] += gq[(((int64_t)b * H + h) * T + t) * hd + d];
            for (int kvh = 0; kvh < K; kvh++)
                for (int d = 0; d < hd; d++) {
                    float sk = 0, sv = 0;
                    for (int h = kvh * rep; h < (kvh + 1) * rep && h < H; h++) {
                        int64_t o = (((int64_t)b * H + h) * T + t) * hd + d;
                        if (gk) sk += gk[o];
                        if (gv) sv += gv[o];
                    }
                    if (gk) dr[C + kvh * hd + d] += sk;
                    if (gv) dr[C + K * hd + kvh * hd + d] += sv;
                }
        }
}

/* train_tape.c:1329-1338 TOP_MERGE: dctx[b,h,t,d] += dy[b,t,h*hd+d] */
void orc_head_merge_bwd(const float *dy, float *dctx, int B, int T, int C, int H, int hd) {
    for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++)
            for (int h = 0; h < H; h++)
                for (int d = 0; d < hd; d++)
                    dctx[(((int64_t)b * H + h) * T + t) * hd + d] += dy[((int64_t)b * T + t) * C + h * hd + d];
}

/* train_tape.c:1339-1350 TOP_HEADSPLIT: dx[b,t,h*hd+d] += dy[b,h,t,d] */
void orc_heads_transpose_bwd(const float *dy, float *dx, int B, int T, int C, int H, int hd) {
    for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++)
            for (int h = 0; h < H; h++)
                for (int d = 0; d < hd; d++)
                    dx[((int64_t)b * T + t) * C + h * hd + d] += dy[(((int64_t)b * H + h) * T + t) * hd + d];
}

/* ncp.c:80-92 build_rope for positions 0..S-1 */
void orc_rope_tables_ncp(int S, int hd, int base, float *cos_t, float *sin_t) {
    int half = hd / 2;
    for (int t = 0; t < S; t++)
        for (int d = 0; d < half; d++) {
            double inv = 1.0 / pow((double)base, (double)d / half);
            double f = t * inv;
            float co = (float)cos(f), si = (float)sin(f);
            cos_t[t * hd + d] = co;
            cos_t[t * hd + half + d] = co;
            sin_t[t * hd + d] = si;
            sin_t[t * hd + half + d] = si;
        }
}

void orc_conv1d_btc(const float *x, const float *W, const float *bias, float *y, int B, int T, int Cin, int Cout,
                    int K, int stride, int pad) {
    orc_conv1d(x, W, bias, y, B, T, Cin, Cout, K, stride, pad);
}

/* ncp.c:441-466 head_logits, tie_heads_to_codebook branch */
void orc_ncp_tied_head(const float *z, const float *E, const float *bias, float invT, float *out, int rows, int V,
                       int Dd) {
    double *Esq = (double *)malloc((size_t)(V > 0 ? V : 1) * sizeof(double));
    double ds = 0;
    for (int v = 0; v < V; v++) {
        double s = 0;
        for (int d = 0; d < Dd; d++) s += (double)E[(size_t)v * Dd + d] * E[(size_t)v * Dd + d];
        Esq[v] = s;
        ds += s;
    }
    ds /= V;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++)
        for (int v = 0; v < V; v++) {
            double dot = 0;
            for (int d = 0; d < Dd; d++) dot += (double)z[(size_t)r * Dd + d] * E[(size_t)v * Dd + d];
            double o = (2 * dot - Esq[v]) / ds * invT;
            if (bias) o += bias[v];
            out[(size_t)r * V + v] = (float)o;
        }
    free(Esq);
}
