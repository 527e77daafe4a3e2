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
