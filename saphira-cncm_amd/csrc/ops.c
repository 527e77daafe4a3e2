/* ops.c -- host side of the row-wise kernels (greedy id). */
#include "internal.h"

#include <limits.h>

/* kernels.c:731-735, on a HOST row, as the reference: strict '>' from index 0. */
int argmax_row(const float *x, int n) {
    int bi = 0;
    float bv = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > bv) {
            bv = x[i];
            bi = i;
        }
    return bi;
}

void argmax_rows(const float *x, int *idx, int64_t rows, int n) {
    if (rows < 0 || rows > INT_MAX || n <= 0) {
        ncm_fail(NCM_E_ARG, "argmax_rows: bad shape rows=%lld n=%d", (long long)rows, n);
        return;
    }
    if (rows == 0) return;
    if (!x || !idx) {
        ncm_fail(NCM_E_ARG, "argmax_rows: null pointer");
        return;
    }
    if (ncm_ready()) return;
    void *args[] = {&x, &n, &idx};
    ncm_launch_named("argmax_rows_k", (unsigned)rows, 1, 1, 256, args);
}
