/* linear.c -- host side of the fp32 linear layer: argument checks, kernel
 * selection (MFMA GEMM vs. GEMV), split-K planning, launches.
 *
 * Reference semantics (kernels.c:38-54, train_tape.c:680-725):
 *   forward  y[r,m]  = b[m] + sum_k x[r,k] W[m,k]
 *   backward dx[r,k] += sum_m dy[r,m] W[m,k]
 *            dW[m,k] += sum_r dy[r,m] x[r,k]
 *            db[m]   += sum_r dy[r,m]
 * The reference accumulates each output in fp64; the MFMA path accumulates
 * in fp32 (the parity contract is |y - ref| <= 1e-4 (|ref| + 1)). */
#include "internal.h"

#include <limits.h>
#include <stdio.h>

/* Must match struct GemmArgs in gemm.hip. */
typedef struct {
    const float *A;
    const float *B;
    float *C;
    const float *bias;
    const float *res;
    float *ws;
    int Mo, No, K;
    int lda, ldb, ldc;
    int k_per_split;
    int act;
    int tiles_m, tiles_n;
} GemmArgs;

/* Must match struct GemvArgs in gemm.hip. */
typedef struct {
    const float *x;
    const float *W;
    const float *bias;
    const float *res;
    float *y;
    int N, K;
    int act;
} GemvArgs;

enum { L_FWD = 0, L_DX = 1, L_DW = 2 };
#define TILE 128
#define BK 16
#define N_CU 256

/* Number of K splits so that the grid covers the chip about twice (two
 * workgroups fit per CU) without cutting a split below 256 reduction steps. */
static int plan_splits(int tiles, int Kred) {
    int s = 1;
    while (tiles * s < 2 * N_CU && Kred / (2 * s) >= 256 && s < 32) s *= 2;
    return s;
}

/* Tiling of one GEMM: tile grid, split count and reduction length per split. */
typedef struct {
    int tiles_m, tiles_n, splits, kps;
} GemmPlan;

static GemmPlan plan_gemm(int Mo, int No, int Kred) {
    GemmPlan g;
    g.tiles_m = (Mo + TILE - 1) / TILE;
    g.tiles_n = (No + TILE - 1) / TILE;
    int splits = Kred > 0 ? plan_splits(g.tiles_m * g.tiles_n, Kred) : 1;
    int kps = (Kred + splits - 1) / splits;
    kps = (kps + BK - 1) / BK * BK;
    if (kps <= 0) kps = BK;
    g.kps = kps;
    g.splits = Kred > 0 ? (Kred + kps - 1) / kps : 1;
    return g;
}

static const char *gemm_names[3][2][2] = {
    /* kind x partial x vec */
    {{"gemm_fwd_store_s", "gemm_fwd_store_v"}, {"gemm_fwd_part_s", "gemm_fwd_part_v"}},
    {{"gemm_dx_accum_s", "gemm_dx_accum_v"}, {"gemm_dx_part_s", "gemm_dx_part_v"}},
    {{"gemm_dw_accum_s", "gemm_dw_accum_v"}, {"gemm_dw_part_s", "gemm_dw_part_v"}},
};

static int run_gemm(int kind, const float *A, const float *B, float *C, const float *bias,
                    const float *res, int Mo, int No, int Kred, int lda, int ldb, int ldc,
                    int act, int vec) {
    if (Mo <= 0 || No <= 0) return 0;
    GemmArgs p = {A, B, C, bias, res, NULL, Mo, No, Kred, lda, ldb, ldc, 0, act, 0, 0};
    GemmPlan g = plan_gemm(Mo, No, Kred);
    p.tiles_m = g.tiles_m;
    p.tiles_n = g.tiles_n;
    p.k_per_split = g.kps;
    int splits = g.splits, tiles = g.tiles_m * g.tiles_n;
    const char *(*names)[2][2] = gemm_names;
    int partial = splits > 1;
    if (partial) {
        p.ws = (float *)ncm_workspace(WS_SPLITK, (size_t)splits * Mo * No * sizeof(float));
        if (!p.ws) return NCM_E_OOM;
    }
    void *args[] = {&p};
    int rc = ncm_launch_named(names[kind][partial][vec ? 1 : 0], (unsigned)tiles, 1,
                              (unsigned)splits, 256, args);
    if (rc || !partial) return rc;

    int accum = kind != L_FWD;
    int64_t total = (int64_t)Mo * No;
    const float *ws = p.ws;
    void *rargs[] = {&ws, &splits, &Mo, &No, &C, &ldc, &bias, &res, &act, &accum};
    return ncm_launch_named("splitk_reduce", (unsigned)((total + 255) / 256), 1, 1, 256, rargs);
}

/* GEMV kernel for a chunk of nb <= 8 batch rows; returns rows per workgroup. */
static int gemv_name(int nb, int N, int vec, char *name, size_t cap) {
    int R = 1;
    if (vec) {
        if (nb == 1) R = N >= 8192 ? 4 : (N >= 2048 ? 2 : 1);
        else if (nb == 8) R = 1;
        else R = 2;
        snprintf(name, cap, "gemv_b%d_r%d_v", nb, R);
    } else {
        snprintf(name, cap, "gemv_b%d_r1_s", nb);
    }
    return R;
}

static int run_gemv(const float *x, const float *W, const float *b, const float *res, float *y,
                    int batch, int N, int K, int act, int vec) {
    int r0 = 0;
    while (r0 < batch) {
        int left = batch - r0;
        int nb = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
        char name[32];
        int R = gemv_name(nb, N, vec, name, sizeof name);
        GemvArgs p = {x + (int64_t)r0 * K, W, b, res ? res + (int64_t)r0 * N : NULL,
                      y + (int64_t)r0 * N, N, K, act};
        void *args[] = {&p};
        int rc = ncm_launch_named(name, (unsigned)((N + R - 1) / R), 1, 1, 256, args);
        if (rc) return rc;
        r0 += nb;
    }
    return 0;
}

static int check_dims(const char *fn, int64_t batch, int M, int K) {
    if (batch < 0 || batch > INT_MAX || M <= 0 || K <= 0)
        return ncm_fail(NCM_E_ARG, "%s: bad shape batch=%lld M=%d K=%d", fn, (long long)batch, M, K);
    if ((int64_t)M * K > INT64_MAX / 4)
        return ncm_fail(NCM_E_ARG, "%s: W too large", fn);
    return 0;
}

static void linear_forward(const char *fn, const float *x, const float *W, const float *b,
                           const float *res, float *y, int64_t batch, int M, int K, int act) {
    if (check_dims(fn, batch, M, K)) return;
    if (act < NCM_ACT_NONE || act > NCM_ACT_GELU_TANH) {
        ncm_fail(NCM_E_ARG, "%s: unknown activation %d", fn, act);
        return;
    }
    if (batch == 0) return;
    if (!x || !W || !y) {
        ncm_fail(NCM_E_ARG, "%s: null x/W/y", fn);
        return;
    }
    if (ncm_ready()) return;
    int vec = (K % 4 == 0) && is_aligned16(x) && is_aligned16(W);
    if (batch <= 8)
        run_gemv(x, W, b, res, y, (int)batch, M, K, act, vec);
    else
        run_gemm(L_FWD, x, W, y, b, res, (int)batch, M, K, K, K, M, act, vec);
}

void linear_fwd(const float *x, const float *W, const float *b, float *y, int64_t batch, int M,
                int K) {
    linear_forward("linear_fwd", x, W, b, NULL, y, batch, M, K, NCM_ACT_NONE);
}

void linear_fwd_ep(const float *x, const float *W, const float *b, const float *res, float *y,
                   int64_t batch, int M, int K, int act) {
    linear_forward("linear_fwd_ep", x, W, b, res, y, batch, M, K, act);
}

void linear_bwd(const float *x, const float *W, const float *dy, float *dx, float *dW, float *db,
                int64_t batch, int M, int K) {
    if (check_dims("linear_bwd", batch, M, K)) return;
    if (batch == 0) return;
    if (!dy || (dx && !W) || (dW && !x)) {
        ncm_fail(NCM_E_ARG, "linear_bwd: null dy, or W for dx, or x for dW");
        return;
    }
    if (ncm_ready()) return;
    int nb = (int)batch;
    if (dx) {
        int vec = (M % 4 == 0) && (K % 4 == 0) && is_aligned16(dy) && is_aligned16(W);
        if (run_gemm(L_DX, dy, W, dx, NULL, NULL, nb, K, M, M, K, K, 0, vec)) return;
    }
    if (dW) {
        int vec = (M % 4 == 0) && (K % 4 == 0) && is_aligned16(dy) && is_aligned16(x);
        if (run_gemm(L_DW, dy, x, dW, NULL, NULL, M, K, nb, M, K, K, 0, vec)) return;
    }
    if (db) {
        int rpc = 512;
        int chunks = (nb + rpc - 1) / rpc;
        double *part = (double *)ncm_workspace(WS_COLSUM, (size_t)chunks * M * sizeof(double));
        if (!part) return;
        int64_t rows = nb;
        void *a1[] = {&dy, &rows, &M, &rpc, &part};
        if (ncm_launch_named("colsum_partial", (unsigned)((M + 255) / 256), (unsigned)chunks, 1, 256, a1))
            return;
        void *a2[] = {&part, &chunks, &M, &db};
        ncm_launch_named("colsum_final", (unsigned)((M + 255) / 256), 1, 1, 256, a2);
    }
}

int ncm_hip_linear_plan(int op, int64_t batch, int M, int K, char *kernel, size_t cap) {
    if (op < 0 || op > 2 || batch <= 0 || batch > INT_MAX || M <= 0 || K <= 0 || !kernel || !cap)
        return ncm_fail(NCM_E_ARG, "ncm_hip_linear_plan: bad arguments"), -1;
    int nb = (int)batch;
    if (op == L_FWD && nb <= 8) {
        gemv_name(nb >= 8 ? 8 : nb >= 4 ? 4 : nb >= 2 ? 2 : 1, M, K % 4 == 0, kernel, cap);
        return 1;
    }
    int Mo = op == L_DW ? M : nb, No = op == L_FWD ? M : K, Kred = op == L_FWD ? K : (op == L_DX ? M : nb);
    int vec = op == L_FWD ? K % 4 == 0 : (M % 4 == 0 && K % 4 == 0);
    GemmPlan g = plan_gemm(Mo, No, Kred);
    snprintf(kernel, cap, "%s", gemm_names[op][g.splits > 1][vec]);
    return g.splits;
}
