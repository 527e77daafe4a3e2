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

#include <stdlib.h>

#include <limits.h>
#include <stdio.h>
#include <string.h>

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
    int act;
    int res_mul;
    int tiles_m, tiles_n;
    int iters;
    int dp_tiles;
    int segs;
    unsigned a_bytes, b_bytes;
    const float *B2;
    const float *bias2;
    int beta;
    float *db;
    double *dbpart;
    float *pre;
    const float *bwd_x;
    int bwd_kind;
    const float *B3[3];
    const float *bias3[3];
    float *C3[3];
    int n3[3];
    unsigned b3_bytes[3];
    int hm_T;
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
#define BK 32
#define MAX_SEGS 16
#define MAX_BUFFER_BYTES ((int64_t)1 << 31)

static const char *const kind_names[3] = {"fwd", "dx", "dw"};

/* Kernel of a tile shape, operation and load width: gemm_<BM>x<BN>_<op>_<v|s>. */
static void gemm_name(int bm, int bn, int kind, int vec, char *out, size_t cap) {
    snprintf(out, cap, "gemm_%dx%d_%s_%c", bm, bn, kind_names[kind], vec ? 'v' : 's');
}

/* Work split of one GEMM over the chip.  Tiles [0, dp) run whole, one
 * workgroup each; every other tile is cut into `segs` k-segments (whole
 * groups of 4 slabs) whose partial tiles a fixup launch sums. */
typedef struct {
    int tiles_m, tiles_n, iters, dp_tiles, segs, blocks;
    double cost;   /* the cost model's makespan, in slabs of a 64 x 64 tile */
} GemmPlan;

/* CU makespan, in slabs, of list-scheduling dp units of I slabs and then n2
 * units of u slabs over C CUs in dispatch order, each unit to the CU with
 * the least work so far.  A CU retires slabs at the same rate however many
 * of its workgroups share it (the MFMA pipes are the bound), so CU load --
 * not workgroup slots -- is what has to balance.  The loads form at most two
 * levels at any time, so whole rounds are added at once. */
static double makespan(int C, int dp, int I, int64_t n2, int u) {
    int64_t ca = C - dp % C, cb = dp % C;   /* group a: ca CUs at level la; group b: cb at lb */
    double la = (double)(dp / C) * I, lb = la + I;
    while (n2 > 0) {
        if (cb > 0 && la > lb) {
            int64_t tc = ca; ca = cb; cb = tc;
            double tl = la; la = lb; lb = tl;
        }
        if (cb > 0 && la == lb) { ca += cb; cb = 0; }
        if (n2 < ca) { la += u; break; }   /* n2 of group a's CUs reach la + u */
        la += u;
        n2 -= ca;
    }
    return cb > 0 && lb > la ? lb : la;
}

/* Cost model of a split, fitted to per-call timings of the linear sweep's
 * GEMMs on MI355X under every forced split count (one slab of a 64x64 tile
 * ~ 0.52 us of a CU): the fixup launch adds ~6 us, and the partial tiles
 * ~0.05 us per MB. */
#define SPLIT_FIXED_SLABS 11.5
#define SPLIT_SLABS_PER_MB 0.1

static GemmPlan plan_gemm_uncached(int Mo, int No, int Kred, int slots, int bm, int bn) {
    GemmPlan g;
    g.tiles_m = (Mo + bm - 1) / bm;
    g.tiles_n = (No + bn - 1) / bn;
    const int groups = Kred > 0 ? (Kred + 4 * BK - 1) / (4 * BK) : 1;
    g.iters = 4 * groups;
    const int T = g.tiles_m * g.tiles_n, C = ncm_cu_count();
    if (slots < C) slots = C;
    /* unsplit: every tile whole */
    double best = makespan(C, T, g.iters, 0, 0);
    g.dp_tiles = T;
    g.segs = 1;
    /* whole rounds of workgroup slots, whole rounds of CUs, or nothing runs
     * whole; the rest split into s segments */
    const int dps[3] = {(T / slots) * slots, (T / C) * C, 0};
    for (int d = 0; d < 3; d++) {
        const int dp = dps[d], R = T - dp;
        if (R <= 0 || (d > 0 && dp == dps[d - 1])) continue;
        for (int s = 2; s <= MAX_SEGS && s <= groups; s++) {
            const int u = 4 * ((groups + s - 1) / s);
            double t = makespan(C, dp, g.iters, (int64_t)R * s, u) + SPLIT_FIXED_SLABS +
                       SPLIT_SLABS_PER_MB * (double)R * s * bm * bn * 4 / 1e6;
            if (t < best - 1e-9) {
                best = t;
                g.dp_tiles = dp;
                g.segs = s;
            }
        }
    }
    g.blocks = g.dp_tiles + (T - g.dp_tiles) * g.segs;
    g.cost = best;
    return g;
}

/* Plans are cached per shape (the library is driven from one host thread). */
static GemmPlan plan_gemm(int Mo, int No, int Kred, int slots, int bm, int bn) {
    static struct { int Mo, No, Kred, slots; GemmPlan g; } cache[64];
    static int used = 0, next = 0;
    for (int i = 0; i < used; i++)
        if (cache[i].Mo == Mo && cache[i].No == No && cache[i].Kred == Kred && cache[i].slots == slots)
            return cache[i].g;
    GemmPlan g = plan_gemm_uncached(Mo, No, Kred, slots, bm, bn);
    cache[next].Mo = Mo;
    cache[next].No = No;
    cache[next].Kred = Kred;
    cache[next].slots = slots;
    cache[next].g = g;
    next = (next + 1) % 64;
    if (used < 64) used++;
    return g;
}

/* Concurrent workgroups of a GEMM kernel on the device (CUs x occupancy). */
static int gemm_slots(const char *name) {
    static char names[32][32];
    static int vals[32], n = 0;
    for (int i = 0; i < n; i++)
        if (strcmp(names[i], name) == 0) return vals[i];
    hipFunction_t f = ncm_kernel(name);
    if (!f) return -1;
    int per_cu = 0;
    if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, 256, 0) != hipSuccess || per_cu < 1)
        per_cu = 1;
    int v = per_cu * ncm_cu_count();
    if (n < 32) {
        snprintf(names[n], sizeof names[n], "%s", name);
        vals[n++] = v;
    }
    return v;
}

/* Bytes spanned by a rows x cols row-major operand with row stride ld. */
static int64_t extent(int64_t rows, int64_t cols, int64_t ld) { return ((rows - 1) * ld + cols) * 4; }

/* Tile shapes: 64 x 64 (every kernel, split-K capable) and 128 x 128 (whole
 * tiles only, the vectorised plain / dW+db / dX-through-activation / head-major
 * kernels), chosen per call by the cost model below. */
#define TILE_M 64
#define TILE_N 64
#define BIG_TILE 128
/* Timing model of the two tile sizes on MI355X, fitted to forward launches
 * of 8192 x 1024 outputs (512 tiles of 128 x 128: one pair per CU) at K =
 * 256 .. 4096 with operands rotated through three copies: a 64 x 64 plan's
 * cost-model slabs take ~0.586 us each plus ~22 us per launch; a pair of
 * 128 x 128 tiles of W slab units each (one unit = one slab of 64 x 64 work)
 * takes 2 W 0.434 + 71.6 us -- near the MFMA peak per slab, but with a large
 * fixed cost per tile (start-up and epilogue are not hidden behind other
 * workgroups at two per CU) -- and a tile alone on its CU (one workgroup per
 * CU) is taken as W 0.6 + 60 us.  So the big tiles pay only for long K (about
 * K >= 2048) with CUs holding whole pairs; in the training step's context
 * (cold operands, activation epilogues) they measured 3-12% slower at K = 768
 * .. 3072. */
#define U64_US 0.586
#define U64_FIXED_US 22.0
#define PAIR_US 0.434
#define PAIR_FIXED_US 71.6
#define SINGLE_US 0.6
#define SINGLE_FIXED_US 60.0
/* 0: cost model; 64 / 128: that tile wherever it applies.  The environment
 * variable NCM_GEMM_TILES sets the starting mode (for tuning runs). */
static int g_tile_mode = -1;

void ncm_hip_set_gemm_tiles(int mode) { g_tile_mode = mode == 64 || mode == 128 ? mode : 0; }

static int tile_mode(void) {
    if (g_tile_mode < 0) {
        const char *e = getenv("NCM_GEMM_TILES");
        ncm_hip_set_gemm_tiles(e ? atoi(e) : 0);
    }
    return g_tile_mode;
}

/* Whether the 128 x 128 kernel of op runs this GEMM: it exists for the
 * vectorised plain, dwb, dxa and head-major products, needs whole rows of
 * tiles within one sequence for the head-major ones, and is chosen when its
 * whole-tile makespan beats the 64 x 64 plan's (or when forced). */
static int use_big(const char *op, int vec, int Mo, int No, int Kred, int hm_T, double cost64, int slots64) {
    const int mode = tile_mode();
    if (!vec || mode == 64 || strcmp(op, "fwd3") == 0) return 0;
    if ((strcmp(op, "fwdh") == 0 || strcmp(op, "dxh") == 0) && hm_T % BIG_TILE != 0) return 0;
    const int64_t T = (int64_t)((Mo + BIG_TILE - 1) / BIG_TILE) * ((No + BIG_TILE - 1) / BIG_TILE);
    if (T > INT_MAX / 4) return 0;
    if (mode == 128) return 1;
    (void)slots64;
    const int groups = Kred > 0 ? (Kred + 4 * BK - 1) / (4 * BK) : 1;
    const int C = ncm_cu_count();
    const int64_t n = (T + C - 1) / C;             /* tiles on the busiest CU */
    const double W = 16.0 * groups;                /* 64 x 64 slab units per 128 x 128 tile */
    const double big_us = (double)(n / 2) * (2 * W * PAIR_US + PAIR_FIXED_US) +
                          (double)(n % 2) * (W * SINGLE_US + SINGLE_FIXED_US);
    return big_us < 0.92 * (cost64 * U64_US + U64_FIXED_US);   /* only a clear win */
}

/* Optional parts of a GEMM launch (NULL for a plain one; vectorised kernels
 * only). */
typedef struct {
    float *db;           /* L_DW: the bias gradient db[i] += sum_k A(i,k), summed by the same launch */
    float *pre;          /* L_FWD: also stores acc + bias before the activation */
    const float *bwd_x;  /* L_DX: C (+)= act'(bwd_x) (0.0f + A.B), the activation backward of bwd_kind */
    int bwd_kind;
    const float *const *W3;   /* L_FWD: three products side by side (B, bias, output, width each) */
    const float *const *b3;
    float *const *y3;
    const int *n3;
    float *const *heads;      /* L_FWD: q | k | v parts of the output to head-major [B][n/64][T][64] */
    int hm_T;
} GemmExtra;

/* beta (accumulating kinds): 1 C += A.B, 0 C = 0.0f + A.B (C is not read). */
static int run_gemm_x(int kind, const float *A, const float *B, float *C, const float *bias,
                      const float *res, int res_mul, int Mo, int No, int Kred, int lda, int ldb, int ldc,
                      int act, int vec, int beta, const GemmExtra *ex) {
    static const GemmExtra none = {NULL, NULL, NULL, 0, NULL, NULL, NULL, NULL, NULL, 0};
    if (!ex) ex = &none;
    float *db = ex->db;
    if (Mo <= 0 || No <= 0) return 0;
    const int bm = TILE_M, bn = TILE_N;
    if ((int64_t)((Mo + bm - 1) / bm) * ((No + bn - 1) / bn) > INT_MAX / 4)
        return ncm_fail(NCM_E_ARG, "linear: %d x %d output has too many tiles", Mo, No);
    char name[48], fix[48];
    /* dwb: the dW kernel that also sums db; dxa: dX through the activation backward */
    const char *op = db           ? "dwb"
                     : ex->bwd_x  ? "dxa"
                     : ex->W3     ? "fwd3"
                     : ex->heads  ? (kind == L_DX ? "dxh" : "fwdh")
                                  : kind_names[kind];
    snprintf(name, sizeof name, "gemm_%dx%d_%s_%c", bm, bn, op, vec ? 'v' : 's');
    int slots = gemm_slots(name);
    if (slots < 0) return NCM_E_INIT;
    GemmPlan g = plan_gemm(Mo, No, Kred, slots, bm, bn);
    int big = use_big(op, vec, Mo, No, Kred, ex->hm_T, g.cost, slots);
    if (big) {
        snprintf(name, sizeof name, "gemm_%dx%d_%s_v", BIG_TILE, BIG_TILE, op);
        g.tiles_m = (Mo + BIG_TILE - 1) / BIG_TILE;
        g.tiles_n = (No + BIG_TILE - 1) / BIG_TILE;
        g.dp_tiles = g.blocks = g.tiles_m * g.tiles_n;
        g.segs = 1;
    }
    /* a dW + db reduction that is not whole groups of four slabs (batch 64 in
     * the sweep) runs the instance that skips the slabs past it */
    const int tail = !big && vec && db && Kred % (4 * BK) != 0;
    if (tail) snprintf(name, sizeof name, "gemm_%dx%d_dwbt_v", bm, bn);
    /* operand extents as stored: A is [Mo][Kred] (k-contiguous) or [Kred][Mo] */
    int64_t ab = kind == L_DW ? extent(Kred, Mo, lda) : extent(Mo, Kred, lda);
    int64_t bb = kind == L_FWD ? extent(No, Kred, ldb) : extent(Kred, No, ldb);
    if (ab >= MAX_BUFFER_BYTES || bb >= MAX_BUFFER_BYTES)
        return ncm_fail(NCM_E_ARG, "linear: operand of %lld / %lld bytes exceeds the 2 GiB buffer range",
                        (long long)ab, (long long)bb);
    GemmArgs p = {A, B, C, bias, res, NULL, Mo, No, Kred, lda, ldb, ldc, act, 0,
                  g.tiles_m, g.tiles_n, g.iters, g.dp_tiles, g.segs, (unsigned)ab, (unsigned)bb, NULL, NULL, beta,
                  db, NULL, ex->pre, ex->bwd_x, ex->bwd_kind, {NULL}, {NULL}, {NULL}, {0}, {0}, ex->hm_T};
    p.res_mul = res_mul;
    if (tail) p.iters = (Kred + BK - 1) / BK;
    if (ex->W3)
        for (int g = 0; g < 3; g++) {
            p.B3[g] = ex->W3[g];
            p.bias3[g] = ex->b3[g];
            p.C3[g] = ex->y3[g];
            p.n3[g] = ex->n3[g];
            p.b3_bytes[g] = (unsigned)extent(ex->n3[g], Kred, ldb);
        }
    if (ex->heads)
        for (int g = 0; g < 3; g++) {
            p.C3[g] = ex->heads[g];
            p.n3[g] = ex->n3[g];
        }
    int split_tiles = g.tiles_m * g.tiles_n - g.dp_tiles;
    if (g.segs > 1) {
        /* partial tiles [units][64 * 64] floats, then the bias partials [units][64] doubles */
        size_t units = (size_t)split_tiles * g.segs;
        p.ws = (float *)ncm_workspace(WS_SPLITK, units * (bm * bn * sizeof(float) + (db ? 64 * sizeof(double) : 0)));
        if (!p.ws) return NCM_E_OOM;
        if (db) p.dbpart = (double *)(p.ws + units * bm * bn);
    }
    void *args[] = {&p};
    int rc = ncm_launch(ncm_kernel(name), (unsigned)g.blocks, 1, 1, 256, args);
    if (rc || g.segs == 1) return rc;
    snprintf(fix, sizeof fix, "gemm_%dx%d_fixup_%s_%c", bm, bn, op, vec ? 'v' : 's');
    return ncm_launch_named(fix, (unsigned)split_tiles * 4u, 1, 1, 256, args);  /* one workgroup per MFMA block */
}

static int run_gemm(int kind, const float *A, const float *B, float *C, const float *bias,
                    const float *res, int res_mul, int Mo, int No, int Kred, int lda, int ldb, int ldc,
                    int act, int vec, int beta, float *db) {
    GemmExtra ex = {db, NULL, NULL, 0, NULL, NULL, NULL, NULL, NULL, 0};
    return run_gemm_x(kind, A, B, C, bias, res, res_mul, Mo, No, Kred, lda, ldb, ldc, act, vec, beta, &ex);
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

/* y = res + act(x W^T + b), or act(x W^T + b) * res when res_mul */
static void linear_forward(const char *fn, const float *x, const float *W, const float *b,
                           const float *res, int res_mul, float *y, int64_t batch, int M, int K, int act) {
    if (check_dims(fn, batch, M, K)) return;
    if (act < NCM_ACT_NONE || act > NCM_ACT_RELU2) {
        ncm_fail(NCM_E_ARG, "%s: unknown activation %d", fn, act);
        return;
    }
    if (batch == 0) return;
    if (!x || !W || !y) {
        ncm_fail(NCM_E_ARG, "%s: null x/W/y", fn);
        return;
    }
    if (res_mul && (!res || res == y)) {
        ncm_fail(NCM_E_ARG, "%s: the multiplier must be a buffer other than y", fn);
        return;
    }
    if (ncm_ready()) return;
    int vec = (K % 4 == 0) && is_aligned16(x) && is_aligned16(W);
    if (batch <= 8 && res_mul) {   /* the GEMVs add only: product in a second pass */
        if (run_gemv(x, W, b, NULL, y, (int)batch, M, K, act, vec) == 0) mul_fwd(y, res, y, batch * M);
    } else if (batch <= 8)
        run_gemv(x, W, b, res, y, (int)batch, M, K, act, vec);
    else
        run_gemm(L_FWD, x, W, y, b, res, res_mul, (int)batch, M, K, K, K, M, act, vec, 1, NULL);
}

void linear_fwd(const float *x, const float *W, const float *b, float *y, int64_t batch, int M,
                int K) {
    linear_forward("linear_fwd", x, W, b, NULL, 0, y, batch, M, K, NCM_ACT_NONE);
}

void linear_fwd_ep(const float *x, const float *W, const float *b, const float *res, float *y,
                   int64_t batch, int M, int K, int act) {
    linear_forward("linear_fwd_ep", x, W, b, res, 0, y, batch, M, K, act);
}

void linear_fwd_glu(const float *x, const float *W, const float *b, const float *mul, float *y,
                    int64_t batch, int M, int K, int act) {
    linear_forward("linear_fwd_glu", x, W, b, mul, 1, y, batch, M, K, act);
}

/* pre = x W^T + b and y = act(pre): the outputs of linear_fwd followed by
 * silu_fwd / gelu_fwd / gelu_tanh_fwd, bit for bit (the GEMM epilogue applies
 * the elementwise kernels' activation function to the same float), in one
 * GEMM launch for batches above 8; otherwise those two calls. */
void ncm_linear_fwd_pre(const float *x, const float *W, const float *b, float *pre, float *y, int64_t batch,
                        int M, int K, int act) {
    const char *fn = "ncm_linear_fwd_pre";
    if (check_dims(fn, batch, M, K)) return;
    if (act != NCM_ACT_SILU && act != NCM_ACT_GELU && act != NCM_ACT_GELU_TANH) {
        ncm_fail(NCM_E_ARG, "%s: activation %d has no elementwise form", fn, act);
        return;
    }
    if (batch == 0) return;
    if (!x || !W || !y || !pre || pre == y) {
        ncm_fail(NCM_E_ARG, "%s: null x/W/y/pre or pre == y", fn);
        return;
    }
    if (ncm_ready()) return;
    if (batch <= 8) {
        linear_forward(fn, x, W, b, NULL, 0, pre, batch, M, K, NCM_ACT_NONE);
        int64_t n = batch * M;
        if (act == NCM_ACT_SILU) silu_fwd(pre, y, n);
        else if (act == NCM_ACT_GELU) gelu_fwd(pre, y, n);
        else gelu_tanh_fwd(pre, y, n);
        return;
    }
    int vec = (K % 4 == 0) && is_aligned16(x) && is_aligned16(W);
    GemmExtra ex = {NULL, pre, NULL, 0, NULL, NULL, NULL, NULL, NULL, 0};
    run_gemm_x(L_FWD, x, W, y, b, NULL, 0, (int)batch, M, K, K, K, M, act, vec, 1, &ex);
}

/* Both products of a gated unit in one GEMM launch when its tiles (64 rows x
 * 32 output columns of each product) fill the CUs; otherwise the up product
 * into a workspace, then the gate product with the multiply epilogue. */
void linear_fwd_gated(const float *x, const float *Wg, const float *bg, const float *Wu, const float *bu, float *y,
                      int64_t batch, int M, int K, int act) {
    const char *fn = "linear_fwd_gated";
    if (check_dims(fn, batch, M, K)) return;
    if (act < NCM_ACT_NONE || act > NCM_ACT_RELU2) {
        ncm_fail(NCM_E_ARG, "%s: unknown activation %d", fn, act);
        return;
    }
    if (batch == 0) return;
    if (!x || !Wg || !Wu || !y || y == x) {
        ncm_fail(NCM_E_ARG, "%s: null x/W/y, or y aliasing x", fn);
        return;
    }
    if (ncm_ready()) return;
    const int vec = (K % 4 == 0) && is_aligned16(x) && is_aligned16(Wg) && is_aligned16(Wu);
    const int tiles_m = (int)((batch + TILE_M - 1) / TILE_M), tiles_n = (M + 31) / 32;
    const int64_t tiles = (int64_t)tiles_m * tiles_n;
    if (batch > 8 && batch <= INT_MAX && vec && tiles >= ncm_cu_count() && tiles <= INT_MAX / 4) {
        int64_t ab = extent(batch, K, K), bb = extent(M, K, K);
        if (ab < MAX_BUFFER_BYTES && bb < MAX_BUFFER_BYTES) {
            const int groups = (K + 4 * BK - 1) / (4 * BK);
            GemmArgs p = {x, Wg, y, bg, NULL, NULL, (int)batch, M, K, K, K, M, act, 0,
                          tiles_m, tiles_n, 4 * groups, tiles_m * tiles_n, 1, (unsigned)ab, (unsigned)bb, Wu, bu, 1, NULL, NULL, NULL, NULL, 0,
                          {NULL}, {NULL}, {NULL}, {0}, {0}, 0};
            void *args[] = {&p};
            ncm_launch_named("gemm_64x64_gated_v", (unsigned)(tiles_m * tiles_n), 1, 1, 256, args);
            return;
        }
    }
    float *u = (float *)ncm_workspace(WS_GATED, (size_t)batch * M * sizeof(float));
    if (!u) return;
    linear_forward(fn, x, Wu, bu, NULL, 0, u, batch, M, K, NCM_ACT_NONE);
    linear_forward(fn, x, Wg, bg, u, 1, y, batch, M, K, act);
}

/* Kernel used for the dX of a batch <= 8 backward (transposed GEMV), or NULL. */
static const char *dxt_name(int nb) {
    static const char *n[9] = {NULL, "dxt_partial_b1", "dxt_partial_b2", NULL, "dxt_partial_b4",
                               NULL, NULL, NULL, "dxt_partial_b8"};
    return nb >= 1 && nb <= 8 ? n[nb] : NULL;
}
#define DXT_ROWS 32
#define COLSUM_ROWS 64
#define COLSUM_SMALL_ROWS 512   /* colsum_small covers up to this many rows */

static int run_dxt(const float *dy, const float *W, float *dx, int nb, int M, int K) {
    int r0 = 0;
    while (r0 < nb) {
        int left = nb - r0;
        int c = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
        int chunks = (M + DXT_ROWS - 1) / DXT_ROWS;
        float *part = (float *)ncm_workspace(WS_DXT, (size_t)chunks * c * K * sizeof(float));
        if (!part) return NCM_E_OOM;
        const float *dyc = dy + (int64_t)r0 * M;
        float *dxc = dx + (int64_t)r0 * K;
        void *a1[] = {&dyc, &W, &M, &K, &part};
        int rc = ncm_launch_named(dxt_name(c), (unsigned)((K + 255) / 256), (unsigned)chunks, 1, 256, a1);
        if (rc) return rc;
        int64_t n = (int64_t)c * K;
        void *a2[] = {&part, &chunks, &c, &K, &dxc};
        if ((rc = ncm_launch_named("dxt_final", (unsigned)((n + 63) / 64), 1, 1, 256, a2))) return rc;
        r0 += c;
    }
    return 0;
}

/* linear_bwd with dx_beta = 0: dx is written (0.0f + the product, the bits of
 * accumulating into zeros) instead of accumulated, so its buffer needs no
 * clearing; dW and db always accumulate. */
void ncm_linear_bwd_ex(const float *x, const float *W, const float *dy, float *dx, float *dW, float *db,
                       int64_t batch, int M, int K, int dx_beta) {
    if (check_dims("linear_bwd", batch, M, K)) return;
    if (batch == 0) return;
    if (!dy || (dx && !W) || (dW && !x)) {
        ncm_fail(NCM_E_ARG, "linear_bwd: null dy, or W for dx, or x for dW");
        return;
    }
    if (ncm_ready()) return;
    int nb = (int)batch;
    if (dx) {
        int rc;
        if (nb <= 8 && K % 4 == 0 && is_aligned16(W)) {
            if (!dx_beta && ncm_zero_async(dx, (size_t)nb * K * sizeof(float))) return;
            rc = run_dxt(dy, W, dx, nb, M, K);
        } else {
            int vec = (M % 4 == 0) && (K % 4 == 0) && is_aligned16(dy) && is_aligned16(W);
            rc = run_gemm(L_DX, dy, W, dx, NULL, NULL, 0, nb, K, M, M, K, K, 0, vec, dx_beta, NULL);
        }
        if (rc) return;
    }
    if (dW) {
        int rc;
        if (nb <= 8) {
            int vec = K % 4 == 0 && is_aligned16(x) && is_aligned16(dW);
            int K4 = (K + 3) / 4;
            int64_t n = (int64_t)M * K4;
            /* the rank-update kernel also adds db from the dy values it loads */
            void *a[] = {&dy, &x, &dW, &db, &nb, &M, &K};
            rc = ncm_launch_named(vec ? "dw_rank_v" : "dw_rank_s", (unsigned)((n + 255) / 256), 1, 1, 256, a);
            db = NULL;
        } else {
            int vec = (M % 4 == 0) && (K % 4 == 0) && is_aligned16(dy) && is_aligned16(x);
            /* the vectorised dW kernel also sums db (from the dy slabs it loads anyway) */
            rc = run_gemm(L_DW, dy, x, dW, NULL, NULL, 0, M, K, nb, M, K, K, 0, vec, 1, vec ? db : NULL);
            if (vec) db = NULL;
        }
        if (rc) return;
    }
    if (db) {
        if (nb <= COLSUM_SMALL_ROWS) {   /* one launch: a workgroup per 64 columns sums every row */
            void *a[] = {&dy, &nb, &M, &db};
            ncm_launch_named("colsum_small", (unsigned)((M + 63) / 64), 1, 1, 1024, a);
            return;
        }
        int chunks = (nb + COLSUM_ROWS - 1) / COLSUM_ROWS;
        double *part = (double *)ncm_workspace(WS_COLSUM, (size_t)chunks * M * sizeof(double));
        if (!part) return;
        int64_t rows = nb;
        int vec = M % 4 == 0 && is_aligned16(dy);
        void *a1[] = {&dy, &rows, &M, &part};
        if (ncm_launch_named(vec ? "colsum_partial_v" : "colsum_partial_s", (unsigned)((M + 255) / 256),
                             (unsigned)chunks, 1, 256, a1))
            return;
        void *a2[] = {&part, &chunks, &M, &db};
        if (chunks > 16)   /* many chunks: 16 waves per 64 columns */
            ncm_launch_named("colsum_final_w", (unsigned)((M + 63) / 64), 1, 1, 1024, a2);
        else
            ncm_launch_named("colsum_final", (unsigned)((M + 255) / 256), 1, 1, 256, a2);
    }
}

/* Three linear_fwd products of the same x (y_g = x W_g^T + b_g, W_g
 * [N_g][K]) in one GEMM launch, the q | k | v projections; N_0 and N_1 must be
 * multiples of 64 (a tile column never straddles two products), else, for
 * batches of at most 8 or unaligned operands, the three calls. */
void ncm_linear_fwd3(const float *x, const float *const W[3], const float *const b[3], float *const y[3],
                     const int N[3], int64_t batch, int K) {
    const char *fn = "ncm_linear_fwd3";
    for (int g = 0; g < 3; g++)
        if (check_dims(fn, batch, N[g], K)) return;
    if (batch == 0) return;
    int whole = N[0] % 64 == 0 && N[1] % 64 == 0 && batch > 8 && K % 4 == 0 && is_aligned16(x);
    for (int g = 0; g < 3; g++) {
        if (!W[g] || !y[g]) {
            ncm_fail(NCM_E_ARG, "%s: null W/y", fn);
            return;
        }
        whole = whole && is_aligned16(W[g]);
    }
    if (!x) {
        ncm_fail(NCM_E_ARG, "%s: null x", fn);
        return;
    }
    if (ncm_ready()) return;
    const int64_t Nt = (int64_t)N[0] + N[1] + N[2];
    if (!whole || Nt > INT_MAX) {
        for (int g = 0; g < 3; g++) linear_fwd(x, W[g], b[g], y[g], batch, N[g], K);
        return;
    }
    GemmExtra ex = {NULL, NULL, NULL, 0, W, b, y, N, NULL, 0};
    run_gemm_x(L_FWD, x, W[0], y[0], NULL, NULL, 0, (int)batch, (int)Nt, K, K, K, (int)Nt, NCM_ACT_NONE, 1, 1,
               &ex);
}

/* linear_fwd into qkv [B*T][C + 2 K hd] followed by qkv_split_fwd(qkv, qq, kk,
 * vv, B, T, C, H, hd, K, rep): for hd = 64, C = H hd, one kv head per query
 * head (K = H, rep = 1: the split copies each kv head once), T a multiple of
 * 64 (a tile's rows stay in one sequence) and aligned operands, the GEMM
 * stores each tile straight into its [64 t][64 d] block of qq, kk or vv (the
 * same values) and qkv is not written; otherwise the two calls. */
void ncm_linear_fwd_qkv_heads(const float *x, const float *W, const float *b, float *qkv, float *qq, float *kk,
                              float *vv, int B, int T, int C, int H, int hd, int K, int rep) {
    const int64_t rows = (int64_t)B * T, N = (int64_t)C + 2LL * K * hd;
    if (B < 0 || T < 0 || N > INT_MAX || rows > INT_MAX) {
        ncm_fail(NCM_E_ARG, "ncm_linear_fwd_qkv_heads: bad shape");
        return;
    }
    int whole = hd == 64 && C == H * hd && C % 64 == 0 && K == H && rep == 1 && rows > 8 && T % 64 == 0 &&
                C % 4 == 0 && x && W && qq && kk && vv && is_aligned16(x) && is_aligned16(W);
    if (!whole) {
        linear_fwd(x, W, b, qkv, rows, (int)N, C);
        qkv_split_fwd(qkv, qq, kk, vv, B, T, C, H, hd, K, rep);
        return;
    }
    if (check_dims("ncm_linear_fwd_qkv_heads", rows, (int)N, C) || ncm_ready()) return;
    float *const heads[3] = {qq, kk, vv};
    const int n3[3] = {C, K * hd, K * hd};
    GemmExtra ex = {NULL, NULL, NULL, 0, NULL, NULL, NULL, n3, heads, T};
    run_gemm_x(L_FWD, x, W, qq, b, NULL, 0, (int)rows, (int)N, C, C, C, (int)N, NCM_ACT_NONE, 1, 1, &ex);
}

/* linear_bwd whose x is the head merge of ctx [B][H][T][64] (x = rows (b, t)
 * of C = 64 H): the dX product is written (beta 0) or added (beta 1) straight
 * into ctx's gradient dctx, each tile one [64 t][64 d] block of a head, which
 * is linear_bwd's dX followed by the merge's backward, bit for bit; dW and db
 * as linear_bwd.  Needs ncm_linear_dx_fusable, T % 64 == 0. */
void ncm_linear_bwd_heads(const float *x, const float *W, const float *dy, float *dctx, int beta, float *dW,
                          float *db, int B, int T, int M, int H) {
    const int64_t batch = (int64_t)B * T;
    const int K = 64 * H;
    if (check_dims("ncm_linear_bwd_heads", batch, M, K)) return;
    if (!ncm_linear_dx_fusable(batch, M, K, dy, W) || T % 64 != 0 || !dctx || (dW && !x)) {
        ncm_fail(NCM_E_ARG, "ncm_linear_bwd_heads: shape or operands not supported");
        return;
    }
    if (ncm_ready()) return;
    float *const heads[3] = {dctx, NULL, NULL};
    const int n3[3] = {K, 0, 0};
    GemmExtra ex = {NULL, NULL, NULL, 0, NULL, NULL, NULL, n3, heads, T};
    if (run_gemm_x(L_DX, dy, W, dctx, NULL, NULL, 0, (int)batch, K, M, M, K, K, 0, 1, beta, &ex)) return;
    ncm_linear_bwd_ex(x, W, dy, NULL, dW, db, batch, M, K, 1);
}

int ncm_linear_dx_fusable(int64_t batch, int M, int K, const float *dy, const float *W) {
    return batch > 8 && batch <= INT_MAX && M > 0 && K > 0 && M % 4 == 0 && K % 4 == 0 && is_aligned16(dy) &&
           is_aligned16(W);
}

/* linear_bwd with the dX product passed back through the activation that
 * produced x: dxa (+)= act'(ax) (0.0f + dy W), i.e. ncm_linear_bwd_ex's fresh
 * dX followed by ncm_act_bwd_ex(kind, ax, dX, dxa, beta) bit for bit, with dX
 * never stored; dW and db as linear_bwd. */
void ncm_linear_bwd_act(const float *x, const float *W, const float *dy, float *dxa, const float *ax, int kind,
                        int beta, float *dW, float *db, int64_t batch, int M, int K) {
    if (check_dims("ncm_linear_bwd_act", batch, M, K)) return;
    if (!ncm_linear_dx_fusable(batch, M, K, dy, W) || !dxa || !ax || (dW && !x)) {
        ncm_fail(NCM_E_ARG, "ncm_linear_bwd_act: shape or operands not supported");
        return;
    }
    if (ncm_ready()) return;
    GemmExtra ex = {NULL, NULL, ax, kind == 0 || kind == 1 ? kind : 2, NULL, NULL, NULL, NULL, NULL, 0};
    if (run_gemm_x(L_DX, dy, W, dxa, NULL, NULL, 0, (int)batch, K, M, M, K, K, 0, 1, beta, &ex)) return;
    ncm_linear_bwd_ex(x, W, dy, NULL, dW, db, batch, M, K, 1);
}

void linear_bwd(const float *x, const float *W, const float *dy, float *dx, float *dW, float *db,
                int64_t batch, int M, int K) {
    ncm_linear_bwd_ex(x, W, dy, dx, dW, db, batch, M, K, 1);
}

int ncm_hip_linear_plan(int op, int64_t batch, int M, int K, char *kernel, size_t cap) {
    if (op < 0 || op > 3 || batch <= 0 || batch > INT_MAX || M <= 0 || K <= 0 || !kernel || !cap)
        return ncm_fail(NCM_E_ARG, "ncm_hip_linear_plan: bad arguments"), -1;
    int nb = (int)batch, with_db = op == 3;
    if (with_db) op = L_DW;
    if (op == L_FWD && nb <= 8) {
        gemv_name(nb >= 8 ? 8 : nb >= 4 ? 4 : nb >= 2 ? 2 : 1, M, K % 4 == 0, kernel, cap);
        return 1;
    }
    if (op == L_DX && nb <= 8 && K % 4 == 0) {
        snprintf(kernel, cap, "%s", dxt_name(nb >= 8 ? 8 : nb >= 4 ? 4 : nb >= 2 ? 2 : 1));
        return 1;
    }
    if (op == L_DW && nb <= 8) {
        snprintf(kernel, cap, "%s", K % 4 == 0 ? "dw_rank_v" : "dw_rank_s");
        return 1;
    }
    int Mo = op == L_DW ? M : nb, No = op == L_FWD ? M : K, Kred = op == L_FWD ? K : (op == L_DX ? M : nb);
    int vec = op == L_FWD ? K % 4 == 0 : (M % 4 == 0 && K % 4 == 0);
    const int bm = TILE_M, bn = TILE_N;
    gemm_name(bm, bn, op, vec, kernel, cap);
    if (with_db && vec) snprintf(kernel, cap, "gemm_%dx%d_%s_v", bm, bn, Kred % (4 * BK) ? "dwbt" : "dwb");
    if ((int64_t)((Mo + bm - 1) / bm) * ((No + bn - 1) / bn) > INT_MAX / 4)
        return ncm_fail(NCM_E_ARG, "ncm_hip_linear_plan: %d x %d output has too many tiles", Mo, No), -1;
    int slots = gemm_slots(kernel);
    if (slots < 0) return -1;
    GemmPlan g = plan_gemm(Mo, No, Kred, slots, bm, bn);
    const char *op_name = with_db && vec ? "dwb" : kind_names[op];
    if (use_big(op_name, vec, Mo, No, Kred, 0, g.cost, slots)) {
        snprintf(kernel, cap, "gemm_%dx%d_%s_v", BIG_TILE, BIG_TILE, op_name);
        return 1;
    }
    return g.segs;
}
