/* ops.c -- host side of the row-wise kernels (greedy id). */
#include "internal.h"

#include <limits.h>
#include <math.h>
#include <stdlib.h>

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

static unsigned grid_of(int64_t n, int per_block) { return (unsigned)((n + per_block - 1) / per_block); }
static int aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

static int ops_ready(const char *fn, int64_t n, int nptr, const void *p0, const void *p1) {
    if (n < 0) return ncm_fail(NCM_E_ARG, "%s: negative size", fn);
    if (n == 0) return 1;
    if ((nptr > 0 && !p0) || (nptr > 1 && !p1)) return ncm_fail(NCM_E_ARG, "%s: null pointer", fn);
    if ((n + 255) / 256 > UINT_MAX) return ncm_fail(NCM_E_ARG, "%s: too large", fn);
    return ncm_ready();
}

/* ---- norms (kernels.c:101-162) ---- */
/* The register-resident norm kernels take rows of C <= 1024 floats,
 * C % 4 == 0, 16-byte aligned. */
static int norm4_ok(const float *x, const float *w, const float *b, const float *y, int C) {
    return C % 4 == 0 && C <= 1024 && aligned16(x) && aligned16(w) && aligned16(b) && aligned16(y);
}

void rmsnorm_fwd(const float *x, const float *w, float *y, int64_t rows, int C) {
    if (C <= 0) { ncm_fail(NCM_E_ARG, "rmsnorm_fwd: C=%d", C); return; }
    if (ops_ready("rmsnorm_fwd", rows, 2, x, y)) return;
    if (norm4_ok(x, w, NULL, y, C)) {
        static const char *const k[4] = {"rmsnorm4_1", "rmsnorm4_2", "rmsnorm4_3", "rmsnorm4_4"};
        const float *none = NULL;
        double eps = 0.0;
        void *a[] = {&x, &w, &none, &y, &rows, &C, &eps};
        ncm_launch_named(k[(C + 255) / 256 - 1], grid_of(rows, 4), 1, 1, 256, a);
        return;
    }
    void *a[] = {&x, &w, &y, &rows, &C};
    ncm_launch_named("rmsnorm_k", grid_of(rows, 4), 1, 1, 256, a);
}

static void layernorm_any(const char *fn, const float *x, const float *w, const float *b, float *y, int64_t rows,
                          int C, double eps) {
    if (C <= 0) { ncm_fail(NCM_E_ARG, "%s: C=%d", fn, C); return; }
    if (ops_ready(fn, rows, 2, x, y)) return;
    void *a[] = {&x, &w, &b, &y, &rows, &C, &eps};
    if (norm4_ok(x, w, b, y, C)) {
        static const char *const k[4] = {"layernorm4_1", "layernorm4_2", "layernorm4_3", "layernorm4_4"};
        ncm_launch_named(k[(C + 255) / 256 - 1], grid_of(rows, 4), 1, 1, 256, a);
        return;
    }
    ncm_launch_named("layernorm_k", grid_of(rows, 4), 1, 1, 256, a);
}

void layernorm_fwd(const float *x, const float *w, const float *b, float *y, int64_t rows, int C) {
    layernorm_any("layernorm_fwd", x, w, b, y, rows, C, 1e-6);
}

void layernorm_eps_fwd(const float *x, const float *w, const float *b, float *y, int64_t rows, int C, float eps) {
    layernorm_any("layernorm_eps_fwd", x, w, b, y, rows, C, (double)eps);
}

/* ---- elementwise (kernels.c:167-226, 829-874) ---- */
static void eltwise(const char *fn, const float *a, const float *b, float *y, float s, int64_t n, int op) {
    if (ops_ready(fn, n, 2, a, y)) return;
    if ((op == 0 || op == 1) && !b) { ncm_fail(NCM_E_ARG, "%s: null operand", fn); return; }
    if (n % 4 == 0 && aligned16(a) && aligned16(y) && (!b || aligned16(b))) {
        int64_t n4 = n / 4;
        void *args[] = {&a, &b, &y, &s, &n4, &op};
        ncm_launch_named("eltwise4_k", grid_of(n4, 256), 1, 1, 256, args);
        return;
    }
    void *args[] = {&a, &b, &y, &s, &n, &op};
    ncm_launch_named("eltwise_k", grid_of(n, 256), 1, 1, 256, args);
}
void add_fwd(const float *a, const float *b, float *y, int64_t n) { eltwise("add_fwd", a, b, y, 0.f, n, 0); }
void mul_fwd(const float *a, const float *b, float *y, int64_t n) { eltwise("mul_fwd", a, b, y, 0.f, n, 1); }
void scale_fwd(const float *x, float s, float *y, int64_t n) { eltwise("scale_fwd", x, NULL, y, s, n, 2); }
void add_inplace_fwd(float *y, const float *x, int64_t n) { eltwise("add_inplace_fwd", x, NULL, y, 0.f, n, 3); }
void ncm_add_inplace_ex(float *y, const float *x, int64_t n, int beta) {
    eltwise("add_inplace_fwd", x, NULL, y, 0.f, n, beta ? 3 : 7);
}
void silu_fwd(const float *x, float *y, int64_t n) { eltwise("silu_fwd", x, NULL, y, 0.f, n, 4); }
void gelu_fwd(const float *x, float *y, int64_t n) { eltwise("gelu_fwd", x, NULL, y, 0.f, n, 5); }
void gelu_tanh_fwd(const float *x, float *y, int64_t n) { eltwise("gelu_tanh_fwd", x, NULL, y, 0.f, n, 6); }

/* ---- RoPE (kernels.c:285-308) ---- */
static void rope_rows(float *x, const float *cos_t, const float *sin_t, int64_t rows, int T, int hd) {
    int64_t n = rows * (hd / 2);
    if (!x || n == 0) return;
    void *a[] = {&x, &cos_t, &sin_t, &rows, &T, &hd};
    ncm_launch_named("rope_k", grid_of(n, 256), 1, 1, 256, a);
}

void rope_apply_gqa(float *q, float *k, const float *cos_t, const float *sin_t, int B, int H, int K, int T, int hd) {
    if (B < 0 || H < 0 || K < 0 || T <= 0 || hd <= 0 || (hd & 1)) {
        ncm_fail(NCM_E_ARG, "rope_apply_gqa: bad shape B=%d H=%d K=%d T=%d hd=%d", B, H, K, T, hd);
        return;
    }
    if ((q || k) && (!cos_t || !sin_t)) { ncm_fail(NCM_E_ARG, "rope_apply_gqa: null tables"); return; }
    if (ncm_ready()) return;
    rope_rows(q, cos_t, sin_t, (int64_t)B * H * T, T, hd);
    rope_rows(k, cos_t, sin_t, (int64_t)B * K * T, T, hd);
}

void rope_apply(float *q, float *k, const float *cos_t, const float *sin_t, int B, int H, int T, int hd) {
    rope_apply_gqa(q, k, cos_t, sin_t, B, H, H, T, hd);
}

/* ---- layout (kernels.c:311-357, 891-936) and embedding (kernels.c:59-74) ---- */
void heads_transpose_fwd_b(const float *in, float *out, int B, int64_t T, int H, int hd) {
    int64_t n = (int64_t)B * T * H * hd;
    if (B < 0 || T < 0 || H < 0 || hd < 0) { ncm_fail(NCM_E_ARG, "heads_transpose_fwd: bad shape"); return; }
    if (ops_ready("heads_transpose_fwd", n, 2, in, out)) return;
    if (hd % 4 == 0 && (int64_t)B * T <= INT_MAX && T <= INT_MAX && aligned16(in) && aligned16(out)) {
        int Ti = (int)T;
        void *a[] = {&in, &out, &Ti, &H, &hd};
        ncm_launch_named("heads_transpose_rows_k", (unsigned)(B * T), 1, 1, 256, a);
        return;
    }
    void *a[] = {&in, &out, &B, &T, &H, &hd};
    ncm_launch_named("heads_transpose_k", grid_of(n, 256), 1, 1, 256, a);
}

void heads_transpose_fwd(const float *in, float *out, int64_t T, int H, int hd) {
    heads_transpose_fwd_b(in, out, 1, T, H, hd);
}

void qkv_split_fwd(const float *in, float *qq, float *kk, float *vv, int B, int T, int C, int H, int hd, int K,
                   int rep) {
    int64_t n = (int64_t)B * H * T * hd;
    if (B < 0 || T < 0 || H < 0 || hd < 0 || K <= 0 || rep <= 0 || (H - 1) / rep >= K ||
        (int64_t)H * hd > C) {
        ncm_fail(NCM_E_ARG, "qkv_split_fwd: bad shape (H=%d K=%d rep=%d)", H, K, rep);
        return;
    }
    if (ops_ready("qkv_split_fwd", n, 2, in, qq)) return;
    if (!kk || !vv) { ncm_fail(NCM_E_ARG, "qkv_split_fwd: null pointer"); return; }
    if (hd % 4 == 0 && C % 4 == 0 && (int64_t)B * T <= INT_MAX && (int64_t)C + 2 * K * hd <= INT_MAX &&
        aligned16(in) && aligned16(qq) && aligned16(kk) && aligned16(vv)) {
        void *a[] = {&in, &qq, &kk, &vv, &T, &C, &H, &hd, &K, &rep};
        ncm_launch_named("qkv_split_rows_k", (unsigned)((int64_t)B * T), 1, 1, 256, a);
        return;
    }
    void *a[] = {&in, &qq, &kk, &vv, &B, &T, &C, &H, &hd, &K, &rep};
    ncm_launch_named("qkv_split_k", grid_of(n, 256), 1, 1, 256, a);
}

void qkv_split_rope_fwd(const float *in, float *qq, float *kk, float *vv, const float *cos_t, const float *sin_t,
                        int B, int T, int C, int H, int hd, int K, int rep) {
    int64_t n = (int64_t)B * H * T * (hd / 2);
    if (B < 0 || T < 0 || H < 0 || hd <= 0 || (hd & 1) || K <= 0 || rep <= 0 || (H - 1) / rep >= K ||
        (int64_t)H * hd > C) {
        ncm_fail(NCM_E_ARG, "qkv_split_rope_fwd: bad shape (H=%d K=%d rep=%d hd=%d)", H, K, rep, hd);
        return;
    }
    if (ops_ready("qkv_split_rope_fwd", n, 2, in, qq)) return;
    if (!kk || !vv || !cos_t || !sin_t) { ncm_fail(NCM_E_ARG, "qkv_split_rope_fwd: null pointer"); return; }
    void *a[] = {&in, &qq, &kk, &vv, &cos_t, &sin_t, &B, &T, &C, &H, &hd, &K, &rep};
    ncm_launch_named("qkv_split_rope_k", grid_of(n, 256), 1, 1, 256, a);
}

void head_merge_fwd(const float *ctx, float *out, int B, int T, int C, int H, int hd) {
    int64_t n = (int64_t)B * T * C;
    if (B < 0 || T < 0 || C < 0 || H <= 0 || hd <= 0 || C > H * hd) {
        ncm_fail(NCM_E_ARG, "head_merge_fwd: bad shape");
        return;
    }
    if (ops_ready("head_merge_fwd", n, 2, ctx, out)) return;
    if (hd % 4 == 0 && C % 4 == 0 && (int64_t)B * T <= INT_MAX && aligned16(ctx) && aligned16(out)) {
        void *a[] = {&ctx, &out, &T, &C, &H, &hd};
        ncm_launch_named("head_merge_rows_k", (unsigned)((int64_t)B * T), 1, 1, 256, a);
        return;
    }
    void *a[] = {&ctx, &out, &B, &T, &C, &H, &hd};
    ncm_launch_named("head_merge_k", grid_of(n, 256), 1, 1, 256, a);
}

void embedding_fwd_v(const float *W, int V, const int *idx, float *y, int64_t n, int D) {
    if (D <= 0 || V <= 0) { ncm_fail(NCM_E_ARG, "embedding_fwd: D=%d V=%d", D, V); return; }
    if (ops_ready("embedding_fwd", n * D, 2, W, y)) return;
    if (!idx) { ncm_fail(NCM_E_ARG, "embedding_fwd: null idx"); return; }
    void *a[] = {&W, &idx, &y, &n, &D, &V};
    ncm_launch_named("embedding_k", grid_of(n * D, 256), 1, 1, 256, a);
}

void embedding_fwd(const float *W, const int *idx, float *y, int64_t n, int D) {
    embedding_fwd_v(W, INT_MAX, idx, y, n, D);
}

/* ---- SDPA (kernels.c:364-507) ---- */
/* out [B][Hq][Tq][hd], or [B][Tq][Hq * hd] (the heads merged) when merged */
/* Key-split attention for grids that cannot fill the chip (few (b, h) pairs
 * and long rows, e.g. a single-sequence prefill): each query tile's key range
 * is cut into parts of at most P key blocks, sized for about four workgroups
 * per CU, and sdpa_hd64_combine merges the parts of the tiles that were cut.
 * The work and tile lists depend only on the shape and are built once per
 * shape (a few cached) on the device.  Returns 0 when launched, 1 when the
 * unsplit kernel should run (the grid already fills the chip, or no tile is
 * long enough to cut). */
#define SPLIT_MAXP 8
typedef struct { int B, Hq, Tq, Tkv, causal; int4 *work; int2 *tiles; int nwork, nsplit, nslots; } SplitPlan;
static SplitPlan g_split[4];
static int g_split_next;

static int sdpa_split(const float *q, const float *k, const float *v, const float *mask, int64_t mask_bs, float *out,
                      int B, int Hq, int Hkv, int Tq, int Tkv, float scale, int causal, int merged) {
    const int ntiles = (Tq + 63) / 64, C = ncm_cu_count();
    const int64_t BH = (int64_t)B * Hq;
    if (BH * ntiles >= 2 * (int64_t)C || BH > INT_MAX / 4096) return 1;
    SplitPlan *sp = NULL;
    for (int i = 0; i < 4; i++)
        if (g_split[i].work && g_split[i].B == B && g_split[i].Hq == Hq && g_split[i].Tq == Tq &&
            g_split[i].Tkv == Tkv && g_split[i].causal == causal)
            sp = &g_split[i];
    if (!sp) {
        int *nkb = (int *)malloc((size_t)ntiles * sizeof(int));
        if (!nkb) return 1;
        int64_t units = 0;
        int maxb = 0;
        for (int t = 0; t < ntiles; t++) {
            const int kend = causal ? (t * 64 + 64 + (Tkv - Tq) < Tkv ? t * 64 + 64 + (Tkv - Tq) : Tkv) : Tkv;
            nkb[t] = (kend + 63) / 64;
            units += nkb[t];
            if (nkb[t] > maxb) maxb = nkb[t];
        }
        int P = (int)((BH * units + 4 * (int64_t)C - 1) / (4 * (int64_t)C));
        if (P < (maxb + SPLIT_MAXP - 1) / SPLIT_MAXP) P = (maxb + SPLIT_MAXP - 1) / SPLIT_MAXP;
        if (P < 2) P = 2;
        if (P >= maxb) { free(nkb); return 1; }
        int nwork = 0, nsplit = 0, nslots = 0;
        for (int t = 0; t < ntiles; t++) {
            const int np = (nkb[t] + P - 1) / P;
            nwork += np;
            if (np > 1) { nsplit++; nslots += np; }
        }
        int4 *work = (int4 *)malloc((size_t)nwork * sizeof(int4));
        int2 *tiles = (int2 *)malloc((size_t)(nsplit + 1) * sizeof(int2));
        if (!work || !tiles) { free(nkb); free(work); free(tiles); return 1; }
        int w = 0, st = 0, slot = 0;
        /* longest parts first: part lengths P, P - 1, ..., 1 in turn */
        for (int len = P; len >= 1; len--)
            for (int t = ntiles - 1; t >= 0; t--) {
                const int np = (nkb[t] + P - 1) / P;
                for (int p = 0; p < np; p++) {
                    const int l = nkb[t] - p * P < P ? nkb[t] - p * P : P;
                    if (l != len) continue;
                    work[w].x = t; work[w].y = p * P; work[w].z = l; work[w].w = -1;
                    w++;
                }
            }
        for (int t = 0; t < ntiles; t++) {   /* slots of the cut tiles, in tile order */
            const int np = (nkb[t] + P - 1) / P;
            if (np < 2) continue;
            tiles[st].x = t; tiles[st].y = slot;
            for (int i = 0; i < nwork; i++)
                if (work[i].x == t) work[i].w = slot + work[i].y / P;
            slot += np;
            st++;
        }
        tiles[nsplit].x = 0; tiles[nsplit].y = nslots;
        free(nkb);
        sp = &g_split[g_split_next];
        g_split_next = (g_split_next + 1) % 4;
        if (sp->work) { ncm_hip_sync(); ncm_hip_free(sp->work); ncm_hip_free(sp->tiles); }
        sp->work = (int4 *)ncm_hip_malloc((size_t)nwork * sizeof(int4));
        sp->tiles = (int2 *)ncm_hip_malloc((size_t)(nsplit + 1) * sizeof(int2));
        if (!sp->work || !sp->tiles) {
            free(work); free(tiles);
            if (sp->work) ncm_hip_free(sp->work);
            if (sp->tiles) ncm_hip_free(sp->tiles);
            sp->work = NULL; sp->tiles = NULL;
            return 1;
        }
        mem_h2d(sp->work, work, (size_t)nwork * sizeof(int4));
        mem_h2d(sp->tiles, tiles, (size_t)(nsplit + 1) * sizeof(int2));
        free(work);
        free(tiles);
        sp->B = B; sp->Hq = Hq; sp->Tq = Tq; sp->Tkv = Tkv; sp->causal = causal;
        sp->nwork = nwork; sp->nsplit = nsplit; sp->nslots = nslots;
    }
    if ((int64_t)sp->nwork * BH > INT_MAX) return 1;
    float *part = (float *)ncm_workspace(WS_ATTN, (size_t)BH * sp->nslots * 64 * 66 * sizeof(float));
    if (!part) return -1;
    float *part_o = part, *part_ml = part + (size_t)BH * sp->nslots * 64 * 64;
    int bh = (int)BH, nslots = sp->nslots;
    void *a[] = {&q, &k, &v, &mask, &out, &Hq, &Hkv, &Tq, &Tkv, &scale, &causal, &merged, &sp->work, &bh, &nslots,
                 &part_o, &part_ml, &mask_bs};
    if (ncm_launch_named("sdpa_hd64_split", (unsigned)(sp->nwork * BH), 1, 1, 256, a)) return -1;
    if (sp->nsplit > 0) {
        void *a2[] = {&sp->tiles, &part_o, &part_ml, &out, &Hq, &Tq, &merged, &nslots};
        if (ncm_launch_named("sdpa_hd64_combine", (unsigned)sp->nsplit, (unsigned)BH, 1, 256, a2)) return -1;
    }
    return 0;
}

/* mask_bs: floats between consecutive boards' masks (0: one [Tq][Tkv] mask
 * for every board) */
static void sdpa_any_bm(const char *fn, const float *q, const float *k, const float *v, const float *mask,
                        int64_t mask_bs, float *out, int B, int Hq, int Hkv, int Tq, int Tkv, int hd, int causal,
                        int merged, float *stats) {
    if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || Tq < 0 || Tkv <= 0 || hd <= 0 || hd > 256) {
        ncm_fail(NCM_E_ARG, "%s: bad shape B=%d Hq=%d Hkv=%d Tq=%d Tkv=%d hd=%d", fn, B, Hq, Hkv, Tq, Tkv, hd);
        return;
    }
    if (causal && Tq > Tkv) {
        ncm_fail(NCM_E_ARG, "%s: causal attention needs Tq <= Tkv (Tq=%d Tkv=%d)", fn, Tq, Tkv);
        return;
    }
    if ((int64_t)B * Tq == 0) return;
    if (!q || !k || !v || !out) { ncm_fail(NCM_E_ARG, "%s: null pointer", fn); return; }
    if (B > 65535 || Hq > 65535 || (Tq + 63) / 64 > 65535) { ncm_fail(NCM_E_ARG, "%s: grid too large", fn); return; }
    if (ncm_ready()) return;
    float scale = 1.0f / sqrtf((float)hd);
    if (hd == 64 && is_aligned16(q) && is_aligned16(k) && is_aligned16(v) && is_aligned16(out)) {
        if (!stats && sdpa_split(q, k, v, mask, mask_bs, out, B, Hq, Hkv, Tq, Tkv, scale, causal, merged) <= 0)
            return;
        void *a[] = {&q, &k, &v, &mask, &out, &Hq, &Hkv, &Tq, &Tkv, &scale, &causal, &merged, &stats, &mask_bs};
        ncm_launch_named("sdpa_hd64", (unsigned)Hq, (unsigned)B, (unsigned)((Tq + 63) / 64), 256, a);
    } else if (stats) {
        ncm_fail(NCM_E_ARG, "%s: row statistics need hd = 64 and 16-byte aligned operands", fn);
    } else {
        int64_t rows = (int64_t)B * Hq * Tq;
        void *a[] = {&q, &k, &v, &mask, &out, &B, &Hq, &Hkv, &Tq, &Tkv, &hd, &scale, &causal, &merged, &mask_bs};
        ncm_launch_named("sdpa_rows", grid_of(rows, 4), 1, 1, 256, a);
    }
}

static void sdpa_any(const char *fn, const float *q, const float *k, const float *v, const float *mask, float *out,
                     int B, int Hq, int Hkv, int Tq, int Tkv, int hd, int causal, int merged, float *stats) {
    sdpa_any_bm(fn, q, k, v, mask, 0, out, B, Hq, Hkv, Tq, Tkv, hd, causal, merged, stats);
}

/* sdpa_fwd_gqa_merged with one [Tq][Tkv] mask per board (board b's at mask +
 * b * Tq * Tkv): the NCP forward's boards with padded prefix tokens, each
 * with its own key mask, in one launch (ncp.c:571-607 runs them one board
 * at a time). */
void ncm_sdpa_fwd_gqa_merged_bmask(const float *q, const float *k, const float *v, const float *masks, float *out,
                                   int B, int Hq, int Hkv, int Tq, int Tkv, int hd) {
    if (!masks) {
        ncm_fail(NCM_E_ARG, "ncm_sdpa_fwd_gqa_merged_bmask: null masks");
        return;
    }
    sdpa_any_bm("ncm_sdpa_fwd_gqa_merged_bmask", q, k, v, masks, (int64_t)Tq * Tkv, out, B, Hq, Hkv, Tq, Tkv, hd, 0,
                1, NULL);
}

void sdpa_fwd_gqa(const float *q, const float *k, const float *v, const float *mask, float *out, int B, int Hq,
                  int Hkv, int Tq, int Tkv, int hd) {
    sdpa_any("sdpa_fwd_gqa", q, k, v, mask, out, B, Hq, Hkv, Tq, Tkv, hd, 0, 0, NULL);
}

void sdpa_fwd(const float *q, const float *k, const float *v, const float *mask, float *out, int B, int H, int Tq,
              int Tkv, int hd) {
    sdpa_any("sdpa_fwd", q, k, v, mask, out, B, H, H, Tq, Tkv, hd, 0, 0, NULL);
}

void sdpa_fwd_gqa_merged(const float *q, const float *k, const float *v, const float *mask, float *out, int B,
                         int Hq, int Hkv, int Tq, int Tkv, int hd) {
    sdpa_any("sdpa_fwd_gqa_merged", q, k, v, mask, out, B, Hq, Hkv, Tq, Tkv, hd, 0, 1, NULL);
}

void sdpa_fwd_gqa_causal(const float *q, const float *k, const float *v, float *out, int B, int Hq, int Hkv, int Tq,
                         int Tkv, int hd) {
    sdpa_any("sdpa_fwd_gqa_causal", q, k, v, NULL, out, B, Hq, Hkv, Tq, Tkv, hd, 1, 0, NULL);
}

void ncm_sdpa_fwd_causal_merged(const float *q, const float *k, const float *v, float *out, int B, int Hq, int Hkv,
                                int Tq, int Tkv, int hd) {
    sdpa_any("ncm_sdpa_fwd_causal_merged", q, k, v, NULL, out, B, Hq, Hkv, Tq, Tkv, hd, 1, 1, NULL);
}

void ncm_sdpa_fwd_stats_merged(const float *q, const float *k, const float *v, const float *mask, float *out,
                               float *stats, int B, int Hq, int Hkv, int Tq, int Tkv, int hd, int causal) {
    sdpa_any("ncm_sdpa_fwd_stats_merged", q, k, v, mask, out, B, Hq, Hkv, Tq, Tkv, hd, causal, 1, stats);
}

void ncm_sdpa_fwd_stats(const float *q, const float *k, const float *v, const float *mask, float *out, float *stats,
                        int B, int Hq, int Hkv, int Tq, int Tkv, int hd, int causal) {
    sdpa_any("ncm_sdpa_fwd_stats", q, k, v, mask, out, B, Hq, Hkv, Tq, Tkv, hd, causal, 0, stats);
}
