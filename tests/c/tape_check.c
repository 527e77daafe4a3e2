/* tape_check.c -- a GPT-2 training step written against the REFERENCE's
 * ncm.h (compiled with -I/root/reference/src; only the header is used) and
 * linked to libncmhip_tape.so + libncmhip.so: the taped forward of
 * train_gpt2.c:42-147 (t_embed x2, t_add, per block t_layernorm_eps,
 * t_linear, t_qkvsplit, t_sdpa with the uploaded causal mask, t_headmerge,
 * t_linear, t_add, t_layernorm_eps, t_linear, t_gelu_tanh, t_linear, t_add;
 * ln_f and the tied head), t_ce, and tape_backward(tp, &pm, 0) as
 * train_gpt2.c:146-159 calls them, with the library's arena and memory
 * calls (ncm.h:29-56).  The step runs twice (tape_clear, arena_reset and
 * zeroed gradients in between), and the second must equal the first bit
 * for bit.
 *
 * Usage: tape_check DIR.  DIR holds dims.txt ("n_layer C H V npos B T"),
 * params.bin (float32, the parameters in the order wte, wpe, 12 tensors per
 * block, ln_f weight and bias), ids.bin and tgt.bin (int32 [B][T]); writes
 * loss.bin (float32) and grads.bin (the gradients in parameter order).
 * Test infrastructure (tests/test_gpu_tape_abi.py). */
#include "ncm.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static const char *g_dir;

static void *read_file(const char *name, size_t bytes) {
    char p[1024];
    snprintf(p, sizeof p, "%s/%s", g_dir, name);
    FILE *f = fopen(p, "rb");
    void *h = malloc(bytes + 16);
    if (!f || !h || fread(h, 1, bytes, f) != bytes) {
        fprintf(stderr, "tape_check: cannot read %zu bytes from %s\n", bytes, p);
        exit(2);
    }
    fclose(f);
    return h;
}

static void write_file(const char *name, const void *h, size_t bytes) {
    char p[1024];
    snprintf(p, sizeof p, "%s/%s", g_dir, name);
    FILE *f = fopen(p, "wb");
    if (!f || fwrite(h, 1, bytes, f) != bytes) {
        fprintf(stderr, "tape_check: cannot write %s\n", p);
        exit(2);
    }
    fclose(f);
}

/* One taped step in the order of train_gpt2.c:42-159; returns the loss. */
static float step(Tape *tp, float **P, int L, int C, int H, int V, int npos, const int *ids, const int *tgt, int B,
                  int T, PMap *pm) {
    const int hd = C / H, I = 4 * C;
    const int64_t R = (int64_t)B * T;
    tape_clear(tp);
    arena_reset();
    float *xe = arena_alloc((size_t)R * C), *pe = arena_alloc((size_t)R * C), *h = arena_alloc((size_t)R * C);
    t_embed(tp, P[0], ids, V, xe, R, C);
    int *ph = (int *)malloc((size_t)R * sizeof(int));
    for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++) ph[(size_t)b * T + t] = t;
    t_embed(tp, P[1], ph, npos, pe, R, C);
    free(ph);
    t_add(tp, xe, pe, h, (size_t)R * C);
    float *hm = (float *)malloc((size_t)T * T * sizeof(float));
    for (int tq = 0; tq < T; tq++)
        for (int tk = 0; tk < T; tk++) hm[(size_t)tq * T + tk] = tk <= tq ? 0.0f : -1e9f;
    float *mask = arena_alloc((size_t)T * T);
    mem_h2d(mask, hm, (size_t)T * T * sizeof(float));
    free(hm);
    for (int li = 0; li < L; li++) {
        float **w = P + 2 + 12 * li;
        float *ln = arena_alloc((size_t)R * C), *qkv = arena_alloc((size_t)R * 3 * C);
        float *qq = arena_alloc((size_t)R * C), *kk = arena_alloc((size_t)R * C), *vv = arena_alloc((size_t)R * C);
        float *ctx = arena_alloc((size_t)R * C), *mo = arena_alloc((size_t)R * C), *ao = arena_alloc((size_t)R * C);
        float *x1 = arena_alloc((size_t)R * C), *mn = arena_alloc((size_t)R * C), *mm = arena_alloc((size_t)R * I);
        float *m2 = arena_alloc((size_t)R * I), *mlpo = arena_alloc((size_t)R * C), *out = arena_alloc((size_t)R * C);
        t_layernorm_eps(tp, h, w[0], w[1], ln, R, C, 1e-5);
        t_linear(tp, ln, w[2], w[3], qkv, R, 3 * C, C);
        t_qkvsplit(tp, qkv, qq, kk, vv, B, T, C, H, hd, H, 1);
        t_sdpa(tp, qq, kk, vv, mask, ctx, B, H, H, T, T, hd);
        t_headmerge(tp, ctx, mo, B, T, C, H, hd);
        t_linear(tp, mo, w[4], w[5], ao, R, C, C);
        t_add(tp, h, ao, x1, (size_t)R * C);
        t_layernorm_eps(tp, x1, w[6], w[7], mn, R, C, 1e-5);
        t_linear(tp, mn, w[8], w[9], mm, R, I, C);
        t_gelu_tanh(tp, mm, m2, R * I);
        t_linear(tp, m2, w[10], w[11], mlpo, R, C, I);
        t_add(tp, x1, mlpo, out, (size_t)R * C);
        h = out;
    }
    const int n = 2 + 12 * L + 2;
    float *lnf = arena_alloc((size_t)R * C), *logits = arena_alloc((size_t)R * V);
    t_layernorm_eps(tp, h, P[n - 2], P[n - 1], lnf, R, C, 1e-5);
    t_linear(tp, lnf, P[0], NULL, logits, R, V, C);
    float *loss = arena_alloc(1), *probs = arena_alloc((size_t)R * V);
    t_ce(tp, logits, tgt, NULL, loss, probs, R, V, 1.0);
    tape_backward(tp, pm, 0);
    float lh;
    float *lp = (float *)backend_to_host(loss, sizeof(float));
    lh = *lp;
    free(lp);
    return lh;
}

int main(int argc, char **argv) {
    if (argc != 2) {
        fprintf(stderr, "usage: tape_check DIR\n");
        return 2;
    }
    g_dir = argv[1];
    char p[1024];
    snprintf(p, sizeof p, "%s/dims.txt", g_dir);
    FILE *f = fopen(p, "r");
    int L, C, H, V, npos, B, T;
    if (!f || fscanf(f, "%d %d %d %d %d %d %d", &L, &C, &H, &V, &npos, &B, &T) != 7) {
        fprintf(stderr, "tape_check: bad dims.txt\n");
        return 2;
    }
    fclose(f);
    const int n = 2 + 12 * L + 2;
    int64_t *sizes = (int64_t *)malloc((size_t)n * sizeof(int64_t));
    sizes[0] = (int64_t)V * C;
    sizes[1] = (int64_t)npos * C;
    const int64_t per[12] = {C, C, 3LL * C * C, 3LL * C, (int64_t)C * C, C, C, C, 4LL * C * C, 4LL * C, 4LL * C * C, C};
    for (int li = 0; li < L; li++)
        for (int j = 0; j < 12; j++) sizes[2 + 12 * li + j] = per[j];
    sizes[n - 2] = sizes[n - 1] = C;
    int64_t total = 0;
    for (int i = 0; i < n; i++) total += sizes[i];

    arena_init((size_t)1 << 30);
    float *ph = (float *)read_file("params.bin", (size_t)total * sizeof(float));
    float *zeros = (float *)calloc((size_t)total, sizeof(float));
    Tensor **pt = (Tensor **)malloc((size_t)n * sizeof(Tensor *)), **gt = (Tensor **)malloc((size_t)n * sizeof(Tensor *));
    float **P = (float **)malloc((size_t)n * sizeof(float *)), **G = (float **)malloc((size_t)n * sizeof(float *));
    int64_t off = 0;
    for (int i = 0; i < n; i++) {
        int64_t shape[1] = {sizes[i]};
        pt[i] = tensor_alloc(1, shape);
        gt[i] = tensor_alloc(1, shape);
        tensor_to_backend(pt[i], ph + off);
        tensor_to_backend(gt[i], zeros);
        P[i] = pt[i]->data;
        G[i] = gt[i]->data;
        off += sizes[i];
    }
    int *ids = (int *)read_file("ids.bin", (size_t)B * T * sizeof(int));
    int *tgt = (int *)read_file("tgt.bin", (size_t)B * T * sizeof(int));
    PMap pm;
    pm.params = P;
    pm.grads = G;
    pm.sizes = sizes;
    pm.n = n;

    Tape *tp = tape_new();
    const float l1 = step(tp, P, L, C, H, V, npos, ids, tgt, B, T, &pm);
    float *g1 = (float *)malloc((size_t)total * sizeof(float));
    off = 0;
    for (int i = 0; i < n; i++) {
        tensor_to_host(gt[i], g1 + off);
        tensor_to_backend(gt[i], zeros);   /* zero for the second step */
        off += sizes[i];
    }
    const float l2 = step(tp, P, L, C, H, V, npos, ids, tgt, B, T, &pm);
    float *g2 = (float *)malloc((size_t)total * sizeof(float));
    off = 0;
    for (int i = 0; i < n; i++) {
        tensor_to_host(gt[i], g2 + off);
        off += sizes[i];
    }
    if (memcmp(&l1, &l2, sizeof l1) != 0 || memcmp(g1, g2, (size_t)total * sizeof(float)) != 0) {
        fprintf(stderr, "tape_check: the second step (after tape_clear) differs from the first\n");
        return 3;
    }
    write_file("loss.bin", &l2, sizeof l2);
    write_file("grads.bin", g2, (size_t)total * sizeof(float));
    tape_free(tp);
    for (int i = 0; i < n; i++) {
        tensor_free(pt[i]);
        tensor_free(gt[i]);
    }
    arena_free();
    printf("tape_check: ok\n");
    return 0;
}
