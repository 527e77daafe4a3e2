/* dropin_check.c -- a C caller written against the REFERENCE's ncm.h
 * (compiled with -I/root/reference/src; only the header is used) and linked
 * to libncmhip.so, to show that the library is a link-level drop-in for the
 * reference's kernel and memory API: the Tensor struct, tensor_alloc /
 * tensor_to_backend / tensor_to_host, arena_init / arena_alloc /
 * arena_reset, mem_h2d / mem_d2h, backend_to_host and the kernel prototypes
 * (ncm.h:29-56, 141-199) are called exactly as the reference's own callers
 * call them, with no library-specific initialisation.
 *
 * Usage: dropin_check DIR.  DIR holds dims.txt and raw float32 inputs
 * written by tests/test_gpu_dropin.py; the outputs are written back as raw
 * float32 / int32 files for that test to compare.  Test infrastructure. */
#include "ncm.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static const char *g_dir;

static float *read_f(const char *name, size_t n) {
    char p[1024];
    snprintf(p, sizeof p, "%s/%s", g_dir, name);
    FILE *f = fopen(p, "rb");
    float *h = (float *)malloc(n * sizeof(float) + 16);
    if (!f || !h || fread(h, sizeof(float), n, f) != n) {
        fprintf(stderr, "dropin_check: cannot read %zu floats from %s\n", n, p);
        exit(2);
    }
    fclose(f);
    return h;
}

static void write_raw(const char *name, const void *h, size_t bytes) {
    char p[1024];
    snprintf(p, sizeof p, "%s/%s", g_dir, name);
    FILE *f = fopen(p, "wb");
    if (!f || fwrite(h, 1, bytes, f) != bytes) {
        fprintf(stderr, "dropin_check: cannot write %s\n", p);
        exit(2);
    }
    fclose(f);
}

/* a backend copy of a host file, from the scratch arena */
static float *upload(const char *name, size_t n) {
    float *h = read_f(name, n);
    float *d = arena_alloc(n);
    mem_h2d(d, h, n * sizeof(float));
    free(h);
    return d;
}

static void download(const char *name, const float *d, size_t n) {
    float *h = (float *)backend_to_host(d, n * sizeof(float));
    write_raw(name, h, n * sizeof(float));
    free(h);
}

int main(int argc, char **argv) {
    if (argc != 2) {
        fprintf(stderr, "usage: dropin_check DIR\n");
        return 2;
    }
    g_dir = argv[1];
    char p[1024];
    snprintf(p, sizeof p, "%s/dims.txt", g_dir);
    FILE *f = fopen(p, "r");
    int lb, lM, lK, hasb, ar, av, aC, B, Hq, Hkv, Tq, Tkv, hd, nr, nc, nv;
    if (!f || fscanf(f, "%d %d %d %d %d %d %d %d %d %d %d %d %d %d %d %d", &lb, &lM, &lK, &hasb, &ar, &av, &aC, &B,
                     &Hq, &Hkv, &Tq, &Tkv, &hd, &nr, &nc, &nv) != 16) {
        fprintf(stderr, "dropin_check: bad dims.txt\n");
        return 2;
    }
    fclose(f);

    arena_init((size_t)256 << 20);

    /* linear_fwd with W held in a Tensor (tensor_alloc + tensor_to_backend) */
    int64_t wshape[2] = {lM, lK};
    Tensor *Wt = tensor_alloc(2, wshape);
    if (Wt->n != (int64_t)lM * lK || Wt->ndim != 2 || Wt->shape[0] != lM || Wt->shape[1] != lK) {
        fprintf(stderr, "dropin_check: Tensor fields differ from ncm.h's layout\n");
        return 3;
    }
    float *Wh = read_f("W.bin", (size_t)lM * lK);
    tensor_to_backend(Wt, Wh);
    float *Wback = (float *)malloc((size_t)lM * lK * sizeof(float));
    tensor_to_host(Wt, Wback);
    if (memcmp(Wback, Wh, (size_t)lM * lK * sizeof(float)) != 0) {
        fprintf(stderr, "dropin_check: tensor_to_host did not return what tensor_to_backend stored\n");
        return 3;
    }
    free(Wh);
    free(Wback);
    float *x = upload("x.bin", (size_t)lb * lK);
    float *b = hasb ? upload("b.bin", (size_t)lM) : NULL;
    float *y = arena_alloc((size_t)lb * lM);
    linear_fwd(x, Wt->data, b, y, lb, lM, lK);
    download("y.bin", y, (size_t)lb * lM);
    tensor_free(Wt);
    arena_reset();

    /* rowwise_l2sq */
    float *a = upload("a.bin", (size_t)ar * aC), *e = upload("e.bin", (size_t)av * aC);
    float *d2 = arena_alloc((size_t)ar * av);
    rowwise_l2sq(a, e, d2, ar, av, aC);
    download("d2.bin", d2, (size_t)ar * av);
    arena_reset();

    /* sdpa_fwd_gqa with a causal additive mask */
    float *q = upload("q.bin", (size_t)B * Hq * Tq * hd), *k = upload("k.bin", (size_t)B * Hkv * Tkv * hd),
          *v = upload("v.bin", (size_t)B * Hkv * Tkv * hd), *mask = upload("mask.bin", (size_t)Tq * Tkv);
    float *o = arena_alloc((size_t)B * Hq * Tq * hd);
    sdpa_fwd_gqa(q, k, v, mask, o, B, Hq, Hkv, Tq, Tkv, hd);
    download("o.bin", o, (size_t)B * Hq * Tq * hd);
    arena_reset();

    /* rmsnorm_fwd and layernorm_fwd */
    float *xr = upload("xr.bin", (size_t)nr * nc), *wr = upload("wr.bin", (size_t)nc),
          *br = upload("br.bin", (size_t)nc);
    float *yr = arena_alloc((size_t)nr * nc), *yl = arena_alloc((size_t)nr * nc);
    rmsnorm_fwd(xr, wr, yr, nr, nc);
    layernorm_fwd(xr, wr, br, yl, nr, nc);
    download("rms.bin", yr, (size_t)nr * nc);
    download("ln.bin", yl, (size_t)nr * nc);
    arena_reset();

    /* argmax_row on a host row fetched with backend_to_host (qwen.c:220-222) */
    float *lg = upload("logits.bin", (size_t)nv);
    float *hl = (float *)backend_to_host(lg, (size_t)nv * sizeof(float));
    int id = argmax_row(hl, nv);
    free(hl);
    write_raw("argmax.bin", &id, sizeof id);
    arena_reset();
    arena_free();
    printf("dropin_check: ok\n");
    return 0;
}
