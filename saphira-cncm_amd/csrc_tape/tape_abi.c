/* tape_abi.c -- libncmhip_tape.so: the reference's tape prototypes
 * (ncm.h:192-195, 468-522) over the device tape of libncmhip.so, so that a
 * trainer compiled against ncm.h links unchanged (include/ncm_hip_tape.h).
 * A Tape is an NcmTape and a PMap has NcmPMap's layout; every record and
 * the backward are libncmhip.so's. */
#include "ncm_hip.h"
#include "ncm_hip_tape.h"

#include <stddef.h>

_Static_assert(sizeof(PMap) == sizeof(NcmPMap) && offsetof(PMap, params) == offsetof(NcmPMap, params) &&
                   offsetof(PMap, grads) == offsetof(NcmPMap, grads) &&
                   offsetof(PMap, sizes) == offsetof(NcmPMap, sizes) && offsetof(PMap, n) == offsetof(NcmPMap, n),
               "PMap (ncm.h:513-518) and NcmPMap must share their layout");

#define NT(t) ((NcmTape *)(t))

Tape *tape_new(void) { return (Tape *)ncm_tape_new(); }
void tape_free(Tape *t) { ncm_tape_free(NT(t)); }
void tape_clear(Tape *t) { ncm_tape_clear(NT(t)); }

void t_linear(Tape *t, const float *x, const float *W, const float *b, float *y, int64_t batch, int M, int K) {
    ncm_t_linear(NT(t), x, W, b, y, batch, M, K);
}
void t_embed(Tape *t, const float *W, const int *idx, int V, float *y, int64_t n, int D) {
    ncm_t_embed(NT(t), W, idx, V, y, n, D);
}
void t_layernorm(Tape *t, const float *x, const float *w, const float *b, float *y, int64_t rows, int C) {
    ncm_t_layernorm(NT(t), x, w, b, y, rows, C);
}
void t_layernorm_eps(Tape *t, const float *x, const float *w, const float *b, float *y, int64_t rows, int C,
                     double eps) {
    ncm_t_layernorm_eps(NT(t), x, w, b, y, rows, C, eps);
}
void t_rmsnorm(Tape *t, const float *x, const float *w, float *y, int64_t rows, int C) {
    ncm_t_rmsnorm(NT(t), x, w, y, rows, C);
}
void t_gelu(Tape *t, const float *x, float *y, int64_t n) { ncm_t_gelu(NT(t), x, y, n); }
void t_gelu_tanh(Tape *t, const float *x, float *y, int64_t n) { ncm_t_gelu_tanh(NT(t), x, y, n); }
void t_mul(Tape *t, const float *a, const float *b, float *y, int64_t n) { ncm_t_mul(NT(t), a, b, y, n); }
void t_silu(Tape *t, const float *x, float *y, int64_t n) { ncm_t_silu(NT(t), x, y, n); }
void t_rope(Tape *t, const float *xq, const float *xk, float *yq, float *yk, const float *cos, const float *sin,
            int B, int H, int Hkv, int T, int hd) {
    ncm_t_rope(NT(t), xq, xk, yq, yk, cos, sin, B, H, Hkv, T, hd);
}
void t_sdpa(Tape *t, const float *q, const float *k, const float *v, const float *mask, float *o, int B, int H,
            int Hkv, int Tq, int Tkv, int hd) {
    ncm_t_sdpa(NT(t), q, k, v, mask, o, B, H, Hkv, Tq, Tkv, hd);
}
void t_headsplit(Tape *t, const float *in, float *out, int B, int T, int C, int H, int hd) {
    ncm_t_headsplit(NT(t), in, out, B, T, C, H, hd);
}
void t_add(Tape *t, const float *a, const float *b, float *y, int64_t n) { ncm_t_add(NT(t), a, b, y, n); }
void t_scale(Tape *t, const float *x, float s, float *y, int64_t n) { ncm_t_scale(NT(t), x, s, y, n); }
void t_ce(Tape *t, const float *logits, const int *tgt, const float *wmask, float *loss, float *probs,
          int64_t rows, int V, double weight) {
    ncm_t_ce(NT(t), logits, tgt, wmask, loss, probs, rows, V, weight);
}
void t_qkvsplit(Tape *t, const float *in, float *qq, float *kk, float *vv, int B, int T, int C, int H, int hd,
                int K, int rep) {
    ncm_t_qkvsplit(NT(t), in, qq, kk, vv, B, T, C, H, hd, K, rep);
}
void t_headmerge(Tape *t, const float *ctx, float *out, int B, int T, int C, int H, int hd) {
    ncm_t_headmerge(NT(t), ctx, out, B, T, C, H, hd);
}

void tape_backward(Tape *t, PMap *pm, float seed) {
    (void)seed;   /* dL/dloss = 1, as the reference's tape takes it */
    ncm_tape_backward(NT(t), (const NcmPMap *)pm);
}
