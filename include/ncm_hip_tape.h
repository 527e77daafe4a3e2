/* ncm_hip_tape.h -- the training tape under the reference's own names:
 * libncmhip_tape.so exports the Tape, PMap, tape_* and t_* prototypes of
 * the reference's src/ncm.h (ncm.h:192-195, 468-522) for the ops the device
 * tape of libncmhip.so implements, so that a trainer written against ncm.h
 * (train_gpt2.c:42-180 is one) links unchanged.  Each function forwards to
 * its ncm_t_* / ncm_tape_* counterpart in ncm_hip.h: the same records, run
 * on the device, the same gradients.
 *
 * A separate library so that these names never clash with the reference's
 * train_tape.c where both are linked into one program; libncmhip_tape.so
 * depends on libncmhip.so, which provides the memory substrate (arena_*,
 * mem_*, tensor_*) and the kernels.
 *
 * Not exported (no device implementation here, so a caller that needs them
 * fails at link time instead of running something else): t_groupnorm,
 * t_relu2, t_softmax, t_conv, t_convt, t_iarea, t_ilin, t_concat, t_join,
 * t_gather_rows, t_mse, t_tied (the VQ-VAE and NCP training records) and the
 * path-specific tape_backward_host / tape_backward_dev /
 * tape_backward_force (train_tape.c:539-565). */
#ifndef NCM_HIP_TAPE_H
#define NCM_HIP_TAPE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ncm.h:192: opaque; here the device tape of libncmhip.so */
typedef struct Tape Tape;
/* ncm.h:513-518; same layout as NcmPMap.  params[i]'s gradient accumulates
 * into grads[i] (device buffers of sizes[i] floats). */
typedef struct {
    float **params;
    float **grads;
    int64_t *sizes;
    int n;
} PMap;

/* tape_new / tape_free / tape_clear, ncm.h:468-470, train_tape.c:59-84 */
Tape *tape_new(void);
void tape_free(Tape *t);
void tape_clear(Tape *t);

/* the records, ncm.h:471-522 (train_tape.c:156-481): the forward runs on the
 * device when the record is made; all pointers are device memory except
 * the token ids of t_embed and the targets / weight mask of t_ce, which are
 * host memory as in the reference */
void t_linear(Tape *t, const float *x, const float *W, const float *b, float *y, int64_t batch, int M, int K);
void t_embed(Tape *t, const float *W, const int *idx, int V, float *y, int64_t n, int D);
void t_layernorm(Tape *t, const float *x, const float *w, const float *b, float *y, int64_t rows, int C);
void t_layernorm_eps(Tape *t, const float *x, const float *w, const float *b, float *y, int64_t rows, int C,
                     double eps);
void t_rmsnorm(Tape *t, const float *x, const float *w, float *y, int64_t rows, int C);
void t_gelu(Tape *t, const float *x, float *y, int64_t n);
void t_gelu_tanh(Tape *t, const float *x, float *y, int64_t n);
void t_mul(Tape *t, const float *a, const float *b, float *y, int64_t n);
void t_silu(Tape *t, const float *x, float *y, int64_t n);
void t_rope(Tape *t, const float *xq, const float *xk, float *yq, float *yk, const float *cos, const float *sin,
            int B, int H, int Hkv, int T, int hd);
void t_sdpa(Tape *t, const float *q, const float *k, const float *v, const float *mask, float *o, int B, int H,
            int Hkv, int Tq, int Tkv, int hd);
void t_headsplit(Tape *t, const float *in, float *out, int B, int T, int C, int H, int hd);
void t_add(Tape *t, const float *a, const float *b, float *y, int64_t n);
void t_scale(Tape *t, const float *x, float s, float *y, int64_t n);
void t_ce(Tape *t, const float *logits, const int *tgt, const float *wmask, float *loss, float *probs,
          int64_t rows, int V, double weight);
/* ncm.h:193-195 */
void t_qkvsplit(Tape *t, const float *in, float *qq, float *kk, float *vv, int B, int T, int C, int H, int hd,
                int K, int rep);
void t_headmerge(Tape *t, const float *ctx, float *out, int B, int T, int C, int H, int hd);

/* tape_backward, ncm.h:519, train_tape.c:545-556: every gradient accumulated
 * on the device.  seed is accepted and not used, as in the reference
 * (train_tape.c:636-641 and 1926-1927 both take dL/dloss = 1; its callers
 * pass 0). */
void tape_backward(Tape *t, PMap *pm, float seed);

#ifdef __cplusplus
}
#endif

#endif /* NCM_HIP_TAPE_H */
