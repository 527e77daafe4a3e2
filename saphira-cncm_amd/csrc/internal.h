/* internal.h -- shared declarations of the libncmhip host runtime (C11). */
#ifndef NCM_INTERNAL_H
#define NCM_INTERNAL_H

#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stddef.h>

#include "ncm_hip.h"

#define NCM_E_HIP   1
#define NCM_E_ARG   2
#define NCM_E_OOM   3
#define NCM_E_INIT  4

/* Records (or, in NCM_ERR_EXIT mode, reports and exits on) an error. Returns code. */
int ncm_fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
/* 0 when the runtime is usable, otherwise an error code (already recorded). */
int ncm_ready(void);
hipStream_t ncm_stream(void);
/* The device selected by ncm_hip_init. */
int ncm_device(void);

/* Looks up a kernel of one of the embedded code objects by name (cached). */
hipFunction_t ncm_kernel(const char *name);
/* Launches `f` on the library stream with one by-value argument block per
 * entry of args (hipModuleLaunchKernel kernelParams convention). */
int ncm_launch(hipFunction_t f, unsigned gx, unsigned gy, unsigned gz, unsigned block,
               void **args);
int ncm_launch_named(const char *name, unsigned gx, unsigned gy, unsigned gz, unsigned block,
                     void **args);

/* Library-owned device workspaces (grown on demand, stream-synchronised
 * before a grow).  Slot ids keep independent users apart. */
enum { WS_SPLITK = 0, WS_COLSUM = 1, WS_VQ = 2, WS_DXT = 3, WS_TRAIN = 4, WS_SAMPLE = 5, WS_VQF = 6, WS_GATED = 7, WS_ATTN = 8, WS_VQSOFT = 9, WS_COUNT = 10 };
/* Host-to-device copy of at most 256 KB through pinned staging, ordered on
 * the library stream, returning without waiting for it (the host buffer is
 * free on return); larger copies synchronise as mem_h2d. */
int ncm_h2d_async(void *d, const void *h, size_t n);
/* Stream-ordered device copy / zero fill on the library stream (no sync). */
int ncm_copy_async(void *d, const void *s, size_t n);
int ncm_zero_async(void *d, size_t n);
/* Device sampler launches (sample.c): id to *out (flag to *flag), or to
 * ids[*pos + 1] (flag[*pos + 1]) with ++*pos when pos is set; temp > 0;
 * launches only (graph-capturable).  ws: a caller-owned workspace of
 * ncm_sample_ws_bytes(V) bytes, or NULL for the library's. */
int ncm_sample_launch(const float *x, int V, float temp, int top_k, float top_p, unsigned long long *rng,
                      int *out, int *ids, int *pos, int *flag, void *ws);
size_t ncm_sample_ws_bytes(int V);

/* adamw_update that also zeroes g after reading it (the training driver's
 * step; the gradient is consumed and the next step accumulates from zero). */
void ncm_adamw_update_clear(float *p, float *g, float *m, float *v, int64_t n, double lr, double b1, double b2,
                            double b1t, double b2t, double eps, double wd);
/* pre = x W^T + b and y = act(pre) for act SILU / GELU / GELU_TANH, bit for
 * bit linear_fwd followed by the elementwise activation (linear.c). */
void ncm_linear_fwd_pre(const float *x, const float *W, const float *b, float *pre, float *y, int64_t batch,
                        int M, int K, int act);
/* Three linear_fwd products of the same x in one GEMM launch (linear.c). */
void ncm_linear_fwd3(const float *x, const float *const W[3], const float *const b[3], float *const y[3],
                     const int N[3], int64_t batch, int K);
/* linear_fwd into qkv then qkv_split_fwd, with the split done by the GEMM's
 * epilogue (qkv not written) when hd = 64, C = H hd, K = H and 64 | T (linear.c). */
void ncm_linear_fwd_qkv_heads(const float *x, const float *W, const float *b, float *qkv, float *qq, float *kk,
                              float *vv, int B, int T, int C, int H, int hd, int K, int rep);
/* 1 when linear_bwd's dX runs as one vectorised GEMM (batch > 8, M and K
 * multiples of 4, dy and W 16-byte aligned): then ncm_linear_bwd_act applies. */
int ncm_linear_dx_fusable(int64_t batch, int M, int K, const float *dy, const float *W);
/* linear_bwd whose dX goes back through the activation (kind 0 GELU, 1 SiLU,
 * 2 GELU tanh form) that produced x from ax: dxa (+)= act'(ax) (0.0f + dy W)
 * (beta 1 accumulates, 0 writes), bit for bit the fresh dX followed by
 * ncm_act_bwd_ex, the dX itself never stored; dW / db accumulate. */
void ncm_linear_bwd_act(const float *x, const float *W, const float *dy, float *dxa, const float *ax, int kind,
                        int beta, float *dW, float *db, int64_t batch, int M, int K);
/* linear_bwd whose x [B*T][64 H] is the head merge of ctx [B][H][T][64]: dX
 * written (beta 0) or added into ctx's gradient directly (T % 64 == 0; the
 * merge's backward bit for bit); dW / db accumulate. */
void ncm_linear_bwd_heads(const float *x, const float *W, const float *dy, float *dctx, int beta, float *dW,
                          float *db, int B, int T, int M, int H);
/* Backward ops with a first-write form: beta 1 accumulates (the public
 * functions' contract), beta 0 writes 0.0f + the gradient -- the bits of an
 * accumulation into zeros -- so the output needs no clearing and is not read.
 * Where a path cannot write every element it clears the output first. */
void ncm_linear_bwd_ex(const float *x, const float *W, const float *dy, float *dx, float *dW, float *db,
                       int64_t batch, int M, int K, int dx_beta);
void ncm_layernorm_bwd_ex(const float *x, const float *w, const float *dy, float *dx, float *dw, float *db,
                          int64_t rows, int C, double eps, int beta);
void ncm_rmsnorm_bwd_ex(const float *x, const float *w, const float *dy, float *dx, float *dw, int64_t rows, int C,
                        int beta);
/* norm backward writing dx = (0.0f + base) + the norm's gradient: a residual
 * gradient's first write and the norm's accumulation onto it, in one pass */
void ncm_layernorm_bwd_base(const float *x, const float *w, const float *dy, float *dx, float *dw, float *db,
                            int64_t rows, int C, double eps, const float *base);
void ncm_rmsnorm_bwd_base(const float *x, const float *w, const float *dy, float *dx, float *dw, int64_t rows, int C,
                          const float *base);
void ncm_act_bwd_ex(int kind, const float *x, const float *dy, float *dx, int64_t n, int beta);
void ncm_add_inplace_ex(float *y, const float *x, int64_t n, int beta);
/* (o_ld > 0: o stored with the heads merged, rows (b, t) of stride o_ld) */
void ncm_sdpa_bwd_flash_ex(const float *q, const float *k, const float *v, const float *o, const float *stats,
                           const float *mask, int causal, const float *dO, float *dq, float *dk, float *dv, int B,
                           int H, int Hkv, int Tq, int Tkv, int hd, int beta, int o_ld);
/* ncm_sdpa_bwd_flash_ex with the three gradients written into the q | k | v
 * rows' gradient dqkv [B*T][(H + 2 Hkv) hd] (q at column 0, k at H hd, v at
 * (H + Hkv) hd): the gradient qkv_split_bwd would form from them, when q, k
 * and v came from such rows by a split with one kv head per kv head. */
void ncm_sdpa_bwd_flash_rows(const float *q, const float *k, const float *v, const float *o, const float *stats,
                             const float *mask, int causal, const float *dO, float *dqkv, int B, int H, int Hkv,
                             int Tq, int Tkv, int hd, int beta, int o_ld);
void ncm_qkv_split_bwd_ex(const float *gq, const float *gk, const float *gv, float *dx, int B, int T, int C, int H,
                          int hd, int K, int rep, int beta);
void ncm_heads_bwd_ex(const float *dy, float *dx, int B, int T, int C, int H, int hd, int dir, int beta);
/* grad_clip_global(G, sizes, count, max_norm) followed by
 * ncm_adamw_update_clear (clear_g) or adamw_update on every tensor, in three
 * launches with no host synchronisation; *g2_dev gets the device address of
 * the gradients' sum of squares before clipping.  Returns -1 (nothing
 * launched) for lists this path does not take (over 2048 tensors). */
int ncm_clip_adamw_multi(float *const *P, float *const *G, float *const *M, float *const *V, const int64_t *sizes,
                         int count, double max_norm, double lr, double b1, double b2, double b1t, double b2t,
                         double eps, double wd, int clear_g, const double **g2_dev);
/* conv1d_fwd (kernels.c:546-566, bit-exact) on [B][T][D] rows with D input
 * and D output channels: y [B][To][D], To = (T + 2 pad - K) / stride + 1;
 * W [D][D][K]; launches only. */
int ncm_conv1d_btd(const float *x, const float *W, const float *b, float *y, int B, int T, int D, int K, int stride,
                   int pad);
/* sdpa_fwd_gqa_causal with the heads merged on output: out [B][Tq][Hq * hd]
 * (the values of sdpa_fwd_gqa_causal followed by head_merge_fwd). */
void ncm_sdpa_fwd_causal_merged(const float *q, const float *k, const float *v, float *out, int B, int Hq, int Hkv,
                                int Tq, int Tkv, int hd);
/* sdpa_fwd_gqa_merged with one [Tq][Tkv] mask per board (board b's at
 * masks + b Tq Tkv). */
void ncm_sdpa_fwd_gqa_merged_bmask(const float *q, const float *k, const float *v, const float *masks, float *out,
                                   int B, int Hq, int Hkv, int Tq, int Tkv, int hd);
/* ncm_sdpa_fwd_stats with the heads merged on output: out [B][Tq][Hq hd]. */
void ncm_sdpa_fwd_stats_merged(const float *q, const float *k, const float *v, const float *mask, float *out,
                               float *stats, int B, int Hq, int Hkv, int Tq, int Tkv, int hd, int causal);
/* SDPA forward (hd 64, 16-byte aligned operands) that also writes each
 * query row's softmax (max, sum) to stats [B][Hq][Tq][2]; causal generates
 * the mask (query t sees keys <= t + Tkv - Tq) instead of reading one. */
void ncm_sdpa_fwd_stats(const float *q, const float *k, const float *v, const float *mask, float *out, float *stats,
                        int B, int Hq, int Hkv, int Tq, int Tkv, int hd, int causal);
/* SDPA backward that recomputes the probabilities from q, k and the row
 * statistics of ncm_sdpa_fwd_stats (no stored P); gradients accumulate. */
void ncm_sdpa_bwd_flash(const float *q, const float *k, const float *v, const float *o, const float *stats,
                        const float *mask, int causal, const float *dO, float *dq, float *dk, float *dv, int B, int H,
                        int Hkv, int Tq, int Tkv, int hd);
/* Compute units of the selected device. */
int ncm_cu_count(void);
void *ncm_workspace(int slot, size_t bytes);

#define HIP_TRY(call)                                                              \
    do {                                                                           \
        hipError_t e_ = (call);                                                    \
        if (e_ != hipSuccess)                                                      \
            return ncm_fail(NCM_E_HIP, "%s:%d %s: %s", __FILE__, __LINE__, #call, \
                            hipGetErrorString(e_));                                \
    } while (0)

static inline int is_aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

/* File helpers shared by the NCM1 / NCK1 code (formats.c): exact reads
 * (0 on success), little-endian integers, and a device buffer streamed to
 * sink() through a bounded host staging buffer that is wiped afterwards. */
#include <stdio.h>
int fmt_read_exact(FILE *f, void *dst, size_t n);
int fmt_read_u32le(FILE *f, uint32_t *v);
int fmt_read_u64le(FILE *f, uint64_t *v);
int fmt_download(const float *dev, uint64_t nbytes, void (*sink)(void *, const void *, size_t), void *ctx);

#endif
