/* ncm_hip.h -- C ABI of libncmhip.so, the MI355X (gfx950) backend for cncm's
 * matrix-multiplication hot path.
 *
 * The library is a drop-in for the kernel/memory surface of the reference's
 * src/ncm.h: every function below that carries a "replaces" citation keeps the
 * reference prototype, argument meaning and out-params-last convention, and all
 * float pointers are DEVICE pointers (the reference's "backend memory",
 * ncm.h:29-34 and ncm.h:141-143).  Entry points marked "extension" have no
 * one-to-one reference prototype: each replaces a sequence of reference calls
 * that the caller would otherwise issue (cited per function).
 *
 * Execution model: one HIP stream per process (ncm_hip_stream()); every kernel
 * entry point is asynchronous on it, every mem_* copy is synchronous (as the
 * reference's cudaMemcpy-based mem_* are, tensor.c:323-344).
 *
 * Errors: by default a failing HIP call or an invalid argument prints a
 * message and calls exit(1), the reference behaviour (tensor.c:10-12,
 * tensor.c:301-305).  ncm_hip_set_error_mode(NCM_ERR_RECORD) switches to
 * "record and return": the call does nothing further and the message is kept
 * for ncm_hip_last_error().
 */
#ifndef NCM_HIP_H
#define NCM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ */
/* runtime (extension: the reference selects its device implicitly)    */
/* ------------------------------------------------------------------ */

#define NCM_ERR_EXIT   0
#define NCM_ERR_RECORD 1

/* Select device, create the stream, load the embedded gfx950 code objects.
 * Called implicitly by the first entry point; returns 0 on success. */
int   ncm_hip_init(int device);
void  ncm_hip_set_error_mode(int mode);
/* Copies the last error message (if any) into buf; returns its error code
 * (0 = no error since the last call) and clears it. */
int   ncm_hip_last_error(char *buf, size_t cap);
/* Blocks until all work queued on the library stream has finished. */
void  ncm_hip_sync(void);
/* The hipStream_t every kernel entry point launches on. */
void *ncm_hip_stream(void);
/* Device allocation helpers for callers that do not use Tensor/arenas. */
void *ncm_hip_malloc(size_t bytes);
void  ncm_hip_free(void *p);
/* Test hook (no counterpart in the reference): after n more successful
 * ncm_hip_malloc calls, the next ones fail with NCM_E_OOM as if the device
 * memory were exhausted; n < 0 (the default) turns it off.  Lets the tests
 * drive the library's allocation-failure paths. */
void  ncm_hip_fail_alloc_after(long n);

/* ------------------------------------------------------------------ */
/* tensor + memory substrate -- replaces src/tensor.c (ncm.h:27-56)     */
/* ------------------------------------------------------------------ */

#define NCM_MAX_DIMS 4

/* Same layout as the reference Tensor (ncm.h:29-34). */
typedef struct {
    float  *data;
    int64_t shape[NCM_MAX_DIMS];
    int     ndim;
    int64_t n;
} Tensor;

/* replaces tensor_alloc / tensor_free / tensor_numel, ncm.h:37-39, tensor.c:15-42 */
Tensor *tensor_alloc(int ndim, const int64_t *shape);
void    tensor_free(Tensor *t);
int64_t tensor_numel(int ndim, const int64_t *shape);
/* replaces tensor_to_host / tensor_to_backend, ncm.h:42-43, tensor.c:44-62 */
void tensor_to_host(const Tensor *t, float *out);
void tensor_to_backend(Tensor *t, const float *in);
/* replaces mem_d2h / mem_h2d / mem_d2d, ncm.h:44-46, tensor.c:323-344 (synchronous) */
void mem_d2h(void *h, const void *d, size_t n);
void mem_h2d(void *d, const void *h, size_t n);
void mem_d2d(void *d, const void *s, size_t n);
/* replaces the scratch bump arena, ncm.h:49-53, tensor.c:268-321:
 * 16-byte aligned bump allocation, overflow is an error. */
void   arena_init(size_t bytes);
void   arena_init_default(void);
float *arena_alloc(size_t n_floats);
void   arena_reset(void);
void   arena_free(void);
/* replaces the persistent arena, ncm.h:54-55, tensor.c:346-365 */
void   parena_init(size_t bytes);
float *parena_alloc(size_t n_floats);
/* replaces backend_to_host, tensor.c:367-371: malloc'd host copy */
void  *backend_to_host(const float *d, size_t nbytes);

/* ------------------------------------------------------------------ */
/* linear (FP32 MFMA GEMM / GEMV)                                      */
/* ------------------------------------------------------------------ */

#define NCM_ACT_NONE      0
#define NCM_ACT_SILU      1  /* v/(1+exp(-v)), kernels.c:220-226 */
#define NCM_ACT_GELU      2  /* exact erf GELU, kernels.c:185-194 */
#define NCM_ACT_GELU_TANH 3  /* HF gelu_new, kernels.c:207-218 */
#define NCM_ACT_RELU2     4  /* relu(v)^2, the NCP MLP's use_relu2 (ncp.c:327-333) */

/* replaces linear_fwd, ncm.h:145-146, kernels.c:38-54:
 * y[r,m] = b[m] + sum_k x[r,k] W[m,k];  x:[batch,K], W:[M,K], b:[M]|NULL, y:[batch,M] */
void linear_fwd(const float *x, const float *W, const float *b,
                float *y, int64_t batch, int M, int K);

/* extension: linear_fwd with a fused epilogue y = res + act(x W^T + b).
 * Replaces linear_fwd followed by silu_fwd/gelu_fwd/gelu_tanh_fwd and/or
 * add_fwd (e.g. ncp.c:296-298, qwen.c:159-161).  res may be NULL; res may
 * alias y (in-place residual update). */
void linear_fwd_ep(const float *x, const float *W, const float *b,
                   const float *res, float *y, int64_t batch, int M, int K, int act);

/* extension: the gated unit y = act(x W^T + b) * mul, elementwise with mul
 * [batch][M] (a buffer other than y).  Replaces linear_fwd + silu_fwd
 * followed by mul_fwd(g, u, g) (ncp.c:301-310, qwen.c:162-166): the product
 * is formed in the GEMM's epilogue, with the same float operations. */
void linear_fwd_glu(const float *x, const float *W, const float *b,
                    const float *mul, float *y, int64_t batch, int M, int K, int act);

/* extension: the whole gated unit y = act(x Wg^T + bg) * (x Wu^T + bu), y
 * [batch][M] (not aliasing x), bg / bu may be NULL.  Replaces the gate
 * linear_fwd + silu_fwd, the up linear_fwd and mul_fwd (ncp.c:301-310,
 * qwen.c:162-166); one GEMM launch computes both products. */
void linear_fwd_gated(const float *x, const float *Wg, const float *bg, const float *Wu,
                      const float *bu, float *y, int64_t batch, int M, int K, int act);

/* extension: the linear backward of the autograd tape, host path
 * train_tape.c:680-725 and device path train_tape.c:1978-2000:
 *   dx[r,k] += sum_m dy[r,m] W[m,k]        (dX = dY . W)
 *   dW[m,k] += sum_r dy[r,m] x[r,k]        (dW = dY^T . X)
 *   db[m]   += sum_r dy[r,m]
 * Any of dx, dW, db may be NULL to skip that gradient.  Accumulates, like
 * the tape's gradient map. */
void linear_bwd(const float *x, const float *W, const float *dy,
                float *dx, float *dW, float *db, int64_t batch, int M, int K);

/* extension: which kernel a linear call launches (op 0 = linear_fwd,
 * 1 = dX of linear_bwd, 2 = dW of linear_bwd, 3 = dW and db of one
 * linear_bwd call: the dW GEMM then also sums db) for 16-byte aligned
 * operands, written to `kernel`; returns the number of K splits (>= 1; a
 * split count above 1 adds a fixup launch), -1 on bad arguments. */
int ncm_hip_linear_plan(int op, int64_t batch, int M, int K, char *kernel, size_t cap);
/* extension for tuning and tests: 64 or 128 runs every GEMM that has a
 * kernel of that tile size (128 x 128: the vectorised ones, whole tiles) on
 * it; 0 (the default) lets the library's cost model choose per call. */
void ncm_hip_set_gemm_tiles(int mode);

/* ------------------------------------------------------------------ */
/* VQ nearest-codeword search                                          */
/* ------------------------------------------------------------------ */

/* replaces rowwise_l2sq, ncm.h:187-188, kernels.c:753-770:
 * d2[i,j] = (float) sum_c ((double)a[i,c] - b[j,c])^2, fp64 serial over c. */
void rowwise_l2sq(const float *a, const float *b, float *d2,
                  int64_t rows, int64_t colsA, int C);

/* extension: fused distance + argmin.  Replaces rowwise_l2sq followed by
 * the device->host copy and the host strict-'<' scan of vq.c:410-443:
 * idx[i] = lowest j minimising (float) sum_c ((double)a[i,c]-E[j,c])^2.
 * Bit-exact with that reference sequence; never materialises the rows x V
 * distance matrix.  idx is a device int32 array. */
void vq_argmin(const float *a, const float *E, int *idx, int64_t rows, int V, int D);
/* extension for tests and profiling: with counting on, every search (of
 * vq_argmin, vq_quantize_multiscale and the quantiser) waits for its rescore
 * and adds up the rows the fp32 screen could not certify: those decided
 * between two tracked codewords (pairs) and those rescored against every
 * codeword (full).  Turning counting on or off clears the totals. */
void ncm_vq_count_rescores(int on);
void ncm_vq_rescore_counts(long long *pairs, long long *full);

/* extension with no counterpart in the reference: vq_argmin for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and the same codes as
 * vq_argmin, but the search's scratch lives in a fixed 9 MiB device array
 * that the library reserves per GPU for the life of the process, so no call
 * allocates.  Limits: rows <= 262144, V <= 65536 (D <= 4096 as vq_argmin);
 * larger shapes are refused with an error.  Calls on one GPU share the
 * array: calls that overlap on one GPU (several host threads) race.
 * Returns 0 or an error code. */
int vq_argmin_noalloc(const float *a, const float *E, int *idx, int64_t rows, int V, int D);

/* extension: the multiscale residual quantiser of vq_z_to_idx
 * (vq.c:378-500) for configurations whose every level has length L
 * (area/linear resampling are identities) and Phi disabled
 * (quant_resi_ratio = 0).  Per level lv: codes = vq_argmin(z_rest, E[lv]);
 * z_hat += E[lv][codes]; z_rest -= E[lv][codes], all in float.
 *   z:[B*L, D]; E[lv]:[vocabs[lv], D] (host array of device pointers);
 *   idx:[B, n_levels*L] level-major per batch row (vq.c:444-445), device int32;
 *   z_hat, z_rest:[B*L, D] outputs. */
void vq_quantize_multiscale(const float *z, const float *const *E, const int *vocabs,
                            int n_levels, int B, int L, int D,
                            int *idx, float *z_hat, float *z_rest);

/* ------------------------------------------------------------------ */
/* norms, RoPE, attention, layout, elementwise                         */
/* ------------------------------------------------------------------ */

/* replaces rmsnorm_fwd, ncm.h:154, kernels.c:150-162 (eps 1e-6; w may be NULL) */
void rmsnorm_fwd(const float *x, const float *w, float *y, int64_t rows, int C);
/* replaces layernorm_fwd (eps 1e-6), ncm.h:149-150, kernels.c:101-117 */
void layernorm_fwd(const float *x, const float *w, const float *b, float *y, int64_t rows, int C);
/* replaces layernorm_eps_fwd, ncm.h:151-152, kernels.c:132-148 */
void layernorm_eps_fwd(const float *x, const float *w, const float *b, float *y, int64_t rows, int C, float eps);
/* replaces gelu_fwd / gelu_tanh_fwd / silu_fwd, ncm.h:153-156, kernels.c:185-226 */
void gelu_fwd(const float *x, float *y, int64_t n);
void gelu_tanh_fwd(const float *x, float *y, int64_t n);
void silu_fwd(const float *x, float *y, int64_t n);
/* replaces rope_apply / rope_apply_gqa, ncm.h:158-161, kernels.c:285-308:
 * rotate-half RoPE in place on [B][H][T][hd] (q) and [B][K][T][hd] (k);
 * tables [T][hd] pair-duplicated; q or k may be NULL. */
void rope_apply(float *q, float *k, const float *cos, const float *sin, int B, int H, int T, int hd);
void rope_apply_gqa(float *q, float *k, const float *cos, const float *sin, int B, int H, int K, int T, int hd);
/* replaces heads_transpose_fwd / _b, ncm.h:162-164, kernels.c:322-357 */
void heads_transpose_fwd(const float *in, float *out, int64_t T, int H, int hd);
void heads_transpose_fwd_b(const float *in, float *out, int B, int64_t T, int H, int hd);
/* replaces sdpa_fwd / sdpa_fwd_gqa, ncm.h:165-170, kernels.c:423-507:
 * softmax(Q K^T / sqrt(hd) + mask) V; q [B][Hq][Tq][hd], k/v [B][Hkv][Tkv][hd],
 * mask [Tq][Tkv] additive or NULL; kv head = h / (Hq/Hkv), Hq % Hkv == 0. */
void sdpa_fwd(const float *q, const float *k, const float *v, const float *mask, float *out,
              int B, int H, int Tq, int Tkv, int hd);
void sdpa_fwd_gqa(const float *q, const float *k, const float *v, const float *mask, float *out,
                  int B, int Hq, int Hkv, int Tq, int Tkv, int hd);
/* extension: sdpa_fwd_gqa with the heads merged on output, out [B][Tq][Hq * hd]
 * = head_merge_fwd of sdpa_fwd_gqa's [B][Hq][Tq][hd] (ncp.c:248-260 runs the
 * two in turn); identical values. */
void sdpa_fwd_gqa_merged(const float *q, const float *k, const float *v, const float *mask, float *out,
                         int B, int Hq, int Hkv, int Tq, int Tkv, int hd);
/* extension: causal SDPA-GQA with the mask generated in the kernel: query tq
 * sees keys <= tq + (Tkv - Tq).  Replaces building the T x T -1e9 mask on the
 * host and uploading it (qwen.c:130-138, gpt2.c:112-121) + sdpa_fwd_gqa. */
void sdpa_fwd_gqa_causal(const float *q, const float *k, const float *v, float *out,
                         int B, int Hq, int Hkv, int Tq, int Tkv, int hd);
/* replaces embedding_fwd, ncm.h:147, kernels.c:67-74 (ids must be valid, as
 * there); embedding_fwd_v is the extension that clamps ids outside [0, V). */
void embedding_fwd(const float *W, const int *idx, float *y, int64_t n, int D);
void embedding_fwd_v(const float *W, int V, const int *idx, float *y, int64_t n, int D);
/* replaces add_fwd / scale_fwd / mul_fwd / add_inplace_fwd, ncm.h:189-192, kernels.c:829-874 */
void add_fwd(const float *a, const float *b, float *y, int64_t n);
void scale_fwd(const float *x, float s, float *y, int64_t n);
void mul_fwd(const float *a, const float *b, float *y, int64_t n);
void add_inplace_fwd(float *y, const float *x, int64_t n);
/* replaces qkv_split_fwd / head_merge_fwd, ncm.h:193-196, kernels.c:891-936 */
void qkv_split_fwd(const float *in, float *qq, float *kk, float *vv,
                   int B, int T, int C, int H, int hd, int K, int rep);
/* extension: qkv_split_fwd followed by rope_apply(qq, kk, cos_t, sin_t, B, H,
 * T, hd) in one pass (ncp.c:213-236 does the two in turn); identical values. */
void qkv_split_rope_fwd(const float *in, float *qq, float *kk, float *vv, const float *cos_t,
                        const float *sin_t, int B, int T, int C, int H, int hd, int K, int rep);
void head_merge_fwd(const float *ctx, float *out, int B, int T, int C, int H, int hd);

/* ------------------------------------------------------------------ */
/* training step: backward rows and optimizer                          */
/* Gradients accumulate (+=) into the caller's buffers; NULL skips one. */
/* ------------------------------------------------------------------ */

/* replaces the TOP_LN / TOP_LNE backward, train_tape.c:569-634 (host) and
 * k_ln_stats / k_ln_param / k_ln_dx, train_tape.c:1560-1620 (device);
 * eps = 1e-6 for layernorm_fwd, the recorded eps for layernorm_eps_fwd. */
void layernorm_bwd(const float *x, const float *w, const float *dy, float *dx, float *dw, float *db,
                   int64_t rows, int C, double eps);
/* replaces the TOP_RMSN backward, train_tape.c:748-792 / k_rmsn_*, :1575-1645 */
void rmsnorm_bwd(const float *x, const float *w, const float *dy, float *dx, float *dw, int64_t rows, int C);
/* replaces t_ce's forward, train_tape.c:442-481: probs [rows][V] and the mean
 * NLL over rows with wmask != 0 (wmask may be NULL) into loss[0]; tgt, wmask
 * and loss are device pointers. */
void ce_fwd(const float *logits, const int *tgt, const float *wmask, float *loss, float *probs,
            int64_t rows, int V);
/* replaces the TOP_CE backward, train_tape.c:657-679 / k_ce_bwd :1801-1810:
 * dlogits += (p - onehot) * w * inv, inv = weight / count */
void ce_bwd(const float *probs, const int *tgt, const float *wmask, float *dlogits, int64_t rows, int V,
            double inv);
/* extension: ce_fwd + ce_bwd without storing probs (count computed on the
 * device); loss[0] as ce_fwd, dlogits accumulates. */
void ce_fwd_bwd(const float *logits, const int *tgt, const float *wmask, float *loss, float *dlogits,
                int64_t rows, int V, double weight);
/* replaces t_sdpa's host computation of the stored probabilities,
 * train_tape.c:289-313: P [B][H][Tq][Tkv] = softmax(Q K^T / sqrt(hd) + mask). */
void sdpa_probs_gqa(const float *q, const float *k, const float *mask, float *P,
                    int B, int H, int Hkv, int Tq, int Tkv, int hd);
/* replaces the TOP_SDPA backward (MHA and GQA), train_tape.c:936-1051 (host)
 * and k_sdpa_* :1691-1799 (device), from the stored P; dO like q. */
void sdpa_bwd_gqa(const float *q, const float *k, const float *v, const float *P, const float *dO,
                  float *dq, float *dk, float *dv, int B, int H, int Hkv, int Tq, int Tkv, int hd);
/* replaces k_adamw, train.c:51-64 (= the host loop :131-141): one tensor,
 * lr already scaled by the schedule and the tensor's multiplier. */
void adamw_update(float *p, const float *g, float *m, float *v, int64_t n, double lr, double b1, double b2,
                  double b1t, double b2t, double eps, double wd);
/* the schedule of train.c:172-178 (static there): linear warm-up, cosine decay */
double sched_cosine_warmup(long step, double warmup, double total);
/* replaces the global-norm clip of train_gpt2.c:160-173: returns the norm of
 * all `count` device gradients (fp64) and scales them by (float)(1/norm) when
 * it exceeds max_norm; -1 on error.  Synchronises the library stream. */
double grad_clip_global(float *const *grads, const int64_t *sizes, int count, double max_norm);

/* replaces the TOP_GELU / TOP_SILU / TOP_GELU_TANH backward,
 * train_tape.c:830-873 / k_gelu_bwd, k_gelu_tanh_bwd: dx += dy * f'(x) */
void gelu_bwd(const float *x, const float *dy, float *dx, int64_t n);
void silu_bwd(const float *x, const float *dy, float *dx, int64_t n);
void gelu_tanh_bwd(const float *x, const float *dy, float *dx, int64_t n);
/* replaces the TOP_MUL backward, train_tape.c:1254-1268 (da or db may be NULL) */
void mul_bwd(const float *a, const float *b, const float *dy, float *da, float *db, int64_t n);
/* replaces the TOP_ROPE backward, train_tape.c:890-930 / k_rope_bwd: gq, gk are
 * the gradients of the rotated q [B][H][T][hd] and k [B][Hkv][T][hd]. */
void rope_bwd_gqa(const float *gq, const float *gk, const float *cos, const float *sin, float *dxq, float *dxk,
                  int B, int H, int Hkv, int T, int hd);
/* replaces the TOP_EMBED backward, train_tape.c:726-741: idx are HOST ints
 * (the tape keeps them on the host); dW [V][D] accumulates, bit-exact. */
void embedding_bwd(const float *dy, const int *idx, int64_t n, int D, float *dW, int V);
/* replaces the TOP_SPLIT backward, train_tape.c:1293-1328 (any of gq/gk/gv NULL) */
void qkv_split_bwd(const float *gq, const float *gk, const float *gv, float *dx,
                   int B, int T, int C, int H, int hd, int K, int rep);
/* replaces the TOP_MERGE / TOP_HEADSPLIT backward, train_tape.c:1329-1350 */
void head_merge_bwd(const float *dy, float *dctx, int B, int T, int C, int H, int hd);
void heads_transpose_bwd(const float *dy, float *dx, int B, int T, int C, int H, int hd);

/* ------------------------------------------------------------------ */
/* device tape                                                         */
/* ------------------------------------------------------------------ */

/* Replaces the reference's Tape for the hot-path ops (train_tape.c:19-162,
 * 277-481, 636-1051; ncm.h:468-522): recorders run the forward on the device
 * and record; ncm_tape_backward accumulates every gradient on the device.
 * Prefixed names, so the library can be linked next to the reference's
 * train_tape.c. */
typedef struct NcmTape NcmTape;
/* same layout as the reference's PMap (ncm.h:513-518): params[i]'s gradient
 * accumulates into grads[i] (device buffers of sizes[i] floats) */
typedef struct {
    float **params;
    float **grads;
    int64_t *sizes;
    int n;
} NcmPMap;

NcmTape *ncm_tape_new(void);                       /* tape_new, train_tape.c:59 */
void ncm_tape_free(NcmTape *t);                    /* tape_free, :83 */
void ncm_tape_clear(NcmTape *t);                   /* tape_clear, :84 */
int ncm_tape_size(const NcmTape *t);               /* number of records */
/* tape_backward, train_tape.c:545-556 (the device path, all on the GPU) */
void ncm_tape_backward(NcmTape *t, const NcmPMap *pm);
/* gradient accumulated for `key` by the last backward (NULL if none) */
float *ncm_tape_grad(NcmTape *t, const float *key);
/* recorders: t_linear :156, t_embed :164 (idx HOST ints), t_layernorm :176,
 * t_layernorm_eps :186, t_rmsnorm :194, t_gelu :209, t_gelu_tanh :217,
 * t_silu :223, t_mul :229, t_rope :260, t_sdpa :277, t_add :361,
 * t_scale :367, t_qkvsplit :386, t_headmerge :397, t_headsplit :405,
 * t_ce :442 (tgt, wmask HOST arrays; loss a device float; probs optional). */
void ncm_t_linear(NcmTape *t, const float *x, const float *W, const float *b, float *y, int64_t batch, int M, int K);
void ncm_t_embed(NcmTape *t, const float *W, const int *idx, int V, float *y, int64_t n, int D);
void ncm_t_layernorm(NcmTape *t, const float *x, const float *w, const float *b, float *y, int64_t rows, int C);
void ncm_t_layernorm_eps(NcmTape *t, const float *x, const float *w, const float *b, float *y, int64_t rows, int C,
                         double eps);
void ncm_t_rmsnorm(NcmTape *t, const float *x, const float *w, float *y, int64_t rows, int C);
void ncm_t_gelu(NcmTape *t, const float *x, float *y, int64_t n);
void ncm_t_gelu_tanh(NcmTape *t, const float *x, float *y, int64_t n);
void ncm_t_silu(NcmTape *t, const float *x, float *y, int64_t n);
void ncm_t_mul(NcmTape *t, const float *a, const float *b, float *y, int64_t n);
void ncm_t_add(NcmTape *t, const float *a, const float *b, float *y, int64_t n);
void ncm_t_scale(NcmTape *t, const float *x, float s, float *y, int64_t n);
void ncm_t_rope(NcmTape *t, const float *xq, const float *xk, float *yq, float *yk, const float *cos,
                const float *sin, int B, int H, int Hkv, int T, int hd);
void ncm_t_sdpa(NcmTape *t, const float *q, const float *k, const float *v, const float *mask, float *o,
                int B, int H, int Hkv, int Tq, int Tkv, int hd);
/* extension: ncm_t_linear (x -> pre) followed by the activation (pre -> y;
 * kind 0 GELU, 1 SiLU, 2 GELU tanh form, as ncm_t_gelu / ncm_t_silu /
 * ncm_t_gelu_tanh) with one GEMM writing both outputs, bit for bit the two
 * calls (train_gpt2.c:87-89) */
void ncm_t_linear_act(NcmTape *t, const float *x, const float *W, const float *b, float *pre, float *y,
                      int64_t batch, int M, int K, int kind);
/* extension: ncm_t_linear then ncm_t_add(res, linear output -> y) with the sum
 * in the GEMM epilogue and the linear output never stored (train_gpt2.c:72-74,
 * 95-97); res must not be y */
void ncm_t_linear_res(NcmTape *t, const float *x, const float *W, const float *b, const float *res, float *y,
                      int64_t batch, int M, int K);
/* extension: ncm_t_linear (x -> qkv, [B*T][C + 2 K hd]) then ncm_t_qkvsplit
 * (qkv -> qq, kk, vv) with the split done by the GEMM's epilogue when hd = 64,
 * C = H hd, K = H and T % 64 == 0 (qkv is then not written; it still keys its
 * gradient),
 * bit for bit the two calls (train_gpt2.c:58-62) */
void ncm_t_linear_qkvsplit(NcmTape *t, const float *x, const float *W, const float *b, float *qkv, float *qq,
                           float *kk, float *vv, int B, int T, int C, int H, int hd, int K, int rep);
/* extension: ncm_t_sdpa_causal (q, k, v -> ctx [B][H][T][hd]) then
 * ncm_t_headmerge (ctx -> out [B*T][H hd]) with the attention writing the
 * merged rows itself (hd 64: ctx is then not written; it still keys its
 * gradient), bit for bit the two calls (train_gpt2.c:64-66) */
void ncm_t_sdpa_causal_merge(NcmTape *t, const float *q, const float *k, const float *v, float *ctx, float *out,
                             int B, int H, int Hkv, int T, int hd);
/* extension: ncm_t_sdpa with the causal mask generated in the kernels (query t
 * sees keys <= t + Tkv - Tq), replacing the T x T -1e9 mask the reference's
 * callers build and upload (train_gpt2.c:112-121) */
void ncm_t_sdpa_causal(NcmTape *t, const float *q, const float *k, const float *v, float *o, int B, int H, int Hkv,
                       int Tq, int Tkv, int hd);
void ncm_t_qkvsplit(NcmTape *t, const float *in, float *qq, float *kk, float *vv, int B, int T, int C, int H, int hd,
                    int K, int rep);
void ncm_t_headmerge(NcmTape *t, const float *ctx, float *out, int B, int T, int C, int H, int hd);
void ncm_t_headsplit(NcmTape *t, const float *in, float *out, int B, int T, int C, int H, int hd);
void ncm_t_ce(NcmTape *t, const float *logits, const int *tgt, const float *wmask, float *loss, float *probs,
              int64_t rows, int V, double weight);

/* ------------------------------------------------------------------ */
/* config-5 driver: the taped GPT-2 training step of train_gpt2.c      */
/* ------------------------------------------------------------------ */

typedef struct {
    int n_layer, n_embd, n_head, vocab, n_pos;
} NcmGpt2Config;

/* flat parameter order: 0 wte [vocab][C], 1 wpe [n_pos][C], then per layer
 * l (base 2 + 12 l): ln_1.weight, ln_1.bias, attn.c_attn.weight [3C][C],
 * attn.c_attn.bias, attn.c_proj.weight [C][C], attn.c_proj.bias, ln_2.weight,
 * ln_2.bias, mlp.c_fc.weight [4C][C], mlp.c_fc.bias, mlp.c_proj.weight
 * [C][4C], mlp.c_proj.bias; last two ln_f.weight, ln_f.bias. */
int ncm_gpt2_param_count(const NcmGpt2Config *c);
/* elements of parameter i (rows x cols written when non-NULL), -1 if out of range */
int64_t ncm_gpt2_param_shape(const NcmGpt2Config *c, int i, int64_t *rows, int64_t *cols);
/* train_gpt2_forward (train_gpt2.c:107-147) on the device tape: ids HOST
 * [B][T] -> logits [B*T][vocab] in the arena (arena_init first). */
float *ncm_gpt2_forward(NcmTape *t, const NcmGpt2Config *c, float *const *params, const int *ids, int B, int T);
/* train_gpt2_step (train_gpt2.c:149-180) + adamw_step (train.c:102-145):
 * forward, mean CE on xout, backward, clip 1.0, AdamW (betas 0.9/0.95,
 * eps 1e-8, decay wd, lr = base_lr * sched_cosine_warmup(step, ...)).
 * grads zero on entry and exit.  Returns the loss (-1 on error). */
float ncm_gpt2_train_step(NcmTape *t, const NcmGpt2Config *c, float *const *params, float *const *grads,
                          float *const *m, float *const *v, const int *xin, const int *xout, int B, int T, long step,
                          double base_lr, double warmup, double total, double wd, double *gnorm_out);

/* ------------------------------------------------------------------ */
/* config-4 driver: the Qwen2 decoder of qwen.c                        */
/* ------------------------------------------------------------------ */

typedef struct {
    int n_layer, n_embd, n_head, n_kv, n_inner, vocab, n_ctx;
    double rope_theta;
} NcmQwenConfig;
typedef struct NcmQwen NcmQwen;

/* flat parameter order (qwen.c:60-75): 0 embed_tokens [vocab][C] (tied head);
 * per layer at 1 + 12 l: input_layernorm, q_proj.weight, q_proj.bias,
 * k_proj.weight, k_proj.bias, v_proj.weight, v_proj.bias, o_proj.weight,
 * post_attention_layernorm, gate_proj, up_proj, down_proj; last norm.weight. */
int ncm_qwen_param_count(const NcmQwenConfig *c);
int64_t ncm_qwen_param_shape(const NcmQwenConfig *c, int i, int64_t *rows, int64_t *cols);
/* model state over borrowed parameter buffers: RoPE tables (qwen.c:85-101),
 * KV cache [n_layer][n_kv][n_ctx][hd], decode scratch */
NcmQwen *ncm_qwen_new(const NcmQwenConfig *c, float *const *params);
void ncm_qwen_free(NcmQwen *m);
/* qwen_forward (qwen.c:121-190): ids HOST [T] -> logits [T][vocab] (or the
 * last row) in the arena; also fills the KV cache for positions 0..T-1. */
float *ncm_qwen_forward(NcmQwen *m, const int *ids, int T, int last_only);
/* one KV-cached step for token `id` at position pos (cache holds 0..pos-1):
 * logits [vocab] in the model's buffer (hd 64, <= 16 query heads per kv head) */
float *ncm_qwen_decode(NcmQwen *m, int id, int pos);
/* greedy generation (qwen_generate with temp 0, qwen.c:204-228): prefill +
 * cached decode, device argmax; stops after eos when eos >= 0. Returns the
 * number of ids written to out (-1 on error). */
int ncm_qwen_generate(NcmQwen *m, const int *prompt, int np, int n_new, int eos, int *out);
/* qwen_generate (qwen.c:204-228) with temperature / top-k / nucleus
 * sampling: each step's id is sample_topkp's draw (kernels.c:782-825) from
 * the xorshift64* state *rng (HOST; advanced once per generated token),
 * computed on the device inside the replayed decode graph.  temp <= 0 is
 * ncm_qwen_generate.  n_flagged (may be NULL): draws whose certification
 * flag was not 0 (see sample_topkp_dev).  Returns the ids written or -1. */
int ncm_qwen_generate_sample(NcmQwen *m, const int *prompt, int np, int n_new, int eos, float temp, int top_k,
                             float top_p, unsigned long long *rng, int *out, int *n_flagged);

/* ------------------------------------------------------------------ */
/* config-1 driver: the NCP transformer forward of ncp.c               */
/* ------------------------------------------------------------------ */

/* The block normalises with LayerNorm (eps 1e-6), as ncp_block always
 * does (ncp.c:199, 277, 352-357): the reference's NCP has no RMSNorm variant. */
typedef struct {
    int n_layer, n_embd, n_head, n_kv, n_inner, vocab;
    int rope_base; /* ncp.c build_rope base (10000) */
} NcmNcpConfig;

/* flat parameter order (biases may be NULL): 0 wte [V][C]; per layer at
 * 1 + 14 l: ln_1.weight, ln_1.bias, attn.c_attn.weight [C + 2 Kv hd][C],
 * attn.c_attn.bias, attn.c_proj.weight, attn.c_proj.bias, ln_2.weight,
 * ln_2.bias, mlp.w_gate.weight [I][C], mlp.w_gate.bias, mlp.w_up.weight,
 * mlp.w_up.bias, mlp.c_proj.weight [C][I], mlp.c_proj.bias; then
 * ln_f.weight, ln_f.bias, head.weight [V][C], head.bias. */
int ncm_ncp_param_count(const NcmNcpConfig *c);
int64_t ncm_ncp_param_shape(const NcmNcpConfig *c, int i, int64_t *rows, int64_t *cols);
/* build_rope (ncp.c:80-92) for positions 0..S-1 into HOST [S][hd] arrays */
int ncm_ncp_rope_tables(int S, int hd, int base, float *cos_host, float *sin_host);
/* ncp_block x n_layer (ncp.c:184-338) + ln_f + head over ids HOST [B][S]
 * (one level, no mask): logits [B*S][V] in the arena (arena_init first). */
float *ncm_ncp_forward(const NcmNcpConfig *c, float *const *params, const int *ids, int B, int S);

/* ------------------------------------------------------------------ */
/* greedy id                                                           */
/* ------------------------------------------------------------------ */

/* replaces argmax_row, ncm.h:186, kernels.c:731-735.  HOST pointer, as in
 * the reference (qwen.c:220-222 copies the logits row to the host first). */
int argmax_row(const float *x, int n);

/* extension: device argmax over each of `rows` rows of length n, lowest
 * index on ties.  Replaces backend_to_host + argmax_row (qwen.c:220-222). */
void argmax_rows(const float *x, int *idx, int64_t rows, int n);

/* ------------------------------------------------------------------ */
/* sampling                                                            */
/* ------------------------------------------------------------------ */

/* replaces rng_next, ncm.h:199, kernels.c:774-780 (xorshift64*). */
unsigned long long rng_next(unsigned long long *state);

/* replaces sample_topkp, ncm.h:197-198, kernels.c:782-825: temperature,
 * top-k (0 = all) and nucleus sampling of one row.  HOST logits and rng, as
 * the reference's callers pass them (qwen.c:220-223, gpt2.c:194); the row is
 * copied to the device and sampled there (sample_topkp_dev).  When the device
 * cannot certify its draw (flag 1 or 2 below), the draw is made again on the
 * host from the same row and starting rng state with the reference's own
 * steps, so the returned id and *rng are always the reference's.  temp <= 0
 * returns argmax_row and leaves *rng as it is.  V <= 262144, top_p >= 0. */
int sample_topkp(const float *logits, int V, float temp, int top_k, float top_p, unsigned long long *rng);
/* device flag of the last sample_topkp call (see sample_topkp_dev); not 0
 * means its id came from the host redraw */
int ncm_hip_sample_flag(void);

/* extension: sample_topkp on the device.  logits [V], rng (the xorshift64*
 * state, advanced once when temp > 0), out (the id) and flag are device
 * pointers; flag may be NULL.  *flag = 0: the id is certified to be the
 * reference's (every decision cleared the combined rounding bound of the
 * device and host exp and of the summation orders); 1: the draw lay within
 * that bound of a cumulative boundary (probability ~1e-10 per draw; the id
 * is then the device's own reading); 2: a non-finite logits/temp value.
 * Asynchronous on the library stream.  Replaces backend_to_host +
 * sample_topkp (qwen.c:220-223). */
void sample_topkp_dev(const float *logits, int V, float temp, int top_k, float top_p,
                      unsigned long long *rng, int *out, int *flag);

/* ------------------------------------------------------------------ */
/* on-disk formats -- replaces the loaders of src/tensor.c (ncm.h:57-70, */
/* 72-139, 262-265) and weights_save (train.c:741-767)                  */
/* ------------------------------------------------------------------ */

/* Same layouts as ncm.h:58-66; every tensor lives in device memory. */
typedef struct {
    char    name[256];
    Tensor *t;
} NamedTensor;

typedef struct {
    NamedTensor *items;
    int          count;
} WeightStore;

/* replaces weights_load, tensor.c:70-132: an "NCM1" file (magic, u32 count,
 * then per tensor u8 name length, name, u8 ndim, u32 dims, u64 byte count,
 * float32 data, all little-endian), or the weights section of an "NCK1"
 * checkpoint.  0 on success; -1 (store left empty) on a missing file, bad
 * magic, truncation or a byte count that does not match the shape. */
int     weights_load(WeightStore *ws, const char *path);
/* replaces weights_free / weights_get, tensor.c:134-143 */
void    weights_free(WeightStore *ws);
Tensor *weights_get(WeightStore *ws, const char *name); /* NULL if missing */
/* replaces weights_save, train.c:741-767: writes the NCM1 layout above */
int     weights_save(WeightStore *ws, const char *path);

#define NCM_MAX_LEVELS 64
#define NCM_MAX_VOCAB_LIST 64

/* Same layout and field meaning as the reference NCMConfig (ncm.h:75-137). */
typedef struct {
    char task[64];
    int  n_layer, n_head, n_embd, context_length, prefix_len;
    int  bias;
    int  raw_token_prefix, contextual_prefix;
    int  prefix_pad_token_id;
    int  vocab_size[NCM_MAX_VOCAB_LIST];
    int  n_levels_out;
    int  predict_level0, query_level0, l0_autoregressive;
    int  attn_pattern_block_diag;
    int  use_positional_encoding, use_level_encoding;
    int  use_rope, rope_base, use_qk_norm, use_flex_attention;
    double rope_theta;
    int  n_kv_heads;
    int  ctx_enabled, ctx_n_layer, ctx_vocab;
    int  puc_enabled, puc_kernel;
    int  shared_output_head, shared_head_per_level_bias, untied_head_bias;
    int  tie_heads_to_codebook, tie_heads_learn_scale, tie_heads_trainable;
    int  tie_heads_bias;
    int  use_swiglu, use_geglu, use_relu2, parallel_block, normformer;
    int  use_layerscale, use_rezero;
    float layerscale_init;
    float dropout;
    int  vq_embed_dim, vq_in_vocab, vq_context_length, vq_n_layers;
    int  vq_compression;
    int  vq_soft_levels;
    double vq_soft_tau;
    int  levels[NCM_MAX_LEVELS];
    int  n_qlevels;
    int  vq_vocab[NCM_MAX_LEVELS];
    float quant_resi_ratio;
    int   quant_resi_enabled;
    int   quant_resi_share_mode;
    int   learned_l1_sampling, learned_l1_cascade;
    int   learned_l1_cascade_base;
    int   learned_l1_norm, learned_l1_norm_final;
    int   learned_all_sampling;
    int   pre_quant_groupnorm;
    int   vq_qk_norm;
    int   enc_layers, enc_attn_window, enc_conv_layers, enc_conv_kernel;
    int   enc_positional;
    int   dec_layers, dec_positional;
    char pre_tok[16];
    int  sudoku_size;
    char hf_model_id[128];
    int  eos_token_id, pad_token_id;
    float gen_temperature;
    int   gen_top_k;
    float gen_top_p, gen_cfg_scale;
    float gen_freq, gen_mu;
    float gen_adj_a; int gen_adj_w; float gen_adj_d;
} NCMConfig;

/* replaces config_load, tensor.c:145-266: `key=value` lines with model.*,
 * vq.*, tok.* and gen.* keys over the reference's defaults; unknown keys and
 * lines without '=' are ignored.  0 on success, -1 if the file cannot be
 * opened.  Host only (no device use). */
int config_load(NCMConfig *c, const char *path);

/* ------------------------------------------------------------------ */
/* the multiscale quantizer -- replaces src/vq.c (ncm.h:205-239)       */
/* ------------------------------------------------------------------ */

typedef struct VQState VQState;
/* replaces vq_load, ncm.h:206, vq.c:76-197: codebooks "embeddings.<i>.weight",
 * the Phi convs "quant_resi.<i>.*" (per level / shared / k partially shared),
 * the learned level-0 cascade "learned_down_l1.<i>.*" / "learned_up_l1.<i>.*"
 * and the refine convs "learned_{down,up}_refine.<i>.*", from the store's
 * DEVICE tensors (borrowed).  Errors (missing or mis-shaped weights, a cascade
 * that does not map L to levels[0] and back, kernels above 16) are reported
 * like the reference's exit(1); NULL in record mode. */
VQState *vq_load(const NCMConfig *c, WeightStore *ws, const char *prefix);
/* replaces vq_free / vq_total_codes and the accessors, ncm.h:207-208, 235-239 */
void vq_free(VQState *vq);
int  vq_total_codes(const VQState *vq);
int  vq_nlevels(const VQState *vq);
int  vq_level_len(const VQState *vq, int k);
int  vq_level_V(const VQState *vq, int k);
int  vq_Ltotal(const VQState *vq);
int  vq_Ddim(const VQState *vq);
/* replaces vq_z_to_idx, ncm.h:210, vq.c:378-500 (argmin at every level):
 * z [B][L][D] device, idx [B][total] HOST level-major codes, as the
 * reference's caller receives them.  Codes bit-exact with the CPU path. */
void vq_z_to_idx(VQState *vq, const float *z, int B, int *idx);
/* replaces vq_z_to_idx_soft, ncm.h:214, vq.c:388-437 (training: levels below
 * soft_levels draw from the tempered softmax over code distances, one
 * xorshift64 step of *rng (host memory) per drawn row, rows in order; idx is
 * host memory as in vq_z_to_idx; soft_levels <= 0, soft_tau <= 0 or rng NULL
 * is vq_z_to_idx) */
void vq_z_to_idx_soft(VQState *vq, const float *z, int B, int *idx, int soft_levels, double soft_tau,
                      unsigned long long *rng);
/* extension: rows of the last vq_z_to_idx_soft call whose draw lay within the
 * rounding bound of the device exp against glibc's and was therefore decided
 * again on the host with the reference's loop and libm exp */
int ncm_vq_soft_host_rows(void);
/* replaces vq_ema_init / vq_ema_update, ncm.h:228-229, vq.c:677-790 (training:
 * EMA codebook maintenance; z device memory, codes host memory [B][total]; the
 * codebooks vq_load bound are rewritten in place, as the reference's are;
 * a code outside its level's [0, V) is NCM_E_ARG) */
void vq_ema_init(VQState *vq);
void vq_ema_update(VQState *vq, const float *z, const int *codes, int B, double decay, double eps);
/* extension: vq_z_to_idx with device codes, and the final z_hat / z_rest
 * [B][L][D] (device, may be NULL); asynchronous on the library stream. */
void vq_z_to_idx_dev(VQState *vq, const float *z, int B, int *idx, float *z_hat, float *z_rest);
/* replaces vq_idx_to_zhats, ncm.h:217, vq.c:502-552: idx HOST; zhats[level]
 * device [B][L][D] buffers receiving z_hat after each level. */
void vq_idx_to_zhats(VQState *vq, const int *idx, int B, float **zhats);
/* replaces vq_next_input, ncm.h:219-220, vq.c:554-597: codes HOST [B][levels[level]];
 * z_hat device [B][L][D] += that level's contribution; x_out device
 * [B][levels[level + 1]][D] = area(z_hat).  level + 1 < n_levels. */
void vq_next_input(VQState *vq, const int *codes, int level_idx, float *z_hat, float *x_out, int B);
/* replaces vq_idx_to_ncm_input, ncm.h:222, vq.c:601-670: idx HOST [B][total];
 * x_out device [B][total - levels[0]][D]: level li's chunk (li < n_levels - 1)
 * is area(z_hat after level li -> levels[li + 1]). */
void vq_idx_to_ncm_input(VQState *vq, const int *idx, int B, float *x_out);


/* ------------------------------------------------------------------ */
/* the NCP transformer forward -- replaces src/ncp.c (ncm.h:249-268)    */
/* ------------------------------------------------------------------ */

typedef struct VQVAEState VQVAEState;
typedef struct NCPState NCPState;
/* replaces ncp_load, ncm.h:250, ncp.c:94-175: reads the block, embedding and
 * head weights under the reference's names from the store's DEVICE tensors
 * (borrowed), builds the RoPE tables of the level positions (prefix 0..P-1,
 * then 0..l_k - 1 per target level), the level embedding rows (wle, plus wpe
 * without RoPE) and the additive mask on the device.  vqvae is kept for the
 * caller and not used by the forward.  Missing weights or a configuration
 * the reference cannot run (n_kv_heads <= 0 or not dividing n_head, odd head
 * size with RoPE, no target level) are reported like its exit(1). */
NCPState *ncp_load(const NCMConfig *c, WeightStore *ws, VQVAEState *vqvae);
/* replaces ncp_free, ncm.h:251 */
void ncp_free(NCPState *m);
/* replace the accessors of ncm.h:252-260 (tables are DEVICE [rows][hd]) */
int ncp_P(NCPState *m);
int ncp_T(NCPState *m);
int ncp_ntgt(NCPState *m);
int ncp_lvlfirst(NCPState *m);
float *ncp_rope_cos(NCPState *m);
float *ncp_rope_sin(NCPState *m);
float *ncp_rope_gen_cos(NCPState *m, int k);
float *ncp_rope_gen_sin(NCPState *m, int k);
/* replaces ncp_forward, ncm.h:267-268, ncp.c:480-640: x DEVICE [B][P+T][D]
 * (D = vq_embed_dim), prefix_ids HOST [B][P] or NULL, logits DEVICE
 * [B][T][max vocab] (-inf past a level's vocabulary).  Every step runs on the
 * device (the reference stages the split, the level embedding, the q/k/v
 * split, the head merge, the gated product and the per-level slices on the
 * host); activations come from the library arena, which the caller resets,
 * as the reference's callers do.  Boards with padded prefix tokens run one
 * at a time with their own mask, as in the reference. */
void ncp_forward(NCPState *m, const float *x, const int *prefix_ids, float *logits, int B);

/* replaces train_data_load / train_data_free, ncm.h:262-264, tensor.c:375-395:
 * "NCMT" magic, u64 rows, u64 row length, int32 tokens; at most max_rows rows
 * when max_rows > 0.  HOST rows; NULL on error.  Host only. */
typedef struct { int *rows; int n_rows, row_len; } TrainData;
TrainData *train_data_load(const char *path, int max_rows);
void       train_data_free(TrainData *d);

/* ------------------------------------------------------------------ */
/* AdamW object + NCK1 checkpoints -- replaces train.c:15-150 and        */
/* src/ckpt.c (ncm.h:416-466, 523-540)                                  */
/* ------------------------------------------------------------------ */

/* The reference AdamW (ncm.h:523-536) with the moments and gradient
 * accumulators resident on the device: params, m, v and g are DEVICE
 * pointers (sizes[i] floats each); lr[i] is the per-tensor multiplier. */
typedef struct AdamW {
    float **params;
    float **m, **v;
    float **g;
    int64_t *sizes;
    double *lr;
    int n;
    double b1, b2, eps, wd;
    long step;
} AdamW;

/* replaces adamw_new, train.c:18-41: every tensor of the store not flagged
 * in `frozen` (may be NULL), zero moments and gradients, b1 0.9, b2 0.95,
 * eps 1e-8, wd 0.01, lr multipliers 1.  NULL on allocation failure. */
AdamW *adamw_new(WeightStore *ws, const int *frozen);
/* replaces adamw_zero_grad, train.c:43-46 (device memset of every g[i]) */
void   adamw_zero_grad(AdamW *o);
/* replaces adamw_step, train.c:102-145: step += 1, lr = base_lr *
 * sched_cosine_warmup(step, warmup, total) * lr[i], the k_adamw update of
 * every tensor (bit-identical to the reference's host loop) */
void   adamw_step(AdamW *o, double base_lr, double warmup, double total);
void   adamw_free(AdamW *o);                 /* train.c:147-159 */
/* replaces adamw_sync_to_host, train.c:85-98: a no-op, the moments have no
 * host copy (a checkpoint save reads them from the device) */
void   adamw_sync_to_host(AdamW *o);

/* Same layouts as ncm.h:426-439 and ncm.h:450-456. */
typedef struct {
    long global_step;
    unsigned long long batch_rng;
    double base_lr, warmup, total;
    int batch_B;
    int accum_pending;
    long n_rows; int row_len;
    uint64_t data_hash;
    const char *data_path;
    uint64_t conf_hash;
    const char *tokenizer_id;
    double noise_sd;
    const char *train_cfg_json;
} CkptRunState;

typedef struct {
    int batch_B; long n_rows; int row_len; uint64_t data_hash;
    uint64_t conf_hash; const char *tokenizer_id;
    double base_lr, warmup, total;
    double b1, b2, eps, wd;
} CkptExpect;

/* replaces ckpt_probe, ckpt.c:67-78: 1 = NCK1, 0 = NCM1, -1 = unreadable */
int ckpt_probe(const char *path);
/* replaces ckpt_file_hash, ckpt.c:50-64: FNV-1a 64 of the file's bytes */
uint64_t ckpt_file_hash(const char *path, uint64_t *nbytes_out);
/* replaces ckpt_save_atomic, ckpt.c:188-328: the NCK1 v1 layout (run state,
 * tensors, "ADAM" section with per-tensor moments, FNV-1a 64 trailer), byte
 * for byte the reference's for the same state; written to path.tmp.<pid>,
 * re-read and validated, fsync'd and renamed over path (then the directory
 * is fsync'd).  Refuses accum_pending != 0.  0 on success, else -1 with a
 * reason in err and path untouched. */
int ckpt_save_atomic(const WeightStore *ws, AdamW *opt, const CkptRunState *rs,
                     const char *path, char *err, size_t errcap);
/* replaces ckpt_load_training, ckpt.c:330-543: checksum first, then every
 * identity check against ex (dataset, config hash, tokenizer, schedule,
 * tensor names/shapes, optimizer hyper-parameters and parameter map) before
 * anything is applied; on success the weights, moments, opt->step and the
 * scalars of *out_rs are restored.  -1 with err set and nothing modified. */
int ckpt_load_training(const char *path, WeightStore *ws, AdamW *opt,
                       const CkptExpect *ex, CkptRunState *out_rs,
                       char *err, size_t errcap);
/* replaces ckpt_info, ckpt.c:628-713: summary on stdout; 0 = valid */
int ckpt_info(const char *path);
/* replaces ckpt_load_weights_only, ckpt.c:549-626: the tensor section into a
 * fresh store (device tensors) */
int ckpt_load_weights_only(const char *path, WeightStore *ws, char *err, size_t errcap);

#ifdef __cplusplus
}
#endif

#endif /* NCM_HIP_H */
