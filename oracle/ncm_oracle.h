/* ncm_oracle.h -- CPU restatement of the reference (SaphiraLinux/saphira-cncm)
 * arithmetic on the matrix-multiplication hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker the HIP library is compared
 * against; it is never linked into libncmhip.so.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Every function reproduces the reference's operation order exactly (fp64
 * accumulators, serial reduction order, float roundings at the same points),
 * so its results are bit-identical to the reference CPU build; the file:line
 * each one follows is given beside it.  Build flags keep IEEE semantics:
 * -std=c11 (no FMA contraction), no -ffast-math.
 */
#ifndef NCM_ORACLE_H
#define NCM_ORACLE_H

#include <stdint.h>

/* src/kernels.c:38-54 linear_fwd (CPU branch) */
void orc_linear_fwd(const float *x, const float *W, const float *b, float *y,
                    int64_t batch, int M, int K);
/* src/train_tape.c:680-725 TOP_LINEAR host backward (accumulating) */
void orc_linear_bwd(const float *x, const float *W, const float *dy,
                    float *dx, float *dW, float *db, int64_t batch, int M, int K);
/* src/kernels.c:753-770 rowwise_l2sq (CPU branch) */
void orc_l2sq(const float *a, const float *b, float *d2, int64_t rows, int64_t cols, int C);
/* rowwise_l2sq + host strict-'<' argmin of src/vq.c:440-443, per row */
void orc_vq_argmin(const float *a, const float *E, int *idx, int64_t rows, int V, int D);
/* src/vq.c:388-500 vq_z_to_idx_soft with rng = NULL, every level of length L
 * (identity resampling) and quant_resi disabled. */
void orc_vq_multiscale(const float *z, const float *const *E, const int *vocabs,
                       int n_levels, int B, int L, int D,
                       int *idx, float *z_hat, float *z_rest);
/* src/kernels.c:731-735 argmax_row */
int orc_argmax_row(const float *x, int n);
/* src/kernels.c:185-194, 207-218, 220-226 activations; :843-849 add */
void orc_gelu(const float *x, float *y, int64_t n);
void orc_gelu_tanh(const float *x, float *y, int64_t n);
void orc_silu(const float *x, float *y, int64_t n);
void orc_add(const float *a, const float *b, float *y, int64_t n);

/* src/kernels.c:150-162 rmsnorm_fwd; :101-148 layernorm_fwd (eps 1e-6) and layernorm_eps_fwd */
void orc_rmsnorm(const float *x, const float *w, float *y, int64_t rows, int C);
void orc_layernorm(const float *x, const float *w, const float *b, float *y, int64_t rows, int C);
void orc_layernorm_eps(const float *x, const float *w, const float *b, float *y, int64_t rows, int C, float eps);
/* src/kernels.c:249-264 rope_one_exact (in place; row position = row % T) */
void orc_rope(float *x, const float *cos_t, const float *sin_t, int64_t rows, int T, int hd);
/* src/qwen.c:85-101 RoPE tables */
void orc_rope_tables_qwen(int T, int hd, double theta, float *cos_t, float *sin_t);
/* src/kernels.c:423-464 sdpa_fwd_gqa (CPU branch) */
void orc_sdpa_gqa(const float *q, const float *k, const float *v, const float *mask, float *out,
                  int B, int Hq, int Hkv, int Tq, int Tkv, int hd);
/* src/kernels.c:67-74, :345-357, :913-936, :859-874 layout and elementwise */
void orc_embedding(const float *W, const int *idx, float *y, int64_t n, int D);
void orc_heads_transpose(const float *in, float *out, int B, int64_t T, int H, int hd);
void orc_qkv_split(const float *in, float *qq, float *kk, float *vv, int B, int T, int C, int H, int hd,
                   int K, int rep);
void orc_head_merge(const float *ctx, float *out, int B, int T, int C, int H, int hd);
void orc_mul(const float *a, const float *b, float *y, int64_t n);
void orc_scale(const float *x, float s, float *y, int64_t n);

/* training backward and optimizer (accumulating into existing gradients;
 * NULL gradient pointers are skipped) */
/* src/train_tape.c:569-634 host_ln_bwd (eps 1e-6 for TOP_LN, recorded eps for TOP_LNE) */
void orc_layernorm_bwd(const float *x, const float *w, const float *dy, float *dx, float *dw, float *db,
                       int64_t rows, int C, double eps);
/* src/train_tape.c:748-792 TOP_RMSN */
void orc_rmsnorm_bwd(const float *x, const float *w, const float *dy, float *dx, float *dw, int64_t rows, int C);
/* src/train_tape.c:442-481 t_ce (returns the weight count) and :657-679 its backward */
double orc_ce_fwd(const float *logits, const int *tgt, const float *wm, float *loss, float *probs, int64_t rows,
                  int V);
void orc_ce_bwd(const float *probs, const int *tgt, const float *wm, float *dl, int64_t rows, int V, double inv);
/* src/train.c:131-141 / :51-64 AdamW update; :172-178 schedule; train_gpt2.c:160-173 clip */
void orc_adamw(float *p, const float *g, float *m, float *v, int64_t n, double lr, double b1, double b2,
               double b1t, double b2t, double eps, double wd);
double orc_sched_cosine_warmup(long step, double warmup, double total);
double orc_grad_clip(float *const *g, const int64_t *n, int count, double max_norm);
/* src/train_tape.c:289-313 stored probabilities, :936-1051 SDPA backward */
void orc_sdpa_probs(const float *q, const float *k, const float *mask, float *P, int B, int H, int Hkv, int Tq,
                    int Tkv, int hd);
void orc_sdpa_bwd(const float *q, const float *k, const float *v, const float *P, const float *dy, float *dq,
                  float *dk, float *dv, int B, int H, int Hkv, int Tq, int Tkv, int hd);

/* src/train_tape.c:830-873 activation backward (kind 0 gelu, 1 silu, 2 gelu_tanh),
 * :1254-1268 mul, :890-930 rope, :726-741 embedding, :1293-1350 split / merge / headsplit */
void orc_act_bwd(const float *x, const float *dy, float *dx, int64_t n, int kind);
void orc_mul_bwd(const float *a, const float *b, const float *dy, float *da, float *db, int64_t n);
void orc_rope_bwd(const float *g, const float *cos_t, const float *sin_t, float *dx, int64_t rows, int T, int hd);
void orc_embedding_bwd(const float *dy, const int *idx, int64_t n, int D, float *dW, int V);
void orc_qkv_split_bwd(const float *gq, const float *gk, const float *gv, float *dx, int B, int T, int C, int H,
                       int hd, int K, int rep);
void orc_head_merge_bwd(const float *dy, float *dctx, int B, int T, int C, int H, int hd);
void orc_heads_transpose_bwd(const float *dy, float *dx, int B, int T, int C, int H, int hd);

/* src/ncp.c:80-92 build_rope (positions 0..S-1) */
void orc_rope_tables_ncp(int S, int hd, int base, float *cos_t, float *sin_t);

/* src/kernels.c:774-780 rng_next (xorshift64*) and the ktest generator of
 * tests/ktest_kernels.c:8-12, for seeded inputs shared with the reference. */
uint64_t orc_rng_next(uint64_t *state);
void orc_fill_ktest(uint64_t *state, float *out, int64_t n);

/* src/kernels.c:782-825 sample_topkp (temperature, top-k, nucleus); rng
 * is the xorshift64* state, advanced once when temp > 0 */
int orc_sample_topkp(const float *logits, int V, float temp, int top_k, float top_p, uint64_t *rng);

/* The multiscale quantizer of src/vq.c in full (vq_load + vq_z_to_idx with
 * rng = NULL, vq_idx_to_zhats): per-level lengths with area down-sampling
 * (kernels.c:681-700) and linear up-sampling (kernels.c:702-727), the Phi
 * residual conv (vq.c:243-277), the learned level-0 conv cascade with
 * optional GroupNorm (vq.c:280-376; kernels.c:546-640) and the learned
 * refine convs of the middle levels.  Tensors are row-major [B][T][D] (the
 * reference's BLD layout); weights keep the reference's PyTorch layouts. */
typedef struct {
    int n_levels, D;
    const int *levels, *vocabs;
    const float *const *E;                       /* [n_levels] codebooks [V][D] */
    int n_phi;                                   /* 0: Phi off */
    float resi_ratio;
    const float *const *phiW, *const *phib;      /* [n_phi]: [D][D][3], [D] */
    int n_down, n_up;                            /* 0: no learned level-0 sampling */
    const float *const *downW, *const *downB;    /* [n_down]: [D][D][k], [D] */
    const int *downK;
    const float *const *upW, *const *upB;        /* [n_up]: [D][D][k] (ConvTranspose1d), [D] */
    const int *upK;
    int l1_norm, l1_norm_final;
    int has_all;                                 /* refine convs (entries may be NULL) */
    const float *const *drefW, *const *drefB, *const *urefW, *const *urefB;  /* [n_levels] */
} OrcVq;
/* idx [B][sum levels] level-major; z_hat / z_rest [B][L][D] may be NULL */
void orc_vq_z_to_idx(const OrcVq *q, const float *z, int B, int *idx, float *z_hat, float *z_rest);
void orc_vq_z_to_idx_soft(const OrcVq *q, const float *z, int B, int *idx, float *z_hat, float *z_rest,
                          int soft_levels, double tau, unsigned long long *rng);
int orc_soft_pick(const float *d, int V, double tau, unsigned long long *rng);
void orc_vq_ema_update(const OrcVq *q, float *const *cs, float *const *w, const float *z, const int *codes, int B,
                       double decay, double eps);
/* zhats [n_levels][B][L][D]: z_hat after each level */
void orc_vq_idx_to_zhats(const OrcVq *q, const int *idx, int B, float *zhats);
void orc_vq_next_input(const OrcVq *q, const int *codes, int lv, float *z_hat, float *x_out, int B);
void orc_vq_idx_to_ncm_input(const OrcVq *q, const int *idx, int B, float *x_out);

/* conv1d_fwd (kernels.c:546-566) on [B][T][Cin] rows -> [B][To][Cout]:
 * fp64 over ci (outer) and k (inner), taps outside [0, T) skipped */
void orc_conv1d_btc(const float *x, const float *W, const float *bias, float *y, int B, int T, int Cin, int Cout,
                    int K, int stride, int pad);
/* the codebook-tied NCP head (ncp.c:429-466): o[r][v] = (float)((2 dot -
 * |E_v|^2) / ds * invT (+ bias[v])), dot and |E_v|^2 serial fp64 over d,
 * ds = the serial fp64 sum of |E_v|^2 over v divided by V */
void orc_ncp_tied_head(const float *z, const float *E, const float *bias, float invT, float *out, int rows, int V,
                       int Dd);

/* threads used by the OpenMP loops (0 = runtime default) */
void orc_set_threads(int n);

#endif
