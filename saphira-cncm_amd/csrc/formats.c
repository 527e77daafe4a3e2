/* formats.c -- the reference's on-disk formats on the host side of the
 * library: NCM1 weight files (tensor.c:64-143, train.c:741-767), the .conf
 * key=value model configuration (tensor.c:145-266) and NCMT training rows
 * (tensor.c:375-395).  Tensors of a WeightStore live in device memory; files
 * are read and written in bounded host chunks. */
#include "internal.h"

#include <limits.h>
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- bytes */

int fmt_read_exact(FILE *f, void *dst, size_t n) { return n == 0 || fread(dst, 1, n, f) == n ? 0 : -1; }

int fmt_read_u32le(FILE *f, uint32_t *v) {
    unsigned char b[4];
    if (fmt_read_exact(f, b, 4)) return -1;
    *v = (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 | (uint32_t)b[3] << 24;
    return 0;
}

int fmt_read_u64le(FILE *f, uint64_t *v) {
    unsigned char b[8];
    if (fmt_read_exact(f, b, 8)) return -1;
    uint64_t x = 0;
    for (int i = 7; i >= 0; i--) x = x << 8 | b[i];
    *v = x;
    return 0;
}

/* Device <-> file copies of one tensor through a bounded staging buffer. */
#define STAGE_BYTES ((size_t)64 << 20)

static int upload_from_file(FILE *f, float *dev, uint64_t nbytes) {
    size_t cap = nbytes < STAGE_BYTES ? (size_t)nbytes : STAGE_BYTES;
    unsigned char *h = (unsigned char *)malloc(cap ? cap : 1);
    if (!h) return -1;
    uint64_t done = 0;
    int rc = 0;
    while (done < nbytes) {
        size_t n = nbytes - done < cap ? (size_t)(nbytes - done) : cap;
        if (fmt_read_exact(f, h, n)) { rc = -1; break; }
        mem_h2d((unsigned char *)dev + done, h, n);
        done += n;
    }
    free(h);
    return rc;
}

/* Calls sink(ctx, bytes, n) for the tensor's bytes in order; the staging
 * buffer is wiped before it is freed (weights are sensitive data). */
int fmt_download(const float *dev, uint64_t nbytes, void (*sink)(void *, const void *, size_t), void *ctx) {
    size_t cap = nbytes < STAGE_BYTES ? (size_t)nbytes : STAGE_BYTES;
    unsigned char *h = (unsigned char *)malloc(cap ? cap : 1);
    if (!h) return -1;
    for (uint64_t done = 0; done < nbytes;) {
        size_t n = nbytes - done < cap ? (size_t)(nbytes - done) : cap;
        mem_d2h(h, (const unsigned char *)dev + done, n);
        sink(ctx, h, n);
        done += n;
    }
    memset(h, 0, cap);
    free(h);
    return 0;
}

/* ---------------------------------------------------------------- NCM1 */

void weights_free(WeightStore *ws) {
    if (!ws) return;
    for (int i = 0; i < ws->count; i++) tensor_free(ws->items[i].t);
    free(ws->items);
    ws->items = NULL;
    ws->count = 0;
}

Tensor *weights_get(WeightStore *ws, const char *name) {
    if (!ws || !name) return NULL;
    for (int i = 0; i < ws->count; i++)
        if (strcmp(ws->items[i].name, name) == 0) return ws->items[i].t;
    return NULL;
}

/* One tensor record: u8 name length, name, u8 ndim, u32 dims, u64 bytes,
 * data.  Appends it to ws (whose items array holds `cap` entries). */
static int ncm1_record(FILE *f, WeightStore *ws, const char *path) {
    NamedTensor *it = &ws->items[ws->count];
    unsigned char nl, nd;
    if (fmt_read_exact(f, &nl, 1) || fmt_read_exact(f, it->name, nl)) return -1;
    it->name[nl] = 0;
    if (fmt_read_exact(f, &nd, 1)) return -1;
    if (nd > NCM_MAX_DIMS) {
        fprintf(stderr, "%s: tensor '%s' has %u dims (at most %d)\n", path, it->name, nd, NCM_MAX_DIMS);
        return -1;
    }
    int64_t shape[NCM_MAX_DIMS] = {0};
    for (int d = 0; d < nd; d++) {
        uint32_t v;
        if (fmt_read_u32le(f, &v)) return -1;
        shape[d] = v;
    }
    uint64_t nbytes;
    if (fmt_read_u64le(f, &nbytes)) return -1;
    if ((uint64_t)tensor_numel(nd, shape) * 4u != nbytes) {
        fprintf(stderr, "%s: size mismatch\n", it->name);
        return -1;
    }
    Tensor *t = tensor_alloc(nd, shape);
    if (!t) return -1;
    if (upload_from_file(f, t->data, nbytes)) {
        tensor_free(t);
        return -1;
    }
    it->t = t;
    ws->count++;
    return 0;
}

int weights_load(WeightStore *ws, const char *path) {
    if (!ws || !path) return ncm_fail(NCM_E_ARG, "weights_load: null argument"), -1;
    ws->items = NULL;
    ws->count = 0;
    if (ckpt_probe(path) == 1) {
        char err[512] = {0};
        if (ckpt_load_weights_only(path, ws, err, sizeof err)) {
            fprintf(stderr, "%s\n", err);
            return -1;
        }
        return 0;
    }
    FILE *f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "cannot open %s\n", path);
        return -1;
    }
    char magic[4];
    uint32_t count = 0;
    if (fmt_read_exact(f, magic, 4) || memcmp(magic, "NCM1", 4) != 0) {
        fprintf(stderr, "%s: bad magic\n", path);
        fclose(f);
        return -1;
    }
    if (fmt_read_u32le(f, &count) || count > (1u << 24)) {
        fclose(f);
        return -1;
    }
    ws->items = (NamedTensor *)calloc(count ? count : 1, sizeof(NamedTensor));
    if (!ws->items) {
        fclose(f);
        return -1;
    }
    int rc = 0;
    for (uint32_t i = 0; i < count && rc == 0; i++) rc = ncm1_record(f, ws, path);
    fclose(f);
    if (rc) weights_free(ws);
    return rc;
}

static void sink_file(void *ctx, const void *p, size_t n) {
    FILE **f = (FILE **)ctx;
    if (*f && fwrite(p, 1, n, *f) != n) {
        fclose(*f);
        *f = NULL;
    }
}

int weights_save(WeightStore *ws, const char *path) {
    if (!ws || !path) return ncm_fail(NCM_E_ARG, "weights_save: null argument"), -1;
    FILE *f = fopen(path, "wb");
    if (!f) {
        fprintf(stderr, "cannot write %s\n", path);
        return -1;
    }
    unsigned char hdr[8] = {'N', 'C', 'M', '1'};
    for (int i = 0; i < 4; i++) hdr[4 + i] = (unsigned char)((uint32_t)ws->count >> (8 * i));
    sink_file(&f, hdr, 8);
    for (int i = 0; i < ws->count && f; i++) {
        const Tensor *t = ws->items[i].t;
        size_t nl = strlen(ws->items[i].name);
        if (nl > 255 || t->ndim < 0 || t->ndim > NCM_MAX_DIMS) {
            fclose(f);
            f = NULL;
            break;
        }
        unsigned char rec[1 + 255 + 1 + 4 * NCM_MAX_DIMS + 8];
        size_t k = 0;
        rec[k++] = (unsigned char)nl;
        memcpy(rec + k, ws->items[i].name, nl);
        k += nl;
        rec[k++] = (unsigned char)t->ndim;
        for (int d = 0; d < t->ndim; d++)
            for (int b = 0; b < 4; b++) rec[k++] = (unsigned char)((uint32_t)t->shape[d] >> (8 * b));
        uint64_t nbytes = (uint64_t)t->n * 4u;
        for (int b = 0; b < 8; b++) rec[k++] = (unsigned char)(nbytes >> (8 * b));
        sink_file(&f, rec, k);
        if (f && fmt_download(t->data, nbytes, sink_file, &f)) {
            fclose(f);
            f = NULL;
        }
    }
    if (!f || fclose(f)) {
        fprintf(stderr, "cannot write %s\n", path);
        return -1;
    }
    return 0;
}

/* ---------------------------------------------------------------- .conf */

/* How a key's value is parsed (tensor.c:147-168 and the key chain of
 * tensor.c:182-259):
 *   K_BOOLINT  leading blanks skipped, "T.."/"t.." = 1, "F.."/"f.." = 0, else atoi
 *   K_ATOI     atoi          K_FLOAT (float)atof      K_DOUBLE atof
 *   K_STR      copied, truncated to the field
 *   K_LIST     comma-separated atoi list; count stored at `aux` (or dropped)
 *   K_PATTERN  1 iff the value is exactly "block_diagonal"
 *   K_ADJ      "a[,w[,d]]" -> gen_adj_a, gen_adj_w (default 1), gen_adj_d (1) */
enum { K_BOOLINT, K_ATOI, K_FLOAT, K_DOUBLE, K_STR, K_LIST, K_PATTERN, K_ADJ };

typedef struct {
    const char *key;
    int kind;
    size_t off;   /* field */
    size_t size;  /* field bytes (K_STR) or list capacity (K_LIST) */
    long aux;     /* K_LIST: offset of the count field, -1 = none */
} ConfKey;

#define F(field) offsetof(NCMConfig, field)
#define BI(key, field) {key, K_BOOLINT, F(field), 0, -1}
#define AI(key, field) {key, K_ATOI, F(field), 0, -1}
#define FL(key, field) {key, K_FLOAT, F(field), 0, -1}
#define DB(key, field) {key, K_DOUBLE, F(field), 0, -1}
#define ST(key, field) {key, K_STR, F(field), sizeof(((NCMConfig *)0)->field), -1}

static const ConfKey conf_keys[] = {
    ST("task", task),
    BI("model.n_layer", n_layer), BI("model.n_head", n_head), BI("model.n_embd", n_embd),
    BI("model.context_length", context_length), BI("model.prefix_len", prefix_len),
    BI("model.raw_token_prefix", raw_token_prefix), BI("model.contextual_prefix", contextual_prefix),
    BI("model.prefix_pad_token_id", prefix_pad_token_id),
    BI("model.predict_level0", predict_level0), BI("model.query_level0", query_level0),
    BI("model.l0_autoregressive", l0_autoregressive),
    BI("model.use_positional_encoding", use_positional_encoding),
    BI("model.use_level_encoding", use_level_encoding),
    BI("model.use_rope", use_rope), BI("model.rope_base", rope_base), BI("model.use_qk_norm", use_qk_norm),
    BI("model.use_flex_attention", use_flex_attention),
    DB("model.rope_theta", rope_theta),
    BI("model.n_kv_heads", n_kv_heads),
    FL("model.dropout", dropout),
    AI("model.bias", bias),
    BI("model.ctx_enabled", ctx_enabled), BI("model.ctx_n_layer", ctx_n_layer), BI("model.ctx_vocab", ctx_vocab),
    BI("model.puc_enabled", puc_enabled), BI("model.puc_kernel", puc_kernel),
    BI("model.shared_output_head", shared_output_head),
    BI("model.shared_head_per_level_bias", shared_head_per_level_bias),
    BI("model.untied_head_bias", untied_head_bias),
    BI("model.tie_heads_to_codebook", tie_heads_to_codebook),
    BI("model.tie_heads_learn_scale", tie_heads_learn_scale),
    BI("model.tie_heads_trainable", tie_heads_trainable), BI("model.tie_heads_bias", tie_heads_bias),
    BI("model.use_swiglu", use_swiglu), BI("model.use_geglu", use_geglu), BI("model.use_relu2", use_relu2),
    BI("model.parallel_block", parallel_block), BI("model.normformer", normformer),
    BI("model.use_layerscale", use_layerscale), BI("model.use_rezero", use_rezero),
    FL("model.layerscale_init", layerscale_init),
    {"model.attn_pattern", K_PATTERN, F(attn_pattern_block_diag), 0, -1},
    {"model.vocab_size", K_LIST, F(vocab_size), NCM_MAX_VOCAB_LIST, (long)F(n_levels_out)},
    AI("vq.embed_dim", vq_embed_dim), AI("vq.in_vocab", vq_in_vocab),
    AI("vq.context_length", vq_context_length), AI("vq.n_layers", vq_n_layers),
    AI("vq.compression", vq_compression), AI("vq.soft_levels", vq_soft_levels),
    DB("vq.soft_tau", vq_soft_tau),
    {"vq.levels", K_LIST, F(levels), NCM_MAX_LEVELS, (long)F(n_qlevels)},
    {"vq.vocab", K_LIST, F(vq_vocab), NCM_MAX_LEVELS, -1},
    AI("vq.qr_enabled", quant_resi_enabled), FL("vq.qr_ratio", quant_resi_ratio),
    AI("vq.qr_share", quant_resi_share_mode),
    AI("vq.l1_sampling", learned_l1_sampling), AI("vq.l1_cascade", learned_l1_cascade),
    AI("vq.l1_base", learned_l1_cascade_base),
    BI("vq.l1_norm", learned_l1_norm), BI("vq.l1_norm_final", learned_l1_norm_final),
    AI("vq.all_sampling", learned_all_sampling), AI("vq.pre_quant_gn", pre_quant_groupnorm),
    BI("vq.qk_norm", vq_qk_norm),
    AI("vq.enc_layers", enc_layers), AI("vq.enc_window", enc_attn_window), AI("vq.enc_convs", enc_conv_layers),
    AI("vq.enc_conv_kernel", enc_conv_kernel), AI("vq.enc_positional", enc_positional),
    AI("vq.dec_layers", dec_layers), AI("vq.dec_positional", dec_positional),
    ST("tok.kind", pre_tok),
    AI("model.sudoku_size", sudoku_size),
    ST("tok.model_id", hf_model_id),
    BI("tok.eos_id", eos_token_id), BI("tok.pad_id", pad_token_id),
    FL("gen.temperature", gen_temperature), AI("gen.top_k", gen_top_k), FL("gen.top_p", gen_top_p),
    FL("gen.cfg_scale", gen_cfg_scale), FL("gen.freq", gen_freq), FL("gen.mu", gen_mu),
    {"gen.adj", K_ADJ, 0, 0, -1},
};

static int boolint(const char *v) {
    while (*v == ' ') v++;
    if (*v == 'T' || *v == 't') return 1;
    if (*v == 'F' || *v == 'f') return 0;
    return atoi(v);
}

/* Comma-separated integers: separators (blanks, commas) are skipped, each
 * entry is atoi of what follows, up to the next comma. */
static int int_list(const char *v, int *out, int cap) {
    int k = 0;
    for (const char *p = v; *p && k < cap;) {
        while (*p == ' ' || *p == ',') p++;
        if (!*p) break;
        out[k++] = atoi(p);
        while (*p && *p != ',') p++;
    }
    return k;
}

static void conf_apply(NCMConfig *c, const ConfKey *e, const char *v) {
    char *base = (char *)c;
    switch (e->kind) {
    case K_BOOLINT: *(int *)(base + e->off) = boolint(v); break;
    case K_ATOI: *(int *)(base + e->off) = atoi(v); break;
    case K_FLOAT: *(float *)(base + e->off) = (float)atof(v); break;
    case K_DOUBLE: *(double *)(base + e->off) = atof(v); break;
    case K_STR: {
        char *dst = base + e->off;
        strncpy(dst, v, e->size - 1);
        dst[e->size - 1] = 0;
        break;
    }
    case K_LIST: {
        int tmp[NCM_MAX_LEVELS > NCM_MAX_VOCAB_LIST ? NCM_MAX_LEVELS : NCM_MAX_VOCAB_LIST];
        int n = int_list(v, tmp, (int)e->size);
        memcpy(base + e->off, tmp, (size_t)n * sizeof(int));
        if (e->aux >= 0) *(int *)(base + e->aux) = n;
        break;
    }
    case K_PATTERN: *(int *)(base + e->off) = strcmp(v, "block_diagonal") == 0; break;
    case K_ADJ:
        if (v[0]) {
            const char *q = strchr(v, ',');
            c->gen_adj_a = (float)atof(v);
            c->gen_adj_w = q ? atoi(q + 1) : 1;
            q = q ? strchr(q + 1, ',') : NULL;
            c->gen_adj_d = q ? (float)atof(q + 1) : 1.0f;
        }
        break;
    }
}

int config_load(NCMConfig *c, const char *path) {
    if (!c || !path) return ncm_fail(NCM_E_ARG, "config_load: null argument"), -1;
    memset(c, 0, sizeof *c);
    /* the defaults of tensor.c:172-177 */
    c->bias = 1;
    c->rope_base = 10000;
    c->rope_theta = 10000.0;
    c->n_kv_heads = -1;
    c->prefix_pad_token_id = -1;
    c->eos_token_id = -1;
    c->pad_token_id = -1;
    c->attn_pattern_block_diag = 1;
    c->gen_top_k = 1;
    c->gen_top_p = 1.0f;
    FILE *f = fopen(path, "r");
    if (!f) {
        fprintf(stderr, "cannot open %s\n", path);
        return -1;
    }
    /* Lines are read in pieces of at most 1023 characters, as the reference
     * reads them (a longer line is parsed as several pieces). */
    char line[1024];
    while (fgets(line, sizeof line, f)) {
        char *eq = strchr(line, '=');
        if (!eq) continue;
        *eq = 0;
        char *v = eq + 1;
        v[strcspn(v, "\r\n")] = 0;
        for (size_t i = 0; i < sizeof conf_keys / sizeof conf_keys[0]; i++)
            if (strcmp(line, conf_keys[i].key) == 0) {
                conf_apply(c, &conf_keys[i], v);
                break;
            }
    }
    fclose(f);
    if (c->n_kv_heads < 0) c->n_kv_heads = c->n_head; /* full multi-head attention */
    return 0;
}

/* ---------------------------------------------------------------- NCMT */

TrainData *train_data_load(const char *path, int max_rows) {
    if (!path) return ncm_fail(NCM_E_ARG, "train_data_load: null path"), NULL;
    FILE *f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "cannot open %s\n", path);
        return NULL;
    }
    char magic[4];
    uint64_t nr = 0, rl = 0;
    if (fmt_read_exact(f, magic, 4) || memcmp(magic, "NCMT", 4) != 0) {
        fprintf(stderr, "%s: bad magic\n", path);
        fclose(f);
        return NULL;
    }
    if (fmt_read_u64le(f, &nr) || fmt_read_u64le(f, &rl)) {
        fclose(f);
        return NULL;
    }
    if (max_rows > 0 && nr > (uint64_t)max_rows) nr = (uint64_t)max_rows;
    if (nr > INT_MAX || rl > INT_MAX || (rl && nr > (uint64_t)SIZE_MAX / sizeof(int) / rl)) {
        fprintf(stderr, "%s: implausible shape %llu x %llu\n", path, (unsigned long long)nr,
                (unsigned long long)rl);
        fclose(f);
        return NULL;
    }
    TrainData *d = (TrainData *)calloc(1, sizeof *d);
    size_t n = (size_t)(nr * rl);
    if (d) d->rows = (int *)malloc(n ? n * sizeof(int) : 1);
    if (!d || !d->rows || fmt_read_exact(f, d->rows, n * sizeof(int))) {
        if (d && d->rows) fprintf(stderr, "%s: short read\n", path);
        train_data_free(d);
        fclose(f);
        return NULL;
    }
    d->n_rows = (int)nr;
    d->row_len = (int)rl;
    fclose(f);
    return d;
}

void train_data_free(TrainData *d) {
    if (!d) return;
    free(d->rows);
    free(d);
}
