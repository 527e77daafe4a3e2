/* ckpt.c -- NCK1 v1 training checkpoints (reference: src/ckpt.c, ncm.h:416-466)
 * for a WeightStore and AdamW whose tensors and moments live on the device.
 *
 * Layout (little-endian; a format, so it is the reference's byte for byte):
 *   "NCK1" u32 version=1
 *   i64 global_step, u64 batch_rng, f64 base_lr, f64 warmup, f64 total,
 *   i32 batch_B, i32 accum_pending, i64 n_rows, i32 row_len, u64 data_hash,
 *   str data_path, u64 conf_hash, str tokenizer_id, str train_cfg_json
 *     (str = u16 length + bytes)
 *   u32 count, then per tensor: u8 name length, name, u8 ndim, u32 dims,
 *     u64 bytes, float32 data
 *   "ADAM" f64 b1, b2, eps, wd, u32 n, i64 step, then per optimised tensor:
 *     u32 store index, f64 lr multiplier, u64 bytes, m, u64 bytes, v
 *   u64 FNV-1a 64 of every byte before it.
 *
 * Saving streams the file through the hash (device data is staged in bounded
 * chunks), then re-reads it to validate before the atomic rename.  Loading
 * reads the whole file, checks the trailer first, then parses into a list of
 * validated sections; only when every check has passed is anything written
 * to the caller's tensors, moments or step. */
#define _POSIX_C_SOURCE 200809L /* fileno, fsync, O_DIRECTORY under -std=c11 */
#include "internal.h"

#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#define NCK1_VERSION 1u
#define NCK1_MAX_FILE ((uint64_t)1 << 40)
#define NCK1_MAX_STR 0xffffu /* the u16 length field */
#define FNV_OFFSET 14695981039346656037ULL
#define FNV_PRIME 1099511628211ULL
#define ADAM_TAG 0x4D414441u /* "ADAM" read as a little-endian u32 */

static uint64_t fnv1a64(uint64_t h, const void *p, size_t n) {
    const unsigned char *b = (const unsigned char *)p;
    for (size_t i = 0; i < n; i++) h = (h ^ b[i]) * FNV_PRIME;
    return h;
}

uint64_t ckpt_file_hash(const char *path, uint64_t *nbytes_out) {
    if (nbytes_out) *nbytes_out = 0;
    FILE *f = path ? fopen(path, "rb") : NULL;
    if (!f) return 0;
    unsigned char *buf = (unsigned char *)malloc(1 << 20);
    uint64_t h = FNV_OFFSET, n = 0;
    size_t r;
    while (buf && (r = fread(buf, 1, 1 << 20, f)) > 0) {
        h = fnv1a64(h, buf, r);
        n += r;
    }
    free(buf);
    fclose(f);
    if (nbytes_out) *nbytes_out = n;
    return h;
}

int ckpt_probe(const char *path) {
    FILE *f = path ? fopen(path, "rb") : NULL;
    if (!f) return -1;
    char m[4];
    int ok = fmt_read_exact(f, m, 4) == 0;
    fclose(f);
    if (!ok) return -1;
    if (memcmp(m, "NCK1", 4) == 0) return 1;
    if (memcmp(m, "NCM1", 4) == 0) return 0;
    return -1;
}

/* ---------------------------------------------------------------- writer */

typedef struct {
    FILE *f;
    uint64_t h;
    int bad;
} Out;

static void out_bytes(void *ctx, const void *p, size_t n) {
    Out *o = (Out *)ctx;
    if (o->bad || n == 0) return;
    if (fwrite(p, 1, n, o->f) != n) {
        o->bad = 1;
        return;
    }
    o->h = fnv1a64(o->h, p, n);
}

static void out_le(Out *o, uint64_t v, int bytes) {
    unsigned char b[8];
    for (int i = 0; i < bytes; i++) b[i] = (unsigned char)(v >> (8 * i));
    out_bytes(o, b, (size_t)bytes);
}

static void out_f64(Out *o, double v) {
    uint64_t u;
    memcpy(&u, &v, 8);
    out_le(o, u, 8);
}

static void out_str(Out *o, const char *s) {
    size_t n = s ? strlen(s) : 0;
    if (n > NCK1_MAX_STR) {
        o->bad = 1;
        return;
    }
    out_le(o, n, 2);
    out_bytes(o, s, n);
}

static void out_device(Out *o, const float *dev, uint64_t nbytes) {
    if (!o->bad && fmt_download(dev, nbytes, out_bytes, o)) o->bad = 1;
}

static int store_index(const WeightStore *ws, const float *p) {
    for (int j = 0; j < ws->count; j++)
        if (ws->items[j].t->data == p) return j;
    return -1;
}

static void write_body(Out *o, const WeightStore *ws, const AdamW *opt, const CkptRunState *rs) {
    out_bytes(o, "NCK1", 4);
    out_le(o, NCK1_VERSION, 4);
    out_le(o, (uint64_t)(int64_t)rs->global_step, 8);
    out_le(o, rs->batch_rng, 8);
    out_f64(o, rs->base_lr);
    out_f64(o, rs->warmup);
    out_f64(o, rs->total);
    out_le(o, (uint32_t)rs->batch_B, 4);
    out_le(o, (uint32_t)rs->accum_pending, 4);
    out_le(o, (uint64_t)(int64_t)rs->n_rows, 8);
    out_le(o, (uint32_t)rs->row_len, 4);
    out_le(o, rs->data_hash, 8);
    out_str(o, rs->data_path ? rs->data_path : "");
    out_le(o, rs->conf_hash, 8);
    out_str(o, rs->tokenizer_id ? rs->tokenizer_id : "");
    out_str(o, rs->train_cfg_json ? rs->train_cfg_json : "");
    out_le(o, (uint32_t)ws->count, 4);
    for (int i = 0; i < ws->count && !o->bad; i++) {
        const Tensor *t = ws->items[i].t;
        size_t nl = strlen(ws->items[i].name);
        if (nl > 255 || t->ndim < 0 || t->ndim > 8) {
            o->bad = 1;
            return;
        }
        out_le(o, nl, 1);
        out_bytes(o, ws->items[i].name, nl);
        out_le(o, (uint64_t)t->ndim, 1);
        for (int d = 0; d < t->ndim; d++) out_le(o, (uint32_t)t->shape[d], 4);
        out_le(o, (uint64_t)t->n * 4u, 8);
        out_device(o, t->data, (uint64_t)t->n * 4u);
    }
    out_bytes(o, "ADAM", 4);
    out_f64(o, opt->b1);
    out_f64(o, opt->b2);
    out_f64(o, opt->eps);
    out_f64(o, opt->wd);
    out_le(o, (uint32_t)opt->n, 4);
    out_le(o, (uint64_t)(int64_t)opt->step, 8);
    for (int i = 0; i < opt->n && !o->bad; i++) {
        int idx = store_index(ws, opt->params[i]);
        if (idx < 0) {
            o->bad = 1;
            return;
        }
        uint64_t nb = (uint64_t)opt->sizes[i] * 4u;
        out_le(o, (uint32_t)idx, 4);
        out_f64(o, opt->lr[i]);
        out_le(o, nb, 8);
        out_device(o, opt->m[i], nb);
        out_le(o, nb, 8);
        out_device(o, opt->v[i], nb);
    }
}

/* ---------------------------------------------------------------- reader */

typedef struct {
    const unsigned char *p, *end;
    int bad;
} In;

static const unsigned char *in_take(In *r, uint64_t n) {
    if (r->bad || (uint64_t)(r->end - r->p) < n) {
        r->bad = 1;
        return NULL;
    }
    const unsigned char *q = r->p;
    r->p += n;
    return q;
}

static uint64_t in_le(In *r, int bytes) {
    const unsigned char *b = in_take(r, (uint64_t)bytes);
    uint64_t v = 0;
    if (b)
        for (int i = bytes - 1; i >= 0; i--) v = v << 8 | b[i];
    return v;
}

static double in_f64(In *r) {
    uint64_t u = in_le(r, 8);
    double v;
    memcpy(&v, &u, 8);
    return v;
}

/* u16-prefixed string: pointer into the buffer (not terminated) */
static const char *in_str(In *r, size_t *len) {
    size_t n = (size_t)in_le(r, 2);
    const char *s = (const char *)in_take(r, n);
    *len = s ? n : 0;
    return s;
}

/* The whole file; trailer checked; r spans the bytes before the trailer. */
static unsigned char *read_checked(const char *path, In *r, size_t *len_out, int *sum_ok, char *err, size_t errcap) {
    FILE *f = fopen(path, "rb");
    if (!f) {
        snprintf(err, errcap, "cannot open checkpoint %s: %s", path, strerror(errno));
        return NULL;
    }
    struct stat st;
    memset(&st, 0, sizeof st);
    if (fstat(fileno(f), &st) || st.st_size < 8 || (uint64_t)st.st_size > NCK1_MAX_FILE) {
        snprintf(err, errcap, "%s: refused, %lld bytes is too small or too large for a checkpoint", path, (long long)st.st_size);
        fclose(f);
        return NULL;
    }
    size_t len = (size_t)st.st_size;
    unsigned char *buf = (unsigned char *)malloc(len);
    if (!buf || fmt_read_exact(f, buf, len)) {
        snprintf(err, errcap, buf ? "%s: cannot read the whole file" : "%s: cannot allocate a buffer for the file", path);
        free(buf);
        fclose(f);
        return NULL;
    }
    fclose(f);
    uint64_t trailer = 0;
    for (int i = 7; i >= 0; i--) trailer = trailer << 8 | buf[len - 8 + i];
    *sum_ok = fnv1a64(FNV_OFFSET, buf, len - 8) == trailer;
    r->p = buf;
    r->end = buf + len - 8;
    r->bad = 0;
    *len_out = len;
    return buf;
}

static void wipe_free(unsigned char *buf, size_t len) {
    if (!buf) return;
    memset(buf, 0, len);
    free(buf);
}

/* Run-state header after "NCK1" + version. */
typedef struct {
    CkptRunState rs;
    const char *dpath, *tokid, *cfg;
    size_t dl, tl, cl;
} Header;

static void in_header(In *r, Header *h) {
    memset(h, 0, sizeof *h);
    h->rs.global_step = (long)(int64_t)in_le(r, 8);
    h->rs.batch_rng = in_le(r, 8);
    h->rs.base_lr = in_f64(r);
    h->rs.warmup = in_f64(r);
    h->rs.total = in_f64(r);
    h->rs.batch_B = (int)(int32_t)in_le(r, 4);
    h->rs.accum_pending = (int)(int32_t)in_le(r, 4);
    h->rs.n_rows = (long)(int64_t)in_le(r, 8);
    h->rs.row_len = (int)(int32_t)in_le(r, 4);
    h->rs.data_hash = in_le(r, 8);
    h->dpath = in_str(r, &h->dl);
    h->rs.conf_hash = in_le(r, 8);
    h->tokid = in_str(r, &h->tl);
    h->cfg = in_str(r, &h->cl);
}

/* ---------------------------------------------------------------- save */

int ckpt_save_atomic(const WeightStore *ws, AdamW *opt, const CkptRunState *rs, const char *path, char *err,
                     size_t errcap) {
    char dummy[8];
    if (!err || !errcap) {
        err = dummy;
        errcap = sizeof dummy;
    }
    err[0] = 0;
    if (!ws || !opt || !rs || !path) {
        snprintf(err, errcap, "ckpt_save_atomic: refused, null argument");
        return -1;
    }
    if (rs->accum_pending != 0) {
        snprintf(err, errcap, "save refused: %d gradient accumulation steps are still pending", rs->accum_pending);
        return -1;
    }
    adamw_sync_to_host(opt);
    char tmp[4096];
    if (snprintf(tmp, sizeof tmp, "%s.tmp.%d", path, (int)getpid()) >= (int)sizeof tmp) {
        snprintf(err, errcap, "ckpt_save_atomic: refused, path too long");
        return -1;
    }
    Out o = {fopen(tmp, "wb"), FNV_OFFSET, 0};
    if (!o.f) {
        snprintf(err, errcap, "cannot create %s: %s", tmp, strerror(errno));
        return -1;
    }
    write_body(&o, ws, opt, rs);
    if (!o.bad) {
        uint64_t sum = o.h;
        unsigned char b[8];
        for (int i = 0; i < 8; i++) b[i] = (unsigned char)(sum >> (8 * i));
        if (fwrite(b, 1, 8, o.f) != 8) o.bad = 1;
    }
    if (fclose(o.f)) o.bad = 1;
    if (o.bad) {
        unlink(tmp);
        snprintf(err, errcap, "writing %s failed; %s was left as it was", tmp, path);
        return -1;
    }
    /* validate the new file by reading it back before it replaces anything */
    {
        In r;
        size_t len = 0;
        int sum_ok = 0;
        char verr[256];
        unsigned char *buf = read_checked(tmp, &r, &len, &sum_ok, verr, sizeof verr);
        int ok = buf && sum_ok && memcmp(buf, "NCK1", 4) == 0;
        wipe_free(buf, len);
        if (!ok) {
            unlink(tmp);
            snprintf(err, errcap, "%s did not verify after writing; %s was left as it was", tmp, path);
            return -1;
        }
    }
    int fd = open(tmp, O_RDONLY);
    if (fd < 0 || fsync(fd)) {
        if (fd >= 0) close(fd);
        unlink(tmp);
        snprintf(err, errcap, "cannot fsync %s", tmp);
        return -1;
    }
    close(fd);
    if (rename(tmp, path)) {
        unlink(tmp);
        snprintf(err, errcap, "cannot rename %s to %s: %s", tmp, path, strerror(errno));
        return -1;
    }
    /* the rename itself must survive a crash: sync the directory */
    char dir[4096];
    snprintf(dir, sizeof dir, "%s", path);
    char *slash = strrchr(dir, '/');
    if (slash) *slash = 0;
    int dfd = open(slash ? (dir[0] ? dir : "/") : ".", O_RDONLY | O_DIRECTORY);
    if (dfd >= 0) {
        fsync(dfd);
        close(dfd);
    }
    return 0;
}

/* ---------------------------------------------------------------- load */

int ckpt_load_training(const char *path, WeightStore *ws, AdamW *opt, const CkptExpect *ex, CkptRunState *out_rs,
                       char *err, size_t errcap) {
    char dummy[8];
    if (!err || !errcap) {
        err = dummy;
        errcap = sizeof dummy;
    }
    err[0] = 0;
    if (!path || !ws || !opt || !ex) {
        snprintf(err, errcap, "ckpt_load_training: refused, null argument");
        return -1;
    }
    In r;
    size_t len = 0;
    int sum_ok = 0;
    unsigned char *buf = read_checked(path, &r, &len, &sum_ok, err, errcap);
    if (!buf) return -1;
    /* per tensor: file data; per optimised tensor: m and v */
    const unsigned char **tdata = (const unsigned char **)calloc((size_t)ws->count + 1, sizeof *tdata);
    const unsigned char **mdata = (const unsigned char **)calloc(2 * (size_t)opt->n + 1, sizeof *mdata);
    int rc = -1;
    Header h;
    if (!tdata || !mdata) {
        snprintf(err, errcap, "cannot allocate memory for the checkpoint");
        goto done;
    }
    if (!sum_ok) {
        snprintf(err, errcap, "%s: refused, the stored checksum does not match the contents (corrupt or truncated file)", path);
        goto done;
    }
    const unsigned char *magic = in_take(&r, 4);
    if (!magic || memcmp(magic, "NCK1", 4) != 0) {
        snprintf(err, errcap, "%s: refused, no NCK1 magic", path);
        goto done;
    }
    if (in_le(&r, 4) != NCK1_VERSION) {
        snprintf(err, errcap, "%s: refused, format version is not %u", path, NCK1_VERSION);
        goto done;
    }
    in_header(&r, &h);
    if (r.bad) {
        snprintf(err, errcap, "%s: refused, the run-state header is truncated", path);
        goto done;
    }
    if (h.rs.accum_pending != 0) {
        snprintf(err, errcap, "%s: refused, written with %d accumulation steps pending", path,
                 h.rs.accum_pending);
        goto done;
    }
    if (h.rs.batch_B != ex->batch_B || h.rs.n_rows != ex->n_rows || h.rs.row_len != ex->row_len ||
        h.rs.data_hash != ex->data_hash) {
        snprintf(err, errcap, "%s: refused, the training data differ from this run's (batch, rows, row_len or hash)", path);
        goto done;
    }
    if (h.rs.conf_hash != ex->conf_hash) {
        snprintf(err, errcap, "%s: refused, the model configuration hash differs", path);
        goto done;
    }
    {
        const char *want = ex->tokenizer_id ? ex->tokenizer_id : "";
        if (strlen(want) != h.tl || memcmp(want, h.tokid, h.tl) != 0) {
            snprintf(err, errcap, "%s: refused, tokenizer '%.*s' in the file, '%s' expected", path, (int)h.tl, h.tokid,
                     want);
            goto done;
        }
    }
    if (h.rs.base_lr != ex->base_lr || h.rs.warmup != ex->warmup || h.rs.total != ex->total) {
        snprintf(err, errcap, "%s: refused, the learning-rate schedule differs (lr, warmup or total)", path);
        goto done;
    }
    /* tensors: names in store order, shapes and sizes as the live store's */
    uint32_t count = (uint32_t)in_le(&r, 4);
    if (r.bad || count != (uint32_t)ws->count) {
        snprintf(err, errcap, "%s: refused, %u tensors in the file, %d in the model", path, r.bad ? 0u : count, ws->count);
        goto done;
    }
    for (int i = 0; i < ws->count; i++) {
        const Tensor *t = ws->items[i].t;
        size_t nl = (size_t)in_le(&r, 1);
        const char *nm = (const char *)in_take(&r, nl);
        if (r.bad || nl == 0) {
            snprintf(err, errcap, "%s: refused, the tensor section is cut short", path);
            goto done;
        }
        if (strlen(ws->items[i].name) != nl || memcmp(nm, ws->items[i].name, nl) != 0) {
            snprintf(err, errcap, "%s: refused, tensor %d is '%.*s' (another name or order)", path, i, (int)nl, nm);
            goto done;
        }
        if ((int)in_le(&r, 1) != t->ndim) {
            snprintf(err, errcap, "%s: refused, tensor '%s' has another rank", path, ws->items[i].name);
            goto done;
        }
        int shape_ok = 1;
        for (int d = 0; d < t->ndim; d++) shape_ok &= (int64_t)in_le(&r, 4) == t->shape[d];
        if (!shape_ok) {
            snprintf(err, errcap, "%s: refused, tensor '%s' has another shape", path, ws->items[i].name);
            goto done;
        }
        uint64_t nb = in_le(&r, 8);
        tdata[i] = nb == (uint64_t)t->n * 4u ? in_take(&r, nb) : NULL;
        if (!tdata[i]) {
            snprintf(err, errcap, "%s: refused, tensor '%s' has another size", path, ws->items[i].name);
            goto done;
        }
    }
    /* optimizer section */
    uint32_t tag = (uint32_t)in_le(&r, 4);
    double b1 = in_f64(&r), b2 = in_f64(&r), eps = in_f64(&r), wd = in_f64(&r);
    uint32_t on = (uint32_t)in_le(&r, 4);
    int64_t ostep = (int64_t)in_le(&r, 8);
    if (r.bad || tag != ADAM_TAG || on != (uint32_t)opt->n || b1 != ex->b1 || b2 != ex->b2 || eps != ex->eps ||
        wd != ex->wd) {
        snprintf(err, errcap, "%s: refused, the optimizer section differs (tag, tensor count or hyperparameters)", path);
        goto done;
    }
    if (ostep < 0 || ostep > ((int64_t)1 << 40)) {
        snprintf(err, errcap, "%s: refused, optimizer step %lld is out of range", path, (long long)ostep);
        goto done;
    }
    for (int i = 0; i < opt->n; i++) {
        uint32_t idx = (uint32_t)in_le(&r, 4);
        double lrm = in_f64(&r);
        uint64_t mnb = in_le(&r, 8);
        mdata[2 * i] = in_take(&r, mnb);
        uint64_t vnb = in_le(&r, 8);
        mdata[2 * i + 1] = in_take(&r, vnb);
        if (r.bad) {
            snprintf(err, errcap, "%s: refused, the moments of tensor %d are cut short", path, i);
            goto done;
        }
        if (idx >= (uint32_t)ws->count || ws->items[idx].t->data != opt->params[i] ||
            mnb != (uint64_t)opt->sizes[i] * 4u || vnb != mnb || lrm != opt->lr[i]) {
            snprintf(err, errcap, "%s: refused, optimizer entry %d differs (index, size or lr scale)", path, i);
            goto done;
        }
    }
    if (r.p != r.end) {
        snprintf(err, errcap, "%s: refused, %ld unexpected bytes after the last section", path, (long)(r.end - r.p));
        goto done;
    }
    /* every check passed: apply */
    for (int i = 0; i < ws->count; i++) mem_h2d(ws->items[i].t->data, tdata[i], (size_t)ws->items[i].t->n * 4u);
    for (int i = 0; i < opt->n; i++) {
        mem_h2d(opt->m[i], mdata[2 * i], (size_t)opt->sizes[i] * 4u);
        mem_h2d(opt->v[i], mdata[2 * i + 1], (size_t)opt->sizes[i] * 4u);
    }
    opt->step = (long)ostep;
    if (out_rs) {
        *out_rs = h.rs;
        out_rs->data_path = NULL; /* the strings stay with the caller */
        out_rs->tokenizer_id = NULL;
        out_rs->train_cfg_json = NULL;
    }
    rc = 0;
done:
    free(tdata);
    free(mdata);
    wipe_free(buf, len);
    return rc;
}

int ckpt_load_weights_only(const char *path, WeightStore *ws, char *err, size_t errcap) {
    char dummy[8];
    if (!err || !errcap) {
        err = dummy;
        errcap = sizeof dummy;
    }
    err[0] = 0;
    if (!path || !ws) {
        snprintf(err, errcap, "ckpt_load_weights_only: refused, null argument");
        return -1;
    }
    ws->items = NULL;
    ws->count = 0;
    In r;
    size_t len = 0;
    int sum_ok = 0;
    unsigned char *buf = read_checked(path, &r, &len, &sum_ok, err, errcap);
    if (!buf) return -1;
    if (!sum_ok) {
        snprintf(err, errcap, "%s: refused, the stored checksum does not match the contents", path);
        wipe_free(buf, len);
        return -1;
    }
    const unsigned char *magic = in_take(&r, 4);
    if (!magic || memcmp(magic, "NCK1", 4) != 0 || in_le(&r, 4) != NCK1_VERSION) {
        snprintf(err, errcap, "%s: refused, no NCK1 magic", path);
        wipe_free(buf, len);
        return -1;
    }
    Header h;
    in_header(&r, &h); /* skipped: the run state is not needed for inference */
    uint32_t n = (uint32_t)in_le(&r, 4);
    if (r.bad || n > (1u << 24)) {
        snprintf(err, errcap, "%s: refused, bad tensor count", path);
        wipe_free(buf, len);
        return -1;
    }
    ws->items = (NamedTensor *)calloc(n ? n : 1, sizeof(NamedTensor));
    if (!ws->items) {
        snprintf(err, errcap, "cannot allocate memory for the checkpoint");
        wipe_free(buf, len);
        return -1;
    }
    for (uint32_t i = 0; i < n; i++) {
        NamedTensor *it = &ws->items[i];
        size_t nl = (size_t)in_le(&r, 1);
        const unsigned char *nm = in_take(&r, nl);
        size_t nd = (size_t)in_le(&r, 1);
        if (r.bad || nl == 0 || nd > NCM_MAX_DIMS) goto fail;
        memcpy(it->name, nm, nl);
        it->name[nl] = 0;
        int64_t shape[NCM_MAX_DIMS] = {0};
        for (size_t d = 0; d < nd; d++) shape[d] = (int64_t)in_le(&r, 4);
        uint64_t nb = in_le(&r, 8);
        const unsigned char *data = in_take(&r, nb);
        if (r.bad) goto fail;
        if ((uint64_t)tensor_numel((int)nd, shape) * 4u != nb) {
            snprintf(err, errcap, "%s: refused, tensor '%s' has another size", path, it->name);
            goto fail;
        }
        Tensor *t = tensor_alloc((int)nd, shape);
        if (!t) goto fail;
        mem_h2d(t->data, data, (size_t)nb);
        it->t = t;
        ws->count++;
    }
    wipe_free(buf, len);
    return 0;
fail:
    if (!err[0]) snprintf(err, errcap, "%s: refused, the tensor section is cut short", path);
    weights_free(ws);
    wipe_free(buf, len);
    return -1;
}

int ckpt_info(const char *path) {
    char err[512] = {0};
    In r;
    size_t len = 0;
    int sum_ok = 0;
    unsigned char *buf = path ? read_checked(path, &r, &len, &sum_ok, err, sizeof err) : NULL;
    if (!buf) {
        fprintf(stderr, "ckpt-info: %s\n", path ? err : "null path");
        return 1;
    }
    const unsigned char *magic = in_take(&r, 4);
    if (!magic || memcmp(magic, "NCK1", 4) != 0) {
        printf("file: %s\nformat: NOT NCK1 (probe=%d)\nchecksum: n/a\n", path, ckpt_probe(path));
        wipe_free(buf, len);
        return 1;
    }
    uint32_t ver = (uint32_t)in_le(&r, 4);
    Header h;
    in_header(&r, &h);
    uint32_t n = (uint32_t)in_le(&r, 4);
    if (r.bad) {
        printf("file: %s\nformat: NCK1 (truncated header)\nchecksum: %s\n", path, sum_ok ? "OK" : "MISMATCH");
        wipe_free(buf, len);
        return 1;
    }
    uint64_t wbytes = 0, mbytes = 0;
    for (uint32_t i = 0; i < n && !r.bad; i++) {
        in_take(&r, in_le(&r, 1));
        uint64_t nd = in_le(&r, 1);
        in_take(&r, 4 * nd);
        uint64_t nb = in_le(&r, 8);
        in_take(&r, nb);
        wbytes += nb;
    }
    uint32_t tag = (uint32_t)in_le(&r, 4);
    double b1 = in_f64(&r), b2 = in_f64(&r), eps = in_f64(&r), wd = in_f64(&r);
    uint32_t on = (uint32_t)in_le(&r, 4);
    long ostep = (long)(int64_t)in_le(&r, 8);
    for (uint32_t i = 0; i < on && !r.bad; i++) {
        in_le(&r, 4);
        in_f64(&r);
        uint64_t mnb = in_le(&r, 8);
        in_take(&r, mnb);
        uint64_t vnb = in_le(&r, 8);
        in_take(&r, vnb);
        mbytes += mnb + vnb;
    }
    printf("file: %s (%llu bytes)\n", path, (unsigned long long)len);
    printf("format: NCK1 v%u  checksum: %s\n", ver, sum_ok ? "OK" : "MISMATCH");
    printf("global_step: %ld  optimizer_step: %ld  accum_pending: %d\n", h.rs.global_step, ostep,
           h.rs.accum_pending);
    printf("schedule: lr=%.6g warmup=%.6g total=%.6g\n", h.rs.base_lr, h.rs.warmup, h.rs.total);
    printf("optimizer: ADAM(%.4f,%.4f,eps=%.1g,wd=%.4g) params=%u moments=%.1f MiB\n", b1, b2, eps, wd, on,
           mbytes / 1048576.0);
    printf("batch: B=%d rng=0x%016llx  data: rows=%ld row_len=%d hash=%016llx\n", h.rs.batch_B, h.rs.batch_rng,
           h.rs.n_rows, h.rs.row_len, (unsigned long long)h.rs.data_hash);
    printf("data_path: %.*s\n", (int)h.dl, h.dpath ? h.dpath : "");
    printf("conf_hash: %016llx  tokenizer: %.*s\n", (unsigned long long)h.rs.conf_hash, (int)h.tl,
           h.tokid ? h.tokid : "");
    printf("tensors: %u weights=%.1f MiB\n", n, wbytes / 1048576.0);
    printf("cfg: %.*s\n", (int)h.cl, h.cfg ? h.cfg : "");
    int rc = 0;
    if (!sum_ok) {
        printf("status: CHECKSUM MISMATCH - refused, do not resume from this file\n");
        rc = 1;
    } else if (r.bad || r.p != r.end || tag != ADAM_TAG) {
        printf("status: STRUCTURALLY INVALID\n");
        rc = 1;
    } else {
        printf("status: valid, exact-resume ready\n");
    }
    fflush(stdout);
    wipe_free(buf, len);
    return rc;
}
