/* ref_glue_qwen.c -- drives the REFERENCE's own Qwen2 decoder for oracle
 * validation.  qwen.c keeps its model functions static, so this
 * translation unit includes /root/reference/src/qwen.c (found through the
 * -I$(REF)/src include path; nothing is copied) and exports thin wrappers.
 * Compiled only into oracle/_ref/libref.so by oracle/Makefile; never part of
 * libncmhip.so.  Test infrastructure only.
 *
 * refg_qwen_open runs qwen_open (qwen.c:43-116) on an NCM1 weights file and
 * an in-memory NCMConfig with the sudoku pre-tokenizer (tok_load then needs
 * no asset files, tok.c:285-291) and eos id -1 (never produced), so
 * qwen_generate never stops early.  refg_qwen_forward returns qwen_forward's
 * logits (qwen.c:121-190); refg_qwen_generate runs the greedy loop of
 * qwen_generate (qwen.c:204-228, temp 0 -> argmax_row). */
#include "qwen.c"

void refg_parena_once(void); /* ref_glue.c */

void *refg_qwen_open(const char *weights, int n_layer, int n_head, int n_kv, int n_embd, int n_ctx,
                     double theta) {
    refg_parena_once();
    NCMConfig *c = (NCMConfig *)calloc(1, sizeof(NCMConfig));
    QWEN *m = (QWEN *)calloc(1, sizeof(QWEN));
    if (!c || !m) {
        free(c);
        free(m);
        return NULL;
    }
    c->n_layer = n_layer;
    c->n_head = n_head;
    c->n_kv_heads = n_kv;
    c->n_embd = n_embd;
    c->context_length = n_ctx;
    c->rope_theta = theta;
    snprintf(c->pre_tok, sizeof(c->pre_tok), "sudoku");
    c->eos_token_id = -1;
    c->pad_token_id = -1;
    int rc = qwen_open(m, c, weights, ".");
    free(c);
    if (rc) {
        free(m);
        return NULL;
    }
    return m;
}

/* logits of ids[T] into out ([T][V], or [V] when last_only) */
int refg_qwen_forward(void *h, const int *ids, int T, int last_only, float *out) {
    QWEN *m = (QWEN *)h;
    if (!m || T <= 0 || T > m->n_ctx) return -1;
    float *lg = qwen_forward(m, ids, T, last_only);
    size_t n = (size_t)(last_only ? 1 : T) * (size_t)m->vocab_size;
    memcpy(out, lg, n * sizeof(float));
    return m->vocab_size;
}

/* greedy continuation of prompt[np] by n_new ids into out; returns the count */
int refg_qwen_generate(void *h, const int *prompt, int np, int n_new, int *out) {
    QWEN *m = (QWEN *)h;
    if (!m) return -1;
    unsigned long long rng = 0x9E3779B97F4A7C15ull;
    return qwen_generate(m, prompt, np, n_new, 0.0f, 0, 1.0f, &rng, out);
}

void refg_qwen_close(void *h) {
    QWEN *m = (QWEN *)h;
    if (!m) return;
    weights_free(&m->ws);
    qwen_close(m);
    free(m);
}
