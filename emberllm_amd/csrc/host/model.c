/* model.c — run state and the forward-pass entry points of ember.h.
 *
 * ember_state_new_ex resolves the same tensors as the reference
 * (src/model.c:144-171, with the same error messages), uploads them to the
 * GPU once per model (ehip_model_upload repacks them for the kernels) and
 * creates the device state (KV cache in HBM, fp32 or fp16).  ember_forward
 * and ember_prefill check their arguments as the reference does
 * (src/model.c:285, 306-307, 368-371) and run on the device; the returned
 * logits are pinned host memory owned by the state.  There is no CPU
 * fallback: without a usable GPU, state creation fails with an error.
 */
#include "ember.h"
#include "ehip.h"
#include "model_internal.h"
#include "util.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

struct EmberState {
    const EmberModel *m;
    EhipState *dev;
    int ctx, vocab;
    float *logits;     /* last logits returned (pinned, owned by dev) */
    float *zeros;      /* returned by a prefill of zero tokens before any call */
};

static size_t stored_bytes(int dtype, long rows, long cols) {
    switch (dtype) {
        case EMBER_DT_F32: return (size_t)(rows * cols * 4);
        case EMBER_DT_Q8_0: return (size_t)(rows * (cols / EMBER_Q_BLOCK) * 34);
        case EMBER_DT_Q4_0: return (size_t)(rows * (cols / EMBER_Q_BLOCK) * 18);
        default: return 0;
    }
}

/* Look a tensor up by printf-style name; NULL data when absent.  The stored
 * size must cover the logical shape the forward pass will read. */
static EhipWeight weight(const EmberModel *m, const char *fmt, int l, long rows, long cols) {
    char name[48];
    if (l >= 0) snprintf(name, sizeof name, fmt, l);
    else snprintf(name, sizeof name, "%s", fmt);
    EhipWeight w = { NULL, EMBER_DT_F32 };
    const EmberTensor *t = ember_model_tensor(m, name);
    if (!t) return w;
    w.data = ember_model_data(m, t);
    w.dtype = t->dtype;
    if (!w.data) ember_die("tensor '%s' lies outside the model file", name);
    if (t->dtype != EMBER_DT_F32 && t->dtype != EMBER_DT_Q8_0 && t->dtype != EMBER_DT_Q4_0)
        ember_die("tensor '%s' has unsupported dtype %d", name, t->dtype);
    if (t->nbytes < stored_bytes(t->dtype, rows, cols))
        ember_die("tensor '%s' is smaller than its [%ld, %ld] shape", name, rows, cols);
    return w;
}

static const float *vec(const EmberModel *m, const char *fmt, int l, long n) {
    EhipWeight w = weight(m, fmt, l, 1, n);
    if (w.data && w.dtype != EMBER_DT_F32) ember_die("vector tensor '%s' must be F32", fmt);
    return (const float *)w.data;
}

void ember_model_release_device(EmberModel *m) {
    if (m && m->dev) { ehip_model_free(m->dev); m->dev = NULL; }
}

static void upload(EmberModel *m) {
    const EmberHeader *h = m->hdr;
    const int L = h->n_layers, dim = h->dim, hid = h->hidden_dim, hd = h->head_dim;
    const long qd = (long)h->n_heads * hd, kvd = (long)h->n_kv_heads * hd;
    if (h->n_heads <= 0 || h->n_kv_heads <= 0 || hd <= 0 || hid <= 0 || hd % 2)
        ember_die("header has invalid attention shape");
    EhipLayer *ly = ember_xcalloc((size_t)L, sizeof *ly, "layer table");
    for (int l = 0; l < L; l++) {
        EhipLayer *y = &ly[l];
        y->wq = weight(m, "layers.%d.wq", l, qd, dim);
        y->wk = weight(m, "layers.%d.wk", l, kvd, dim);
        y->wv = weight(m, "layers.%d.wv", l, kvd, dim);
        y->wo = weight(m, "layers.%d.wo", l, dim, qd);
        y->w1 = weight(m, "layers.%d.w1", l, hid, dim);
        y->w2 = weight(m, "layers.%d.w2", l, dim, hid);
        y->w3 = weight(m, "layers.%d.w3", l, hid, dim);
        y->attn_norm = vec(m, "layers.%d.attn_norm", l, dim);
        y->ffn_norm = vec(m, "layers.%d.ffn_norm", l, dim);
        y->q_norm = vec(m, "layers.%d.q_norm", l, hd);
        y->k_norm = vec(m, "layers.%d.k_norm", l, hd);
        y->bq = vec(m, "layers.%d.wq_bias", l, qd);
        y->bk = vec(m, "layers.%d.wk_bias", l, kvd);
        y->bv = vec(m, "layers.%d.wv_bias", l, kvd);
    }
    EhipWeight emb = weight(m, "tok_embeddings", -1, h->vocab_size, dim);
    const float *fnorm = vec(m, "final_norm", -1, dim);
    EhipWeight head = (h->flags & EMBER_FLAG_TIED_EMBED) ? emb : weight(m, "lm_head", -1, h->vocab_size, dim);
    if (!emb.data) ember_die("model is missing tensor 'tok_embeddings'");
    if (!fnorm) ember_die("model is missing tensor 'final_norm'");
    if (!head.data) ember_die("model is missing tensor 'lm_head' (and is not tied)");
    for (int l = 0; l < L; l++) {
        const EhipLayer *y = &ly[l];
        if (!y->wq.data || !y->wk.data || !y->wv.data || !y->wo.data || !y->w1.data ||
            !y->w2.data || !y->w3.data || !y->attn_norm || !y->ffn_norm)
            ember_die("model is missing a required tensor in layer %d", l);
    }
    /* RoPE inverse frequencies with the reference's expression (model.c:69) */
    float *inv_freq = ember_xmalloc(sizeof(float) * (size_t)(hd / 2), "rope table");
    for (int i = 0; i < hd / 2; i++) inv_freq[i] = 1.0f / powf(h->rope_theta, (float)(2 * i) / hd);
    EhipConfig cfg = { dim, hid, L, h->n_heads, h->n_kv_heads, hd, h->vocab_size,
                       h->rope_theta, h->norm_eps, h->rope_style,
                       (h->flags & EMBER_FLAG_QK_NORM) != 0 };
    if (ehip_device_count() <= 0) ember_die("no GPU is visible to the HIP runtime");
    m->dev = ehip_model_upload(&cfg, ly, emb, head, fnorm, inv_freq);
    free(ly);
    free(inv_freq);
    if (!m->dev) ember_die("weight upload failed: %s", ehip_last_error());
}

EmberState *ember_state_new(const EmberModel *m, int ctx_len) {
    return ember_state_new_ex(m, ctx_len, 0);
}

EmberState *ember_state_new_ex(const EmberModel *mc, int ctx_len, int kv_fp16) {
    EmberModel *m = (EmberModel *)mc;  /* the device weight cache is mutable state of the model */
    const EmberHeader *h = m->hdr;
    if (!m->dev) upload(m);
    EmberState *s = ember_xcalloc(1, sizeof *s, "EmberState");
    s->m = m;
    s->ctx = (ctx_len > 0 && ctx_len < h->max_seq_len) ? ctx_len : h->max_seq_len;
    s->vocab = h->vocab_size;
    if (s->ctx <= 0) ember_die("model has no usable context length");
    s->dev = ehip_state_create(m->dev, s->ctx, kv_fp16 ? 1 : 0);
    if (!s->dev) ember_die("device state creation failed: %s", ehip_last_error());
    s->zeros = ember_xcalloc((size_t)s->vocab, sizeof(float), "logits");
    s->logits = s->zeros;
    return s;
}

void ember_state_free(EmberState *s) {
    if (!s) return;
    ehip_state_destroy(s->dev);
    free(s->zeros);
    free(s);
}

float *ember_forward(EmberModel *m, EmberState *s, int tok, int pos) {
    (void)m;
    if (tok < 0 || tok >= s->vocab) ember_die("token id %d out of range [0,%d)", tok, s->vocab);
    if (pos < 0 || pos >= s->ctx) ember_die("position %d out of range [0,%d)", pos, s->ctx);
    float *lg = ehip_forward(s->dev, tok, pos);
    if (!lg) ember_die("decode step failed: %s", ehip_last_error());
    return s->logits = lg;
}

float *ember_prefill(EmberModel *m, EmberState *s, const int *ids, int n, int start) {
    (void)m;
    if (n <= 0) return s->logits;
    for (int b = 0; b < n; b++)
        if (ids[b] < 0 || ids[b] >= s->vocab) ember_die("token id %d out of range [0,%d)", ids[b], s->vocab);
    if (start < 0 || (long)start + n > s->ctx)
        ember_die("prefill of %d tokens at position %d exceeds the context of %d", n, start, s->ctx);
    float *lg = ehip_prefill(s->dev, ids, n, start);
    if (!lg) ember_die("prefill failed: %s", ehip_last_error());
    return s->logits = lg;
}

/* Access to the device state for the package's measurement and test hooks. */
EhipState *ember_state_device(EmberState *s) { return s->dev; }
