/* ehip_stub.c — a test double of the device layer (include/ehip.h) for
 * sanitizer runs of the host C library (emberllm_amd/csrc/host) on a machine
 * without a GPU.  TEST INFRASTRUCTURE: it is linked only into the driver
 * built by tests/host_asan/Makefile, never into libember.so.
 *
 * It computes nothing of the model.  It reads every byte the real layer
 * reads from the caller's buffers (each weight matrix over its full
 * [rows][in_len] extent in the mapped file, norms, biases, the RoPE
 * frequencies, prompt ids, the requantizer's fp32 rows) and writes every
 * byte the real layer writes to them (the requantizer's blocks, through the
 * host row quantizers), so AddressSanitizer checks the host library's
 * pointers and sizes exactly as the device layer consumes them.  The logits
 * it returns are a fixed pattern of (token, position), with the error-flag
 * word behind them cleared as the real layer's is. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ehip.h"

void ember_quant_q8_row(const float *x, uint8_t *out, int n);
void ember_quant_q4_row(const float *x, uint8_t *out, int n);

struct EhipModel { EhipConfig cfg; uint64_t sum; };
struct EhipState { EhipModel *m; int ctx; float *logits; uint64_t sum; };

static char err[256];
const char *ehip_last_error(void) { return err; }
int ehip_device_count(void) { return 1; }

static volatile uint64_t g_sink;

static uint64_t touch(const void *p, size_t n) {
    const uint8_t *b = p;
    uint64_t s = 0;
    for (size_t i = 0; i < n; i++) s = s * 31 + b[i];
    return s;
}

static size_t enc_bytes(int dtype, long rows, long cols) {
    switch (dtype) {
        case EMBER_DT_F32: return (size_t)rows * cols * 4;
        case EMBER_DT_Q8_0: return (size_t)rows * (cols / 32) * 34;
        case EMBER_DT_Q4_0: return (size_t)rows * (cols / 32) * 18;
        default: return 0;
    }
}

static int mat(uint64_t *s, EhipWeight w, long rows, long cols, const char *what) {
    if (!w.data || !enc_bytes(w.dtype, rows, cols) || cols % 32) {
        snprintf(err, sizeof err, "ehip_model_upload: bad %s", what);
        return -1;
    }
    *s += touch(w.data, enc_bytes(w.dtype, rows, cols));
    return 0;
}

static void vec(uint64_t *s, const float *v, long n) { if (v) *s += touch(v, 4 * (size_t)n); }

EhipModel *ehip_model_upload(const EhipConfig *c, const EhipLayer *ly, EhipWeight emb, EhipWeight head,
                             const float *fnorm, const float *inv_freq) {
    const long dim = c->dim, hid = c->hidden_dim, hd = c->head_dim, V = c->vocab_size;
    const long qd = (long)c->n_heads * hd, kvd = (long)c->n_kv_heads * hd;
    uint64_t s = 0;
    for (int l = 0; l < c->n_layers; l++) {
        const EhipLayer *y = &ly[l];
        if (mat(&s, y->wq, qd, dim, "wq") || mat(&s, y->wk, kvd, dim, "wk") || mat(&s, y->wv, kvd, dim, "wv") ||
            mat(&s, y->wo, dim, qd, "wo") || mat(&s, y->w1, hid, dim, "w1") || mat(&s, y->w3, hid, dim, "w3") ||
            mat(&s, y->w2, dim, hid, "w2"))
            return NULL;
        vec(&s, y->attn_norm, dim); vec(&s, y->ffn_norm, dim);
        vec(&s, y->q_norm, hd); vec(&s, y->k_norm, hd);
        vec(&s, y->bq, qd); vec(&s, y->bk, kvd); vec(&s, y->bv, kvd);
    }
    if (mat(&s, emb, V, dim, "tok_embeddings") || mat(&s, head, V, dim, "lm_head")) return NULL;
    vec(&s, fnorm, dim);
    vec(&s, inv_freq, hd / 2);
    EhipModel *m = calloc(1, sizeof *m);
    if (!m) return NULL;
    m->cfg = *c;
    m->sum = s;
    return m;
}

void ehip_model_free(EhipModel *m) { if (m) g_sink += m->sum; free(m); }
uint64_t ehip_model_bytes(const EhipModel *m) { (void)m; return 0; }

EhipState *ehip_state_create(EhipModel *m, int ctx, int kv_fp16) {
    (void)kv_fp16;
    if (!m || ctx <= 0) { snprintf(err, sizeof err, "ehip_state_create: bad arguments"); return NULL; }
    EhipState *s = calloc(1, sizeof *s);
    if (!s) return NULL;
    s->m = m;
    s->ctx = ctx;
    s->logits = calloc((size_t)m->cfg.vocab_size + 4, sizeof(float));
    if (!s->logits) { free(s); return NULL; }
    return s;
}

void ehip_state_destroy(EhipState *s) {
    if (!s) return;
    g_sink += s->sum;
    free(s->logits);
    free(s);
}

static float *fill(EhipState *s, int tok, int pos) {
    const int V = s->m->cfg.vocab_size;
    for (int i = 0; i < V; i++) s->logits[i] = (float)((i * 7 + tok * 3 + pos) % 97) * 0.01f;
    s->logits[V] = 0.0f;   /* the error-flag word */
    return s->logits;
}

float *ehip_forward(EhipState *s, int tok, int pos) {
    if (tok < 0 || tok >= s->m->cfg.vocab_size || pos < 0 || pos >= s->ctx) {
        snprintf(err, sizeof err, "ehip_forward: tok %d pos %d out of range", tok, pos);
        return NULL;
    }
    return fill(s, tok, pos);
}

float *ehip_prefill(EhipState *s, const int *ids, int n, int start) {
    if (n <= 0 || start < 0 || (long)start + n > s->ctx) {
        snprintf(err, sizeof err, "ehip_prefill: %d tokens at %d", n, start);
        return NULL;
    }
    s->sum += touch(ids, 4 * (size_t)n);
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= s->m->cfg.vocab_size) { snprintf(err, sizeof err, "ehip_prefill: id"); return NULL; }
    return fill(s, ids[n - 1], start + n - 1);
}

int ehip_quantize_rows(const EhipQuantJob *jobs, int n_jobs) {
    for (int j = 0; j < n_jobs; j++) {
        const EhipQuantJob *q = &jobs[j];
        if (q->cols % 32 || q->rows < 0 || (q->dtype != EMBER_DT_Q8_0 && q->dtype != EMBER_DT_Q4_0)) {
            snprintf(err, sizeof err, "ehip_quantize_rows: bad job %d", j);
            return -1;
        }
        const size_t rb = (size_t)(q->cols / 32) * (q->dtype == EMBER_DT_Q8_0 ? 34 : 18);
        for (int64_t r = 0; r < q->rows; r++) {
            const float *x = q->src + (size_t)r * q->cols;
            uint8_t *o = (uint8_t *)q->dst + (size_t)r * rb;
            if (q->dtype == EMBER_DT_Q8_0) ember_quant_q8_row(x, o, q->cols);
            else ember_quant_q4_row(x, o, q->cols);
        }
    }
    return 0;
}
