/* synth.c — seeded synthetic .ember models (include/ember_synth.h).
 *
 * Benchmarks and tests need model files of the real shapes without network
 * access.  Weights are drawn N(0, std) from a documented generator so every
 * machine regenerates identical bytes:
 *   stream key   = splitmix64(seed ^ fnv1a64(tensor name)), then per row r
 *                  state = key + (r+1) * 0x9E3779B97F4A7C15
 *   draws        = splitmix64 outputs, two per Box-Muller pair:
 *                  u1 = ((a >> 11) + 1) * 2^-53,  u2 = (b >> 11) * 2^-53,
 *                  z0 = sqrt(-2 ln u1) cos(2 pi u2), z1 = ... sin(2 pi u2)
 *                  (double precision), stored as (float)(std * z)
 * Norm weights (attn/ffn/final/q/k norms) are 1.0; biases are drawn like
 * matrices.  2-D tensors are then encoded with the file rules of
 * ember_quantize_file (src/quant.c:26-75): Q8_0 / Q4_0 rows when the row
 * length is a multiple of 32, and tok_embeddings / lm_head kept at Q8_0 in
 * Q4_0 mode.  Tensor order and alignment follow tools/convert.py:57-112 and
 * 294-390.  The tokenizer blob is a SentencePiece-style vocabulary
 * ("<unk>", "<s>", "</s>", 256 byte pieces "<0xNN>", then "t<id>").
 */
#define _DEFAULT_SOURCE
#include "ember_synth.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ember.h"
#include "util.h"

static uint64_t splitmix(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static uint64_t fnv1a64(const char *s) {
    uint64_t h = 1469598103934665603ULL;
    for (; *s; s++) { h ^= (unsigned char)*s; h *= 1099511628211ULL; }
    return h;
}

uint64_t ember_synth_row_state(uint64_t seed, const char *name, int row) {
    uint64_t k = seed ^ fnv1a64(name);
    uint64_t key = splitmix(&k);
    return key + (uint64_t)(row + 1) * 0x9E3779B97F4A7C15ULL;
}

void ember_synth_fill_row(uint64_t seed, const char *name, int row, float std, float *out, int n) {
    uint64_t st = ember_synth_row_state(seed, name, row);
    for (int i = 0; i < n; i += 2) {
        const double u1 = (double)((splitmix(&st) >> 11) + 1) * 0x1.0p-53;
        const double u2 = (double)(splitmix(&st) >> 11) * 0x1.0p-53;
        const double r = sqrt(-2.0 * log(u1)), a = 6.283185307179586 * u2;
        out[i] = (float)(std * r * cos(a));
        if (i + 1 < n) out[i + 1] = (float)(std * r * sin(a));
    }
}

typedef struct {
    char name[48];
    int kind;            /* 0 = matrix (random), 1 = norm (ones), 2 = bias (random) */
    int rows, cols, ndim, dtype;
    uint64_t offset, nbytes;
} Spec;

static uint64_t up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

static void add(Spec *t, int *n, const char *name, int kind, int rows, int cols, int file_dtype, int q_emb) {
    Spec *s = &t[(*n)++];
    memset(s, 0, sizeof *s);
    snprintf(s->name, sizeof s->name, "%s", name);
    s->kind = kind; s->rows = rows; s->cols = cols;
    s->ndim = cols > 1 ? 2 : 1;
    int dt = EMBER_DT_F32;
    if (s->ndim >= 2 && cols % EMBER_Q_BLOCK == 0 && file_dtype != EMBER_DT_F32)
        dt = (file_dtype == EMBER_DT_Q4_0 && q_emb) ? EMBER_DT_Q8_0 : file_dtype;
    s->dtype = dt;
    s->nbytes = dt == EMBER_DT_F32 ? (uint64_t)rows * cols * 4
                                   : (uint64_t)rows * (cols / EMBER_Q_BLOCK) * (dt == EMBER_DT_Q8_0 ? 34 : 18);
}

typedef struct {
    const Spec *s; uint64_t seed; float std; uint8_t *dst; int r0, r1;
} Job;

static void *fill_job(void *p) {
    const Job *j = p;
    const Spec *s = j->s;
    float *row = ember_xmalloc(sizeof(float) * (size_t)s->cols, "synth row");
    const size_t rb = s->nbytes / (uint64_t)s->rows;
    for (int r = j->r0; r < j->r1; r++) {
        if (s->kind == 1) for (int i = 0; i < s->cols; i++) row[i] = 1.0f;
        else ember_synth_fill_row(j->seed, s->name, r, j->std, row, s->cols);
        uint8_t *o = j->dst + (size_t)r * rb;
        if (s->dtype == EMBER_DT_Q8_0) ember_quant_q8_row(row, o, s->cols);
        else if (s->dtype == EMBER_DT_Q4_0) ember_quant_q4_row(row, o, s->cols);
        else memcpy(o, row, sizeof(float) * (size_t)s->cols);
    }
    free(row);
    return NULL;
}

static void fill_tensor(const Spec *s, uint64_t seed, float std, uint8_t *dst, int nthreads) {
    /* norms and biases are stored as one row of `cols` values */
    Spec one = *s;
    if (s->ndim == 1) { one.cols = s->rows * s->cols; one.rows = 1; }
    if (nthreads > one.rows) nthreads = one.rows;
    if (nthreads < 1) nthreads = 1;
    pthread_t th[64];
    Job jobs[64];
    if (nthreads > 64) nthreads = 64;
    for (int t = 0; t < nthreads; t++) {
        jobs[t] = (Job){ &one, seed, std, dst, (int)((long)one.rows * t / nthreads),
                         (int)((long)one.rows * (t + 1) / nthreads) };
        if (t) pthread_create(&th[t], NULL, fill_job, &jobs[t]);
    }
    fill_job(&jobs[0]);
    for (int t = 1; t < nthreads; t++) pthread_join(th[t], NULL);
}

int ember_synth_write(const char *path, const EmberSynthConfig *c) {
    const int L = c->n_layers, hd = c->head_dim, qd = c->n_heads * hd, kvd = c->n_kv_heads * hd;
    const int dt = c->dtype;
    const int cap = 4 + L * 16;
    Spec *t = ember_xcalloc((size_t)cap, sizeof(Spec), "synth specs");
    int n = 0;
    char nm[48];
    add(t, &n, "tok_embeddings", 0, c->vocab_size, c->dim, dt, 1);
    for (int l = 0; l < L; l++) {
#define NM(fmt) (snprintf(nm, sizeof nm, fmt, l), nm)
        add(t, &n, NM("layers.%d.attn_norm"), 1, c->dim, 1, dt, 0);
        add(t, &n, NM("layers.%d.wq"), 0, qd, c->dim, dt, 0);
        add(t, &n, NM("layers.%d.wk"), 0, kvd, c->dim, dt, 0);
        add(t, &n, NM("layers.%d.wv"), 0, kvd, c->dim, dt, 0);
        add(t, &n, NM("layers.%d.wo"), 0, c->dim, qd, dt, 0);
        if (c->qkv_bias) {
            add(t, &n, NM("layers.%d.wq_bias"), 2, qd, 1, dt, 0);
            add(t, &n, NM("layers.%d.wk_bias"), 2, kvd, 1, dt, 0);
            add(t, &n, NM("layers.%d.wv_bias"), 2, kvd, 1, dt, 0);
        }
        if (c->qk_norm) {
            add(t, &n, NM("layers.%d.q_norm"), 1, hd, 1, dt, 0);
            add(t, &n, NM("layers.%d.k_norm"), 1, hd, 1, dt, 0);
        }
        add(t, &n, NM("layers.%d.ffn_norm"), 1, c->dim, 1, dt, 0);
        add(t, &n, NM("layers.%d.w1"), 0, c->hidden_dim, c->dim, dt, 0);
        add(t, &n, NM("layers.%d.w2"), 0, c->dim, c->hidden_dim, dt, 0);
        add(t, &n, NM("layers.%d.w3"), 0, c->hidden_dim, c->dim, dt, 0);
#undef NM
    }
    add(t, &n, "final_norm", 1, c->dim, 1, dt, 0);
    if (!c->tied) add(t, &n, "lm_head", 0, c->vocab_size, c->dim, dt, 1);

    /* tokenizer blob: int32 max_len, then per id {float score, int32 len, bytes} */
    size_t tcap = 16 + (size_t)c->vocab_size * 24, tlen = 4;
    uint8_t *tok = ember_xmalloc(tcap, "synth tokenizer");
    int32_t maxlen = 0;
    for (int i = 0; i < c->vocab_size; i++) {
        char piece[32];
        if (i == 0) snprintf(piece, sizeof piece, "<unk>");
        else if (i == 1) snprintf(piece, sizeof piece, "<s>");
        else if (i == 2) snprintf(piece, sizeof piece, "</s>");
        else if (i < 259) snprintf(piece, sizeof piece, "<0x%02X>", i - 3);
        else snprintf(piece, sizeof piece, "t%d", i);
        const int32_t len = (int32_t)strlen(piece);
        const float score = -(float)i;
        if (len > maxlen) maxlen = len;
        memcpy(tok + tlen, &score, 4); memcpy(tok + tlen + 4, &len, 4);
        memcpy(tok + tlen + 8, piece, (size_t)len);
        tlen += 8 + (size_t)len;
    }
    memcpy(tok, &maxlen, 4);

    EmberHeader h;
    memset(&h, 0, sizeof h);
    memcpy(h.magic, "EMBR", 4);
    h.version = EMBER_VERSION;
    h.dim = c->dim; h.hidden_dim = c->hidden_dim; h.n_layers = L;
    h.n_heads = c->n_heads; h.n_kv_heads = c->n_kv_heads; h.head_dim = hd;
    h.vocab_size = c->vocab_size; h.max_seq_len = c->max_seq_len;
    h.rope_theta = c->rope_theta; h.norm_eps = c->norm_eps;
    h.flags = (c->tied ? EMBER_FLAG_TIED_EMBED : 0u) | (c->qk_norm ? EMBER_FLAG_QK_NORM : 0u);
    h.rope_style = c->rope_style;
    h.bos_token_id = 1; h.eos_token_id = 2; h.eos_token_id2 = -1;
    h.n_tensors = n;
    h.tokenizer_type = EMBER_TOK_LLAMA_SP;
    h.default_top_k = 0; h.default_temp = 1.0f; h.default_top_p = 0.9f;
    h.tokenizer_offset = sizeof(EmberHeader);
    h.tokenizer_size = tlen;
    h.tensor_table_offset = up(h.tokenizer_offset + tlen, 8);
    h.tensor_table_size = (uint64_t)n * sizeof(EmberTensor);
    h.header_bytes = up(h.tensor_table_offset + h.tensor_table_size, 64);
    uint64_t cur = h.header_bytes;
    EmberTensor *tab = ember_xcalloc((size_t)n, sizeof(EmberTensor), "synth table");
    for (int i = 0; i < n; i++) {
        cur = up(cur, 64);
        t[i].offset = cur;
        cur += t[i].nbytes;
        memcpy(tab[i].name, t[i].name, sizeof tab[i].name);
        tab[i].dtype = t[i].dtype;
        tab[i].ndim = t[i].ndim;
        tab[i].shape[0] = t[i].rows;
        tab[i].shape[1] = t[i].ndim == 2 ? t[i].cols : 1;
        tab[i].shape[2] = tab[i].shape[3] = 1;
        tab[i].offset = t[i].offset;
        tab[i].nbytes = t[i].nbytes;
    }
    FILE *f = fopen(path, "wb");
    if (!f) { free(t); free(tok); free(tab); return 1; }
    int rc = 0;
    uint64_t at = 0;
    static const uint8_t zeros[64];
#define PUT(p, len) do { if (fwrite((p), 1, (len), f) != (size_t)(len)) rc = 1; at += (len); } while (0)
#define PAD_TO(o)   do { while (at < (o)) { uint64_t k_ = (o) - at > 64 ? 64 : (o) - at; PUT(zeros, k_); } } while (0)
    PUT(&h, sizeof h);
    PUT(tok, tlen);
    PAD_TO(h.tensor_table_offset);
    PUT(tab, sizeof(EmberTensor) * (size_t)n);
    PAD_TO(h.header_bytes);
    const int nth = c->threads > 0 ? c->threads : 8;
    for (int i = 0; i < n && !rc; i++) {
        PAD_TO(t[i].offset);
        uint8_t *buf = ember_xmalloc(t[i].nbytes, "synth tensor");
        fill_tensor(&t[i], c->seed, c->std, buf, nth);
        PUT(buf, t[i].nbytes);
        free(buf);
    }
#undef PUT
#undef PAD_TO
    if (fclose(f) != 0) rc = 1;
    free(t); free(tok); free(tab);
    return rc;
}
