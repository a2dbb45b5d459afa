/* oracle.c — CPU restatement of emberllm's token loop.  TEST INFRASTRUCTURE:
 * the checker for the GPU path, loaded only by tests/, the smoke check and
 * bench.py's CPU-baseline leg.  Nothing in the product links it.
 *
 * Every function restates the reference operation for operation, in the
 * same evaluation order, so that with -O2 -fno-fast-math -ffp-contract=off
 * its outputs equal the reference's deterministic build bit for bit.
 *
 * How each part is pinned (tests/test_oracle.py):
 *   f16 conversions ........ exhaustive over all 65,536 halves vs numpy, and
 *                            float->half RNE vs numpy on 2M random floats
 *                            plus every boundary case (subnormals, ties, inf)
 *   Q8_0 / Q4_0 quantizers . golden rows quantized by the compiled reference,
 *                            plus closed-form invariants (max element -> +-127
 *                            or nibble 0, zero block -> zero, clamp, ties)
 *   block dots ............. brute-force int64 on random blocks
 *   matmul ................. float64 numpy bound + reference goldens
 *   forward / prefill ...... full-logit goldens of the compiled reference on
 *                            seeded tiny models covering every variant
 *                            (tests/golden, npz files), and the invariant that
 *                            prefill's last logits equal sequential forwards
 *   sampler ................ RNG sequence from the seed, hand-computed
 *                            top-k/top-p cuts, and reference goldens
 * No function is left unpinned.
 */
#define _DEFAULT_SOURCE
#include "oracle.h"

#include <fcntl.h>
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

enum { DT_F32 = 0, DT_Q8 = 1, DT_Q4 = 2 };
enum { ROPE_NEOX = 1 };
#define QB 32
#define PAR_FLOOR 32768L

#pragma pack(push, 1)
typedef struct { uint16_t d; int8_t q[QB]; } Q8Blk;      /* 34 B */
typedef struct { uint16_t d; uint8_t q[QB / 2]; } Q4Blk; /* 18 B */
typedef struct {
    char magic[4]; uint32_t version; uint64_t header_bytes;
    int32_t dim, hidden, n_layers, n_heads, n_kv, head_dim, vocab, max_seq;
    float theta, eps; uint32_t flags; int32_t rope_style;
    int32_t bos, eos, eos2, n_tensors, tok_type, top_k; float temp, top_p;
    uint64_t tok_off, tok_size, table_off, table_size; uint8_t pad[128];
} Hdr;
typedef struct {
    char name[48]; int32_t dtype, ndim, shape[4]; uint64_t offset, nbytes;
} TEnt;
#pragma pack(pop)

static void fatal(const char *msg) { fprintf(stderr, "oracle: %s\n", msg); exit(1); }
static void *xalloc(size_t n) { void *p = malloc(n ? n : 1); if (!p) fatal("out of memory"); return p; }

/* ------------------------------------------------------------------------- */
/* thread pool (restates src/threads.c:61-104: static slices, main runs 0)    */
/* ------------------------------------------------------------------------- */
typedef void (*RangeFn)(void *, int, int);
static int g_nth = 1;
static pthread_t *g_workers;
static pthread_mutex_t g_mu = PTHREAD_MUTEX_INITIALIZER;
static pthread_cond_t g_go = PTHREAD_COND_INITIALIZER, g_fin = PTHREAD_COND_INITIALIZER;
static unsigned long g_round;
static int g_finished, g_quit;
static RangeFn g_job;
static void *g_arg;
static int g_len;

static void slice(int id) {
    long lo = (long)id * g_len / g_nth, hi = (long)(id + 1) * g_len / g_nth;
    if (hi > lo) g_job(g_arg, (int)lo, (int)hi);
}

static void *worker(void *p) {
    int id = (int)(long)p;
    unsigned long seen = 0;
    for (;;) {
        pthread_mutex_lock(&g_mu);
        while (g_round == seen && !g_quit) pthread_cond_wait(&g_go, &g_mu);
        if (g_quit) { pthread_mutex_unlock(&g_mu); return NULL; }
        seen = g_round;
        pthread_mutex_unlock(&g_mu);
        slice(id);
        pthread_mutex_lock(&g_mu);
        if (++g_finished == g_nth - 1) pthread_cond_signal(&g_fin);
        pthread_mutex_unlock(&g_mu);
    }
}

void orc_threads_init(int n) {
    orc_threads_shutdown();
    g_nth = n < 1 ? 1 : n;
    g_round = 0; g_finished = 0; g_quit = 0;
    if (g_nth == 1) return;
    g_workers = xalloc(sizeof(pthread_t) * (size_t)(g_nth - 1));
    for (int i = 1; i < g_nth; i++) pthread_create(&g_workers[i - 1], NULL, worker, (void *)(long)i);
}

void orc_threads_shutdown(void) {
    if (g_nth <= 1) { g_nth = 1; return; }
    pthread_mutex_lock(&g_mu);
    g_quit = 1;
    pthread_cond_broadcast(&g_go);
    pthread_mutex_unlock(&g_mu);
    for (int i = 0; i < g_nth - 1; i++) pthread_join(g_workers[i], NULL);
    free(g_workers); g_workers = NULL; g_nth = 1;
}

static int want_par(long work) { return g_nth > 1 && work >= PAR_FLOOR * g_nth; }

static void par_for(RangeFn fn, void *arg, int n) {
    if (g_nth <= 1) { fn(arg, 0, n); return; }
    pthread_mutex_lock(&g_mu);
    g_job = fn; g_arg = arg; g_len = n; g_finished = 0; g_round++;
    pthread_cond_broadcast(&g_go);
    pthread_mutex_unlock(&g_mu);
    slice(0);
    pthread_mutex_lock(&g_mu);
    while (g_finished != g_nth - 1) pthread_cond_wait(&g_fin, &g_mu);
    pthread_mutex_unlock(&g_mu);
}

/* ------------------------------------------------------------------------- */
/* half precision (src/kernels.c:25-68)                                      */
/* ------------------------------------------------------------------------- */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    int e = (h >> 10) & 31;
    uint32_t m = h & 1023u, bits;
    if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        bits = sign | ((uint32_t)(e + 112) << 23) | (m << 13);
    } else if (m == 0) {
        bits = sign;
    } else { /* subnormal: renormalise */
        int k = 0;
        while (!(m & 1024u)) { m <<= 1; k++; }
        bits = sign | ((uint32_t)(113 - k) << 23) | ((m & 1023u) << 13);
    }
    float f; memcpy(&f, &bits, 4);
    return f;
}

/* round-to-nearest-even; NaN maps to infinity like the reference's scalar
 * converter (kernels.c:61-62 sends every exponent >= 31 to inf). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t u; memcpy(&u, &f, 4);
    uint16_t s = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    int e = (int)(a >> 23) - 112;
    if (e >= 31) return (uint16_t)(s | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return s;
        uint32_t m = (a & 0x7fffffu) | 0x800000u;
        int sh = 14 - e;
        uint32_t q = m >> sh, r = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (r > half || (r == half && (q & 1u))) q++;
        return (uint16_t)(s | q);
    }
    uint32_t q = ((uint32_t)e << 10) | ((a >> 13) & 1023u);
    uint32_t r = a & 0x1fffu;
    if (r > 0x1000u || (r == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(s | q);
}

/* ------------------------------------------------------------------------- */
/* quantizers (src/kernels.c:73-115)                                         */
/* ------------------------------------------------------------------------- */
void orc_quantize_q8_0(const float *x, void *out, int n) {
    Q8Blk *o = out;
    for (int b = 0; b < n / QB; b++) {
        const float *v = x + (size_t)b * QB;
        float amax = 0.0f;
        for (int i = 0; i < QB; i++) { float a = fabsf(v[i]); if (a > amax) amax = a; }
        float d = amax / 127.0f;
        float inv = d > 0.0f ? 1.0f / d : 0.0f;
        o[b].d = orc_f32_to_f16(d);
        for (int i = 0; i < QB; i++) {
            int q = (int)lroundf(v[i] * inv);   /* as kernels.c:86: LONG_MIN (NaN, inf) -> 0 */
            o[b].q[i] = (int8_t)(q > 127 ? 127 : (q < -127 ? -127 : q));
        }
    }
}

void orc_quantize_q4_0(const float *x, void *out, int n) {
    Q4Blk *o = out;
    for (int b = 0; b < n / QB; b++) {
        const float *v = x + (size_t)b * QB;
        float amax = 0.0f, peak = 0.0f;   /* peak keeps the sign of the max-|.| element */
        for (int i = 0; i < QB; i++) { float a = fabsf(v[i]); if (a > amax) { amax = a; peak = v[i]; } }
        float d = peak / -8.0f;
        float inv = d != 0.0f ? 1.0f / d : 0.0f;
        o[b].d = orc_f32_to_f16(d);
        for (int i = 0; i < QB / 2; i++) {
            int lo = (int)(v[i] * inv + 8.5f), hi = (int)(v[i + QB / 2] * inv + 8.5f);
            lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
            hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
            o[b].q[i] = (uint8_t)(lo | (hi << 4));
        }
    }
}

/* ------------------------------------------------------------------------- */
/* dots and matmul (src/kernels.c:120-264, scalar paths)                     */
/* ------------------------------------------------------------------------- */
int32_t orc_block_dot_q8(const void *wb, const void *xb) {
    const Q8Blk *w = wb, *x = xb;
    int32_t acc = 0;
    for (int i = 0; i < QB; i++) acc += (int32_t)w->q[i] * (int32_t)x->q[i];
    return acc;
}

int32_t orc_block_dot_q4(const void *wb, const void *xb) {
    const Q4Blk *w = wb; const Q8Blk *x = xb;
    int32_t acc = 0;
    for (int i = 0; i < QB / 2; i++) {
        int lo = (int)(w->q[i] & 15) - 8, hi = (int)(w->q[i] >> 4) - 8;
        acc += lo * (int32_t)x->q[i] + hi * (int32_t)x->q[i + QB / 2];
    }
    return acc;
}

static float row_dot(const void *wrow, const void *xv, int dtype, int n_in) {
    float s = 0.0f;
    if (dtype == DT_F32) {
        const float *w = wrow, *x = xv;
        for (int i = 0; i < n_in; i++) s += w[i] * x[i];
    } else if (dtype == DT_Q8) {
        const Q8Blk *w = wrow, *x = xv;
        for (int b = 0; b < n_in / QB; b++)
            s += (float)orc_block_dot_q8(&w[b], &x[b]) * orc_f16_to_f32(w[b].d) * orc_f16_to_f32(x[b].d);
    } else {
        const Q4Blk *w = wrow; const Q8Blk *x = xv;
        for (int b = 0; b < n_in / QB; b++)
            s += (float)orc_block_dot_q4(&w[b], &x[b]) * orc_f16_to_f32(w[b].d) * orc_f16_to_f32(x[b].d);
    }
    return s;
}

static size_t row_bytes(int dtype, int n_in) {
    return dtype == DT_F32 ? (size_t)n_in * 4 : (size_t)(n_in / QB) * (dtype == DT_Q8 ? 34 : 18);
}

typedef struct { float *out; const void *x; const uint8_t *w; int dtype, n_in, d_out, B; } MM;

static void mm_job(void *p, int r0, int r1) {
    MM *c = p;
    size_t rb = row_bytes(c->dtype, c->n_in);
    size_t xb = c->dtype == DT_F32 ? (size_t)c->n_in * 4 : (size_t)(c->n_in / QB) * 34;
    for (int r = r0; r < r1; r++)
        for (int b = 0; b < c->B; b++)
            c->out[(size_t)b * c->d_out + r] =
                row_dot(c->w + (size_t)r * rb, (const uint8_t *)c->x + (size_t)b * xb, c->dtype, c->n_in);
}

static void matmul_b(float *out, const float *x, const void *w, int dtype, int n_in, int d_out,
                     int B, Q8Blk *scratch) {
    const void *xin = x;
    if (dtype != DT_F32) {
        for (int b = 0; b < B; b++)
            orc_quantize_q8_0(x + (size_t)b * n_in, scratch + (size_t)b * (n_in / QB), n_in);
        xin = scratch;
    }
    MM c = { out, xin, w, dtype, n_in, d_out, B };
    if (want_par((long)n_in * d_out * B)) par_for(mm_job, &c, d_out);
    else mm_job(&c, 0, d_out);
}

void orc_matmul(float *out, const float *x, const void *w, int dtype, int n_in, int d_out) {
    Q8Blk *s = xalloc(sizeof(Q8Blk) * (size_t)(n_in / QB + 1));
    matmul_b(out, x, w, dtype, n_in, d_out, 1, s);
    free(s);
}

void orc_matmul_batch(float *out, const float *x, const void *w, int dtype, int n_in, int d_out, int B) {
    Q8Blk *s = xalloc(sizeof(Q8Blk) * (size_t)B * (n_in / QB + 1));
    matmul_b(out, x, w, dtype, n_in, d_out, B, s);
    free(s);
}

/* ------------------------------------------------------------------------- */
/* model file                                                                */
/* ------------------------------------------------------------------------- */
struct OrcModel { int fd; size_t size; const uint8_t *base; const Hdr *h; const TEnt *tab; };

OrcModel *orc_model_open(const char *path) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) return NULL;
    struct stat st;
    if (fstat(fd, &st) != 0 || (size_t)st.st_size < sizeof(Hdr)) { close(fd); return NULL; }
    void *p = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) { close(fd); return NULL; }
    OrcModel *m = xalloc(sizeof *m);
    m->fd = fd; m->size = (size_t)st.st_size; m->base = p; m->h = p;
    if (memcmp(m->h->magic, "EMBR", 4) != 0 || m->h->table_off + m->h->table_size > m->size) {
        munmap(p, m->size); close(fd); free(m); return NULL;
    }
    m->tab = (const TEnt *)(m->base + m->h->table_off);
    return m;
}

void orc_model_close(OrcModel *m) {
    if (!m) return;
    munmap((void *)m->base, m->size); close(m->fd); free(m);
}

static const TEnt *find(const OrcModel *m, const char *name) {
    for (int i = 0; i < m->h->n_tensors; i++)
        if (strncmp(m->tab[i].name, name, 48) == 0) return &m->tab[i];
    return NULL;
}

typedef struct { const void *p; int dt; } W;

static W weight(const OrcModel *m, const char *fmt, int l) {
    char nm[64];
    if (l >= 0) snprintf(nm, sizeof nm, fmt, l); else snprintf(nm, sizeof nm, "%s", fmt);
    const TEnt *t = find(m, nm);
    W w = { NULL, DT_F32 };
    if (t) { w.p = m->base + t->offset; w.dt = t->dtype; }
    return w;
}

/* ------------------------------------------------------------------------- */
/* state (src/model.c:16-35, 120-205)                                        */
/* ------------------------------------------------------------------------- */
typedef struct {
    W wq, wk, wv, wo, w1, w2, w3;
    const float *an, *fn, *qn, *kn, *bq, *bk, *bv;
} Layer;

struct OrcState {
    int dim, hid, L, nh, nkv, hd, kvd, V, ctx, qk, rope_style, f16kv;
    float theta, eps;
    W emb, head; const float *fnorm;
    Layer *ly;
    float *x, *xb, *xb2, *hb, *hb2, *q, *k, *v, *att, *logits;
    void *kc, *vc;
    Q8Blk *xq;
    int cap_layer;        /* orc_capture: layer whose vectors are copied out, or -1 */
    float *cap[6];
};

OrcState *orc_state_new(OrcModel *m, int ctx_len, int kv_fp16) {
    const Hdr *h = m->h;
    OrcState *s = calloc(1, sizeof *s);
    s->dim = h->dim; s->hid = h->hidden; s->L = h->n_layers; s->nh = h->n_heads;
    s->nkv = h->n_kv; s->hd = h->head_dim; s->kvd = h->n_kv * h->head_dim; s->V = h->vocab;
    s->theta = h->theta; s->eps = h->eps; s->rope_style = h->rope_style;
    s->qk = (h->flags & 2u) != 0; s->f16kv = kv_fp16 != 0;
    s->ctx = (ctx_len > 0 && ctx_len < h->max_seq) ? ctx_len : h->max_seq;
    s->ly = calloc((size_t)s->L, sizeof(Layer));
    for (int l = 0; l < s->L; l++) {
        Layer *y = &s->ly[l];
        y->wq = weight(m, "layers.%d.wq", l); y->wk = weight(m, "layers.%d.wk", l);
        y->wv = weight(m, "layers.%d.wv", l); y->wo = weight(m, "layers.%d.wo", l);
        y->w1 = weight(m, "layers.%d.w1", l); y->w2 = weight(m, "layers.%d.w2", l);
        y->w3 = weight(m, "layers.%d.w3", l);
        y->an = weight(m, "layers.%d.attn_norm", l).p; y->fn = weight(m, "layers.%d.ffn_norm", l).p;
        y->qn = weight(m, "layers.%d.q_norm", l).p;    y->kn = weight(m, "layers.%d.k_norm", l).p;
        y->bq = weight(m, "layers.%d.wq_bias", l).p;   y->bk = weight(m, "layers.%d.wk_bias", l).p;
        y->bv = weight(m, "layers.%d.wv_bias", l).p;
        if (!y->wq.p || !y->wk.p || !y->wv.p || !y->wo.p || !y->w1.p || !y->w2.p || !y->w3.p || !y->an || !y->fn)
            fatal("missing layer tensor");
    }
    s->emb = weight(m, "tok_embeddings", -1);
    s->fnorm = weight(m, "final_norm", -1).p;
    s->head = (h->flags & 1u) ? s->emb : weight(m, "lm_head", -1);
    if (!s->emb.p || !s->fnorm || !s->head.p) fatal("missing global tensor");

    int qd = s->nh * s->hd, wide = s->hid > s->dim ? s->hid : s->dim;
    if (qd > wide) wide = qd;
    s->x = xalloc(4 * (size_t)s->dim);
    s->xb = xalloc(4 * (size_t)(qd > s->dim ? qd : s->dim));
    s->xb2 = xalloc(4 * (size_t)s->dim);
    s->hb = xalloc(4 * (size_t)s->hid); s->hb2 = xalloc(4 * (size_t)s->hid);
    s->q = xalloc(4 * (size_t)qd);
    s->k = xalloc(4 * (size_t)s->kvd); s->v = xalloc(4 * (size_t)s->kvd);
    s->att = xalloc(4 * (size_t)s->nh * s->ctx);
    s->logits = calloc((size_t)s->V, 4);
    size_t kvb = (size_t)s->L * s->ctx * s->kvd * (s->f16kv ? 2 : 4);
    s->kc = calloc(1, kvb); s->vc = calloc(1, kvb);
    if (!s->kc || !s->vc || !s->logits) fatal("out of memory (kv)");
    s->xq = xalloc(sizeof(Q8Blk) * (size_t)(wide / QB + 1));
    s->cap_layer = -1;
    return s;
}

void orc_capture(OrcState *s, int layer, float *const *slots) {
    s->cap_layer = layer;
    for (int i = 0; i < 6; i++) s->cap[i] = slots ? slots[i] : NULL;
}

/* copy n floats to capture slot i (row `row` of width n) when layer l is captured */
static void cap_put(OrcState *s, int l, int i, size_t row, const float *src, size_t n) {
    if (l == s->cap_layer && s->cap[i]) memcpy(s->cap[i] + row * n, src, 4 * n);
}

void orc_state_free(OrcState *s) {
    if (!s) return;
    free(s->ly); free(s->x); free(s->xb); free(s->xb2); free(s->hb); free(s->hb2);
    free(s->q); free(s->k); free(s->v); free(s->att); free(s->logits);
    free(s->kc); free(s->vc); free(s->xq); free(s);
}

int orc_state_ctx(const OrcState *s) { return s->ctx; }
void *orc_kv_cache(OrcState *s, int which) { return which ? s->vc : s->kc; }
uint64_t orc_kv_bytes(const OrcState *s) { return (uint64_t)s->L * s->ctx * s->kvd * (s->f16kv ? 2 : 4); }

/* ------------------------------------------------------------------------- */
/* forward-pass pieces (src/model.c:39-100)                                  */
/* ------------------------------------------------------------------------- */
static void norm(float *out, const float *x, const float *w, int n, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    float r = 1.0f / sqrtf(ss / n + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * r * w[i];
}

static void rotate(float *v, int n, int hd, int pos, float theta, int style) {
    for (int base = 0; base < n; base += hd)
        for (int i = 0; i < hd / 2; i++) {
            float fr = 1.0f / powf(theta, (float)(2 * i) / hd);
            float ang = pos * fr;
            float c = cosf(ang), sn = sinf(ang);
            int a = style == ROPE_NEOX ? base + i : base + 2 * i;
            int b = style == ROPE_NEOX ? base + i + hd / 2 : base + 2 * i + 1;
            float v0 = v[a], v1 = v[b];
            v[a] = v0 * c - v1 * sn;
            v[b] = v0 * sn + v1 * c;
        }
}

static void store_kv(OrcState *s, int l, int pos, const float *k, const float *v) {
    size_t off = ((size_t)l * s->ctx + pos) * s->kvd;
    if (s->f16kv) {
        uint16_t *kc = (uint16_t *)s->kc + off, *vc = (uint16_t *)s->vc + off;
        for (int i = 0; i < s->kvd; i++) { kc[i] = orc_f32_to_f16(k[i]); vc[i] = orc_f32_to_f16(v[i]); }
    } else {
        memcpy((float *)s->kc + off, k, 4 * (size_t)s->kvd);
        memcpy((float *)s->vc + off, v, 4 * (size_t)s->kvd);
    }
}

static void embed(const OrcState *s, int tok, float *out) {
    if (s->emb.dt == DT_F32) {
        memcpy(out, (const float *)s->emb.p + (size_t)tok * s->dim, 4 * (size_t)s->dim);
    } else if (s->emb.dt == DT_Q8) {
        const Q8Blk *row = (const Q8Blk *)s->emb.p + (size_t)tok * (s->dim / QB);
        for (int b = 0; b < s->dim / QB; b++) {
            float d = orc_f16_to_f32(row[b].d);
            for (int i = 0; i < QB; i++) out[b * QB + i] = row[b].q[i] * d;
        }
    } else {
        fatal("embedding must be F32 or Q8_0");
    }
}

/* attention over positions 0..pos of layer l (src/model.c:207-278) */
typedef struct { OrcState *s; const float *q; float *out; int l, pos; } AttJob;

static float kv_at(const OrcState *s, const void *base, size_t i) {
    return s->f16kv ? orc_f16_to_f32(((const uint16_t *)base)[i]) : ((const float *)base)[i];
}

static void att_heads(void *p, int h0, int h1) {
    AttJob *j = p; OrcState *s = j->s;
    int hd = s->hd, kvd = s->kvd, grp = s->nh / s->nkv;
    float scale = 1.0f / sqrtf((float)hd);
    size_t lbase = (size_t)j->l * s->ctx * kvd;
    for (int h = h0; h < h1; h++) {
        const float *qh = j->q + (size_t)h * hd;
        float *sc = s->att + (size_t)h * s->ctx, *o = j->out + (size_t)h * hd;
        size_t hoff = (size_t)(h / grp) * hd;
        for (int i = 0; i < hd; i++) o[i] = 0.0f;
        for (int t = 0; t <= j->pos; t++) {
            size_t row = lbase + (size_t)t * kvd + hoff;
            float a = 0.0f;
            for (int i = 0; i < hd; i++) a += qh[i] * kv_at(s, s->kc, row + i);
            sc[t] = a * scale;
        }
        /* softmax (src/model.c:57-64) */
        float mx = sc[0];
        for (int t = 1; t <= j->pos; t++) if (sc[t] > mx) mx = sc[t];
        float sum = 0.0f;
        for (int t = 0; t <= j->pos; t++) { sc[t] = expf(sc[t] - mx); sum += sc[t]; }
        float inv = 1.0f / sum;
        for (int t = 0; t <= j->pos; t++) sc[t] *= inv;
        for (int t = 0; t <= j->pos; t++) {
            size_t row = lbase + (size_t)t * kvd + hoff;
            float p = sc[t];
            for (int i = 0; i < hd; i++) o[i] += p * kv_at(s, s->vc, row + i);
        }
    }
}

static void attend(OrcState *s, const float *q, float *out, int l, int pos) {
    AttJob j = { s, q, out, l, pos };
    if (want_par((long)s->nh * (pos + 1) * s->hd)) par_for(att_heads, &j, s->nh);
    else att_heads(&j, 0, s->nh);
}

static void add_vec(float *y, const float *b, int n) { for (int i = 0; i < n; i++) y[i] += b[i]; }

/* ------------------------------------------------------------------------- */
/* ember_forward (src/model.c:362-414)                                       */
/* ------------------------------------------------------------------------- */
float *orc_forward(OrcState *s, int tok, int pos) {
    if (tok < 0 || tok >= s->V) fatal("token out of range");
    if (pos < 0 || pos >= s->ctx) fatal("position out of range");
    int dim = s->dim, hd = s->hd, qd = s->nh * s->hd, kvd = s->kvd;
    embed(s, tok, s->x);
    for (int l = 0; l < s->L; l++) {
        Layer *y = &s->ly[l];
        cap_put(s, l, 0, 0, s->x, (size_t)dim);
        norm(s->xb, s->x, y->an, dim, s->eps);
        matmul_b(s->q, s->xb, y->wq.p, y->wq.dt, dim, qd, 1, s->xq);
        matmul_b(s->k, s->xb, y->wk.p, y->wk.dt, dim, kvd, 1, s->xq);
        matmul_b(s->v, s->xb, y->wv.p, y->wv.dt, dim, kvd, 1, s->xq);
        if (y->bq) add_vec(s->q, y->bq, qd);
        if (y->bk) add_vec(s->k, y->bk, kvd);
        if (y->bv) add_vec(s->v, y->bv, kvd);
        if (l == s->cap_layer && s->cap[1]) {   /* raw q|k|v */
            memcpy(s->cap[1], s->q, 4 * (size_t)qd);
            memcpy(s->cap[1] + qd, s->k, 4 * (size_t)kvd);
            memcpy(s->cap[1] + qd + kvd, s->v, 4 * (size_t)kvd);
        }
        if (s->qk && y->qn) {
            for (int h = 0; h < s->nh; h++) norm(s->q + h * hd, s->q + h * hd, y->qn, hd, s->eps);
            for (int h = 0; h < s->nkv; h++) norm(s->k + h * hd, s->k + h * hd, y->kn, hd, s->eps);
        }
        rotate(s->q, qd, hd, pos, s->theta, s->rope_style);
        rotate(s->k, kvd, hd, pos, s->theta, s->rope_style);
        store_kv(s, l, pos, s->k, s->v);
        attend(s, s->q, s->xb, l, pos);
        cap_put(s, l, 2, 0, s->xb, (size_t)qd);
        matmul_b(s->xb2, s->xb, y->wo.p, y->wo.dt, qd, dim, 1, s->xq);
        add_vec(s->x, s->xb2, dim);
        cap_put(s, l, 3, 0, s->x, (size_t)dim);
        norm(s->xb, s->x, y->fn, dim, s->eps);
        matmul_b(s->hb, s->xb, y->w1.p, y->w1.dt, dim, s->hid, 1, s->xq);
        matmul_b(s->hb2, s->xb, y->w3.p, y->w3.dt, dim, s->hid, 1, s->xq);
        for (int i = 0; i < s->hid; i++) { float g = s->hb[i]; s->hb[i] = g / (1.0f + expf(-g)) * s->hb2[i]; }
        cap_put(s, l, 4, 0, s->hb, (size_t)s->hid);
        matmul_b(s->xb, s->hb, y->w2.p, y->w2.dt, s->hid, dim, 1, s->xq);
        add_vec(s->x, s->xb, dim);
        cap_put(s, l, 5, 0, s->x, (size_t)dim);
    }
    norm(s->x, s->x, s->fnorm, dim, s->eps);
    matmul_b(s->logits, s->x, s->head.p, s->head.dt, dim, s->V, 1, s->xq);
    return s->logits;
}

/* ------------------------------------------------------------------------- */
/* ember_prefill (src/model.c:283-360)                                       */
/* ------------------------------------------------------------------------- */
float *orc_prefill(OrcState *s, const int *ids, int n, int start) {
    if (n <= 0) return s->logits;
    int dim = s->dim, hd = s->hd, qd = s->nh * s->hd, kvd = s->kvd, hid = s->hid;
    int wide = dim > hid ? dim : hid;
    if (qd > wide) wide = qd;
    size_t N = (size_t)n;
    float *X = xalloc(4 * N * dim), *Xn = xalloc(4 * N * dim), *T = xalloc(4 * N * dim);
    float *Q = xalloc(4 * N * qd), *K = xalloc(4 * N * kvd), *Vv = xalloc(4 * N * kvd);
    float *O = xalloc(4 * N * qd), *H1 = xalloc(4 * N * hid), *H2 = xalloc(4 * N * hid);
    Q8Blk *sq = xalloc(sizeof(Q8Blk) * N * (size_t)(wide / QB + 1));
    for (int b = 0; b < n; b++) {
        if (ids[b] < 0 || ids[b] >= s->V) fatal("token out of range");
        embed(s, ids[b], X + (size_t)b * dim);
    }
    for (int l = 0; l < s->L; l++) {
        Layer *y = &s->ly[l];
        for (int b = 0; b < n; b++) cap_put(s, l, 0, (size_t)b, X + (size_t)b * dim, (size_t)dim);
        for (int b = 0; b < n; b++) norm(Xn + (size_t)b * dim, X + (size_t)b * dim, y->an, dim, s->eps);
        matmul_b(Q, Xn, y->wq.p, y->wq.dt, dim, qd, n, sq);
        matmul_b(K, Xn, y->wk.p, y->wk.dt, dim, kvd, n, sq);
        matmul_b(Vv, Xn, y->wv.p, y->wv.dt, dim, kvd, n, sq);
        for (int b = 0; b < n; b++) {
            if (y->bq) add_vec(Q + (size_t)b * qd, y->bq, qd);
            if (y->bk) add_vec(K + (size_t)b * kvd, y->bk, kvd);
            if (y->bv) add_vec(Vv + (size_t)b * kvd, y->bv, kvd);
        }
        if (l == s->cap_layer && s->cap[1])   /* raw q|k|v rows */
            for (int b = 0; b < n; b++) {
                float *r = s->cap[1] + (size_t)b * (qd + 2 * kvd);
                memcpy(r, Q + (size_t)b * qd, 4 * (size_t)qd);
                memcpy(r + qd, K + (size_t)b * kvd, 4 * (size_t)kvd);
                memcpy(r + qd + kvd, Vv + (size_t)b * kvd, 4 * (size_t)kvd);
            }
        for (int b = 0; b < n; b++) {
            float *qb = Q + (size_t)b * qd, *kb = K + (size_t)b * kvd;
            if (s->qk && y->qn) {
                for (int h = 0; h < s->nh; h++) norm(qb + h * hd, qb + h * hd, y->qn, hd, s->eps);
                for (int h = 0; h < s->nkv; h++) norm(kb + h * hd, kb + h * hd, y->kn, hd, s->eps);
            }
            rotate(qb, qd, hd, start + b, s->theta, s->rope_style);
            rotate(kb, kvd, hd, start + b, s->theta, s->rope_style);
            store_kv(s, l, start + b, kb, Vv + (size_t)b * kvd);
        }
        for (int b = 0; b < n; b++) attend(s, Q + (size_t)b * qd, O + (size_t)b * qd, l, start + b);
        for (int b = 0; b < n; b++) cap_put(s, l, 2, (size_t)b, O + (size_t)b * qd, (size_t)qd);
        matmul_b(T, O, y->wo.p, y->wo.dt, qd, dim, n, sq);
        for (size_t i = 0; i < N * dim; i++) X[i] += T[i];
        for (int b = 0; b < n; b++) cap_put(s, l, 3, (size_t)b, X + (size_t)b * dim, (size_t)dim);
        for (int b = 0; b < n; b++) norm(Xn + (size_t)b * dim, X + (size_t)b * dim, y->fn, dim, s->eps);
        matmul_b(H1, Xn, y->w1.p, y->w1.dt, dim, hid, n, sq);
        matmul_b(H2, Xn, y->w3.p, y->w3.dt, dim, hid, n, sq);
        if (l == s->cap_layer && s->cap[4])   /* w1 | w3 products before SwiGLU */
            for (int b = 0; b < n; b++) {
                memcpy(s->cap[4] + (size_t)b * 2 * hid, H1 + (size_t)b * hid, 4 * (size_t)hid);
                memcpy(s->cap[4] + (size_t)b * 2 * hid + hid, H2 + (size_t)b * hid, 4 * (size_t)hid);
            }
        for (size_t i = 0; i < N * hid; i++) { float g = H1[i]; H1[i] = g / (1.0f + expf(-g)) * H2[i]; }
        matmul_b(T, H1, y->w2.p, y->w2.dt, hid, dim, n, sq);
        for (size_t i = 0; i < N * dim; i++) X[i] += T[i];
        for (int b = 0; b < n; b++) cap_put(s, l, 5, (size_t)b, X + (size_t)b * dim, (size_t)dim);
    }
    norm(s->x, X + (size_t)(n - 1) * dim, s->fnorm, dim, s->eps);
    matmul_b(s->logits, s->x, s->head.p, s->head.dt, dim, s->V, 1, s->xq);
    free(X); free(Xn); free(T); free(Q); free(K); free(Vv); free(O); free(H1); free(H2); free(sq);
    return s->logits;
}

/* ------------------------------------------------------------------------- */
/* sampler (src/sample.c:17-175)                                             */
/* ------------------------------------------------------------------------- */
void orc_sampler_init(OrcSampler *s, float temp, float top_p, int top_k, uint64_t seed) {
    memset(s, 0, sizeof *s);
    s->temperature = temp; s->top_p = top_p; s->top_k = top_k;
    s->repeat_penalty = 1.0f;
    s->rng_state = seed ? seed : 0x9E3779B97F4A7C15ULL;
}

void orc_sampler_set_penalties(OrcSampler *s, float rp, int last_n, float pres, float freq, float min_p) {
    s->repeat_penalty = rp; s->presence_penalty = pres; s->frequency_penalty = freq;
    s->min_p = min_p; s->repeat_last_n = last_n;
    int need = last_n > 0 && (rp != 1.0f || pres != 0.0f || freq != 0.0f);
    if (need) {
        if (s->hist_cap != last_n) {
            int *p = realloc(s->history, sizeof(int) * (size_t)last_n);
            if (!p) fatal("out of memory (history)");
            s->history = p; s->hist_cap = last_n;
        }
    } else {
        free(s->history); s->history = NULL; s->hist_cap = 0;
    }
    s->hist_len = s->hist_pos = 0;
}

void orc_sampler_accept(OrcSampler *s, int token) {
    if (!s->history || s->hist_cap == 0) return;
    s->history[s->hist_pos] = token;
    s->hist_pos = (s->hist_pos + 1) % s->hist_cap;
    if (s->hist_len < s->hist_cap) s->hist_len++;
}

void orc_sampler_free(OrcSampler *s) {
    free(s->history); s->history = NULL; s->hist_cap = s->hist_len = s->hist_pos = 0;
}

uint32_t orc_rng_u32(OrcSampler *s) {
    uint64_t x = s->rng_state;
    x ^= x >> 12; x ^= x << 25; x ^= x >> 27;
    s->rng_state = x;
    return (uint32_t)((x * 0x2545F4914F6CDD1DULL) >> 32);
}

typedef struct { float p; int i; } Cand;

static int by_prob_desc(const void *a, const void *b) {
    float x = ((const Cand *)a)->p, y = ((const Cand *)b)->p;
    return (x < y) - (x > y);
}

static int first_max(const float *v, int n) {
    int best = 0;
    for (int i = 1; i < n; i++) if (v[i] > v[best]) best = i;
    return best;
}

int orc_sample(OrcSampler *s, float *logits, int n) {
    /* penalties (src/sample.c:76-96) */
    if (s->history && s->hist_len > 0) {
        int rep = s->repeat_penalty != 1.0f, fr = s->frequency_penalty != 0.0f, pr = s->presence_penalty != 0.0f;
        if (rep || fr || pr)
            for (int i = 0; i < s->hist_len; i++) {
                int t = s->history[i];
                if (t < 0 || t >= n) continue;
                int seen = 0;
                for (int j = 0; j < i; j++) if (s->history[j] == t) { seen = 1; break; }
                if (!seen) {
                    if (rep) logits[t] = logits[t] > 0.0f ? logits[t] / s->repeat_penalty : logits[t] * s->repeat_penalty;
                    if (pr) logits[t] -= s->presence_penalty;
                }
                if (fr) logits[t] -= s->frequency_penalty;
            }
    }
    if (s->temperature <= 0.0f) {
        int c = first_max(logits, n);
        orc_sampler_accept(s, c);
        return c;
    }
    for (int i = 0; i < n; i++) logits[i] /= s->temperature;
    float mx = logits[first_max(logits, n)], sum = 0.0f;
    for (int i = 0; i < n; i++) { logits[i] = expf(logits[i] - mx); sum += logits[i]; }
    for (int i = 0; i < n; i++) logits[i] /= sum;
    Cand *c = xalloc(sizeof(Cand) * (size_t)n);
    for (int i = 0; i < n; i++) { c[i].p = logits[i]; c[i].i = i; }
    qsort(c, (size_t)n, sizeof(Cand), by_prob_desc);
    int m = n;
    if (s->top_k > 0 && s->top_k < m) m = s->top_k;
    if (s->min_p > 0.0f && s->min_p < 1.0f) {
        float th = s->min_p * c[0].p;
        int keep = 1;
        while (keep < m && c[keep].p >= th) keep++;
        m = keep;
    }
    float mass;
    if (s->top_p > 0.0f && s->top_p < 1.0f) {
        float cum = 0.0f;
        int last = m - 1;
        for (int i = 0; i < m; i++) { cum += c[i].p; if (cum >= s->top_p) { last = i; break; } }
        m = last + 1;
        mass = cum;
    } else {
        mass = 0.0f;
        for (int i = 0; i < m; i++) mass += c[i].p;
    }
    float r = (float)(orc_rng_u32(s) >> 8) / 16777216.0f * mass;
    float cum = 0.0f;
    int pick = c[m - 1].i;
    for (int i = 0; i < m; i++) { cum += c[i].p; if (r < cum) { pick = c[i].i; break; } }
    free(c);
    orc_sampler_accept(s, pick);
    return pick;
}

/* The C library's expf over an array: the exponential the reference's softmax
 * and SwiGLU call (src/model.c:61, 405), for checking restatements of it. */
void orc_expf_n(const float *x, float *y, long n) {
    for (long i = 0; i < n; i++) y[i] = expf(x[i]);
}
