/* sample.c — the sampler of ember.h (replaces src/sample.c:17-175).
 *
 * Same controls and the same xorshift64* stream as the reference, so a seed
 * reproduces its choices: penalties over the history ring, then greedy
 * (first maximum) or temperature -> softmax -> candidates ordered by
 * probability -> top-k -> min-p -> top-p -> one uniform draw.  The
 * reference orders candidates with glibc qsort, which sorts stably (merge
 * sort), so ties keep ascending token order; this file orders by
 * (probability desc, index asc) explicitly and, when top-k is set, selects
 * only the k best with a bounded heap instead of sorting the whole vocabulary.
 */
#include "ember.h"
#include "util.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* seed 0 selects this fixed nonzero state (a zero xorshift state stays zero) */
#define RNG_ZERO_SEED 0x9E3779B97F4A7C15ULL

void ember_sampler_init(EmberSampler *s, float temp, float top_p, int top_k, uint64_t seed) {
    /* every penalty starts at its no-op value; no history ring */
    const EmberSampler fresh = {
        .temperature = temp,
        .top_p = top_p,
        .top_k = top_k,
        .repeat_penalty = 1.0f,
        .rng_state = seed != 0 ? seed : RNG_ZERO_SEED,
    };
    *s = fresh;
}

/* Give the history ring `cap` slots (cap <= 0 releases it) and empty it. */
static void ring_resize(EmberSampler *s, int cap) {
    if (cap <= 0) {
        free(s->history);
        s->history = NULL;
        s->hist_cap = 0;
    } else if (cap != s->hist_cap) {
        s->history = ember_xrealloc(s->history, sizeof(int) * (size_t)cap, "sampler history ring");
        s->hist_cap = cap;
    }
    s->hist_len = 0;
    s->hist_pos = 0;
}

void ember_sampler_set_penalties(EmberSampler *s, float repeat_penalty, int repeat_last_n,
                                 float presence_penalty, float frequency_penalty, float min_p) {
    s->repeat_penalty = repeat_penalty;
    s->repeat_last_n = repeat_last_n;
    s->presence_penalty = presence_penalty;
    s->frequency_penalty = frequency_penalty;
    s->min_p = min_p;
    /* a ring is kept only when some penalty would read it */
    const int reads_history = repeat_penalty != 1.0f || presence_penalty != 0.0f || frequency_penalty != 0.0f;
    ring_resize(s, reads_history ? repeat_last_n : 0);
}

void ember_sampler_accept(EmberSampler *s, int token) {
    if (s->history == NULL || s->hist_cap <= 0) return;
    s->history[s->hist_pos] = token;
    s->hist_pos = s->hist_pos + 1 < s->hist_cap ? s->hist_pos + 1 : 0;
    if (s->hist_len < s->hist_cap) s->hist_len += 1;
}

void ember_sampler_reset(EmberSampler *s) {
    s->hist_len = 0;
    s->hist_pos = 0;
}

void ember_sampler_free(EmberSampler *s) {
    if (s != NULL) ring_resize(s, 0);
}

/* Penalties over the ring's hist_len valid entries (src/sample.c:76-96).
 * Each distinct in-range token t is handled once, at its first entry: the
 * repetition penalty (divide a positive logit, multiply a negative one) and
 * the presence penalty, then the frequency penalty subtracted once per entry
 * holding t.  Per logit that is the reference's sequence of operations, so
 * the results are bit-identical; different logits are independent. */
static void penalize(EmberSampler *s, float *logits, int n) {
    const int rep = s->repeat_penalty != 1.0f, pres = s->presence_penalty != 0.0f,
              freq = s->frequency_penalty != 0.0f;
    if (s->history == NULL || s->hist_len <= 0 || !(rep || pres || freq)) return;
    const int *h = s->history, len = s->hist_len;
    for (int i = 0; i < len; i++) {
        const int t = h[i];
        if (t < 0 || t >= n) continue;
        int seen = 0;
        for (int j = 0; j < i && !seen; j++) seen = h[j] == t;
        if (seen) continue;
        float v = logits[t];
        if (rep) v = v > 0.0f ? v / s->repeat_penalty : v * s->repeat_penalty;
        if (pres) v -= s->presence_penalty;
        if (freq)
            for (int k = i; k < len; k++)
                if (h[k] == t) v -= s->frequency_penalty;
        logits[t] = v;
    }
}

static uint32_t next_u32(EmberSampler *s) {
    uint64_t x = s->rng_state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    s->rng_state = x;
    return (uint32_t)((x * 0x2545F4914F6CDD1DULL) >> 32);
}

static int first_argmax(const float *v, int n) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

typedef struct { float p; int id; } Cand;

/* strict "a ranks before b": higher probability, then lower token id */
static int before(const Cand *a, const Cand *b) { return a->p > b->p || (a->p == b->p && a->id < b->id); }

static int cand_cmp(const void *x, const void *y) {
    const Cand *a = x, *b = y;
    return before(a, b) ? -1 : (before(b, a) ? 1 : 0);
}

/* min-heap on rank (root = worst of the kept k) */
static void sift_down(Cand *h, int k, int i) {
    for (;;) {
        int l = 2 * i + 1, r = l + 1, w = i;
        if (l < k && before(&h[w], &h[l])) w = l;
        if (r < k && before(&h[w], &h[r])) w = r;
        if (w == i) return;
        Cand t = h[i]; h[i] = h[w]; h[w] = t;
        i = w;
    }
}

/* first k of the (prob desc, id asc) order of p[0..n), sorted */
static int top_candidates(const float *p, int n, int k, Cand *out) {
    if (k <= 0 || k >= n) {
        for (int i = 0; i < n; i++) { out[i].p = p[i]; out[i].id = i; }
        qsort(out, (size_t)n, sizeof(Cand), cand_cmp);
        return n;
    }
    for (int i = 0; i < k; i++) { out[i].p = p[i]; out[i].id = i; }
    for (int i = k / 2 - 1; i >= 0; i--) sift_down(out, k, i);
    for (int i = k; i < n; i++) {
        Cand c = { p[i], i };
        if (before(&c, &out[0])) { out[0] = c; sift_down(out, k, 0); }
    }
    qsort(out, (size_t)k, sizeof(Cand), cand_cmp);
    return k;
}

int ember_sample(EmberSampler *s, float *logits, int n) {
    penalize(s, logits, n);
    if (s->temperature <= 0.0f) {
        const int c = first_argmax(logits, n);
        ember_sampler_accept(s, c);
        return c;
    }
    for (int i = 0; i < n; i++) logits[i] /= s->temperature;
    const float mx = logits[first_argmax(logits, n)];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) { logits[i] = expf(logits[i] - mx); sum += logits[i]; }
    for (int i = 0; i < n; i++) logits[i] /= sum;

    const int k = (s->top_k > 0 && s->top_k < n) ? s->top_k : 0;
    Cand *c = ember_xmalloc(sizeof(Cand) * (size_t)(k ? k : n), "sampler candidates");
    int m = top_candidates(logits, n, k, c);
    if (s->min_p > 0.0f && s->min_p < 1.0f) {
        const float floor_p = s->min_p * c[0].p;
        int keep = 1;
        while (keep < m && c[keep].p >= floor_p) keep++;
        m = keep;
    }
    float mass = 0.0f;
    if (s->top_p > 0.0f && s->top_p < 1.0f) {
        int last = m - 1;
        for (int i = 0; i < m; i++) {
            mass += c[i].p;
            if (mass >= s->top_p) { last = i; break; }
        }
        m = last + 1;
    } else {
        for (int i = 0; i < m; i++) mass += c[i].p;
    }
    const float r = (float)(next_u32(s) >> 8) / 16777216.0f * mass;
    float cum = 0.0f;
    int chosen = c[m - 1].id;
    for (int i = 0; i < m; i++) {
        cum += c[i].p;
        if (r < cum) { chosen = c[i].id; break; }
    }
    free(c);
    ember_sampler_accept(s, chosen);
    return chosen;
}
