/* drive.c — runs the host C library (with the device-layer test double of
 * ehip_stub.c) through the call sequences of the reference's callers, for
 * AddressSanitizer / UndefinedBehaviorSanitizer.  TEST INFRASTRUCTURE.
 *
 *   drive MODEL [MODEL ...]
 * For each model file:
 *   - the `ember bench` loop (src/main.c:230-294): ember_threads_init,
 *     ember_state_new_ex(pp + tg + 2), ember_prefill of pp ids, tg calls of
 *     ember_forward from pos = pp, each logits vector read in full, twice
 *     (a warmup rep and a timed one);
 *   - the generate / chat loop (src/main.c:143-221, 296-330): tokenizer,
 *     ember_encode, prefill, sampled decode with penalties (ember_sample,
 *     ember_sampler_accept), ember_decode of each token, a continuation
 *     prefill at start > 0, a prefill of zero tokens, ember_sampler_reset;
 *   - the ctypes binding's use (bindings/python/emberllm.py): header, tensor
 *     lookup and data, ember_state_new with ctx 0;
 *   - ember_quantize_file to Q8_0 and Q4_0 when the model is F32, each
 *     result loaded and run through the bench loop.
 * Prints "drive ok" at the end; any sanitizer report aborts with an error. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ember.h"

static double g_sum;

static void read_all(const float *lg, int n) {
    double s = 0;
    for (int i = 0; i < n; i++) s += lg[i];
    g_sum += s;
}

static void bench_loop(const char *path, int pp, int tg) {
    EmberModel *m = ember_model_load(path);
    if (!m) { fprintf(stderr, "drive: cannot load %s\n", path); exit(2); }
    const EmberHeader *h = ember_model_header(m);
    ember_threads_init(2);
    if (pp + tg + 2 > h->max_seq_len) { pp = h->max_seq_len / 2; tg = h->max_seq_len / 2 - 3; }
    EmberState *st = ember_state_new_ex(m, pp + tg + 2, 0);
    int *ids = malloc(sizeof(int) * (size_t)pp);
    for (int i = 0; i < pp; i++) ids[i] = (i * 131 + 7) % h->vocab_size;
    for (int r = 0; r < 2; r++) {
        read_all(ember_prefill(m, st, ids, pp, 0), h->vocab_size);
        int pos = pp;
        for (int i = 0; i < tg; i++, pos++)
            read_all(ember_forward(m, st, (pos * 131 + 7) % h->vocab_size, pos), h->vocab_size);
    }
    free(ids);
    ember_state_free(st);
    ember_threads_shutdown();
    ember_model_free(m);
}

static void generate_loop(const char *path) {
    EmberModel *m = ember_model_load(path);
    if (!m) { fprintf(stderr, "drive: cannot load %s\n", path); exit(2); }
    const EmberHeader *h = ember_model_header(m);
    const int V = h->vocab_size;
    /* the binding's lookups */
    const EmberTensor *t = ember_model_tensor(m, "tok_embeddings");
    if (!t || !ember_model_data(m, t)) { fprintf(stderr, "drive: no tok_embeddings\n"); exit(2); }
    if (ember_model_tensor(m, "no.such.tensor")) { fprintf(stderr, "drive: lookup\n"); exit(2); }
    EmberState *st = ember_state_new(m, 0);
    EmberTokenizer *tok = ember_tokenizer_new(m);
    int *ids = NULL, n = 0;
    if (tok) n = ember_encode(tok, "Once upon a time, there was a tiny model.", 1, &ids);
    if (n <= 0) {   /* no tokenizer in the file: a fixed prompt */
        free(ids);
        n = 8;
        ids = malloc(sizeof(int) * 8);
        for (int i = 0; i < n; i++) ids[i] = (i * 37 + 1) % V;
    }
    EmberSampler smp;
    ember_sampler_init(&smp, 0.8f, 0.9f, 40, 1234);
    ember_sampler_set_penalties(&smp, 1.1f, 16, 0.2f, 0.1f, 0.05f);
    for (int i = 0; i < n; i++) ember_sampler_accept(&smp, ids[i]);
    float *lg = ember_prefill(m, st, ids, n, 0);
    int pos = n, prev = ids[n - 1];
    const int steps = h->max_seq_len - n - 12 < 24 ? h->max_seq_len - n - 12 : 24;
    for (int i = 0; i < steps; i++, pos++) {
        const int next = ember_sample(&smp, lg, V);
        if (next < 0 || next >= V) { fprintf(stderr, "drive: sampled %d\n", next); exit(2); }
        ember_sampler_accept(&smp, next);
        if (tok) { const char *piece = ember_decode(tok, prev, next); if (piece) g_sum += strlen(piece); }
        prev = next;
        lg = ember_forward(m, st, next, pos);
    }
    /* a chat turn: continuation at start > 0, then a prefill of nothing */
    int more[3] = { 1 % V, 2 % V, 3 % V };
    read_all(ember_prefill(m, st, more, 3, pos), V);
    read_all(ember_prefill(m, st, more, 0, pos + 3), V);
    ember_sampler_reset(&smp);
    EmberSampler greedy;
    ember_sampler_init(&greedy, 0.0f, 1.0f, 0, 0);
    g_sum += ember_sample(&greedy, ember_forward(m, st, 5 % V, pos + 3), V);
    ember_sampler_free(&greedy);
    ember_sampler_free(&smp);
    free(ids);
    if (tok) ember_tokenizer_free(tok);
    ember_state_free(st);
    ember_model_free(m);
}

int main(int argc, char **argv) {
    if (argc < 3) { fprintf(stderr, "usage: drive TMPDIR MODEL...\n"); return 2; }
    const char *tmp = argv[1];
    for (int a = 2; a < argc; a++) {
        const char *path = argv[a];
        bench_loop(path, 24, 16);
        generate_loop(path);
        EmberModel *m = ember_model_load(path);
        if (!m) return 2;
        const EmberHeader *h = ember_model_header(m);
        const EmberTensor *tab = (const EmberTensor *)((const uint8_t *)h + h->tensor_table_offset);
        const int f32 = tab[0].dtype == EMBER_DT_F32;
        ember_model_free(m);
        if (f32) {
            for (int target = EMBER_DT_Q8_0; target <= EMBER_DT_Q4_0; target++) {
                char out[4096];
                snprintf(out, sizeof out, "%s/drive_q%d.ember", tmp, target);
                if (ember_quantize_file(path, out, target)) { fprintf(stderr, "drive: quantize failed\n"); return 2; }
                bench_loop(out, 24, 16);
                generate_loop(out);
            }
        }
        fprintf(stderr, "drive: %s done\n", path);
    }
    printf("drive ok %.3f\n", g_sum);
    return 0;
}
