/* ember_synth.h — seeded synthetic .ember model files.
 *
 * Not part of the reference's API: benchmarks and tests use it to build model
 * files of the reference's shapes with no network access.  The generator and
 * the file rules are documented in emberllm_amd/csrc/host/synth.c.
 */
#ifndef EMBER_SYNTH_H
#define EMBER_SYNTH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int32_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim, vocab_size, max_seq_len;
    float   rope_theta, norm_eps;
    int32_t rope_style;   /* EMBER_ROPE_*                                   */
    int32_t qk_norm;      /* emit q_norm / k_norm and set EMBER_FLAG_QK_NORM */
    int32_t qkv_bias;     /* emit wq_bias / wk_bias / wv_bias                */
    int32_t tied;         /* lm_head shares tok_embeddings                  */
    int32_t dtype;        /* EMBER_DT_F32, EMBER_DT_Q8_0 or EMBER_DT_Q4_0    */
    int32_t threads;      /* generator threads (<= 0: 8)                    */
    uint64_t seed;
    float   std;          /* standard deviation of matrices and biases      */
} EmberSynthConfig;

/* Write the model; returns 0 on success. */
int ember_synth_write(const char *path, const EmberSynthConfig *cfg);
/* The fp32 values of one row of a randomly drawn tensor (before encoding). */
void ember_synth_fill_row(uint64_t seed, const char *name, int row, float std, float *out, int n);
uint64_t ember_synth_row_state(uint64_t seed, const char *name, int row);

#ifdef __cplusplus
}
#endif
#endif
