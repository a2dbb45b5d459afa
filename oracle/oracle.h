/* oracle.h — CPU restatement of emberllm's token loop.  TEST INFRASTRUCTURE.
 *
 * This library is the checker for the GPU product, never the product: only
 * tests/, the smoke check and the CPU-baseline leg of bench.py load it.  It
 * restates, operation for operation, the reference's CPU path so that its
 * results equal those of the reference built with its deterministic flags
 * (-O2 -fno-fast-math -ffp-contract=off, Makefile:57-59):
 *
 *   orc_f32_to_f16 / orc_f16_to_f32  <- src/kernels.c:25-68
 *   orc_quantize_q8_0 / _q4_0        <- src/kernels.c:73-115
 *   orc_matmul / orc_matmul_batch    <- src/kernels.c:120-264 (scalar paths)
 *   orc_state_* / orc_forward        <- src/model.c:16-205, 207-278, 362-414
 *   orc_prefill                      <- src/model.c:283-360
 *   orc_sample and the sampler       <- src/sample.c:17-175
 *   orc_threads_init                 <- src/threads.c:61-104 (timed baseline)
 *
 * Pinning status of each function is recorded at the top of oracle.c.
 */
#ifndef EMBER_ORACLE_H
#define EMBER_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct OrcModel OrcModel;
typedef struct OrcState OrcState;

/* same field layout as EmberSampler (src/ember.h:141-155) */
typedef struct {
    float temperature, top_p;
    int   top_k;
    float min_p, repeat_penalty, presence_penalty, frequency_penalty;
    int   repeat_last_n;
    uint64_t rng_state;
    int  *history;
    int   hist_cap, hist_len, hist_pos;
} OrcSampler;

uint16_t orc_f32_to_f16(float f);
float    orc_f16_to_f32(uint16_t h);
void     orc_expf_n(const float *x, float *y, long n);   /* the C library's expf, as model.c:61, 405 call it */
void     orc_quantize_q8_0(const float *x, void *out, int n);
void     orc_quantize_q4_0(const float *x, void *out, int n);
/* out[d_out] = W[d_out, n_in] . x (activation re-quantized to Q8_0 first) */
void     orc_matmul(float *out, const float *x, const void *w, int dtype, int n_in, int d_out);
void     orc_matmul_batch(float *out, const float *x, const void *w, int dtype,
                          int n_in, int d_out, int B);
/* the integer part of one Q8_0 x Q8_0 / Q4_0 x Q8_0 block dot (exact) */
int32_t  orc_block_dot_q8(const void *wblock, const void *xblock);
int32_t  orc_block_dot_q4(const void *wblock, const void *xblock);

OrcModel *orc_model_open(const char *path);
void      orc_model_close(OrcModel *m);
OrcState *orc_state_new(OrcModel *m, int ctx_len, int kv_fp16);
void      orc_state_free(OrcState *s);
int       orc_state_ctx(const OrcState *s);
float    *orc_forward(OrcState *s, int tok, int pos);
float    *orc_prefill(OrcState *s, const int *ids, int n, int start);
/* raw KV cache access: which = 0 keys, 1 values; layout [L][ctx][kv_dim] of
 * fp32 or fp16 (per kv_fp16).  Used to hand a GPU-filled cache to the oracle. */
void     *orc_kv_cache(OrcState *s, int which);
/* Copy layer `layer`'s vectors out during the following orc_forward /
 * orc_prefill calls (layer -1 or slots NULL: stop).  slots[i] (NULL to skip)
 * receives per token, as [n][width] rows: 0 the residual entering the layer,
 * 1 the raw q|k|v after bias, 2 the attention output, 3 the residual after
 * wo, 4 the SwiGLU output (orc_forward) or the w1|w3 products before it
 * ([n][2*hidden], orc_prefill), 5 the residual after w2.  The same slots as
 * the GPU layer's debug capture, for checking the checker itself. */
void      orc_capture(OrcState *s, int layer, float *const *slots);
uint64_t  orc_kv_bytes(const OrcState *s);

void orc_sampler_init(OrcSampler *s, float temp, float top_p, int top_k, uint64_t seed);
void orc_sampler_set_penalties(OrcSampler *s, float repeat_penalty, int repeat_last_n,
                               float presence_penalty, float frequency_penalty, float min_p);
void orc_sampler_accept(OrcSampler *s, int token);
void orc_sampler_free(OrcSampler *s);
int  orc_sample(OrcSampler *s, float *logits, int n);
uint32_t orc_rng_u32(OrcSampler *s);

void orc_threads_init(int n);
void orc_threads_shutdown(void);

#ifdef __cplusplus
}
#endif
#endif
