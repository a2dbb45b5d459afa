/* ehip.h — the thin C-ABI device layer beneath ember.h.
 *
 * The host library (C11) resolves tensors from the mmap'd .ember file and
 * hands plain host pointers to this layer, which repacks and uploads them to
 * one MI355X (gfx950) and runs the forward pass there.  No C++ or HIP type
 * crosses this boundary: only pointers, sizes and the structs below.
 *
 * Each entry point replaces the work of a reference function:
 *   ehip_model_upload   <- weight resolution in ember_state_new_ex (src/model.c:120-171)
 *   ehip_state_create   <- activation/KV allocation (src/model.c:173-193)
 *   ehip_state_destroy  <- ember_state_free (src/model.c:195-205)
 *   ehip_forward        <- ember_forward (src/model.c:362-414)
 *   ehip_prefill        <- ember_prefill (src/model.c:283-360)
 * Errors: functions returning a pointer return NULL, functions returning int
 * return nonzero; ehip_last_error() then names the failing call.
 */
#ifndef EMBER_EHIP_H
#define EMBER_EHIP_H

#include <stdint.h>

#include "ember.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct EhipModel EhipModel;  /* weights resident in HBM         */
typedef struct EhipState EhipState;  /* KV cache, activations, stream   */

typedef struct {
    int32_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim, vocab_size;
    float   rope_theta, norm_eps;
    int32_t rope_style;   /* EMBER_ROPE_*                                       */
    int32_t qk_norm;      /* nonzero: per-head RMSNorm of q and k before RoPE   */
} EhipConfig;

/* A weight matrix in its file encoding: `data` points at rows*in_len weights
 * stored as EMBER_DT_F32, EMBER_DT_Q8_0 (34-byte blocks) or EMBER_DT_Q4_0
 * (18-byte blocks), row-major [rows][in_len]. */
typedef struct { const void *data; int32_t dtype; } EhipWeight;

typedef struct {
    EhipWeight wq, wk, wv, wo, w1, w2, w3;
    const float *attn_norm, *ffn_norm;   /* [dim]                      */
    const float *q_norm, *k_norm;        /* [head_dim] or NULL          */
    const float *bq, *bk, *bv;           /* [n_heads*hd], [kv_dim] or NULL */
} EhipLayer;

const char *ehip_last_error(void);
/* Number of visible devices (0 when no GPU); initialises the runtime. */
int ehip_device_count(void);

/* Repack and upload all weights.  `rope_inv_freq` holds head_dim/2 values
 * 1/theta^(2i/head_dim) computed on the host; each state tabulates
 * cosf/sinf of pos * freq_i for its positions with the host libm, as the
 * reference computes them per call (src/model.c:66-71). */
EhipModel *ehip_model_upload(const EhipConfig *cfg, const EhipLayer *layers,
                             EhipWeight tok_emb, EhipWeight lm_head,
                             const float *final_norm, const float *rope_inv_freq);
void       ehip_model_free(EhipModel *m);
/* Device bytes held by the uploaded weights. */
uint64_t   ehip_model_bytes(const EhipModel *m);

EhipState *ehip_state_create(EhipModel *m, int ctx, int kv_fp16);
void       ehip_state_destroy(EhipState *s);

/* Decode one token; returns host-readable logits owned by the state (pinned). */
float *ehip_forward(EhipState *s, int tok, int pos);
/* Prefill ids[0..n) at positions start..; returns last-token logits. */
float *ehip_prefill(EhipState *s, const int *ids, int n, int start);

/* Greedy decode held entirely on the device, replacing the caller's loop of
 * ember_sample (temperature <= 0: the first maximum, src/sample.c:114-127)
 * followed by ember_forward (the generate loop of src/main.c:197-206).
 * Starting from token `tok` at position `pos`, run n decode steps; after
 * each, the argmax of the logits becomes the next input token on the device,
 * with no host round trip (one hipGraph replayed n times).  The n chosen
 * tokens are copied to out_tokens (if non-NULL); the last step's logits stay
 * in device memory (ehip_debug_buffer 4).  *ms (if non-NULL) receives the
 * device time of the n steps, from HIP events on the state's stream.  No
 * stop-token handling: exactly n tokens are generated.  Returns 0, or
 * nonzero with ehip_last_error() set. */
int ehip_generate_greedy(EhipState *s, int tok, int pos, int n, int *out_tokens, float *ms);

/* ember_sample(smp, logits, n) (src/sample.c:120-175) on the device:
 * penalties over the sampler's history ring, then the first maximum
 * (temperature <= 0) or temperature -> softmax -> top-k -> min-p -> top-p
 * -> one draw from the sampler's xorshift64* stream; the token is accepted
 * into the ring.  `logits` (host, n <= vocab floats) is copied to the device
 * and left unmodified; NULL samples (and overwrites) the logits the last
 * decode step left on the device.  The sampler's rng_state, history,
 * hist_len and hist_pos are updated as ember_sample would.  Any top_k:
 * 1..64 keeps the first 64 candidates by bounds; 0 (no cap) or more than 64
 * sorts every token's probability and walks the running sum in that order,
 * one addition per candidate as the reference does.  Returns 0 and *token,
 * or nonzero. */
int ehip_sample(EhipState *s, const float *logits, int n, EmberSampler *smp, int *token);

/* The generate loop of src/main.c:197-206 held on the device with the full
 * sampler: starting from token `tok` at position `pos`, n steps of decode
 * followed by ehip_sample's selection, the chosen token feeding the next step
 * with no host round trip (one hipGraph per step, captured for the sampler's
 * parameters).  Tokens go to out_tokens (if non-NULL), the sampler state is
 * updated as after n ember_sample calls, *ms (if non-NULL) receives the
 * device time.  Same parameter support as ehip_sample. */
int ehip_generate_sampled(EhipState *s, int tok, int pos, int n, EmberSampler *smp, int *out_tokens, float *ms);

/* ehip_sample's selection on logits already in device memory, allocating
 * nothing.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  All pointers are device memory:
 * logits[n] (penalties update them in place, as ember_sample does), the
 * xorshift64* state *rng_state (advanced), the history ring history[cap]
 * and hist_meta[2] = {hist_len, hist_pos} (both NULL: no ring; else
 * cap = params->hist_cap, updated as ember_sampler_accept would), and
 * *token (written).  params (host) supplies temperature, top_k, top_p,
 * min_p, the penalties and hist_cap; its history pointer and RNG fields are
 * not read.  The launches are enqueued on `stream` (a hipStream_t; NULL for
 * the default stream) and the call returns without waiting.  Every
 * intermediate lives in one fixed device array per GPU (about 36 KB, held
 * until the process ends); n is limited to 262,144 logits and top_k to
 * [1, 64] when temperature > 0.  Calls that overlap on one GPU race on that
 * array.  Returns 0, or nonzero with ehip_last_error() set. */
int ehip_sample_noalloc(float *logits, int n, const EmberSampler *params, uint64_t *rng_state,
                        int *history, int *hist_meta, int *token, void *stream);
/* Looks up that array's device address on the current device (done by
 * ehip_state_create; needed before graph capture on a device without a
 * state).  Returns 0 or nonzero. */
int ehip_noalloc_setup(void);

/* One tensor for the requantizer: `rows` x `cols` fp32 values (row-major,
 * host memory, cols a multiple of 32) to be encoded as `dtype`
 * (EMBER_DT_Q8_0: 34-byte blocks, EMBER_DT_Q4_0: 18-byte blocks) into
 * rows*(cols/32) blocks at `dst` (host memory). */
typedef struct {
    const float *src;
    int64_t rows;
    int32_t cols, dtype;
    void *dst;
} EhipQuantJob;

/* Block quantization of every job on the device, replacing the per-row
 * quantizer loops of quantize_tensor (src/quant.c:26-57, with
 * ember_quantize_q8_0 / ember_quantize_q4_0 of src/kernels.c:73-115) that
 * ember_quantize_file runs.  The blocks equal the host quantizers'
 * (ember_quant_q8_row / ember_quant_q4_row) byte for byte.  Synchronous:
 * returns once every block is in its destination; 0, or nonzero with
 * ehip_last_error() set (bad job, no GPU, failed copy). */
int ehip_quantize_rows(const EhipQuantJob *jobs, int n_jobs);

/* ---- inspection and measurement (tests and bench) ----------------------- */
/* Copy the KV cache of the given layers to/from host memory in the cache's
 * own element type; which = 0 keys, 1 values; rows [0, n_pos). */
int ehip_kv_read(EhipState *s, int which, int layer, int n_pos, void *host);
int ehip_kv_write(EhipState *s, int which, int layer, int n_pos, const void *host);
/* Copy a per-step device buffer to the host after a call: which = 0 the
 * residual stream x [dim], 1 the last layer's raw q|k|v, 2 its attention
 * output [n_heads*hd], 3 its SwiGLU output [hidden], 4 logits [vocab]. */
int ehip_debug_buffer(EhipState *s, int which, void *host, uint64_t bytes);
/* Record one layer's intermediate vectors during every following decode
 * step (ember_forward / ehip_forward and the device loops; layer -1 stops
 * recording).  Slots, each fp32, as the layer computes them (the layer
 * structure of src/model.c:374-409):
 *   0 the residual stream entering the layer [dim] (layer 0: the embedding row)
 *   1 the raw q|k|v product, bias added [n_heads*hd + 2*kv_dim]
 *   2 the attention output [n_heads*hd]
 *   3 the residual after wo [dim]
 *   4 the SwiGLU output [hidden]
 *   5 the residual after w2 [dim]
 * No counterpart in the reference: a test hook for checking each decode
 * kernel at full model shapes against a recomputation on the same inputs.
 * Changing the layer drops the state's captured step graphs. */
int ehip_debug_capture(EhipState *s, int layer);
int ehip_debug_read(EhipState *s, int slot, void *host, uint64_t bytes);
/* The same for prefill: record `layer` of prefill pass `pass` (passes cover
 * ehip_prefill_pass_tokens() tokens each) in the following ehip_prefill
 * calls, as [n_tok][width] fp32 rows; slot 4 holds the w1|w3 product before
 * SwiGLU ([n_tok][2*hidden], the w1 rows first).  ehip_debug_read_prefill
 * also returns the pass's token count and first position. */
int ehip_debug_capture_prefill(EhipState *s, int layer, int pass);
int ehip_debug_read_prefill(EhipState *s, int slot, void *host, uint64_t bytes, int *n_tok, int *pos0);
int ehip_prefill_pass_tokens(const EhipState *s);
/* 0: eager launches, 1: one hipGraph per decode step (default). */
int ehip_set_graph_mode(EhipState *s, int mode);
/* How the state's decode step is scheduled: bit 0 = the attention kernel
 * merges its chunks itself (no merge kernel), which needs every workgroup of
 * a kv head on one XCD; the state checks that at creation.  Bit 1 = the
 * attention kernel also computes the wo product (no wo matvec launch).  A
 * step whose kernels find a workgroup on another XCD, whose wo product
 * times out, or whose merge reads a chunk's partial of another launch (each
 * carries a token of its launch), clears both bits for the rest of the
 * state's life. */
int ehip_decode_fusion(const EhipState *s);
/* Time `steps` decode steps at positions pos0.. with HIP events recorded on
 * the state's stream; writes the average step time in ms.  Tokens follow the
 * reference bench stream (pos*131+7) % vocab. */
int ehip_time_decode(EhipState *s, int pos0, int steps, float *ms_per_step);
/* Time `reps` back-to-back launches of one decode-step kernel on the
 * state's stream with HIP events, at position pos; writes average ms.
 * kernel: 0 = the split-K attention kernel (with its in-kernel chunk merge
 * and folded wo product when ehip_decode_fusion reports them; the separate
 * merge kernel is not timed), 1 = lm_head matvec, 2 = fused w1|w3 matvec
 * (adding the wo partials when they are folded).  Launches of kernels 0
 * and 2 walk through the layers, so each streams its own cache rows or
 * weights from HBM as in a decode step. */
int ehip_time_kernel(EhipState *s, int kernel, int pos, int reps, float *ms_per_launch);
/* The GPU's measured streaming read bandwidth: `reps` passes of a plain
 * 16-byte-load kernel (32 KB per workgroup) over a fresh device buffer of
 * `bytes` (1 MiB to 64 GiB), timed with HIP events on the state's stream;
 * writes GB/s.  No counterpart in the reference: the measured peak that
 * decode roofline fractions are also quoted against, beside the 8 TB/s
 * datasheet figure. */
int ehip_measure_read_bw(EhipState *s, uint64_t bytes, int reps, float *gb_per_s);
/* y[i] = expf(x[i]) for i < n, evaluated on the host with the restatement of
 * the C library's expf that the reference-order kernels (EHIP_ORDER=reference)
 * run on the device.  No counterpart in the reference: exported so the
 * restatement can be checked against the host's libm without a GPU. */
void ehip_libm_expf(const float *x, float *y, long n);

#ifdef __cplusplus
}
#endif
#endif
