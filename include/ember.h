/* ember.h — the public C API and the on-disk .ember weight format.
 *
 * This header is the drop-in boundary: it keeps the exact ABI of emberllm's
 * public header (src/ember.h:1-173) so that existing C callers and the ctypes
 * binding (bindings/python/emberllm.py:48-109) link against this library
 * unchanged.  Behind these entry points the forward pass runs on an MI355X
 * (gfx950) through the device layer declared in ehip.h.
 *
 * File layout (all offsets absolute from the start of the file, little-endian):
 *   EmberHeader (256 B) | tokenizer blob | tensor table (n * 88 B, 8-aligned)
 *   | zero pad to 64 | tensor data, each tensor 64-byte aligned.
 * Quantized blocks hold 32 weights: Q8_0 = {fp16 scale, int8[32]} (34 B),
 * Q4_0 = {fp16 scale, 16 bytes of nibbles} (18 B).
 */
#ifndef EMBER_H
#define EMBER_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EMBER_MAGIC   0x52424d45u /* the bytes "EMBR" read as a little-endian u32 */
#define EMBER_VERSION 1u

/* stored tensor encodings (src/ember.h:24-30) */
enum {
    EMBER_DT_F32  = 0,
    EMBER_DT_Q8_0 = 1,
    EMBER_DT_Q4_0 = 2,
    EMBER_DT_F16  = 3  /* defined by the format; no forward pass consumes it */
};

/* header flags (src/ember.h:32-37) */
enum {
    EMBER_FLAG_TIED_EMBED = 1u << 0, /* lm_head is the token-embedding table     */
    EMBER_FLAG_QK_NORM    = 1u << 1, /* per-head RMSNorm of q and k before RoPE   */
    EMBER_FLAG_THINKING   = 1u << 2  /* model has a reasoning mode (chat front-end only) */
};

/* rotary pairing (src/ember.h:39-43) */
enum {
    EMBER_ROPE_INTERLEAVED = 0, /* pairs (2i, 2i+1) inside each head  */
    EMBER_ROPE_NEOX        = 1  /* pairs (i, i + head_dim/2)          */
};

/* tokenizer blob kinds (src/ember.h:45-49) */
enum {
    EMBER_TOK_LLAMA_SP = 0, /* SentencePiece-style pieces with merge scores */
    EMBER_TOK_BYTE_BPE = 1  /* byte-level BPE with merge ranks              */
};

#define EMBER_Q_BLOCK 32

#pragma pack(push, 1)
/* 256-byte file header (src/ember.h:54-83). */
typedef struct {
    char     magic[4];
    uint32_t version;
    uint64_t header_bytes;         /* start of the tensor data region        */
    int32_t  dim;
    int32_t  hidden_dim;
    int32_t  n_layers;
    int32_t  n_heads;
    int32_t  n_kv_heads;
    int32_t  head_dim;
    int32_t  vocab_size;
    int32_t  max_seq_len;
    float    rope_theta;
    float    norm_eps;
    uint32_t flags;
    int32_t  rope_style;
    int32_t  bos_token_id;
    int32_t  eos_token_id;
    int32_t  eos_token_id2;
    int32_t  n_tensors;
    int32_t  tokenizer_type;
    int32_t  default_top_k;
    float    default_temp;
    float    default_top_p;
    uint64_t tokenizer_offset;
    uint64_t tokenizer_size;
    uint64_t tensor_table_offset;
    uint64_t tensor_table_size;
    uint8_t  reserved[128];
} EmberHeader;

/* 88-byte tensor table entry (src/ember.h:85-92).  2-D tensors are
 * shape = [out_rows, in_len]; unused trailing dims are 1. */
typedef struct {
    char     name[48];
    int32_t  dtype;
    int32_t  ndim;
    int32_t  shape[4];
    uint64_t offset;
    uint64_t nbytes;
} EmberTensor;
#pragma pack(pop)

#ifdef __cplusplus
static_assert(sizeof(EmberHeader) == 256, "EmberHeader is 256 bytes");
static_assert(sizeof(EmberTensor) == 88, "EmberTensor is 88 bytes");
#else
_Static_assert(sizeof(EmberHeader) == 256, "EmberHeader is 256 bytes");
_Static_assert(sizeof(EmberTensor) == 88, "EmberTensor is 88 bytes");
#endif

typedef struct EmberModel EmberModel;
typedef struct EmberTokenizer EmberTokenizer;
typedef struct EmberState EmberState;

/* ---- model file (replaces src/io.c:30-96) ---------------------------------
 * ember_model_load returns NULL and prints "ember: <reason>" on a file that is
 * missing, too small, has a bad magic/version, or points outside itself. */
EmberModel        *ember_model_load(const char *path);
void               ember_model_free(EmberModel *m);
const EmberHeader *ember_model_header(const EmberModel *m);
const EmberTensor *ember_model_tensor(const EmberModel *m, const char *name);
const void        *ember_model_data(const EmberModel *m, const EmberTensor *t);

/* ---- run state and the forward pass (replaces src/model.c:116-414) -------
 * ember_state_new_ex uploads the weights to the GPU (repacked for the
 * kernels; the file is not modified) and allocates the KV cache there, fp32
 * or (kv_fp16 != 0) fp16.  ctx_len <= 0 or >= max_seq_len selects
 * max_seq_len.  ember_forward / ember_prefill return host-readable logits
 * (vocab_size floats) owned by the state and valid until the next call.
 * Out-of-range tokens or positions, missing tensors and device failures print
 * "ember: <reason>" and exit(1), as the reference does. */
EmberState *ember_state_new(const EmberModel *m, int ctx_len);
EmberState *ember_state_new_ex(const EmberModel *m, int ctx_len, int kv_fp16);
void        ember_state_free(EmberState *s);
float      *ember_forward(EmberModel *m, EmberState *s, int tok, int pos);
float      *ember_prefill(EmberModel *m, EmberState *s, const int *ids, int n, int start);

/* ---- tokenizer (replaces src/tokenizer.c:176-420) ------------------------
 * ember_encode stores a malloc'd id array in *out_ids (free with free()). */
EmberTokenizer *ember_tokenizer_new(const EmberModel *m);
void            ember_tokenizer_free(EmberTokenizer *t);
int             ember_encode(EmberTokenizer *t, const char *text, int add_bos, int **out_ids);
const char     *ember_decode(EmberTokenizer *t, int prev_tok, int tok);

/* ---- sampler (replaces src/sample.c:17-175; field layout is ABI) --------- */
typedef struct {
    float temperature;
    float top_p;
    int   top_k;
    float min_p;
    float repeat_penalty;
    float presence_penalty;
    float frequency_penalty;
    int   repeat_last_n;
    uint64_t rng_state;
    int  *history;
    int   hist_cap, hist_len, hist_pos;
} EmberSampler;

void ember_sampler_init(EmberSampler *s, float temp, float top_p, int top_k, uint64_t seed);
void ember_sampler_set_penalties(EmberSampler *s, float repeat_penalty, int repeat_last_n,
                                 float presence_penalty, float frequency_penalty, float min_p);
void ember_sampler_accept(EmberSampler *s, int token);
void ember_sampler_reset(EmberSampler *s);
void ember_sampler_free(EmberSampler *s);
/* Picks the next token from `logits` (n floats).  Like the reference it may
 * overwrite the logits in place (penalties, temperature, softmax). */
int  ember_sample(EmberSampler *s, float *logits, int n);

/* ---- offline requantizer (replaces src/quant.c:59-125) -------------------
 * target is EMBER_DT_Q8_0 or EMBER_DT_Q4_0; returns 0 on success. */
int ember_quantize_file(const char *in_path, const char *out_path, int target);

/* ---- pool symbols the reference CLI links against (src/kernels.h:71-83) --
 * The GPU path has no host thread pool; these keep the CLI link surface and
 * record the requested count, which nothing on the device path consumes. */
void ember_threads_init(int nthreads);
void ember_threads_shutdown(void);
int  ember_nthreads(void);

#ifdef __cplusplus
}
#endif

#endif /* EMBER_H */
