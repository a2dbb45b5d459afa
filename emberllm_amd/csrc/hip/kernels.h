// kernels.h — launch interface of the gfx950 kernels (host side, C++).
#pragma once
#include "dev_common.h"

namespace ehip {

// ---------------------------------------------------------------- matvec --
// One decode-step matrix-vector product with a fused prologue and epilogue:
//   prologue  PRO_NORM        x' = rmsnorm(in) then Q8_0-quantize x'
//             PRO_PLAIN       Q8_0-quantize in
//             PRO_EMBED_NORM  in = embedding row of the device token, written
//                             to x_out, then as PRO_NORM
//             PRO_NORM_PARTS  in + (parts[0] + ... + parts[n_parts - 1]) (the
//                             kv groups' wo partials of the decode attention),
//                             written to x_out, then as PRO_NORM; workgroup 0
//                             clears flag_reset[p * XM_CNT_STRIDE], p < n_parts
//   epilogue  EPI_STORE   out[r] = W[r].x' (+ bias[r])
//             EPI_RESID   out[r] += W[r].x'
//             EPI_SWIGLU  out[u] = silu(W[u].x') * W[u+pair_off].x'
enum { PRO_NORM = 0, PRO_PLAIN = 1, PRO_EMBED_NORM = 2, PRO_NORM_PARTS = 3 };
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_QKPOST = 3 };

struct MatvecArgs {
    DMat W;
    int units;            // number of outputs
    int pair_off;         // EPI_SWIGLU: row offset of the second matrix
    const float *in;      // [W.cols]
    const float *norm_w;  // [W.cols]
    float eps;
    const int *tokpos;    // device {tok, pos}
    union {   // (one storage: no prologue uses both)
        DMat emb;         // embedding table (PRO_EMBED_NORM)
        // PRO_NORM_PARTS: n_parts vectors of W.cols floats, n_parts <= MATVEC_MAX_PARTS
        struct { const float *parts; int n_parts; int *flag_reset; };
    };
    float *x_out;
    float *out;
    const float *bias;
    // EPI_STORE only, optional: greedy selection over the outputs (first
    // maximum).  Per-workgroup winners go to am_val/am_idx (MATVEC_MAX_GRID
    // entries); a merge kernel then writes am_tokpos = {token, pos + 1, n + 1}
    // and am_out[n] = token (when n < am_cap).
    float *am_val; int *am_idx;
    int *am_tokpos; int *am_out; int am_cap;
    // EPI_STORE only, optional: the outputs also stored straight into this
    // pinned host buffer (the API's logits), and the word after the last
    // output (out[units], the step's error flag) copied behind them, so the
    // PCIe writes overlap the product's weight stream instead of following it
    float *out_host;
};
constexpr int MATVEC_MAX_GRID = 2048;
constexpr int MATVEC_MAX_PARTS = 8;
int launch_matvec(hipStream_t st, int pro, int epi, const MatvecArgs &a);
// EPI_STORE with am_val/am_idx set and no merge: returns the number of
// per-workgroup winners written (the sampler's per-part maxima), or -1.
int launch_matvec_parts(hipStream_t st, int pro, const MatvecArgs &a);
// the same products in the reference's order (one thread per output, block
// sums added block after block; reforder.hip)
int launch_matvec_ref(hipStream_t st, int pro, int epi, const MatvecArgs &a);

// ------------------------------------------------------------- attention --
// GQA attention against the cache.  Prefill: causal attention of n_tok query
// tokens in the reference's floating-point order.  Decode: one token, split
// over chunks of positions (flash-decoding), merged in-kernel or by a merge
// kernel; the token's raw q/k/v (straight out of the QKV matvec) is
// QK-normed and rotated in the prologue and its k/v are written to the cache
// at `pos` by the chunk that owns it.
struct AttnArgs {
    const float *q;        // fused: raw q|k|v row; else rotated Q rows
    int q_stride;          // floats between consecutive tokens' q
    const float *q_norm, *k_norm;  // [hd] or nullptr
    const float2 *rope;            // [ctx][hd/2] (cos, sin) of pos * freq_i
    float eps, inv_sqrt;
    int rope_style;
    void *kc, *vc;         // layer cache base, [ctx][kv_dim]
    int kv_dim, hd, n_heads, n_kv, ctx;
    const int *tokpos;     // fused (decode): device {tok, pos}
    int pos_base;          // unfused (prefill): token b sits at pos_base + b
    int n_tok;
    // decode: chunk partials, o [n_heads][max_chunks][hd], then (m, l)
    // [n_heads][max_chunks], then (with xm_cnt) the launch token of each
    // chunk's partials, int [n_kv][max_chunks]
    float *part;
    int max_chunks;
    // decode, optional: merge the chunks of each kv head inside the chunk
    // kernel through the L2 of the one XCD all of them run on.  xm_cnt:
    // arrival counters of this layer, [n_kv] spaced XM_CNT_STRIDE ints apart,
    // zero between launches; xm_xcc: the XCD of each kv head's workgroups;
    // xm_err: set nonzero by a workgroup that finds itself on another XCD
    // (1), by a folded wo product that times out (2) or by a merge that
    // reads a partial of another launch (4: each carries a token from the
    // position and tokpos[3]).
    int *xm_cnt; const int *xm_xcc; int *xm_err;
    // with xm_cnt: the grid is 1-D, 8 * xm_slots workgroups (max_chunks =
    // xm_slots); workgroup L takes slot L / 8 of XCD L % 8 (where round-robin
    // dispatch places it), whose slots the kv heads g = L % 8, L % 8 + 8, ...
    // share as their chunks.  With n_kv a multiple of 8 that is the 2-D grid
    // (n_kv, max_chunks = 8 xm_slots / n_kv), which is what runs.
    int xm_slots;
    float *out;            // [n_tok][n_heads*hd]
    // The prefill fields and the decode-only folded wo product share their
    // storage (no launch uses both), which keeps the struct's size and layout
    // those of the prefill fields alone: a larger argument struct measured
    // 1-1.3% slower decode steps.
    union {
        struct {
            // prefill scratch: scores [n_heads][n_tok][ldk] (ldk >= pos_base +
            // n_tok, a multiple of 4); the maximum of each 64-key tile of a
            // row, [n_heads][n_tok][attn_prefill_tiles(ldk)]; per row the
            // maximum and 1/sum of the exponentials [n_heads][n_tok]
            float *scores, *tmax, *rowmax, *rowinv;
            int ldk;
            // prefill, optional: the output's Q8_0 codes, fp16-rounded block
            // scales and code sums ([n_tok][n_heads*hd / 32]), as the
            // quantization kernel would make them from `out`; written when the
            // launch reports it
            int8_t *qx; float *qdx; int *qxs;
            // prefill on matrix cores (head_dim 64 / 128): the pass's K/V
            // converted once into per-(kv head, 64-key tile) images,
            // kvimg_tiles tiles per head (attn_kvimg_bytes)
            uint8_t *kvimg; int kvimg_tiles;
            // nonzero: the tiles from pos_base / 64 on were written by the
            // q|k|v product (launch_gemm_qkpost or launch_gemm_qkv); only the
            // earlier ones are converted here (pos_base a multiple of 64)
            int kvimg_fused;
        };
        struct {
            // decode with xm_cnt on the 2-D grid, or on the 1-D grid with at
            // most 8 kv heads, optional: the wo product folded in (Q8_0 wo,
            // or Q4_0 on the 2-D grid; every kv group's G * hd columns in
            // whole 32-weight blocks).
            // Once kv head g's output is merged into `out`, its workgroup c
            // computes rows [c wo_rows, (c + 1) wo_rows) of W_o[:, the
            // group's columns] . o_g (on the 1-D grid wo_rows is the kernel's
            // own, from the kv head's chunk count) into
            // wo_part[g][row], with o_g Q8_0-quantized as the decode matvec
            // quantizes its input.  wo_flag[g * XM_CNT_STRIDE] is raised when
            // o_g is complete and must be zero at launch (the next w1|w3
            // matvec clears it).  wo_spin bounds the polls of that flag
            // (ATT_DEC_FW_SPIN; a time-out raises the error flag).
            DMat wo; float *wo_part; int *wo_flag; int wo_rows, wo_spin;
            // decode with xm_cnt (test hook, 0): added to chunk 0's launch
            // token, so that the merge finds a stale partial
            int tok_skew;
        };
    };
};
// prefill: q rows already normed and rotated, k/v already in the cache.
// *quantized (if non-null) says whether the launch also wrote a.qx/qdx/qxs.
int launch_attention(hipStream_t st, bool f16kv, const AttnArgs &a, bool *quantized = nullptr);
// prefill on matrix cores with a running softmax (no score scratch): fp16
// matrix cores with split operands for head_dim 64 / 128 (which also write
// a.qx/qdx/qxs when set, reported in *quantized), fp32 ones for 48
int launch_attention_mfma(hipStream_t st, bool f16kv, const AttnArgs &a, bool *quantized = nullptr);
// bytes of the K/V tile images the matrix-core prefill attention needs for
// ctx positions (0: head_dim without images)
size_t attn_kvimg_bytes(int hd, bool f16kv, int ctx, int n_kv);
// passes whose keys fit in PF_FUSE_KEYS run the whole exact-order attention
// (and the output's quantization) in one kernel
constexpr int PF_FUSE_KEYS = 256;
// products over at least GEMM_SPLIT_MIN_K inputs may split their block sums
// over pipelines and fuse each block's scaling into one fma (prefill GEMM);
// shorter ones keep one sequential sum in the reference's order
constexpr int GEMM_SPLIT_MIN_K = 1024;
inline int attn_prefill_ldk(int pos_base, int n_tok) { return (pos_base + n_tok + 3) & ~3; }
// tile-maximum slots per prefill score row (64-key tiles, padded to 4)
__host__ __device__ inline int attn_prefill_tiles(int ldk) { return ((ldk + 63) / 64 + 3) & ~3; }
// decode (one token, fused QK-norm / RoPE / KV store) over a grid of
// (n_kv, max_chunks) workgroups, max_chunks = attn_decode_chunks(...).
// Without xm_cnt the merge is a second kernel; with_merge = false leaves it
// out (measurement).
int launch_attn_decode(hipStream_t st, bool f16kv, const AttnArgs &a, bool with_merge = true);
// decode attention in the reference's order (one workgroup per query head,
// the softmax and P.V sums in position order; att: [n_heads][ctx] scratch)
int launch_attn_ref(hipStream_t st, bool f16kv, const AttnArgs &a, float *att);
// workgroups per kv head: two per CU over all kv heads, or more when a chunk
// would exceed ATT_DEC_CR rows (0: head_dim not supported)
int attn_decode_chunks(int ctx, int n_kv, int hd, int n_cu);
// slots per XCD of the in-kernel-merge grid: two workgroups per CU, or more
// when a chunk of the XCD with the most kv heads would exceed ATT_DEC_CR rows
int attn_decode_slots(int ctx, int n_kv, int n_cu);
constexpr int ATT_DEC_NL = 5;       // K and V pieces per thread per batch in the decode attention
constexpr int ATT_DEC_FW_SPIN = 1 << 18;   // polls of the folded wo's flag before the error flag is raised
constexpr int ATT_DEC_NW = 4;       // waves per decode attention workgroup
constexpr int ATT_DEC_WPC = 2;      // decode attention workgroups per CU
constexpr int ATT_DEC_CR = 160;     // positions per decode attention workgroup before more are added
constexpr int ATT_DEC_RMIN = 32;    // positions per decode attention chunk at least (short contexts)
constexpr int ATT_DEC_R1MAX = 96;   // positions per chunk up to which a kv head uses one workgroup per CU (fp32 KV)
// rows per chunk of the decode attention at position pos: (pos + 1) spread
// over one workgroup per CU (max_chunks / ATT_DEC_WPC of the kv head) while
// that gives at most ATT_DEC_R1MAX rows, else over all max_chunks; at least
// ATT_DEC_RMIN, so short contexts use a few chunks and a short merge.  A chunk
// count a little above the CUs a kv head spreads over would put two
// workgroups on a few CUs, and those set the kernel's end (Qwen3-0.6B shape at
// positions 1024..1151: 33-36 chunks of 32 rows 7.8 us per layer, 32 chunks of
// 33-36 rows 6.7 us).  Past that, chunks of fewer than ATT_DEC_RMIN2 rows
// lose to fewer chunks of ATT_DEC_RMIN2 (positions 3072..3199: 64 chunks of
// 49-50 rows 11.2 us per layer, 49-50 chunks of 64 rows 10.8 us).  An fp16
// cache row is half the bytes, and both thresholds double (the SmolLM2-135M
// shape at positions 4096..4223: 64 chunks of 65-66 rows 11.3 us per layer,
// 32-33 chunks of 128 rows 9.4 us); a chunk may then exceed ATT_DEC_CR rows,
// which only sizes the grid.  One division, as it follows the position's read.
constexpr int ATT_DEC_RMIN2 = 64;
__host__ __device__ inline int dec_chunk_rows(int pos, int max_chunks, bool f16) {
    const int one = max_chunks / ATT_DEC_WPC > 0 ? max_chunks / ATT_DEC_WPC : 1, sh = f16 ? 1 : 0;
    const bool spread = pos + 1 <= (ATT_DEC_R1MAX << sh) * one;
    const int d = spread ? one : max_chunks, m = spread ? ATT_DEC_RMIN : ATT_DEC_RMIN2 << sh;
    const int r = (pos + d) / d;
    return r > m ? r : m;
}
constexpr int XM_CNT_STRIDE = 32;   // ints between arrival counters (one 128-byte line each)
// out[y * gx + x] = the XCD that workgroup (x, y) of a (gx, gy) grid ran on
int launch_xcc_probe(hipStream_t st, int gx, int gy, int *out);

// QK-norm + RoPE of n_tok tokens' q (in place) and k, and the k/v cache
// store, for prefill.  qkv rows are [q | k | v] with row stride `stride`.
struct QkPostArgs {
    float *qkv; int stride;
    const float *q_norm, *k_norm;
    const float2 *rope;            // [ctx][hd/2] (cos, sin)
    float eps; int rope_style;
    void *kc, *vc;
    int kv_dim, hd, n_heads, n_kv, pos_base, n_tok;
    int kv_f16;                    // (launch_gemm_qkpost) the cache rows are fp16
    // (launch_gemm_qkpost, launch_gemm_qkv; optional) the K/V tile images of
    // the matrix-core prefill attention (AttnArgs::kvimg): the pass's own
    // tiles are written too; pos_base a multiple of 64
    uint8_t *kvimg; int kvimg_tiles;
};
int launch_qkpost(hipStream_t st, bool f16kv, const QkPostArgs &a);

// ------------------------------------------------------------ prefill GEMM --
// Q8_0-quantize n rows of activations (optionally RMSNorm-ed first):
//   qx[n][cols] int8, dx[n][cols/32] fp32 (the fp16-rounded block scales),
//   xs[n][cols/32] int32 block sums of the codes (Q4_0 weights need them).
struct QuantRowsArgs {
    const float *x; int x_stride, cols, n;
    int swiglu;                           // row value i = silu(x[i]) * x[cols + i]
    const float *norm_w; float eps;       // nullptr: no norm
    const int *ids; DMat emb; float *x_out;  // ids != nullptr: embed rows first
    float *xf;                            // fp32 copy of the (normed) rows, F32 weights
    int8_t *qx; float *dx; int *xs;
};
int launch_quant_rows(hipStream_t st, const QuantRowsArgs &a);

// Y = X . W^T over n tokens, fused epilogues as in matvec (EPI_*), with the
// activations already quantized by launch_quant_rows.
struct GemmArgs {
    DMat W;
    int units, pair_off, n;
    const int8_t *qx; const float *dx; const int *xs;  // quantized X
    const float *xf;                                     // fp32 X (F32 weights)
    float *out; int out_stride;
    const float *bias;
    // launch_gemm_swiglu: the SwiGLU rows' Q8_0 codes [n][units], fp16-rounded
    // block scales and code sums [n][units / 32], for the next product
    int8_t *oq; float *odx; int *oxs;
};
int launch_gemm(hipStream_t st, int epi, const GemmArgs &a);
// The w1|w3 product of a short prompt with the SwiGLU and its Q8_0
// quantization in the epilogue: W holds the gate rows, then the up rows at
// pair_off; units = hidden units (a multiple of 32).  out, when set, also
// receives the gate | up products (out_stride floats per token).  Returns -1
// where gemm_swiglu_fits() is false.
bool gemm_swiglu_fits(const GemmArgs &a);
// the same for the passes launch_gemm gives the matrix-core tiles: the
// gate | up rows paired per tile, SwiGLU and quantization in the epilogue
// (units a multiple of 64)
bool gemm_swiglu_long_fits(const GemmArgs &a);
int launch_gemm_swiglu(hipStream_t st, const GemmArgs &a);
// The q|k|v product of a short prompt with launch_qkpost's work (bias, then
// QK-norm and RoPE of the q and k heads, q written back into p.qkv, k and v
// stored to the cache) in the epilogue: one head vector per workgroup.  g is
// the product (units = (n_heads + 2 n_kv) hd, out unused); raw, when set,
// receives the product with its bias ([n][p.stride]).  Returns -1 where
// gemm_qkv_fits() is false.
bool gemm_qkv_fits(const GemmArgs &g, const QkPostArgs &p);
// The q|k|v product of a longer prompt (k_gemm_mfma's shapes) with
// launch_qkpost's work in the epilogue, for 128-dim heads with neox RoPE;
// a.out, when set, also receives the raw product.  Returns -1 where
// gemm_qkpost_fits() is false.
bool gemm_qkpost_fits(const GemmArgs &g, const QkPostArgs &p);
int launch_gemm_qkpost(hipStream_t st, bool f16kv, const GemmArgs &a, const QkPostArgs &p);
int launch_gemm_qkv(hipStream_t st, bool f16kv, const GemmArgs &g, const QkPostArgs &p, float *raw);

// ---------------------------------------------------------------- sample --
// Greedy selection (first maximum) over n logits; writes tokpos[0] = token,
// tokpos[1] += 1 and appends the token to out[tokpos[2]++] (when < cap).
struct ArgmaxArgs {
    const float *logits; int n;
    float *pval; int *pidx;     // [ARGMAX_MAX_BLOCKS] per-workgroup winners
    int *tokpos;                // device {tok, pos, n_generated}
    int *out; int cap;
};
constexpr int ARGMAX_MAX_BLOCKS = 256;
int launch_argmax(hipStream_t st, const ArgmaxArgs &a);
// The merge step alone: first maximum over `nparts` (value, index) winners,
// n = the number of logits they cover (for the out-of-range guard).
int launch_argmax_merge(hipStream_t st, const float *pval, const int *pidx, int nparts, int n,
                        int *tokpos, int *out, int cap);

// ---------------------------------------------------------- full sampler --
// ember_sample (src/sample.c:76-175) on the device: penalties over a device
// history ring, then either the first maximum (temperature <= 0) or
// temperature -> softmax -> top-k -> min-p -> top-p -> one xorshift64* draw,
// for any top_k (0 = no cap).  The chosen token is accepted into the ring and
// fed to the decode loop as the argmax path does (tokpos/out).
struct SampleParams {
    float temperature, top_p, min_p, repeat_penalty, presence_penalty, frequency_penalty;
    int top_k;
};
constexpr int SAMPLE_TOPK_MAX = 64, SAMPLE_GRID = 64, SAMPLE_SLICE_MAX = 4096;
struct SampleArgs {
    float *logits; int n;            // device logits (penalties update them in place, as the reference does)
    SampleParams p;
    unsigned long long *rng;         // device xorshift64* state
    int *hist, *hist_meta;           // ring [hist_cap]; {hist_len, hist_pos}
    int hist_cap;
    float *psum;                     // [SAMPLE_GRID] slice sums of e
    int *scnt;                       // [SAMPLE_GRID] tokens per slice, then the arrival counter (zeroed)
    float *cval; int *cidx;          // [SAMPLE_GRID][SAMPLE_TOPK_MAX] tokens passed on
    float *am_val; int *am_idx;      // per-part maxima (the greedy winners)
    int nparts;                      // > 0: am_val already holds that many for these logits
    int *tokpos; int *out; int cap;  // as ArgmaxArgs
    // top_k = 0 or > SAMPLE_TOPK_MAX: every token's e [n], the sort keys
    // [2][sample_wide_pad(n)] and the running sums of the walk [n]
    float *we; unsigned long long *wkeys; float *wcum;
    // 1: that whole-vocabulary path for every top_k, so the softmax sum is
    // the reference's sequential one too (the reference-order mode)
    int exact;
};
int launch_sample(hipStream_t st, const SampleArgs &a);
// keys sorted per sampler call with any top_k: n rounded up to a power of two
// of at least one sort tile
constexpr int SAMPLE_WIDE_TILE = 4096;
inline int sample_wide_pad(int n) {
    int p = SAMPLE_WIDE_TILE;
    while (p < n) p <<= 1;
    return p;
}
// ehip_last_error()'s text for this thread (ehip.hip)
void set_error_text(const char *msg);
// Whether launch_sample applies penalties (which change the logits after the
// per-part maxima were taken).
bool sample_penalized(const SampleArgs &a);

}  // namespace ehip
