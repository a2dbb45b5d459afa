// ehip.hip — the C-ABI device layer (include/ehip.h): weight upload and
// repacking, per-state device buffers, and the decode / prefill schedules.
//
// Decode step (replaces ember_forward, src/model.c:362-414), 5 kernels per
// layer plus one for the head, all on the state's stream:
//   qkv   : matvec  RMSNorm(attn_norm) + Q8_0 prologue, [wq;wk;wv] rows,
//           bias epilogue          (layer 0 also gathers the embedding row)
//   attn  : fused QK-norm + RoPE + KV store + split-K GQA attention
//   wo    : matvec  Q8_0 prologue, residual epilogue
//   w13   : matvec  RMSNorm(ffn_norm) + Q8_0 prologue, [w1;w3] rows, SwiGLU
//   w2    : matvec  Q8_0 prologue, residual epilogue
//   head  : matvec  RMSNorm(final_norm) + Q8_0 prologue -> logits
// The token and position live in device memory, copied from pinned host
// memory by the first node, so one captured hipGraph replays every step.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../../include/ember.h"
#include "../../../include/ehip.h"
#include "kernels.h"
#include "libm_expf.h"
#include "staging.h"

using namespace ehip;

static thread_local char g_err[512];

static void set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

#define HCHK(call, ret)                                                                  \
    do {                                                                                 \
        hipError_t e_ = (call);                                                          \
        if (e_ != hipSuccess) {                                                          \
            set_err("%s failed: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, __LINE__); \
            return ret;                                                                  \
        }                                                                                \
    } while (0)

extern "C" const char *ehip_last_error(void) { return g_err; }

void ehip::set_error_text(const char *msg) { snprintf(g_err, sizeof g_err, "%s", msg); }

extern "C" int ehip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

// ---------------------------------------------------------------- model ----
struct DevLayer {
    DMat qkv, wo, w13, w2;
    float *attn_norm, *ffn_norm, *q_norm, *k_norm, *bias_qkv;
};

struct EhipModel {
    EhipConfig cfg;
    std::vector<DevLayer> layers;
    DMat emb, head;
    float *final_norm;
    std::vector<float> inv_freq;   // host copy: 1/theta^(2i/hd), the reference's expression
    std::vector<void *> allocs;
    uint64_t bytes;
    bool any_f32;
};

static void *dev_alloc(EhipModel *m, size_t n) {
    void *p = nullptr;
    if (hipMalloc(&p, n ? n : 1) != hipSuccess) return nullptr;
    m->allocs.push_back(p);
    m->bytes += n;
    return p;
}

static size_t file_row_bytes(int dt, int cols) {
    return dt == DT_F32 ? (size_t)cols * 4 : (size_t)(cols / QB) * (dt == DT_Q8 ? 34 : 18);
}

// Weight upload.  Every matrix is first allocated in its device layout and
// described by one job per file tensor; the jobs' row bytes then stream
// through a ring of pinned host slots, several tensors to a slot: host
// threads copy the slot's rows out of the mapped file, the slot's DMA to a
// device staging buffer and one repack launch per tensor in it are queued on
// the upload stream, and the slot is reused once its event has passed, so the
// host copy of one slot overlaps the transfer and repack of the previous ones.
// The repack only moves bytes (each block's fp16 scale to the scale array,
// its 32 or 16 quant bytes to the row's payload), so the device matrix holds
// the file's values exactly.
__global__ void k_repack_blocks(const uint16_t *__restrict__ src, int nrows, int nb, int bs_half,
                                uint8_t *__restrict__ q, size_t qrow, uint16_t *__restrict__ d, size_t row0) {
    const size_t nblk = (size_t)nrows * nb;
    const int pay_half = bs_half - 1;
    for (size_t b = blockIdx.x * (size_t)blockDim.x + threadIdx.x; b < nblk; b += (size_t)gridDim.x * blockDim.x) {
        const size_t r = b / nb, j = b % nb;
        const uint16_t *blk = src + b * bs_half;
        d[(row0 + r) * nb + j] = blk[0];
        uint16_t *dst = reinterpret_cast<uint16_t *>(q + (row0 + r) * qrow + j * (size_t)(2 * pay_half));
        for (int i = 0; i < pay_half; i++) dst[i] = blk[1 + i];
    }
}

namespace {

// Rows [0, nrows) of one file tensor (row bytes frb) into rows row0.. of a
// device matrix (payload q with row pitch qrow, scales d; F32: q only).
struct UploadJob {
    const uint8_t *src;
    int nrows, dt, nb;
    size_t frb, qrow, row0;
    uint8_t *q;
    uint16_t *d;
};

struct WeightStager {
    static constexpr int SLOTS = 3;
    static constexpr size_t SLOT_MAX = (size_t)32 << 20;
    struct Seg { size_t job, r, n, off; };   // rows [r, r+n) of a job at slot offset off
    size_t slot_bytes;
    hipStream_t st = nullptr;
    uint8_t *pin[SLOTS] = {}, *dev[SLOTS] = {};
    hipEvent_t ev[SLOTS] = {};
    int next = 0, threads = 1;
    bool ok = false;

    // `total`: the file bytes of all weight tensors; slots need not exceed it.
    explicit WeightStager(size_t total) : slot_bytes(std::min(SLOT_MAX, std::max<size_t>(total, 4096))) {
        if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) { st = nullptr; return; }
        for (int i = 0; i < SLOTS; i++) {
            if (hipHostMalloc(reinterpret_cast<void **>(&pin[i]), slot_bytes, hipHostMallocDefault) != hipSuccess) {
                pin[i] = nullptr;
                return;
            }
            if (hipMalloc(reinterpret_cast<void **>(&dev[i]), slot_bytes) != hipSuccess) { dev[i] = nullptr; return; }
            if (hipEventCreateWithFlags(&ev[i], hipEventDisableTiming) != hipSuccess) { ev[i] = nullptr; return; }
        }
        threads = staging_threads();
        ok = true;
    }
    ~WeightStager() {
        if (st) (void)hipStreamSynchronize(st);
        for (int i = 0; i < SLOTS; i++) {
            if (ev[i]) (void)hipEventDestroy(ev[i]);
            if (dev[i]) (void)hipFree(dev[i]);
            if (pin[i]) (void)hipHostFree(pin[i]);
        }
        if (st) (void)hipStreamDestroy(st);
    }

    // Copy the slot's segments out of the mapped file into pin[k].
    void fill(int k, const std::vector<UploadJob> &jobs, const std::vector<Seg> &segs) {
        std::vector<CopySpan> spans;
        for (const Seg &g : segs)
            spans.push_back({ pin[k] + g.off, jobs[g.job].src + g.r * jobs[g.job].frb, g.n * jobs[g.job].frb });
        parallel_copy(spans, threads);
    }

    bool flush(const std::vector<UploadJob> &jobs, std::vector<Seg> &segs, size_t used) {
        if (segs.empty()) return true;
        const int k = next;
        next = (next + 1) % SLOTS;
        HCHK(hipEventSynchronize(ev[k]), false);   // the DMA and repacks that last used the slot are done
        fill(k, jobs, segs);
        HCHK(hipMemcpyAsync(dev[k], pin[k], used, hipMemcpyHostToDevice, st), false);
        for (const Seg &g : segs) {
            const UploadJob &j = jobs[g.job];
            if (j.dt == DT_F32) {
                HCHK(hipMemcpyAsync(j.q + (j.row0 + g.r) * j.qrow, dev[k] + g.off, g.n * j.frb,
                                    hipMemcpyDeviceToDevice, st), false);
                continue;
            }
            const size_t nblk = g.n * (size_t)j.nb;
            const int grid = (int)std::min<size_t>(4096, (nblk + 255) / 256);
            k_repack_blocks<<<grid, 256, 0, st>>>(reinterpret_cast<const uint16_t *>(dev[k] + g.off), (int)g.n,
                                                  j.nb, j.dt == DT_Q8 ? 17 : 9, j.q, j.qrow, j.d, j.row0 + g.r);
            HCHK(hipGetLastError(), false);
        }
        HCHK(hipEventRecord(ev[k], st), false);
        segs.clear();
        return true;
    }

    // Stream every job through the slots, then wait for the last repack.
    bool run(const std::vector<UploadJob> &jobs) {
        std::vector<Seg> segs;
        size_t used = 0;
        for (size_t i = 0; i < jobs.size(); i++) {
            const UploadJob &j = jobs[i];
            if (j.frb > slot_bytes) { set_err("a weight row of %zu bytes exceeds the upload slot", j.frb); return false; }
            for (size_t r = 0; r < (size_t)j.nrows;) {
                const size_t fit = (slot_bytes - used) / j.frb;
                if (fit == 0) {
                    if (!flush(jobs, segs, used)) return false;
                    used = 0;
                    continue;
                }
                const size_t n = std::min(fit, (size_t)j.nrows - r);
                segs.push_back({ i, r, n, used });
                used = std::min(slot_bytes, (used + n * j.frb + 15) & ~(size_t)15);
                r += n;
            }
        }
        if (!flush(jobs, segs, used)) return false;
        HCHK(hipStreamSynchronize(st), false);
        return true;
    }
};

}  // namespace

// Allocate row-concatenated matrices (all of one dtype and width) in the
// device layout described in dev_common.h and queue one upload job per file
// tensor.
static bool upload_mat(EhipModel *m, std::vector<UploadJob> &jobs, DMat *out, const EhipWeight *parts,
                       const int *rows, int nparts, int cols, const char *what) {
    const int dt = parts[0].dtype;
    int R = 0;
    for (int i = 0; i < nparts; i++) {
        if (!parts[i].data) { set_err("missing tensor for %s", what); return false; }
        if (parts[i].dtype != dt) { set_err("%s: mixed weight encodings are not supported", what); return false; }
        R += rows[i];
    }
    if (dt != DT_F32 && dt != DT_Q8 && dt != DT_Q4) { set_err("%s: unsupported dtype %d", what, dt); return false; }
    if (dt != DT_F32 && cols % QB) { set_err("%s: row length %d not a multiple of 32", what, cols); return false; }
    const int nb = cols / QB;
    const size_t qrow = dt == DT_F32 ? (size_t)cols * 4 : (dt == DT_Q8 ? (size_t)cols : (size_t)cols / 2);
    const size_t qbytes = qrow * R, dbytes = dt == DT_F32 ? 0 : (size_t)R * nb * 2;
    const size_t qpad = (qbytes + 255) & ~(size_t)255;
    uint8_t *dev = static_cast<uint8_t *>(dev_alloc(m, qpad + dbytes));
    if (!dev) { set_err("hipMalloc of %zu bytes for %s failed", qpad + dbytes, what); return false; }
    uint16_t *dsc = dt == DT_F32 ? nullptr : reinterpret_cast<uint16_t *>(dev + qpad);
    const size_t frb = file_row_bytes(dt, cols);
    size_t r0 = 0;
    for (int p = 0; p < nparts; p++) {
        jobs.push_back({ static_cast<const uint8_t *>(parts[p].data), rows[p], dt, nb, frb, qrow, r0, dev, dsc });
        r0 += rows[p];
    }
    out->dtype = dt; out->rows = R; out->cols = cols;
    out->q = dev;
    out->d = dsc;
    if (dt == DT_F32) m->any_f32 = true;
    return true;
}

static float *upload_f32(EhipModel *m, const float *const *parts, const int *lens, int nparts) {
    size_t n = 0;
    for (int i = 0; i < nparts; i++) n += lens[i];
    std::vector<float> host(n, 0.0f);
    size_t o = 0;
    for (int i = 0; i < nparts; i++) {
        if (parts[i]) memcpy(host.data() + o, parts[i], lens[i] * sizeof(float));
        o += lens[i];
    }
    float *dev = static_cast<float *>(dev_alloc(m, n * 4));
    if (!dev) { set_err("hipMalloc of %zu bytes failed", n * 4); return nullptr; }
    if (hipMemcpy(dev, host.data(), n * 4, hipMemcpyHostToDevice) != hipSuccess) {
        set_err("hipMemcpy of a vector failed");
        return nullptr;
    }
    return dev;
}

extern "C" void ehip_model_free(EhipModel *m) {
    if (!m) return;
    for (void *p : m->allocs) (void)hipFree(p);
    delete m;
}

extern "C" uint64_t ehip_model_bytes(const EhipModel *m) { return m ? m->bytes : 0; }

static bool upload_weights(EhipModel *m, std::vector<UploadJob> &jobs, const EhipLayer *layers, EhipWeight tok_emb,
                           EhipWeight lm_head, const float *final_norm) {
    const EhipConfig &c = m->cfg;
    const int hd = c.head_dim, qd = c.n_heads * hd, kvd = c.n_kv_heads * hd;
    m->layers.resize(c.n_layers);
    for (int l = 0; l < c.n_layers; l++) {
        const EhipLayer &y = layers[l];
        DevLayer &d = m->layers[l];
        char what[64];
        snprintf(what, sizeof what, "layer %d qkv", l);
        EhipWeight qkv[3] = { y.wq, y.wk, y.wv };
        int qkv_rows[3] = { qd, kvd, kvd };
        if (!upload_mat(m, jobs, &d.qkv, qkv, qkv_rows, 3, c.dim, what)) return false;
        snprintf(what, sizeof what, "layer %d wo", l);
        if (!upload_mat(m, jobs, &d.wo, &y.wo, &c.dim, 1, qd, what)) return false;
        EhipWeight w13[2] = { y.w1, y.w3 };
        int rows13[2] = { c.hidden_dim, c.hidden_dim };
        snprintf(what, sizeof what, "layer %d w1|w3", l);
        if (!upload_mat(m, jobs, &d.w13, w13, rows13, 2, c.dim, what)) return false;
        snprintf(what, sizeof what, "layer %d w2", l);
        if (!upload_mat(m, jobs, &d.w2, &y.w2, &c.dim, 1, c.hidden_dim, what)) return false;
        const float *an = y.attn_norm, *fn = y.ffn_norm;
        if (!(d.attn_norm = upload_f32(m, &an, &c.dim, 1))) return false;
        if (!(d.ffn_norm = upload_f32(m, &fn, &c.dim, 1))) return false;
        d.q_norm = d.k_norm = nullptr;
        if (c.qk_norm && y.q_norm) {
            if (!y.k_norm) { set_err("layer %d has q_norm but no k_norm", l); return false; }
            if (!(d.q_norm = upload_f32(m, &y.q_norm, &hd, 1))) return false;
            if (!(d.k_norm = upload_f32(m, &y.k_norm, &hd, 1))) return false;
        }
        d.bias_qkv = nullptr;
        if (y.bq || y.bk || y.bv) {
            const float *bp[3] = { y.bq, y.bk, y.bv };
            int bl[3] = { qd, kvd, kvd };
            if (!(d.bias_qkv = upload_f32(m, bp, bl, 3))) return false;
        }
    }
    if (!upload_mat(m, jobs, &m->emb, &tok_emb, &c.vocab_size, 1, c.dim, "tok_embeddings")) return false;
    if (lm_head.data == tok_emb.data) m->head = m->emb;
    else if (!upload_mat(m, jobs, &m->head, &lm_head, &c.vocab_size, 1, c.dim, "lm_head")) return false;
    if (!(m->final_norm = upload_f32(m, &final_norm, &c.dim, 1))) return false;
    return true;
}

extern "C" EhipModel *ehip_model_upload(const EhipConfig *cfg, const EhipLayer *layers, EhipWeight tok_emb,
                                        EhipWeight lm_head, const float *final_norm,
                                        const float *rope_inv_freq) {
    const EhipConfig &c = *cfg;
    const int hd = c.head_dim;
    if (c.n_kv_heads <= 0 || c.n_heads % c.n_kv_heads) { set_err("n_heads must be a multiple of n_kv_heads"); return nullptr; }
    if (hd != 48 && hd != 64 && hd != 128) { set_err("head_dim %d not supported by the attention kernel", hd); return nullptr; }
    if (c.n_heads / c.n_kv_heads > 8) { set_err("more than 8 query heads per kv head"); return nullptr; }
    if (tok_emb.dtype != DT_F32 && tok_emb.dtype != DT_Q8) { set_err("embedding must be F32 or Q8_0"); return nullptr; }
    if (hipSetDevice(0) != hipSuccess) { set_err("hipSetDevice(0) failed: no usable GPU"); return nullptr; }
    EhipModel *m = new EhipModel();
    m->cfg = c;
    m->bytes = 0;
    m->any_f32 = false;
    m->inv_freq.assign(rope_inv_freq, rope_inv_freq + hd / 2);
    std::vector<UploadJob> jobs;
    bool ok = upload_weights(m, jobs, layers, tok_emb, lm_head, final_norm);
    if (ok) {
        size_t total = 0;
        for (const UploadJob &j : jobs) total += j.nrows * j.frb;
        WeightStager up(total);   // its destructor waits for the upload stream
        if (!up.ok) set_err("allocating the weight upload buffers failed");
        ok = up.ok && up.run(jobs);
    }
    if (!ok) {
        ehip_model_free(m);
        return nullptr;
    }
    return m;
}

// ---------------------------------------------------------------- state ----
constexpr int PF_CHUNK = 4096;  // prefill tokens per pass through the layers (at most)
constexpr size_t PF_SCORES_MAX = (size_t)1 << 30;   // bytes of attention scores per pass (at most)
// Prefill attention in the reference's summation order (the exact-order
// kernels) or on matrix cores (a running softmax over fp16 products of split
// operands).  A model whose every product has fewer than GEMM_SPLIT_MIN_K
// inputs keeps one sequential block sum per output in the prefill GEMMs, so
// with exact-order attention its prefill matches the reference's
// deterministic build to rounding: its passes of up to PF_EXACT_KEYS keys
// use the exact-order kernels.  Wider models split their longer block sums
// over pipelines (and sum decode products across lanes), so they run at the
// reference builds' own noise floor in any case: their attention runs on
// the matrix cores at every length (the one-kernel exact form, once the
// faster for passes of up to PF_FUSE_KEYS keys over at least 256
// workgroups, lost to the split key-tile attention: Qwen3-0.6B shape pp128
// 1.90 -> 1.82 ms, pp256 2.79 -> 2.50, stories110M shape pp128 0.62 ->
// 0.61; EHIP_PF_ATTN=exact still selects it).
constexpr int PF_EXACT_KEYS = 512;
constexpr int PF_GRAPHS = 8;   // prefill pass graphs kept per state
enum { PF_AUTO = 0, PF_EXACT = 1, PF_MFMA = 2 };

// A captured run of device-loop steps.  One graph launch per token leaves
// the GPU idle for ~7 us between graphs (against ~1.5 us between the kernels
// inside one), so the device loops capture GEN_UNROLL steps per graph; the
// steps read their token and position from device memory, so one graph
// serves any starting point.
constexpr int GEN_UNROLL = 8;
struct StepGraph {
    hipGraph_t g = nullptr;
    hipGraphExec_t x = nullptr;
};

static void graph_free(StepGraph &sg) {
    if (sg.x) (void)hipGraphExecDestroy(sg.x);
    if (sg.g) (void)hipGraphDestroy(sg.g);
    sg.x = nullptr;
    sg.g = nullptr;
}

struct EhipState {
    EhipModel *m;
    int ctx, f16kv, esize, graph_mode;
    hipStream_t st;
    void *kc, *vc;
    int *tokpos_d, *tokpos_h;   // {token, position, steps generated, API step ticket}
    int *done_h;                // pinned: the ticket of the last completed API step
    int ticket;
    float *x, *qkv, *o, *h, *logits_d, *logits_h;
    // the decode attention with the wo product folded in (attn_decode.hip,
    // merge mode 3): the kv groups' wo partials [n_kv][dim], their flags
    // [n_layers][n_kv][XM_CNT_STRIDE] (zero between launches), and a second
    // residual buffer: the w1|w3 matvec writes x + the partials there, so
    // the layers' residual alternates between x and x2
    float *x2, *wo_part;
    int *wo_flag;
    bool fw_cur;   // whether the decode launches enqueued last fold the wo product in
    // polls of a kv group's wo flag before the folded product gives up
    // (ATT_DEC_FW_SPIN; EHIP_FW_TEST_SPIN=n sets it, a test hook: 0 makes
    // every workgroup that finds the flag still down time out, so the
    // fallback can be exercised while the kernels run as usual)
    int fw_spin;
    // added to chunk 0's launch token in the in-kernel merge
    // (EHIP_XMERGE_TEST_TOK, a test hook: 1 makes every merge of a partial
    // of chunk 0 find a stale token, so the check's fallback can be
    // exercised while the kernels run as usual)
    int tok_skew;
    float *part;
    float2 *rope;   // [ctx][hd/2] (cos, sin) of pos * freq_i
    int mc_dec;     // chunks per kv head, two-kernel merge
    int xm_slots;   // slots per XCD, in-kernel merge (attn_decode.hip)
    // in-kernel merge of the decode attention chunks (see attn_decode.hip):
    // arrival counters [n_layers][n_kv][XM_CNT_STRIDE], the XCD of each kv
    // head's workgroups, and the error flag, which sits at logits_d[vocab] so
    // the per-step logits copy brings it to the host
    bool xm_on;
    int *xm_cnt, *xm_xcc, *xm_err;
    // prefill scratch
    float *X, *QKV, *O, *H, *xf, *dxp;
    int8_t *qx; int *xsum, *ids_d;
    int8_t *qx2; float *dxp2; int *xsum2;   // the w2 input's codes when the w1|w3 product quantizes them
    // prefill attention scratch: scores [n_heads][pf_chunk][ldk], tile maxima
    // [n_heads][pf_chunk][attn_prefill_tiles(ldk)], row max and 1/sum [n_heads][pf_chunk]
    float *pf_scores, *pf_tmax, *pf_rowmax, *pf_rowinv;
    uint8_t *pf_kvimg;  // K/V tile images of the matrix-core prefill attention
    int pf_kvimg_tiles;
    int pf_chunk;       // tokens per prefill pass
    // prefill attention: the reference's summation order (three kernels and
    // the score scratch above) for passes whose keys fit in PF_EXACT_KEYS,
    // the matrix-core kernel with a running softmax beyond (PF_AUTO);
    // EHIP_PF_ATTN=exact or =mfma forces one of them for every pass
    int pf_mode;
    bool pf_seq;        // every product has fewer than GEMM_SPLIT_MIN_K inputs
    // EHIP_ORDER=reference: every decode kernel in the reference's floating-
    // point order (reforder.hip), prefill as one decode step per token (the
    // reference's prefill computes exactly its forward steps); att_ref is the
    // attention's score scratch [n_heads][ctx]
    bool ref_order;
    float *att_ref;
    // device greedy loop: argmax partials, counter, generated tokens [ctx]
    float *am_val; int *am_idx; int *gen_tok;
    hipGraph_t graph; hipGraphExec_t gexec;
    // one hipGraph per prefill pass shape (first position, tokens, whether it
    // ends the prompt and so runs the head), least recently used evicted
    struct PfGraph { StepGraph sg; int pos0 = -1, n = 0, last = 0; unsigned long long used = 0; };
    PfGraph pfg[PF_GRAPHS];
    unsigned long long pf_clock = 0;
    StepGraph gen[2];   // device greedy loop: 1 step, GEN_UNROLL steps
    // device sampler: xorshift64* state, history ring, candidates; the
    // sampling decode graph is captured for one parameter set
    unsigned long long *smp_rng; int *smp_meta, *smp_hist; int smp_hist_cap;
    float *smp_psum, *smp_cval; int *smp_cidx, *smp_cnt;
    // sampling with any top_k: every token's e, sort keys, running sums
    float *smp_we, *smp_wcum; unsigned long long *smp_wk;
    StepGraph smp[2];   // device sampling loop: 1 step, GEN_UNROLL steps
    SampleParams smp_graph_p; int smp_graph_cap;
    hipEvent_t ev0, ev1;
    // per-layer capture of the decode step's intermediate vectors
    // (ehip_debug_capture): layer, or -1; one device buffer per DBG_* slot
    int dbg_layer = -1;
    float *dbg[6] = {};
    // the same for one layer of one prefill pass (ehip_debug_capture_prefill)
    int pdbg_layer = -1, pdbg_pass = 0, pdbg_n = 0, pdbg_pos = 0;
    float *pdbg[6] = {};
    std::vector<void *> allocs;
};
// slots of ehip_debug_capture
enum { DBG_XIN = 0, DBG_QKV = 1, DBG_O = 2, DBG_XMID = 3, DBG_H = 4, DBG_XOUT = 5 };

template <class F>
static int graph_capture(EhipState *s, StepGraph &sg, int steps, F enq) {
    graph_free(sg);
    HCHK(hipStreamBeginCapture(s->st, hipStreamCaptureModeThreadLocal), -1);
    int rc = 0;
    for (int i = 0; i < steps && !rc; i++) rc = enq();
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(s->st, &g);
    if (rc) { if (g) (void)hipGraphDestroy(g); return -1; }
    if (e != hipSuccess) { set_err("hipStreamEndCapture: %s", hipGetErrorString(e)); return -1; }
    sg.g = g;
    HCHK(hipGraphInstantiate(&sg.x, g, nullptr, nullptr, 0), -1);
    return 0;
}

static void *salloc(EhipState *s, size_t n, bool zero = false) {
    void *p = nullptr;
    if (hipMalloc(&p, n ? n : 1) != hipSuccess) return nullptr;
    if (zero && hipMemset(p, 0, n ? n : 1) != hipSuccess) { (void)hipFree(p); return nullptr; }
    s->allocs.push_back(p);
    return p;
}

extern "C" void ehip_state_destroy(EhipState *s) {
    if (!s) return;
    (void)hipStreamSynchronize(s->st);
    if (s->gexec) (void)hipGraphExecDestroy(s->gexec);
    if (s->graph) (void)hipGraphDestroy(s->graph);
    for (StepGraph &g : s->gen) graph_free(g);
    for (StepGraph &g : s->smp) graph_free(g);
    for (auto &pg : s->pfg) graph_free(pg.sg);
    if (s->smp_hist) (void)hipFree(s->smp_hist);
    for (void *p : s->allocs) (void)hipFree(p);
    if (s->tokpos_h) (void)hipHostFree(s->tokpos_h);
    if (s->done_h) (void)hipHostFree(s->done_h);
    if (s->logits_h) (void)hipHostFree(s->logits_h);
    if (s->ev0) (void)hipEventDestroy(s->ev0);
    if (s->ev1) (void)hipEventDestroy(s->ev1);
    (void)hipStreamDestroy(s->st);
    delete s;
}

static int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

// Decide whether the decode attention merges its chunks in-kernel: run the
// probe kernel on the attention's 1-D grid of 8 * xm_slots workgroups and
// require the workgroups L, L + 8, L + 16, ... (the chunks of the kv heads
// g = L % 8, L % 8 + 8, ...) to report one XCD (the dispatcher deals a
// grid's workgroups to the XCDs round-robin).  EHIP_XMERGE=0 forces the
// merge kernel.
static int xm_probe(EhipState *s) {
    const int nkv = s->m->cfg.n_kv_heads, gx = 8 * s->xm_slots;
    s->xm_on = false;
    if (!env_int("EHIP_XMERGE", 1) || s->ref_order) return 0;
    std::vector<int> h((size_t)gx, -1);
    int *d = nullptr;
    HCHK(hipMalloc(&d, 4 * h.size()), -1);
    const int rc = launch_xcc_probe(s->st, gx, 1, d);
    const hipError_t e1 = hipStreamSynchronize(s->st);
    const hipError_t e2 = hipMemcpy(h.data(), d, 4 * h.size(), hipMemcpyDeviceToHost);
    (void)hipFree(d);
    if (rc || e1 != hipSuccess || e2 != hipSuccess) { set_err("XCD probe kernel failed"); return -1; }
    bool ok = true;
    for (int L = 8; L < gx && ok; L++) ok = h[L] == h[L % 8];
    if (!ok) return 0;
    std::vector<int> xcc((size_t)nkv);
    for (int g = 0; g < nkv; g++) xcc[g] = h[g % 8];
    // EHIP_XMERGE_TEST_SKEW=k records every kv head's XCD as k further on
    // (test hook): each workgroup's own check then fails, so the error path
    // can be exercised while the kernels run exactly as usual
    const int skew = env_int("EHIP_XMERGE_TEST_SKEW", 0);
    if (skew)
        for (int g = 0; g < nkv; g++) xcc[g] = (xcc[g] + skew) & 7;
    HCHK(hipMemcpy(s->xm_xcc, xcc.data(), 4 * (size_t)nkv, hipMemcpyHostToDevice), -1);
    s->xm_on = true;
    return 0;
}

// After a launch that found a workgroup on an unexpected XCD (or whose folded
// wo product timed out) the counters and flags may hold stale values: clear
// them with the error flag.
static int xm_reset(EhipState *s) {
    const EhipConfig &c = s->m->cfg;
    HCHK(hipMemsetAsync(s->xm_cnt, 0, 4 * (size_t)c.n_layers * c.n_kv_heads * XM_CNT_STRIDE, s->st), -1);
    HCHK(hipMemsetAsync(s->wo_flag, 0, 4 * (size_t)c.n_layers * c.n_kv_heads * XM_CNT_STRIDE, s->st), -1);
    HCHK(hipMemsetAsync(s->xm_err, 0, 4, s->st), -1);
    HCHK(hipStreamSynchronize(s->st), -1);
    return 0;
}

static void drop_step_graphs(EhipState *s);

// The fused merge found a workgroup off the XCD its kv head was recorded on,
// so that launch's merge (and every result after it) is invalid.  Switch the
// state to the two-kernel merge for good: clear the counters and the flag,
// and drop the captured graphs, which hold the fused kernel.  The caller
// re-runs the work from its start, which rewrites the KV rows it wrote.
static int xm_fallback(EhipState *s) {
    if (xm_reset(s)) return -1;
    s->xm_on = false;
    drop_step_graphs(s);
    return 0;
}

extern "C" EhipState *ehip_state_create(EhipModel *m, int ctx, int kv_fp16) {
    const EhipConfig &c = m->cfg;
    const int hd = c.head_dim, qd = c.n_heads * hd, kvd = c.n_kv_heads * hd;
    EhipState *s = new EhipState();  // value-initialised: every pointer starts null
    s->m = m; s->ctx = ctx; s->f16kv = kv_fp16 ? 1 : 0; s->esize = kv_fp16 ? 2 : 4;
    s->graph_mode = env_int("EHIP_GRAPH", 1);
    s->fw_spin = env_int("EHIP_FW_TEST_SPIN", ATT_DEC_FW_SPIN);
    s->tok_skew = env_int("EHIP_XMERGE_TEST_TOK", 0);
    if (hipStreamCreateWithFlags(&s->st, hipStreamNonBlocking) != hipSuccess) {
        set_err("hipStreamCreate failed");
        delete s;
        return nullptr;
    }
    const size_t kvb = (size_t)c.n_layers * ctx * kvd * s->esize;
    int n_cu = 0;
    if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess || n_cu <= 0) n_cu = 1;
    s->mc_dec = attn_decode_chunks(ctx, c.n_kv_heads, hd, n_cu);
    s->xm_slots = attn_decode_slots(ctx, c.n_kv_heads, n_cu);
    if (s->mc_dec <= 0) {
        set_err("head_dim %d not supported by the attention kernel", hd);
        ehip_state_destroy(s);
        return nullptr;
    }
    const size_t ldk_max = (size_t)attn_prefill_ldk(0, ctx);
    {
        const char *pa = getenv("EHIP_PF_ATTN");
        s->pf_mode = pa && !strcmp(pa, "exact") ? PF_EXACT : (pa && !strcmp(pa, "mfma") ? PF_MFMA : PF_AUTO);
    }
    s->pf_chunk = std::min(PF_CHUNK, ctx);
    if (s->pf_mode == PF_EXACT)
        s->pf_chunk = (int)std::max<size_t>(1, std::min<size_t>(s->pf_chunk, PF_SCORES_MAX / (4 * ldk_max * c.n_heads)));
    const size_t pfc = (size_t)s->pf_chunk;
    // exact-order score scratch: every pass (PF_EXACT), or passes of up to
    // PF_EXACT_KEYS keys (PF_AUTO)
    const size_t ex_rows = s->pf_mode == PF_EXACT ? pfc : std::min<size_t>(pfc, PF_EXACT_KEYS);
    const size_t ex_ldk = s->pf_mode == PF_EXACT ? ldk_max : (size_t)attn_prefill_ldk(0, std::min(PF_EXACT_KEYS, ctx));
    const int wide = std::max(std::max(c.dim, c.hidden_dim), qd);
    s->pf_seq = wide < GEMM_SPLIT_MIN_K;
    {
        const char *ord = getenv("EHIP_ORDER");
        s->ref_order = ord && !strcmp(ord, "reference");
    }
    bool ok = (s->kc = salloc(s, kvb, true)) && (s->vc = salloc(s, kvb, true)) &&
              (s->tokpos_d = (int *)salloc(s, 16, true)) &&
              (s->x = (float *)salloc(s, 4 * (size_t)c.dim)) &&
              (s->qkv = (float *)salloc(s, 4 * (size_t)(qd + 2 * kvd))) &&
              (s->o = (float *)salloc(s, 4 * (size_t)qd)) &&
              (s->h = (float *)salloc(s, 4 * (size_t)c.hidden_dim)) &&
              (s->logits_d = (float *)salloc(s, 4 * ((size_t)c.vocab_size + 4), true)) &&
              (s->xm_cnt = (int *)salloc(s, 4 * (size_t)c.n_layers * c.n_kv_heads * XM_CNT_STRIDE, true)) &&
              (s->xm_xcc = (int *)salloc(s, 4 * (size_t)c.n_kv_heads)) &&
              (s->part = (float *)salloc(s, 4 * (size_t)c.n_heads * std::max(s->mc_dec, s->xm_slots) * (hd + 3))) &&
              (s->X = (float *)salloc(s, 4 * pfc * c.dim)) &&
              (s->QKV = (float *)salloc(s, 4 * pfc * (qd + 2 * kvd))) &&
              (s->O = (float *)salloc(s, 4 * pfc * qd)) &&
              (s->H = (float *)salloc(s, 4 * pfc * 2 * c.hidden_dim)) &&
              (s->qx = (int8_t *)salloc(s, pfc * wide)) &&
              (s->dxp = (float *)salloc(s, 4 * pfc * (wide / QB + 1))) &&
              (s->xsum = (int *)salloc(s, 4 * pfc * (wide / QB + 1))) &&
              (s->qx2 = (int8_t *)salloc(s, pfc * c.hidden_dim)) &&
              (s->dxp2 = (float *)salloc(s, 4 * pfc * (c.hidden_dim / QB + 1))) &&
              (s->xsum2 = (int *)salloc(s, 4 * pfc * (c.hidden_dim / QB + 1))) &&
              (s->ids_d = (int *)salloc(s, 4 * pfc)) &&

              (s->am_val = (float *)salloc(s, 4 * (size_t)std::max(ARGMAX_MAX_BLOCKS, MATVEC_MAX_GRID))) &&
              (s->am_idx = (int *)salloc(s, 4 * (size_t)std::max(ARGMAX_MAX_BLOCKS, MATVEC_MAX_GRID))) &&
              (s->gen_tok = (int *)salloc(s, 4 * (size_t)ctx, true)) &&
              (s->smp_rng = (unsigned long long *)salloc(s, 8)) &&
              (s->smp_meta = (int *)salloc(s, 8, true)) &&
              (s->smp_cnt = (int *)salloc(s, 4 * 2 * SAMPLE_GRID, true)) &&
              (s->smp_psum = (float *)salloc(s, 4 * SAMPLE_GRID)) &&
              (s->smp_cval = (float *)salloc(s, 4 * SAMPLE_GRID * SAMPLE_TOPK_MAX)) &&
              (s->smp_cidx = (int *)salloc(s, 4 * SAMPLE_GRID * SAMPLE_TOPK_MAX)) &&
              (s->smp_we = (float *)salloc(s, 4 * (size_t)c.vocab_size)) &&
              (s->smp_wcum = (float *)salloc(s, 4 * (size_t)c.vocab_size)) &&
              (s->smp_wk = (unsigned long long *)salloc(s, 8 * 2 * (size_t)sample_wide_pad(c.vocab_size))) &&
              (s->x2 = (float *)salloc(s, 4 * (size_t)c.dim)) &&
              (s->wo_part = (float *)salloc(s, 4 * (size_t)c.n_kv_heads * c.dim)) &&
              (s->wo_flag = (int *)salloc(s, 4 * (size_t)c.n_layers * c.n_kv_heads * XM_CNT_STRIDE, true));
    if (ok && m->any_f32) ok = (s->xf = (float *)salloc(s, 4 * pfc * wide)) != nullptr;
    if (ok && s->ref_order) ok = (s->att_ref = (float *)salloc(s, 4 * (size_t)c.n_heads * ctx)) != nullptr;
    if (ok && s->pf_mode != PF_EXACT && attn_kvimg_bytes(hd, s->f16kv, ctx, c.n_kv_heads) > 0) {
        s->pf_kvimg_tiles = (ctx + 63) / 64;
        ok = (s->pf_kvimg = (uint8_t *)salloc(s, attn_kvimg_bytes(hd, s->f16kv, ctx, c.n_kv_heads))) != nullptr;
    }
    if (ok && s->pf_mode != PF_MFMA)
        ok = (s->pf_scores = (float *)salloc(s, 4 * ex_rows * ex_ldk * c.n_heads)) &&
             (s->pf_rowinv = (float *)salloc(s, 4 * ex_rows * c.n_heads)) &&
             (s->pf_rowmax = (float *)salloc(s, 4 * ex_rows * c.n_heads)) &&
             (s->pf_tmax = (float *)salloc(s, 4 * ex_rows * c.n_heads * (size_t)attn_prefill_tiles((int)ex_ldk)));
    if (ok) {
        // RoPE table with the reference's arithmetic (model.c:69-71): the
        // angle pos * freq in fp32, then the host libm cosf / sinf
        const int half = hd / 2;
        std::vector<float2> tab((size_t)ctx * half);
        for (int p = 0; p < ctx; p++)
            for (int i = 0; i < half; i++) {
                const float ang = (float)p * m->inv_freq[i];
                tab[(size_t)p * half + i] = make_float2(cosf(ang), sinf(ang));
            }
        ok = (s->rope = (float2 *)salloc(s, sizeof(float2) * tab.size())) != nullptr &&
             hipMemcpy(s->rope, tab.data(), sizeof(float2) * tab.size(), hipMemcpyHostToDevice) == hipSuccess;
    }
    if (!ok) {
        set_err("device allocation for a state with ctx %d failed (KV %zu bytes)", ctx, 2 * kvb);
        ehip_state_destroy(s);
        return nullptr;
    }
    s->xm_err = reinterpret_cast<int *>(s->logits_d + c.vocab_size);
    if (ehip_noalloc_setup()) {   // ehip_sample_noalloc's scratch address on this device
        ehip_state_destroy(s);
        return nullptr;
    }
    if (xm_probe(s)) {
        ehip_state_destroy(s);
        return nullptr;
    }
    if (hipHostMalloc(&s->tokpos_h, 16, hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc(&s->done_h, 64, hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc(&s->logits_h, 4 * ((size_t)c.vocab_size + 4), hipHostMallocDefault) != hipSuccess ||
        hipEventCreate(&s->ev0) != hipSuccess || hipEventCreate(&s->ev1) != hipSuccess) {
        set_err("pinned host allocation failed");
        ehip_state_destroy(s);
        return nullptr;
    }
    memset(s->logits_h, 0, 4 * ((size_t)c.vocab_size + 4));
    memset(s->tokpos_h, 0, 16);
    *s->done_h = 0;
    return s;
}

// ------------------------------------------------------------ schedules ----
static AttnArgs attn_args(EhipState *s, int l) {
    const EhipConfig &c = s->m->cfg;
    const DevLayer &y = s->m->layers[l];
    const int kvd = c.n_kv_heads * c.head_dim;
    AttnArgs a{};
    a.q_norm = y.q_norm; a.k_norm = y.k_norm; a.rope = s->rope;
    a.eps = c.norm_eps; a.inv_sqrt = 1.0f / sqrtf((float)c.head_dim);
    a.rope_style = c.rope_style;
    const size_t loff = (size_t)l * s->ctx * kvd * s->esize;
    a.kc = static_cast<uint8_t *>(s->kc) + loff;
    a.vc = static_cast<uint8_t *>(s->vc) + loff;
    a.kv_dim = kvd; a.hd = c.head_dim; a.n_heads = c.n_heads; a.n_kv = c.n_kv_heads; a.ctx = s->ctx;
    return a;
}

// a decode-step matvec: the fast kernel, or the reference-order one
static int mv(EhipState *s, int pro, int epi, const MatvecArgs &a) {
    return s->ref_order ? launch_matvec_ref(s->st, pro, epi, a) : launch_matvec(s->st, pro, epi, a);
}

// Whether the decode step folds the wo product into the attention: the
// in-kernel merge on the 2-D grid (kv heads a multiple of 8, merge mode 3,
// or 5 with a Q4_0 wo: query heads per kv head a power of two, one round of
// wo rows per workgroup) or on the 1-D grid (at most 8 kv heads, one per
// XCD, merge mode 4, Q8_0 wo: up to two rounds), with G * head_dim whole
// 32-weight blocks of 8-64 chunk lanes per row (the kernel's GM * head_dim
// / 16 for Q8_0, / 32 for Q4_0), and Q8_0 or Q4_0 w1|w3 in every layer.
// EHIP_FUSE_WO=0 turns it off.
static bool fw_usable(EhipState *s) {
    const EhipModel *m = s->m;
    const EhipConfig &c = m->cfg;
    if (!s->xm_on || s->ref_order || !env_int("EHIP_FUSE_WO", 1)) return false;
    const int nkv = c.n_kv_heads, G = c.n_heads / nkv, hd = c.head_dim;
    const int wdt = m->layers[0].wo.dtype;
    if (wdt != DT_Q8 && !(wdt == DT_Q4 && nkv % 8 == 0)) return false;
    const int GM = G <= 1 ? 1 : (G <= 2 ? 2 : (G <= 4 ? 4 : 8));
    const int cpr = GM * hd / (wdt == DT_Q4 ? 32 : 16), rpr = ATT_DEC_NW * 64 / cpr;
    if (G > 8 || (hd != 64 && hd != 128) || (G * hd) % QB || cpr < 8 || cpr > 64) return false;
    if (nkv > MATVEC_MAX_PARTS) return false;
    if (nkv % 8 == 0) {
        const int mc = 8 * s->xm_slots / nkv;
        if (G != GM || (c.dim + mc - 1) / mc > rpr) return false;
    } else if ((c.dim + s->xm_slots - 1) / s->xm_slots > (cpr >= 32 ? 2 : 1) * rpr) {
        return false;
    }
    for (int l = 0; l < c.n_layers; l++) {
        const DevLayer &y = m->layers[l];
        if (y.wo.dtype != wdt || (y.w13.dtype != DT_Q8 && y.w13.dtype != DT_Q4)) return false;
    }
    return true;
}

static int enq_attn_decode(EhipState *s, int l, bool with_merge = true, bool fw = false) {
    AttnArgs a = attn_args(s, l);
    a.q = s->qkv; a.q_stride = 0; a.tokpos = s->tokpos_d; a.pos_base = 0; a.n_tok = 1;
    if (s->ref_order) {
        a.out = s->o;
        return launch_attn_ref(s->st, s->f16kv, a, s->att_ref);
    }
    a.part = s->part; a.max_chunks = s->mc_dec;
    if (s->xm_on) {
        const int nkv = s->m->cfg.n_kv_heads;
        a.xm_slots = s->xm_slots;
        a.max_chunks = nkv % 8 == 0 ? 8 * s->xm_slots / nkv : s->xm_slots;
        a.xm_cnt = s->xm_cnt + (size_t)l * s->m->cfg.n_kv_heads * XM_CNT_STRIDE;
        a.xm_xcc = s->xm_xcc;
        a.xm_err = s->xm_err;
        a.tok_skew = s->tok_skew;
        if (fw) {
            const EhipConfig &c = s->m->cfg;
            a.wo = s->m->layers[l].wo;
            a.wo_part = s->wo_part;
            a.wo_flag = s->wo_flag + (size_t)l * c.n_kv_heads * XM_CNT_STRIDE;
            a.wo_rows = (c.dim + a.max_chunks - 1) / a.max_chunks;
            a.wo_spin = s->fw_spin;
        }
    }
    a.out = s->o;
    return launch_attn_decode(s->st, s->f16kv, a, with_merge);
}

static MatvecArgs head_args(EhipState *s, const float *xin) {
    const EhipModel *m = s->m;
    MatvecArgs a{};
    a.W = m->head; a.units = m->cfg.vocab_size; a.in = xin; a.norm_w = m->final_norm;
    a.eps = m->cfg.norm_eps; a.out = s->logits_d;
    return a;
}

static int enq_head(EhipState *s, const float *xin) {
    return mv(s, PRO_NORM, EPI_STORE, head_args(s, xin));
}

// w1|w3 + SwiGLU of layer l on the residual xin; with xnext (the folded wo
// product) the input is xin + the kv groups' wo partials, written to xnext
static int enq_w13(EhipState *s, int l, const float *xin, float *xnext = nullptr) {
    const EhipModel *m = s->m;
    const DevLayer &y = m->layers[l];
    MatvecArgs a{};
    a.W = y.w13; a.units = m->cfg.hidden_dim; a.pair_off = m->cfg.hidden_dim;
    a.in = xin; a.norm_w = y.ffn_norm; a.eps = m->cfg.norm_eps; a.out = s->h;
    if (!xnext) return mv(s, PRO_NORM, EPI_SWIGLU, a);
    a.parts = s->wo_part; a.n_parts = m->cfg.n_kv_heads; a.x_out = xnext;
    a.flag_reset = s->wo_flag + (size_t)l * m->cfg.n_kv_heads * XM_CNT_STRIDE;
    return mv(s, PRO_NORM_PARTS, EPI_SWIGLU, a);
}

// the residual after the last layer of the enqueued decode launches
static float *x_final(EhipState *s) {
    return s->fw_cur && (s->m->cfg.n_layers & 1) ? s->x2 : s->x;
}

// The layer launches of one decode step (the tokpos copy is the caller's).
static int enq_layers(EhipState *s) {
    const EhipModel *m = s->m;
    const EhipConfig &c = m->cfg;
    const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
    // copies of the captured layer's vectors into the debug slots
    auto snap = [&](int l, int slot, const float *src, int n) -> int {
        if (l != s->dbg_layer) return 0;
        HCHK(hipMemcpyAsync(s->dbg[slot], src, 4 * (size_t)n, hipMemcpyDeviceToDevice, s->st), -1);
        return 0;
    };
    // with the folded wo product the residual alternates: layer l reads
    // xs[l & 1], its w1|w3 matvec writes x + the attention's wo partials to
    // xs[(l + 1) & 1], which the w2 matvec then updates in place
    const bool fw = s->fw_cur = fw_usable(s);
    float *xs[2] = { s->x, fw ? s->x2 : s->x };
    for (int l = 0; l < c.n_layers; l++) {
        const DevLayer &y = m->layers[l];
        float *xin = xs[l & 1], *xnext = xs[(l + 1) & 1];
        MatvecArgs a{};
        a.W = y.qkv; a.units = qd + 2 * kvd; a.in = xin; a.norm_w = y.attn_norm; a.eps = c.norm_eps;
        a.tokpos = s->tokpos_d; a.emb = m->emb; a.x_out = xin; a.out = s->qkv; a.bias = y.bias_qkv;
        if (l > 0 && snap(l, DBG_XIN, xin, c.dim)) return -1;
        if (mv(s, l == 0 ? PRO_EMBED_NORM : PRO_NORM, EPI_STORE, a)) return -1;
        if (l == 0 && snap(l, DBG_XIN, xin, c.dim)) return -1;   // the embedding row it gathered
        if (snap(l, DBG_QKV, s->qkv, qd + 2 * kvd)) return -1;
        if (enq_attn_decode(s, l, true, fw)) return -1;
        if (snap(l, DBG_O, s->o, qd)) return -1;
        if (!fw) {
            MatvecArgs b{};
            b.W = y.wo; b.units = c.dim; b.in = s->o; b.out = xin;
            if (mv(s, PRO_PLAIN, EPI_RESID, b)) return -1;
            if (snap(l, DBG_XMID, xin, c.dim)) return -1;
        }
        if (enq_w13(s, l, xin, fw ? xnext : nullptr)) return -1;
        if (fw && snap(l, DBG_XMID, xnext, c.dim)) return -1;
        if (snap(l, DBG_H, s->h, c.hidden_dim)) return -1;
        MatvecArgs d{};
        d.W = y.w2; d.units = c.dim; d.in = s->h; d.out = xnext;
        if (mv(s, PRO_PLAIN, EPI_RESID, d)) return -1;
        if (snap(l, DBG_XOUT, xnext, c.dim)) return -1;
    }
    return 0;
}

static int enq_decode(EhipState *s) {
    if (enq_layers(s)) return -1;
    return enq_head(s, x_final(s));
}

// The API step's completion: its ticket (tokpos[3], copied in with the token)
// stored into pinned host memory by one lane after the head, with a
// system-scope release, so the host sees it once the logits are in host
// memory.  The host polls that word instead of waking from
// hipStreamSynchronize (about 5 us sooner per step).
__global__ void k_step_done(const int *tokpos, int *done_h) {
    if (threadIdx.x == 0) __hip_atomic_store(done_h, tokpos[3], __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// One API decode step: token, position and ticket in (one 16-byte copy), the
// layers, the head, the logits out, the ticket back.  The quantized heads
// store the logits (and the error flag behind them) straight into the pinned
// host buffer as they are produced, so the PCIe writes overlap the head's
// weight stream (a copy after the head added about 12 us per step); the F32
// and reference-order heads are followed by a copy.
static int enq_step(EhipState *s) {
    const int V = s->m->cfg.vocab_size;
    HCHK(hipMemcpyAsync(s->tokpos_d, s->tokpos_h, 16, hipMemcpyHostToDevice, s->st), -1);
    if (enq_layers(s)) { set_err("a decode kernel could not be launched for this shape"); return -1; }
    const bool direct = !s->ref_order && s->m->head.dtype != DT_F32;
    MatvecArgs a = head_args(s, x_final(s));
    if (direct) a.out_host = s->logits_h;
    if (mv(s, PRO_NORM, EPI_STORE, a)) { set_err("lm_head launch failed"); return -1; }
    if (!direct)
        HCHK(hipMemcpyAsync(s->logits_h, s->logits_d, 4 * ((size_t)V + 1), hipMemcpyDeviceToHost, s->st), -1);
    hipLaunchKernelGGL(k_step_done, dim3(1), dim3(64), 0, s->st, (const int *)s->tokpos_d, s->done_h);
    HCHK(hipGetLastError(), -1);
    return 0;
}

// Wait for the API step holding `ticket`: poll the pinned word its last
// kernel writes, querying the stream now and then so that a failed launch
// ends the wait with an error.
static int wait_step(EhipState *s, int ticket) {
    for (unsigned long k = 1;; k++) {
        if (__atomic_load_n(s->done_h, __ATOMIC_ACQUIRE) == ticket) return 0;
        if ((k & 1023) == 0) {
            const hipError_t q = hipStreamQuery(s->st);
            if (q == hipErrorNotReady) continue;
            if (q != hipSuccess) { set_err("decode step: %s", hipGetErrorString(q)); return -1; }
            if (__atomic_load_n(s->done_h, __ATOMIC_ACQUIRE) == ticket) return 0;
            set_err("decode step: the stream finished without the step's completion word");
            return -1;
        }
        __builtin_ia32_pause();
    }
}

static int run_step(EhipState *s) {
    if (s->graph_mode) {
        if (!s->gexec) {
            HCHK(hipStreamBeginCapture(s->st, hipStreamCaptureModeThreadLocal), -1);
            int rc = enq_step(s);
            hipGraph_t g = nullptr;
            hipError_t e = hipStreamEndCapture(s->st, &g);
            if (rc) { if (g) (void)hipGraphDestroy(g); return -1; }
            if (e != hipSuccess) { set_err("hipStreamEndCapture: %s", hipGetErrorString(e)); return -1; }
            s->graph = g;
            HCHK(hipGraphInstantiate(&s->gexec, g, nullptr, nullptr, 0), -1);
        }
        HCHK(hipGraphLaunch(s->gexec, s->st), -1);
    } else if (enq_step(s)) {
        return -1;
    }
    return 0;
}

extern "C" float *ehip_forward(EhipState *s, int tok, int pos) {
    s->tokpos_h[0] = tok;
    s->tokpos_h[1] = pos;
    s->tokpos_h[2] = 0;
    for (int attempt = 0; attempt < 2; attempt++) {
        const int ticket = s->tokpos_h[3] = ++s->ticket;
        if (run_step(s)) return nullptr;
        if (wait_step(s, ticket)) return nullptr;
        int flag;
        memcpy(&flag, s->logits_h + s->m->cfg.vocab_size, 4);
        if (!flag) return s->logits_h;
        if (!s->xm_on || xm_fallback(s)) break;   // re-run the step on the two-kernel schedule
    }
    set_err("decode attention: the chunk merge reported an error on the two-kernel schedule");
    return nullptr;
}

// The error flag after a device-held loop: 0 clear, 1 raised (and the state
// switched to the two-kernel schedule: re-run the loop), -1 failure.
static int xm_flag(EhipState *s) {
    int flag = 0;
    HCHK(hipMemcpy(&flag, s->xm_err, 4, hipMemcpyDeviceToHost), -1);
    if (!flag) return 0;
    if (!s->xm_on) { set_err("decode attention: the chunk merge reported an error on the two-kernel schedule"); return -1; }
    return xm_fallback(s) ? -1 : 1;
}

// One step of the device-resident greedy loop: the decode launches, then the
// argmax that feeds the chosen token back into tokpos.
static int enq_gen_step(EhipState *s) {
    if (s->m->head.dtype != DT_F32) {   // argmax fused into the lm_head matvec
        if (enq_layers(s)) { set_err("a decode kernel could not be launched for this shape"); return -1; }
        MatvecArgs a = head_args(s, x_final(s));
        a.am_val = s->am_val; a.am_idx = s->am_idx;
        a.am_tokpos = s->tokpos_d; a.am_out = s->gen_tok; a.am_cap = s->ctx;
        if (mv(s, PRO_NORM, EPI_STORE, a)) { set_err("lm_head launch failed"); return -1; }
        return 0;
    }
    if (enq_decode(s)) { set_err("a decode kernel could not be launched for this shape"); return -1; }
    ArgmaxArgs g{};
    g.logits = s->logits_d; g.n = s->m->cfg.vocab_size;
    g.pval = s->am_val; g.pidx = s->am_idx;
    g.tokpos = s->tokpos_d; g.out = s->gen_tok; g.cap = s->ctx;
    if (launch_argmax(s->st, g)) { set_err("argmax launch failed"); return -1; }
    return 0;
}

// A device loop of n steps replays graphs of GEN_UNROLL steps, then single
// steps.  prepare_steps captures and instantiates the graphs the loop will
// replay (once per state and parameter set), so that run_steps, which the
// callers bracket with their timing events, only launches them; without
// graphs run_steps enqueues the plain launches.
template <class F>
static int prepare_steps(EhipState *s, StepGraph (&gr)[2], int n, F enq) {
    if (!s->graph_mode) return 0;
    if (n / GEN_UNROLL && !gr[1].x && graph_capture(s, gr[1], GEN_UNROLL, enq)) return -1;
    if (n % GEN_UNROLL && !gr[0].x && graph_capture(s, gr[0], 1, enq)) return -1;
    return 0;
}

template <class F>
static int run_steps(EhipState *s, StepGraph (&gr)[2], int n, F enq) {
    if (!s->graph_mode) {
        for (int i = 0; i < n; i++)
            if (enq()) return -1;
        return 0;
    }
    const int big = n / GEN_UNROLL, small = n % GEN_UNROLL;
    if ((big && !gr[1].x) || (small && !gr[0].x)) { set_err("device loop: graphs not prepared"); return -1; }
    for (int i = 0; i < big; i++) HCHK(hipGraphLaunch(gr[1].x, s->st), -1);
    for (int i = 0; i < small; i++) HCHK(hipGraphLaunch(gr[0].x, s->st), -1);
    return 0;
}

static int generate_greedy_once(EhipState *s, int tok, int pos, int n, int *out_tokens, float *ms);

extern "C" int ehip_generate_greedy(EhipState *s, int tok, int pos, int n, int *out_tokens, float *ms) {
    const int V = s->m->cfg.vocab_size;
    if (n <= 0 || pos < 0 || (long)pos + n > s->ctx) { set_err("generate: positions %d..%d exceed the context of %d", pos, pos + n - 1, s->ctx); return -1; }
    if (tok < 0 || tok >= V) { set_err("generate: token id %d out of range [0,%d)", tok, V); return -1; }
    int rc = generate_greedy_once(s, tok, pos, n, out_tokens, ms);
    if (rc == 1) rc = generate_greedy_once(s, tok, pos, n, out_tokens, ms);   // after the schedule fallback
    return rc == 0 ? 0 : -1;
}

// One run of the greedy loop: 0, 1 when the fused merge's check fired (the
// state has switched schedules; nothing was returned), or -1.
static int generate_greedy_once(EhipState *s, int tok, int pos, int n, int *out_tokens, float *ms) {
    s->tokpos_h[0] = tok;
    s->tokpos_h[1] = pos;
    s->tokpos_h[2] = 0;
    s->tokpos_h[3] = 0;
    auto enq = [&]() { return enq_gen_step(s); };
    if (prepare_steps(s, s->gen, n, enq)) return -1;
    HCHK(hipMemcpyAsync(s->tokpos_d, s->tokpos_h, 16, hipMemcpyHostToDevice, s->st), -1);
    HCHK(hipStreamSynchronize(s->st), -1);
    HCHK(hipEventRecord(s->ev0, s->st), -1);
    if (run_steps(s, s->gen, n, enq)) return -1;
    HCHK(hipEventRecord(s->ev1, s->st), -1);
    HCHK(hipEventSynchronize(s->ev1), -1);
    if (ms) {
        float t = 0.0f;
        HCHK(hipEventElapsedTime(&t, s->ev0, s->ev1), -1);
        *ms = t;
    }
    const int f = xm_flag(s);
    if (f) return f;
    if (out_tokens) HCHK(hipMemcpy(out_tokens, s->gen_tok, 4 * (size_t)n, hipMemcpyDeviceToHost), -1);
    return 0;
}

// ---------------------------------------------------------- sampling ----
static bool same_params(const SampleParams &a, const SampleParams &b) {
    return a.temperature == b.temperature && a.top_p == b.top_p && a.min_p == b.min_p &&
           a.repeat_penalty == b.repeat_penalty && a.presence_penalty == b.presence_penalty &&
           a.frequency_penalty == b.frequency_penalty && a.top_k == b.top_k;
}

static SampleParams sampler_params(const EmberSampler *smp) {
    SampleParams p{};
    p.temperature = smp->temperature; p.top_p = smp->top_p; p.min_p = smp->min_p;
    p.repeat_penalty = smp->repeat_penalty; p.presence_penalty = smp->presence_penalty;
    p.frequency_penalty = smp->frequency_penalty; p.top_k = smp->top_k;
    return p;
}

// Bring the sampler's RNG and history ring to the device (ring storage is
// grown outside any capture).
static int sampler_upload(EhipState *s, const EmberSampler *smp) {
    const int cap = smp->history ? smp->hist_cap : 0;
    if (cap > s->smp_hist_cap) {
        for (StepGraph &g : s->smp) graph_free(g);
        if (s->smp_hist) (void)hipFree(s->smp_hist);
        s->smp_hist = nullptr;
        s->smp_hist_cap = 0;
        HCHK(hipMalloc(&s->smp_hist, 4 * (size_t)cap), -1);
        s->smp_hist_cap = cap;
    }
    const unsigned long long rng = smp->rng_state;
    const int meta[2] = { smp->hist_len, smp->hist_pos };
    HCHK(hipMemcpyAsync(s->smp_rng, &rng, 8, hipMemcpyHostToDevice, s->st), -1);
    HCHK(hipMemcpyAsync(s->smp_meta, meta, 8, hipMemcpyHostToDevice, s->st), -1);
    if (cap > 0) HCHK(hipMemcpyAsync(s->smp_hist, smp->history, 4 * (size_t)cap, hipMemcpyHostToDevice, s->st), -1);
    HCHK(hipStreamSynchronize(s->st), -1);
    return 0;
}

static int sampler_download(EhipState *s, EmberSampler *smp) {
    const int cap = smp->history ? smp->hist_cap : 0;
    unsigned long long rng = 0;
    int meta[2] = { 0, 0 };
    HCHK(hipStreamSynchronize(s->st), -1);
    HCHK(hipMemcpy(&rng, s->smp_rng, 8, hipMemcpyDeviceToHost), -1);
    HCHK(hipMemcpy(meta, s->smp_meta, 8, hipMemcpyDeviceToHost), -1);
    if (cap > 0) HCHK(hipMemcpy(smp->history, s->smp_hist, 4 * (size_t)cap, hipMemcpyDeviceToHost), -1);
    smp->rng_state = rng;
    smp->hist_len = meta[0];
    smp->hist_pos = meta[1];
    return 0;
}

static SampleArgs sample_args(EhipState *s, const SampleParams &p, int cap, int n) {
    SampleArgs a{};
    a.logits = s->logits_d; a.n = n; a.p = p;
    a.rng = s->smp_rng; a.hist = cap > 0 ? s->smp_hist : nullptr; a.hist_meta = s->smp_meta; a.hist_cap = cap;
    a.psum = s->smp_psum; a.scnt = s->smp_cnt; a.cval = s->smp_cval; a.cidx = s->smp_cidx;
    a.am_val = s->am_val; a.am_idx = s->am_idx;
    a.tokpos = s->tokpos_d; a.out = s->gen_tok; a.cap = s->ctx;
    a.we = s->smp_we; a.wkeys = s->smp_wk; a.wcum = s->smp_wcum;
    a.exact = s->ref_order;   // every operation in the reference's order, the softmax sum included
    return a;
}

extern "C" int ehip_sample(EhipState *s, const float *logits, int n, EmberSampler *smp, int *token) {
    if (n <= 0 || n > s->m->cfg.vocab_size) { set_err("device sampler: %d logits for a vocabulary of %d", n, s->m->cfg.vocab_size); return -1; }
    if (logits) HCHK(hipMemcpyAsync(s->logits_d, logits, 4 * (size_t)n, hipMemcpyHostToDevice, s->st), -1);
    if (sampler_upload(s, smp)) return -1;
    s->tokpos_h[2] = 0;
    HCHK(hipMemcpyAsync(s->tokpos_d + 2, s->tokpos_h + 2, 4, hipMemcpyHostToDevice, s->st), -1);
    const int cap = smp->history ? smp->hist_cap : 0;
    if (launch_sample(s->st, sample_args(s, sampler_params(smp), cap, n))) { set_err("sampler launch failed"); return -1; }
    if (sampler_download(s, smp)) return -1;
    HCHK(hipMemcpy(token, s->gen_tok, 4, hipMemcpyDeviceToHost), -1);
    return 0;
}

static int generate_sampled_once(EhipState *s, int tok, int pos, int n, EmberSampler *smp, int *out_tokens,
                                 float *ms);

extern "C" int ehip_generate_sampled(EhipState *s, int tok, int pos, int n, EmberSampler *smp, int *out_tokens,
                                     float *ms) {
    const int V = s->m->cfg.vocab_size;
    if (n <= 0 || pos < 0 || (long)pos + n > s->ctx) { set_err("generate: positions %d..%d exceed the context of %d", pos, pos + n - 1, s->ctx); return -1; }
    if (tok < 0 || tok >= V) { set_err("generate: token id %d out of range [0,%d)", tok, V); return -1; }
    // the host sampler is updated only after a run whose merge check passed,
    // so a re-run after the schedule fallback starts from the same state
    int rc = generate_sampled_once(s, tok, pos, n, smp, out_tokens, ms);
    if (rc == 1) rc = generate_sampled_once(s, tok, pos, n, smp, out_tokens, ms);
    return rc == 0 ? 0 : -1;
}

static int generate_sampled_once(EhipState *s, int tok, int pos, int n, EmberSampler *smp, int *out_tokens,
                                 float *ms) {
    const int V = s->m->cfg.vocab_size;
    if (sampler_upload(s, smp)) return -1;
    const SampleParams p = sampler_params(smp);
    const int cap = smp->history ? smp->hist_cap : 0;
    s->tokpos_h[0] = tok;
    s->tokpos_h[1] = pos;
    s->tokpos_h[2] = 0;
    s->tokpos_h[3] = 0;
    HCHK(hipMemcpyAsync(s->tokpos_d, s->tokpos_h, 16, hipMemcpyHostToDevice, s->st), -1);
    HCHK(hipStreamSynchronize(s->st), -1);
    SampleArgs sa = sample_args(s, p, cap, V);
    // the lm_head's per-workgroup winners serve as the sampler's per-part
    // maxima unless penalties change the logits afterwards
    const bool parts = p.temperature > 0.0f && !sample_penalized(sa) && s->m->head.dtype != DT_F32 && !s->ref_order;
    auto enq = [&]() -> int {
        if (parts) {
            if (enq_layers(s)) { set_err("a decode kernel could not be launched for this shape"); return -1; }
            MatvecArgs h = head_args(s, x_final(s));
            h.am_val = s->am_val; h.am_idx = s->am_idx;
            sa.nparts = launch_matvec_parts(s->st, PRO_NORM, h);
            if (sa.nparts <= 0) { set_err("lm_head launch failed"); return -1; }
        } else if (enq_decode(s)) {
            set_err("a decode kernel could not be launched for this shape");
            return -1;
        }
        if (launch_sample(s->st, sa)) { set_err("sampler launch failed"); return -1; }
        return 0;
    };
    if (!same_params(p, s->smp_graph_p) || cap != s->smp_graph_cap) {   // graphs hold the parameters
        for (StepGraph &g : s->smp) graph_free(g);
        s->smp_graph_p = p;
        s->smp_graph_cap = cap;
    }
    if (prepare_steps(s, s->smp, n, enq)) return -1;
    HCHK(hipStreamSynchronize(s->st), -1);
    HCHK(hipEventRecord(s->ev0, s->st), -1);
    if (run_steps(s, s->smp, n, enq)) return -1;
    HCHK(hipEventRecord(s->ev1, s->st), -1);
    HCHK(hipEventSynchronize(s->ev1), -1);
    if (ms) {
        float t = 0.0f;
        HCHK(hipEventElapsedTime(&t, s->ev0, s->ev1), -1);
        *ms = t;
    }
    const int f = xm_flag(s);
    if (f) return f;
    if (sampler_download(s, smp)) return -1;
    if (out_tokens) HCHK(hipMemcpy(out_tokens, s->gen_tok, 4 * (size_t)n, hipMemcpyDeviceToHost), -1);
    return 0;
}

// The launches of one prefill pass: tokens pos0 .. pos0 + mt - 1, whose ids
// are in ids_d; `last` adds the head over the final token and the logits copy.
static int enq_prefill_pass(EhipState *s, int pos0, int mt, bool last, int pass) {
    const EhipModel *m = s->m;
    const EhipConfig &c = m->cfg;
    const int hd = c.head_dim, qd = c.n_heads * hd, kvd = c.n_kv_heads * hd, hid = c.hidden_dim;
    const int stride = qd + 2 * kvd;
    {
        for (int l = 0; l < c.n_layers; l++) {
            const DevLayer &y = m->layers[l];
            QuantRowsArgs q{};
            q.x = s->X; q.x_stride = c.dim; q.cols = c.dim; q.n = mt;
            q.norm_w = y.attn_norm; q.eps = c.norm_eps;
            if (l == 0) { q.ids = s->ids_d; q.emb = m->emb; q.x_out = s->X; }
            q.xf = m->any_f32 ? s->xf : nullptr; q.qx = s->qx; q.dx = s->dxp; q.xs = s->xsum;
            // copies of the captured layer's tensors of this pass
            const bool snap = l == s->pdbg_layer && pass == s->pdbg_pass;
            auto psnap = [&](int slot, const float *src, int stride, int width) -> int {
                if (!snap) return 0;
                HCHK(hipMemcpy2DAsync(s->pdbg[slot], 4 * (size_t)width, src, 4 * (size_t)stride, 4 * (size_t)width,
                                      mt, hipMemcpyDeviceToDevice, s->st), -1);
                return 0;
            };
            if (snap) { s->pdbg_n = mt; s->pdbg_pos = pos0; }
            if (l > 0 && psnap(DBG_XIN, s->X, c.dim, c.dim)) return -1;
            int rc = launch_quant_rows(s->st, q);
            if (l == 0 && psnap(DBG_XIN, s->X, c.dim, c.dim)) return -1;   // the embedded rows
            GemmArgs g{};
            g.W = y.qkv; g.units = stride; g.n = mt; g.qx = s->qx; g.dx = s->dxp; g.xs = s->xsum; g.xf = q.xf;
            g.out = s->QKV; g.out_stride = stride; g.bias = y.bias_qkv;
            QkPostArgs p{};
            p.qkv = s->QKV; p.stride = stride; p.q_norm = y.q_norm; p.k_norm = y.k_norm;
            p.rope = s->rope; p.eps = c.norm_eps; p.rope_style = c.rope_style;
            AttnArgs at = attn_args(s, l);
            p.kc = at.kc; p.vc = at.vc; p.kv_dim = kvd; p.hd = hd; p.n_heads = c.n_heads;
            p.n_kv = c.n_kv_heads; p.pos_base = pos0; p.n_tok = mt;
            bool exact = s->pf_mode == PF_EXACT;
            if (s->pf_mode == PF_AUTO)
                exact = s->pf_seq && pos0 + mt <= PF_EXACT_KEYS;
            bool img_fused = false;   // the q|k|v product wrote the pass's K/V tile images
            // the matrix-core attention's K/V tile images of the pass, in the
            // fused q|k|v epilogues (EHIP_PF_KVIMG=0 leaves them to
            // k_pf_kvsplit)
            const bool img_ok = !exact && (hd == 64 || hd == 128) && s->pf_kvimg && pos0 % 64 == 0 &&
                                s->pf_kvimg_tiles >= (pos0 + mt + 63) / 64 && env_int("EHIP_PF_KVIMG", 1);
            if (!q.xf && gemm_qkv_fits(g, p)) {
                // short prompts: the QK-norm, RoPE and cache stores in the
                // product's epilogue (the raw product goes straight to a capture)
                if (img_ok) {
                    p.kvimg = s->pf_kvimg;
                    p.kvimg_tiles = s->pf_kvimg_tiles;
                    img_fused = true;
                }
                rc |= launch_gemm_qkv(s->st, s->f16kv, g, p, snap ? s->pdbg[DBG_QKV] : nullptr);
            } else if (!q.xf && env_int("EHIP_PF_QKPOST", 1) && gemm_qkpost_fits(g, p)) {
                // longer ones, 128-dim heads: the same in the matrix-core
                // product's epilogue (EHIP_PF_QKPOST=0 keeps the product and
                // k_qkpost apart)
                GemmArgs gq = g;
                gq.out = snap ? s->pdbg[DBG_QKV] : nullptr;
                if (img_ok) {
                    p.kvimg = s->pf_kvimg;
                    p.kvimg_tiles = s->pf_kvimg_tiles;
                    img_fused = true;
                }
                rc |= launch_gemm_qkpost(s->st, s->f16kv, gq, p);
            } else {
                rc |= launch_gemm(s->st, EPI_STORE, g);
                if (psnap(DBG_QKV, s->QKV, stride, stride)) return -1;
                rc |= launch_qkpost(s->st, s->f16kv, p);
            }
            at.q = s->QKV; at.q_stride = stride; at.pos_base = pos0; at.n_tok = mt;
            at.out = s->O;
            at.scores = s->pf_scores; at.tmax = s->pf_tmax; at.rowmax = s->pf_rowmax; at.rowinv = s->pf_rowinv;
            at.kvimg = s->pf_kvimg; at.kvimg_tiles = s->pf_kvimg_tiles;
            at.ldk = attn_prefill_ldk(pos0, mt);
            at.kvimg_fused = img_fused ? 1 : 0;
            // the attention can quantize its own output for wo (not for F32
            // weights, whose product reads the fp32 rows)
            bool quantized = false;
            if (!q.xf) { at.qx = s->qx; at.qdx = s->dxp; at.qxs = s->xsum; }
            rc |= exact ? launch_attention(s->st, s->f16kv, at, &quantized)
                        : launch_attention_mfma(s->st, s->f16kv, at, &quantized);
            if (psnap(DBG_O, s->O, qd, qd)) return -1;
            if (!quantized) {
                QuantRowsArgs q2{};
                q2.x = s->O; q2.x_stride = qd; q2.cols = qd; q2.n = mt;
                q2.xf = q.xf; q2.qx = s->qx; q2.dx = s->dxp; q2.xs = s->xsum;
                rc |= launch_quant_rows(s->st, q2);
            }
            GemmArgs g2{};
            g2.W = y.wo; g2.units = c.dim; g2.n = mt; g2.qx = s->qx; g2.dx = s->dxp; g2.xs = s->xsum;
            g2.xf = q.xf; g2.out = s->X; g2.out_stride = c.dim;
            rc |= launch_gemm(s->st, EPI_RESID, g2);
            if (psnap(DBG_XMID, s->X, c.dim, c.dim)) return -1;
            QuantRowsArgs q3 = q;
            q3.ids = nullptr; q3.norm_w = y.ffn_norm;
            rc |= launch_quant_rows(s->st, q3);
            GemmArgs g3{};
            g3.W = y.w13; g3.units = 2 * hid; g3.n = mt; g3.qx = s->qx; g3.dx = s->dxp; g3.xs = s->xsum;
            g3.xf = q.xf; g3.out = s->H; g3.out_stride = 2 * hid;
            GemmArgs g4{};
            g4.W = y.w2; g4.units = c.dim; g4.n = mt; g4.qx = s->qx; g4.dx = s->dxp; g4.xs = s->xsum;
            // the SwiGLU and its quantization in the w1|w3 product's epilogue
            // (the gate | up rows written only for a capture): the short-prompt
            // kernel, or the matrix-core tiles (EHIP_PF_SWIGLU=0 keeps those
            // passes on the product + k_quant_rows)
            GemmArgs gs = g3;
            gs.units = hid; gs.pair_off = hid; gs.oq = s->qx2; gs.odx = s->dxp2; gs.oxs = s->xsum2;
            gs.out = snap ? s->H : nullptr;
            if (!q.xf && (gemm_swiglu_fits(gs) || (env_int("EHIP_PF_SWIGLU", 1) && gemm_swiglu_long_fits(gs)))) {
                rc |= launch_gemm_swiglu(s->st, gs);
                if (psnap(DBG_H, s->H, 2 * hid, 2 * hid)) return -1;
                g4.qx = s->qx2; g4.dx = s->dxp2; g4.xs = s->xsum2;
            } else {
                rc |= launch_gemm(s->st, EPI_STORE, g3);
                if (psnap(DBG_H, s->H, 2 * hid, 2 * hid)) return -1;
                QuantRowsArgs q4{};
                q4.x = s->H; q4.x_stride = 2 * hid; q4.cols = hid; q4.n = mt; q4.swiglu = 1;
                q4.xf = q.xf; q4.qx = s->qx; q4.dx = s->dxp; q4.xs = s->xsum;
                rc |= launch_quant_rows(s->st, q4);
            }
            g4.xf = q.xf; g4.out = s->X; g4.out_stride = c.dim;
            rc |= launch_gemm(s->st, EPI_RESID, g4);
            if (psnap(DBG_XOUT, s->X, c.dim, c.dim)) return -1;
            if (rc) { set_err("a prefill kernel could not be launched for this shape"); return -1; }
        }
        if (last) {
            if (enq_head(s, s->X + (size_t)(mt - 1) * c.dim)) { set_err("head launch failed"); return -1; }
            HCHK(hipMemcpyAsync(s->logits_h, s->logits_d, 4 * (size_t)c.vocab_size, hipMemcpyDeviceToHost, s->st), -1);
        }
    }
    return 0;
}

// The graph of a prefill pass shape, captured on first use.
static hipGraphExec_t prefill_graph(EhipState *s, int pos0, int mt, bool last, int pass) {
    EhipState::PfGraph *hit = nullptr, *lru = &s->pfg[0];
    for (auto &pg : s->pfg) {
        if (pg.sg.x && pg.pos0 == pos0 && pg.n == mt && pg.last == (int)last) hit = &pg;
        if (pg.used < lru->used) lru = &pg;
    }
    if (!hit) {
        hit = lru;
        graph_free(hit->sg);
        HCHK(hipStreamBeginCapture(s->st, hipStreamCaptureModeThreadLocal), nullptr);
        const int rc = enq_prefill_pass(s, pos0, mt, last, pass);
        hipGraph_t g = nullptr;
        const hipError_t e = hipStreamEndCapture(s->st, &g);
        if (rc) { if (g) (void)hipGraphDestroy(g); return nullptr; }
        if (e != hipSuccess) { set_err("hipStreamEndCapture: %s", hipGetErrorString(e)); return nullptr; }
        hit->sg.g = g;
        if (hipGraphInstantiate(&hit->sg.x, g, nullptr, nullptr, 0) != hipSuccess) {
            graph_free(hit->sg);
            set_err("prefill graph instantiation failed");
            return nullptr;
        }
        hit->pos0 = pos0; hit->n = mt; hit->last = last;
    }
    hit->used = ++s->pf_clock;
    return hit->sg.x;
}

extern "C" float *ehip_prefill(EhipState *s, const int *ids, int n, int start) {
    if (s->ref_order) {   // the reference's prefill computes exactly its forward steps
        for (int i = 0; i < n; i++)
            if (!ehip_forward(s, ids[i], start + i)) return nullptr;
        return s->logits_h;
    }
    for (int c0 = 0; c0 < n; c0 += s->pf_chunk) {
        const int mt = std::min(s->pf_chunk, n - c0), pass = c0 / s->pf_chunk;
        const bool last = c0 + mt == n;
        HCHK(hipMemcpyAsync(s->ids_d, ids + c0, 4 * (size_t)mt, hipMemcpyHostToDevice, s->st), nullptr);
        // one graph per pass shape; eager launches while a layer's tensors
        // are being captured for inspection, or with graphs switched off
        if (s->graph_mode && s->pdbg_layer < 0) {
            const hipGraphExec_t x = prefill_graph(s, start + c0, mt, last, pass);
            if (!x) return nullptr;
            HCHK(hipGraphLaunch(x, s->st), nullptr);
        } else if (enq_prefill_pass(s, start + c0, mt, last, pass)) {
            return nullptr;
        }
    }
    HCHK(hipStreamSynchronize(s->st), nullptr);
    return s->logits_h;
}


// ------------------------------------------------------- inspection ----
extern "C" int ehip_kv_read(EhipState *s, int which, int layer, int n_pos, void *host) {
    const EhipConfig &c = s->m->cfg;
    const size_t row = (size_t)c.n_kv_heads * c.head_dim * s->esize;
    if (layer < 0 || layer >= c.n_layers || n_pos < 0 || n_pos > s->ctx) { set_err("kv_read out of range"); return -1; }
    const uint8_t *base = static_cast<const uint8_t *>(which ? s->vc : s->kc) + (size_t)layer * s->ctx * row;
    HCHK(hipStreamSynchronize(s->st), -1);
    HCHK(hipMemcpy(host, base, row * n_pos, hipMemcpyDeviceToHost), -1);
    return 0;
}

extern "C" int ehip_kv_write(EhipState *s, int which, int layer, int n_pos, const void *host) {
    const EhipConfig &c = s->m->cfg;
    const size_t row = (size_t)c.n_kv_heads * c.head_dim * s->esize;
    if (layer < 0 || layer >= c.n_layers || n_pos < 0 || n_pos > s->ctx) { set_err("kv_write out of range"); return -1; }
    uint8_t *base = static_cast<uint8_t *>(which ? s->vc : s->kc) + (size_t)layer * s->ctx * row;
    HCHK(hipStreamSynchronize(s->st), -1);
    HCHK(hipMemcpy(base, host, row * n_pos, hipMemcpyHostToDevice), -1);
    return 0;
}

extern "C" int ehip_debug_buffer(EhipState *s, int which, void *host, uint64_t bytes) {
    const EhipConfig &c = s->m->cfg;
    const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
    const void *src[5] = { x_final(s), s->qkv, s->o, s->h, s->logits_d };
    const uint64_t len[5] = { 4ull * c.dim, 4ull * (qd + 2 * kvd), 4ull * qd, 4ull * c.hidden_dim,
                              4ull * c.vocab_size };
    if (which < 0 || which > 4 || bytes > len[which]) { set_err("debug_buffer: bad request"); return -1; }
    HCHK(hipStreamSynchronize(s->st), -1);
    HCHK(hipMemcpy(host, src[which], bytes, hipMemcpyDeviceToHost), -1);
    return 0;
}

static void drop_step_graphs(EhipState *s) {
    (void)hipStreamSynchronize(s->st);
    if (s->gexec) (void)hipGraphExecDestroy(s->gexec);
    if (s->graph) (void)hipGraphDestroy(s->graph);
    s->gexec = nullptr;
    s->graph = nullptr;
    for (StepGraph &g : s->gen) graph_free(g);
    for (StepGraph &g : s->smp) graph_free(g);
}

extern "C" int ehip_debug_capture(EhipState *s, int layer) {
    const EhipConfig &c = s->m->cfg;
    if (layer < -1 || layer >= c.n_layers) { set_err("debug_capture: layer %d out of range", layer); return -1; }
    const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
    const size_t len[6] = { (size_t)c.dim, (size_t)(qd + 2 * kvd), (size_t)qd, (size_t)c.dim,
                            (size_t)c.hidden_dim, (size_t)c.dim };
    for (int i = 0; i < 6 && layer >= 0; i++)
        if (!s->dbg[i] && !(s->dbg[i] = (float *)salloc(s, 4 * len[i], true))) {
            set_err("debug_capture: allocation failed");
            return -1;
        }
    drop_step_graphs(s);   // captured graphs hold the previous choice
    s->dbg_layer = layer;
    return 0;
}

extern "C" int ehip_debug_read(EhipState *s, int slot, void *host, uint64_t bytes) {
    const EhipConfig &c = s->m->cfg;
    const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
    const uint64_t len[6] = { 4ull * c.dim, 4ull * (qd + 2 * kvd), 4ull * qd, 4ull * c.dim,
                              4ull * c.hidden_dim, 4ull * c.dim };
    if (slot < 0 || slot > 5 || !s->dbg[slot] || bytes > len[slot]) { set_err("debug_read: bad request"); return -1; }
    HCHK(hipStreamSynchronize(s->st), -1);
    HCHK(hipMemcpy(host, s->dbg[slot], bytes, hipMemcpyDeviceToHost), -1);
    return 0;
}

// widths of the prefill capture slots (per token)
static void pdbg_widths(const EhipConfig &c, size_t w[6]) {
    const size_t qd = (size_t)c.n_heads * c.head_dim, kvd = (size_t)c.n_kv_heads * c.head_dim;
    w[DBG_XIN] = c.dim; w[DBG_QKV] = qd + 2 * kvd; w[DBG_O] = qd;
    w[DBG_XMID] = c.dim; w[DBG_H] = 2 * (size_t)c.hidden_dim; w[DBG_XOUT] = c.dim;
}

extern "C" int ehip_debug_capture_prefill(EhipState *s, int layer, int pass) {
    const EhipConfig &c = s->m->cfg;
    if (layer < -1 || layer >= c.n_layers || pass < 0) { set_err("debug_capture_prefill: bad layer or pass"); return -1; }
    size_t w[6];
    pdbg_widths(c, w);
    for (int i = 0; i < 6 && layer >= 0; i++)
        if (!s->pdbg[i] && !(s->pdbg[i] = (float *)salloc(s, 4 * w[i] * (size_t)s->pf_chunk, true))) {
            set_err("debug_capture_prefill: allocation failed");
            return -1;
        }
    s->pdbg_layer = layer;
    s->pdbg_pass = pass;
    s->pdbg_n = 0;
    return 0;
}

extern "C" int ehip_debug_read_prefill(EhipState *s, int slot, void *host, uint64_t bytes, int *n_tok, int *pos0) {
    size_t w[6];
    pdbg_widths(s->m->cfg, w);
    if (slot < 0 || slot > 5 || !s->pdbg[slot]) { set_err("debug_read_prefill: bad request"); return -1; }
    if (n_tok) *n_tok = s->pdbg_n;
    if (pos0) *pos0 = s->pdbg_pos;
    if (bytes > 4 * w[slot] * (size_t)s->pdbg_n) { set_err("debug_read_prefill: %llu bytes requested", (unsigned long long)bytes); return -1; }
    HCHK(hipStreamSynchronize(s->st), -1);
    if (bytes) HCHK(hipMemcpy(host, s->pdbg[slot], bytes, hipMemcpyDeviceToHost), -1);
    return 0;
}

extern "C" int ehip_prefill_pass_tokens(const EhipState *s) { return s->pf_chunk; }

extern "C" int ehip_decode_fusion(const EhipState *s) {
    return (s->xm_on ? 1 : 0) | (fw_usable(const_cast<EhipState *>(s)) ? 2 : 0);
}

extern "C" int ehip_set_graph_mode(EhipState *s, int mode) {
    s->graph_mode = mode ? 1 : 0;
    return 0;
}

extern "C" int ehip_time_decode(EhipState *s, int pos0, int steps, float *ms) {
    const int V = s->m->cfg.vocab_size;
    if (pos0 < 0 || pos0 + steps > s->ctx || steps <= 0) { set_err("time_decode: positions out of range"); return -1; }
    HCHK(hipStreamSynchronize(s->st), -1);
    HCHK(hipEventRecord(s->ev0, s->st), -1);
    for (int i = 0; i < steps; i++) {
        const int pos = pos0 + i;
        s->tokpos_h[0] = (int)(((long)pos * 131 + 7) % V);
        s->tokpos_h[1] = pos;
        if (run_step(s)) return -1;
        HCHK(hipStreamSynchronize(s->st), -1);
    }
    HCHK(hipEventRecord(s->ev1, s->st), -1);
    HCHK(hipEventSynchronize(s->ev1), -1);
    float t = 0.0f;
    HCHK(hipEventElapsedTime(&t, s->ev0, s->ev1), -1);
    *ms = t / steps;
    return 0;
}

// Streaming read: workgroup b reads the SR_PER_WG 16-byte pieces from
// b * SR_PER_WG on, each thread SR_UNROLL of them 4 KB apart, all loads in
// flight at once (the pattern of the decode matvecs: contiguous bytes per
// workgroup, many workgroups).  The XOR of the data is kept alive by a store
// that only a (practically impossible) zero checksum takes.
constexpr int SR_UNROLL = 8, SR_PER_WG = SR_UNROLL * WG;   // 32 KB per workgroup
__global__ __launch_bounds__(WG) void k_stream_read(const uint4 *__restrict__ p, size_t n16, unsigned *sink) {
    const size_t base = (size_t)blockIdx.x * SR_PER_WG;
    uint4 v[SR_UNROLL];
#pragma unroll
    for (int u = 0; u < SR_UNROLL; u++) v[u] = p[min(base + threadIdx.x + u * WG, n16 - 1)];
    unsigned acc = 0;
#pragma unroll
    for (int u = 0; u < SR_UNROLL; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (acc == 0u && threadIdx.x == 0) sink[blockIdx.x & 63] = acc + 1u;
}

extern "C" void ehip_libm_expf(const float *x, float *y, long n) {
    for (long i = 0; i < n; i++) y[i] = libm_expf(x[i]);
}

extern "C" int ehip_measure_read_bw(EhipState *s, uint64_t bytes, int reps, float *gbs) {
    if (bytes < (1u << 20) || reps <= 0 || !gbs) { set_err("measure_read_bw: bad arguments"); return -1; }
    if (bytes > (1ull << 36)) { set_err("measure_read_bw: at most 64 GiB"); return -1; }
    const size_t n16 = (size_t)(bytes / 16);
    void *buf = nullptr;
    unsigned *sink = nullptr;
    HCHK(hipMalloc(&buf, n16 * 16), -1);
    if (hipMalloc(&sink, 64 * 4) != hipSuccess) { (void)hipFree(buf); set_err("hipMalloc failed"); return -1; }
    int rc = 0;
    float t = 0.0f;
    const dim3 grid((unsigned)((n16 + SR_PER_WG - 1) / SR_PER_WG));
    if (hipMemsetAsync(buf, 1, n16 * 16, s->st) != hipSuccess) rc = -1;
    if (!rc) hipLaunchKernelGGL(k_stream_read, grid, dim3(WG), 0, s->st, (const uint4 *)buf, n16, sink);   // warm-up
    if (!rc && (hipEventRecord(s->ev0, s->st) != hipSuccess)) rc = -1;
    for (int r = 0; r < reps && !rc; r++)
        hipLaunchKernelGGL(k_stream_read, grid, dim3(WG), 0, s->st, (const uint4 *)buf, n16, sink);
    if (!rc && (hipEventRecord(s->ev1, s->st) != hipSuccess || hipEventSynchronize(s->ev1) != hipSuccess ||
                hipEventElapsedTime(&t, s->ev0, s->ev1) != hipSuccess || hipGetLastError() != hipSuccess))
        rc = -1;
    (void)hipStreamSynchronize(s->st);
    (void)hipFree(buf);
    (void)hipFree(sink);
    if (rc || t <= 0.0f) { set_err("measure_read_bw: launch or timing failed"); return -1; }
    *gbs = (float)((double)n16 * 16 * reps / (t * 1e-3) / 1e9);
    return 0;
}

extern "C" int ehip_time_kernel(EhipState *s, int kernel, int pos, int reps, float *ms) {
    if (pos < 0 || pos >= s->ctx || reps <= 0) { set_err("time_kernel: bad arguments"); return -1; }
    s->tokpos_h[0] = 0;
    s->tokpos_h[1] = pos;
    HCHK(hipMemcpyAsync(s->tokpos_d, s->tokpos_h, 8, hipMemcpyHostToDevice, s->st), -1);
    // successive launches walk through the layers, so each reads weights or
    // cache rows of its own, as in a decode step (the lm_head is one matrix)
    // The kernels run in the form the decode step uses: with the wo product
    // folded into the attention, the attention raises each kv group's flag
    // and the w1|w3 prologue adds the partials and clears the flags, so the
    // attention's launches clear every layer's flags before each pass over
    // the layers (a fill of a few KB per n_layers launches, timed with them).
    const int L = s->m->cfg.n_layers;
    const bool fw = fw_usable(s);
    const size_t nflag = (size_t)L * s->m->cfg.n_kv_heads * XM_CNT_STRIDE;
    int i = 0;
    auto one = [&]() -> int {
        const int l = i++ % L;
        if (kernel == 0) {
            if (fw && l == 0) HCHK(hipMemsetAsync(s->wo_flag, 0, 4 * nflag, s->st), -1);
            return enq_attn_decode(s, l, false, fw);
        }
        if (kernel == 1) return enq_head(s, s->x);
        if (kernel == 2) return enq_w13(s, l, s->x, fw ? s->x2 : nullptr);
        return -1;
    };
    if (one()) { set_err("time_kernel: unknown kernel %d", kernel); return -1; }  // warm-up
    HCHK(hipStreamSynchronize(s->st), -1);
    HCHK(hipEventRecord(s->ev0, s->st), -1);
    for (int r = 0; r < reps; r++) if (one()) return -1;
    HCHK(hipEventRecord(s->ev1, s->st), -1);
    HCHK(hipEventSynchronize(s->ev1), -1);
    float t = 0.0f;
    HCHK(hipEventElapsedTime(&t, s->ev0, s->ev1), -1);
    *ms = t / reps;
    if (fw && kernel == 0) {   // the flags the last launches raised
        HCHK(hipMemsetAsync(s->wo_flag, 0, 4 * nflag, s->st), -1);
        HCHK(hipStreamSynchronize(s->st), -1);
    }
    return 0;
}
