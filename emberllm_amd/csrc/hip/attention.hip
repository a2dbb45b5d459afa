// attention.hip — prefill GQA attention over the HBM-resident KV cache (gfx950).
//
// Replaces the per-token attention calls of ember_prefill (src/model.c:335-337
// -> attention -> attn_heads + softmax, model.c:57-64, 207-278) and its
// QK-norm / RoPE / kv_store loop (model.c:323-333, k_qkpost).  The decode
// form lives in attn_decode.hip.
//
// The reference's activations are re-quantized to Q8_0 before every matmul,
// so a one-ulp difference in an attention output can move an int8 code and
// cascade through the following layers.  Prefill attention therefore keeps
// the reference's floating-point order exactly, and gets its speed from
// parallelism across (head, token, key) and from sharing every K/V tile in
// LDS among many rows, in three kernels per layer:
//   k_pf_scores   s[h][b][t] = (sum over d in order of q*k) / sqrt(hd), one
//                 lane per key, each lane carrying up to 8 (token, head)
//                 rows of its kv group; K tile and Q rows staged in LDS; also
//                 the maximum of each row over the tile's 64 keys
//   k_pf_rowsum   per row: max = the maximum of its tile maxima; the
//                 exponentials e_t = expf(s_t - max) computed by the whole
//                 workgroup, then added in t order by one lane per row; 1/sum
//                 (model.c:57-64)
//   k_pf_pv       o[b][h][d] = sum over t in order of (e_t * (1/sum)) * v_t[d],
//                 e_t recomputed while staging (expf gives the same value),
//                 one thread per (row set, d); V tile and probabilities
//                 staged in LDS
// The score rows are written once and read twice (the sum, then P.V).
// Roofline: VALU-bound, 2 * hd multiply-adds per (head, token, key) pair,
// each as a separately rounded multiply and add like the reference's
// -ffp-contract=off build.
#include <cstdlib>

#include "kernels.h"
#include "flimg.h"

namespace ehip {

constexpr int PF_KT = 64;   // keys per tile

// rows of (token, head) per lane or thread: tokens x heads <= 8
template <int GM> struct PfRows { static constexpr int QW = GM >= 8 ? 1 : 8 / GM; };

// One tile of PF_KT cache rows (hd elements of one kv head, widened to fp32)
// held in registers between its loads and its LDS stores, so the loads of the
// next tile can be in flight while the current one is used.
template <int HD, bool F16> struct RowTile {
    static constexpr int F4 = HD / 4, N = PF_KT * F4 / WG;
    static_assert(PF_KT * F4 % WG == 0, "whole float4 chunks per thread");
    f32x4 v[N];   // native vectors (HIP's float4 struct kept this array in scratch)
    __device__ __forceinline__ void load(const void *cache, int kv_dim, size_t hoff, int t0, int tmax, int tid) {
#pragma unroll
        for (int i = 0; i < N; i++) {
            const int f = tid + i * WG, t = f / F4, c = (f % F4) * 4;
            const size_t off = (size_t)min(t0 + t, tmax) * kv_dim + hoff + c;
            if (F16) {
                const uint2 u = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(cache) + off);
                v[i] = f32x4{h2f(u.x & 0xffff), h2f(u.x >> 16), h2f(u.y & 0xffff), h2f(u.y >> 16)};
            } else {
                v[i] = *reinterpret_cast<const f32x4 *>(reinterpret_cast<const float *>(cache) + off);
            }
        }
    }
    __device__ __forceinline__ void store(float *dst, int pitch, int tid) const {
#pragma unroll
        for (int i = 0; i < N; i++) {
            const int f = tid + i * WG;
            *reinterpret_cast<f32x4 *>(dst + (f / F4) * pitch + (f % F4) * 4) = v[i];
        }
    }
};

template <int HD, bool F16>
__device__ __forceinline__ void stage_rows(float *dst, int pitch, const void *cache, int kv_dim, size_t hoff,
                                           int t0, int tmax, int tid) {
    // PF_KT rows of hd elements of one kv head, widened to fp32, row t at dst + t * pitch;
    // every load of the thread is issued before the first store
    RowTile<HD, F16> r;
    r.load(cache, kv_dim, hoff, t0, tmax, tid);
    r.store(dst, pitch, tid);
}

// grid (key tiles, token tiles of 4*QW, kv groups); wave w carries tokens
// b0 + w*QW .. + QW-1 and the group's heads; lane = key
template <int HD, int GM, bool F16, int QW>
__global__ __launch_bounds__(WG) void k_pf_scores(AttnArgs a) {
    constexpr int QT = 4 * QW, KP = HD + 4;   // QW token rows per wave
    __shared__ __align__(16) float ks[PF_KT * KP];
    __shared__ __align__(16) float qs[QT * GM * HD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = a.n_heads / a.n_kv, g = blockIdx.z;
    const int kt0 = blockIdx.x * PF_KT, b0 = blockIdx.y * QT;
    const int blast = min(a.n_tok, b0 + QT) - 1;
    if (b0 >= a.n_tok || kt0 > a.pos_base + blast) return;   // causal: no key of this tile is visible
    // the Q rows' loads go out with the K tile's, then both are stored
    constexpr int NQ = (QT * GM * (HD / 4) + WG - 1) / WG;
    f32x4 qv[NQ];
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        const int f = tid + i * WG;
        if (f < QT * GM * (HD / 4)) {
            const int r = f / (HD / 4), c = (f % (HD / 4)) * 4;
            const int qb = r / GM, h = r % GM;
            const int b = min(b0 + qb, a.n_tok - 1);
            qv[i] = *reinterpret_cast<const f32x4 *>(
                a.q + (size_t)b * a.q_stride + (size_t)(g * G + min(h, G - 1)) * HD + c);
        }
    }
    stage_rows<HD, F16>(ks, KP, a.kc, a.kv_dim, (size_t)g * HD, kt0, a.pos_base + blast, tid);
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        const int f = tid + i * WG;
        if (f < QT * GM * (HD / 4))
            *reinterpret_cast<f32x4 *>(&qs[(f / (HD / 4)) * HD + (f % (HD / 4)) * 4]) = qv[i];
    }
    __syncthreads();
    float acc[QW][GM];
#pragma unroll
    for (int i = 0; i < QW; i++)
#pragma unroll
        for (int h = 0; h < GM; h++) acc[i][h] = 0.0f;
    const float *kr = &ks[lane * KP];
    const float *qw = &qs[wave * QW * GM * HD];
#pragma unroll(HD > 64 ? 1 : 4)   // full unrolling at HD 64 spilled registers
    for (int d = 0; d < HD; d += 4) {
        const float4 kf = *reinterpret_cast<const float4 *>(kr + d);
#pragma unroll
        for (int i = 0; i < QW; i++)
#pragma unroll
            for (int h = 0; h < GM; h++) {
                const float4 qf = *reinterpret_cast<const float4 *>(qw + (i * GM + h) * HD + d);
                float s = acc[i][h];            // dims in order, multiply and add rounded apart
                s = s + qf.x * kf.x;
                s = s + qf.y * kf.y;
                s = s + qf.z * kf.z;
                s = s + qf.w * kf.w;
                acc[i][h] = s;
            }
    }
    const int t = kt0 + lane, ntl = attn_prefill_tiles(a.ldk);
#pragma unroll
    for (int i = 0; i < QW; i++) {
        const int b = b0 + wave * QW + i;   // uniform over the wave
        const bool rowok = b < a.n_tok && kt0 <= a.pos_base + b;
        const bool ok = rowok && t <= a.pos_base + b;
#pragma unroll
        for (int h = 0; h < GM; h++) {
            if (h >= G) continue;
            const size_t row = (size_t)(g * G + h) * a.n_tok + b;
            const float sv = acc[i][h] * a.inv_sqrt;
            if (ok) a.scores[row * a.ldk + t] = sv;
            const float mx = wave_max(ok ? sv : -INFINITY);
            if (lane == 0 && rowok) a.tmax[row * ntl + blockIdx.x] = mx;
        }
    }
}

// Passes whose keys fit in PF_SM_KEYS: the scores and the softmax of a row
// in one kernel.  grid (token tiles of 4, kv groups); wave w carries token
// b0 + w and the group's G heads (GM rows), lane = key of the tile.  Each
// 64-key tile of K is staged in LDS and scored as in k_pf_scores (dims in
// order, multiply and add rounded apart, then times 1/sqrt(hd)); a row's
// scores stay in LDS.  Then per row: the maximum, the exponentials
// expf(s - max) (positions past the row's length 0), their sum added in
// position order by one lane per row (k_pf_rowsum's sequential sum: the
// zeros leave it unchanged), and the probabilities e * (1/sum), which go to
// the score rows for k_pf_pv2 to read instead of recomputing them.
//
// FUSE: the workgroup then also multiplies its rows' probabilities into V
// (each (row, four dims) summing its positions in order, multiply and add
// rounded apart, as k_pf_pv2 does; V tiles staged in the LDS the K tiles
// used), writes the output, and, with a.qx, the output's Q8_0 blocks: eight
// lanes hold a block's 32 dims, so its maximum and code sum are 8-lane DPP
// reductions, with k_quant_rows's arithmetic.
constexpr int PF_SM_KEYS = 512;    // keys of a pass the one-kernel softmax takes (LDS rows)
template <int HD, int GM, bool F16, bool FUSE>
__global__ __launch_bounds__(WG) void k_pf_softmax(AttnArgs a) {
    constexpr int QT = 4, KP = HD + 4, NR = QT * GM, SP = PF_SM_KEYS + 4;
    __shared__ __align__(16) float ks[PF_KT * KP];
    __shared__ __align__(16) float qs[NR * HD];
    __shared__ __align__(16) float ss[NR * SP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = a.n_heads / a.n_kv, g = blockIdx.y;
    const int b0 = blockIdx.x * QT;
    if (b0 >= a.n_tok) return;
    const int kend = a.pos_base + min(a.n_tok, b0 + QT) - 1;   // the last key any row here sees
    const int nkt = kend / PF_KT + 1;
    const int b = b0 + wave;                                     // this wave's token (uniform)
    const bool tok_ok = b < a.n_tok;
    const int len = tok_ok ? a.pos_base + b + 1 : 0;             // keys visible to its rows
    constexpr int NQ = (NR * (HD / 4) + WG - 1) / WG;
    f32x4 qv[NQ];
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        const int f = tid + i * WG;
        if (f < NR * (HD / 4)) {
            const int r = f / (HD / 4), c = (f % (HD / 4)) * 4;
            const int qb = min(b0 + r / GM, a.n_tok - 1), h = r % GM;
            qv[i] = *reinterpret_cast<const f32x4 *>(
                a.q + (size_t)qb * a.q_stride + (size_t)(g * G + min(h, G - 1)) * HD + c);
        }
    }
    float mx[GM];
#pragma unroll
    for (int h = 0; h < GM; h++) mx[h] = -INFINITY;
    float *srow = &ss[wave * GM * SP];
    // the next tile's rows are loaded into registers while the current one is
    // scored: K tiles, then (FUSE) the first V tile during the softmax
    RowTile<HD, F16> nxt;
    nxt.load(a.kc, a.kv_dim, (size_t)g * HD, 0, kend, tid);
    for (int kt = 0; kt < nkt; kt++) {
        const int kt0 = kt * PF_KT;
        if (kt > 0) __syncthreads();   // every wave has scored the previous tile
        nxt.store(ks, KP, tid);
        if (kt + 1 < nkt) nxt.load(a.kc, a.kv_dim, (size_t)g * HD, kt0 + PF_KT, kend, tid);
        else if (FUSE) nxt.load(a.vc, a.kv_dim, (size_t)g * HD, 0, kend, tid);
        if (kt == 0) {
#pragma unroll
            for (int i = 0; i < NQ; i++) {
                const int f = tid + i * WG;
                if (f < NR * (HD / 4))
                    *reinterpret_cast<f32x4 *>(&qs[(f / (HD / 4)) * HD + (f % (HD / 4)) * 4]) = qv[i];
            }
        }
        __syncthreads();
        float acc[GM];
#pragma unroll
        for (int h = 0; h < GM; h++) acc[h] = 0.0f;
        const float *kr = &ks[lane * KP];
        const float *qw = &qs[wave * GM * HD];
#pragma unroll 4   // 16 dims per step: their LDS reads are in flight together
        for (int d = 0; d < HD; d += 4) {
            const float4 kf = *reinterpret_cast<const float4 *>(kr + d);
#pragma unroll
            for (int h = 0; h < GM; h++) {
                const float4 qf = *reinterpret_cast<const float4 *>(qw + h * HD + d);
                float s = acc[h];               // dims in order, multiply and add rounded apart
                s = s + qf.x * kf.x;
                s = s + qf.y * kf.y;
                s = s + qf.z * kf.z;
                s = s + qf.w * kf.w;
                acc[h] = s;
            }
        }
        const int t = kt0 + lane;
#pragma unroll
        for (int h = 0; h < GM; h++) {
            const float sv = acc[h] * a.inv_sqrt;
            srow[h * SP + t] = sv;
            if (t < len) mx[h] = fmaxf(mx[h], sv);
        }
    }
#pragma unroll
    for (int h = 0; h < GM; h++) mx[h] = wave_max(mx[h]);
    // exponentials of the wave's own rows (positions past the length: 0)
    const int npos = nkt * PF_KT;
#pragma unroll
    for (int h = 0; h < GM; h++)
        for (int t = lane; t < npos; t += 64) {
            float *e = &srow[h * SP + t];
            *e = t < len ? expf(*e - mx[h]) : 0.0f;
        }
    __syncthreads();
    // lane h adds row h's exponentials in position order
    float inv = 0.0f;
    if (lane < GM && len > 0) {
        const float *er = &srow[lane * SP];
        float sum = 0.0f;
        for (int t = 0; t < len; t += 4) {
            const float4 e = *reinterpret_cast<const float4 *>(er + t);
            sum = sum + e.x;
            sum = sum + e.y;
            sum = sum + e.z;
            sum = sum + e.w;
        }
        inv = 1.0f / sum;
    }
    if constexpr (!FUSE) {
        if (!tok_ok) return;
#pragma unroll
        for (int h = 0; h < GM; h++) {
            const float ih = __shfl(inv, h);
            if (h >= G) continue;
            float *prow = a.scores + ((size_t)(g * G + h) * a.n_tok + b) * a.ldk;
            for (int t = lane; t < len; t += 64) prow[t] = srow[h * SP + t] * ih;   // model.c:62-63
        }
    } else {
        // probabilities in place: p = e * (1/sum), 0 past the row's length
#pragma unroll
        for (int h = 0; h < GM; h++) {
            const float ih = __shfl(inv, h);
            for (int t = lane; t < npos; t += 64) {
                float *e = &srow[h * SP + t];
                *e = t < len ? *e * ih : 0.0f;
            }
        }
        // P.V: thread slot rq = tid + i * WG is (row rq / QPR, dims 4 (rq % QPR) ..)
        constexpr int QPR = HD / 4, NRQ = (NR * QPR + WG - 1) / WG;
        f32x4 acc[NRQ];
#pragma unroll
        for (int i = 0; i < NRQ; i++) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        for (int kt = 0; kt < nkt; kt++) {
            const int kt0 = kt * PF_KT;
            __syncthreads();   // scores / probabilities written, the previous V tile read
            nxt.store(ks, KP, tid);
            if (kt + 1 < nkt) nxt.load(a.vc, a.kv_dim, (size_t)g * HD, kt0 + PF_KT, kend, tid);
            __syncthreads();
#pragma unroll
            for (int i = 0; i < NRQ; i++) {
                const int rq = tid + i * WG;
                if (rq >= NR * QPR) break;
                const float *pr = &ss[(rq / QPR) * SP + kt0];
                const float *vp = &ks[(rq % QPR) * 4];
                f32x4 o = acc[i];
#pragma unroll 8
                for (int t = 0; t < PF_KT; t++) {   // positions in order, multiply and add rounded apart
                    const float pv = pr[t];
                    const float4 v = *reinterpret_cast<const float4 *>(vp + t * KP);
                    o.x = o.x + pv * v.x;
                    o.y = o.y + pv * v.y;
                    o.z = o.z + pv * v.z;
                    o.w = o.w + pv * v.w;
                }
                acc[i] = o;
            }
        }
        const int nbk = a.n_heads * HD / QB;   // Q8_0 blocks per token row
#pragma unroll
        for (int i = 0; i < NRQ; i++) {
            const int rq = tid + i * WG;
            if (rq >= NR * QPR) break;         // uniform per 8-lane group (NR * QPR is a multiple of 8)
            const int r = rq / QPR, dq = rq % QPR, rb = b0 + r / GM, h = r % GM;
            const bool ok = rb < a.n_tok && h < G;
            const size_t col = (size_t)(g * G + min(h, G - 1)) * HD + 4 * dq;
            const f32x4 o = acc[i];
            if (ok) *reinterpret_cast<float4 *>(a.out + (size_t)rb * a.n_heads * HD + col) = make_float4(o.x, o.y, o.z, o.w);
            if (a.qx) {
                // the block of dims 32 (dq / 8) .. of this row: 8 consecutive lanes
                float mx = fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w)));
                mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0xb1, 0xf, 0xf, false)));
                mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0x4e, 0xf, 0xf, false)));
                mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0x141, 0xf, 0xf, false)));
                const float d = mx / 127.0f;
                const float id = d > 0.0f ? 1.0f / d : 0.0f;
                const int c0 = (int)fminf(fmaxf(roundf(o.x * id), -127.0f), 127.0f);
                const int c1 = (int)fminf(fmaxf(roundf(o.y * id), -127.0f), 127.0f);
                const int c2 = (int)fminf(fmaxf(roundf(o.z * id), -127.0f), 127.0f);
                const int c3 = (int)fminf(fmaxf(roundf(o.w * id), -127.0f), 127.0f);
                int cs = c0 + c1 + c2 + c3;
                cs += __builtin_amdgcn_mov_dpp(cs, 0xb1, 0xf, 0xf, false);
                cs += __builtin_amdgcn_mov_dpp(cs, 0x4e, 0xf, 0xf, false);
                cs += __builtin_amdgcn_mov_dpp(cs, 0x141, 0xf, 0xf, false);
                if (ok) {
                    *reinterpret_cast<uint32_t *>(a.qx + (size_t)rb * a.n_heads * HD + col) =
                        ((uint32_t)c0 & 0xffu) | (((uint32_t)c1 & 0xffu) << 8) |
                        (((uint32_t)c2 & 0xffu) << 16) | (((uint32_t)c3 & 0xffu) << 24);
                    if ((dq & 7) == 0) {
                        const size_t blk = (size_t)rb * nbk + col / QB;
                        a.qdx[blk] = h2f(f2h(d));
                        a.qxs[blk] = cs;
                    }
                }
            }
        }
    }
}

// grid (n_heads * n_tok / 64 rounded up), 64 rows per workgroup (rows of one
// head, consecutive tokens, so their lengths differ by at most 63).  The four
// waves compute the exponentials of a 64-position tile of all 64 rows into
// LDS (double-buffered); wave 0 then adds each row's tile in position order,
// one lane per row, while the next tile is computed.  Positions past a row's
// length contribute +0, which leaves the (positive) sum unchanged, so the sum
// is the reference's sequential one.
constexpr int RS_P = PF_KT + 4;   // es row pitch
__global__ __launch_bounds__(WG) void k_pf_rowsum(AttnArgs a) {
    __shared__ __align__(16) float es[2][64 * RS_P];
    __shared__ float smx[64];
    __shared__ int slen[64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nrows = a.n_heads * a.n_tok, r0 = blockIdx.x * 64;
    const int ntl = attn_prefill_tiles(a.ldk);
    if (wave == 0) {   // row maximum = the maximum of the row's tile maxima
        const int r = min(r0 + lane, nrows - 1);
        const int b = r % a.n_tok, len = a.pos_base + b + 1, nt = (len + PF_KT - 1) / PF_KT;
        const float4 *tm = reinterpret_cast<const float4 *>(a.tmax + (size_t)r * ntl);
        float mx = -INFINITY;
        for (int k = 0; k < nt; k += 16) {
            float4 v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = tm[min(k / 4 + i, ntl / 4 - 1)];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int k0 = k + 4 * i;
                if (k0 < nt) mx = fmaxf(mx, v[i].x);
                if (k0 + 1 < nt) mx = fmaxf(mx, v[i].y);
                if (k0 + 2 < nt) mx = fmaxf(mx, v[i].z);
                if (k0 + 3 < nt) mx = fmaxf(mx, v[i].w);
            }
        }
        smx[lane] = mx;
        slen[lane] = r0 + lane < nrows ? len : 0;
    }
    __syncthreads();
    int maxlen = 0;
#pragma unroll 4
    for (int i = 0; i < 64; i++) maxlen = max(maxlen, slen[i]);
    const int nk = (maxlen + PF_KT - 1) / PF_KT;
    // exponentials of tile k: thread -> row tid / 4, positions 16 * (tid % 4) ..
    const int er = tid / 4, eseg = (tid % 4) * 16;
    const float emx = smx[er];
    const int elen = slen[er];
    const float *erow = a.scores + (size_t)min(r0 + er, nrows - 1) * a.ldk;
    const int last4 = a.ldk - 4;
    auto stage = [&](int k, int buf) {
        float4 v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = *reinterpret_cast<const float4 *>(erow + min(k * PF_KT + eseg + 4 * i, last4));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = k * PF_KT + eseg + 4 * i;
            float4 e;
            e.x = t < elen ? expf(v[i].x - emx) : 0.0f;
            e.y = t + 1 < elen ? expf(v[i].y - emx) : 0.0f;
            e.z = t + 2 < elen ? expf(v[i].z - emx) : 0.0f;
            e.w = t + 3 < elen ? expf(v[i].w - emx) : 0.0f;
            *reinterpret_cast<float4 *>(&es[buf][er * RS_P + eseg + 4 * i]) = e;
        }
    };
    float sum = 0.0f;
    if (nk > 0) stage(0, 0);
    __syncthreads();
    for (int k = 0; k < nk; k++) {
        if (k + 1 < nk) stage(k + 1, (k + 1) & 1);
        if (wave == 0) {
            const float *er0 = &es[k & 1][lane * RS_P];
#pragma unroll 4
            for (int j = 0; j < PF_KT; j += 4) {
                const float4 e = *reinterpret_cast<const float4 *>(er0 + j);
                sum = sum + e.x;
                sum = sum + e.y;
                sum = sum + e.z;
                sum = sum + e.w;
            }
        }
        __syncthreads();
    }
    if (wave == 0 && r0 + lane < nrows) {
        a.rowmax[r0 + lane] = smx[lane];
        a.rowinv[r0 + lane] = 1.0f / sum;
    }
}

// grid (token tiles of QT, kv groups); thread (row set, d) with d = tid % HD.
// V is staged transposed (vt[d][t]) so a thread reads four positions of its
// dim in one 16-byte load; probabilities past a row's position are staged as
// zero, and adding a zero product leaves a nonzero sum bit-identical (a sum
// that is exactly zero can at most change the sign of that zero, which no
// later operation observes).
template <int HD, int GM, bool F16>
__global__ __launch_bounds__(WG) void k_pf_pv(AttnArgs a) {
    constexpr int QW = PfRows<GM>::QW, QT = 4 * QW, R = QT * GM;
    constexpr int NSET = WG / HD, RS = (R + NSET - 1) / NSET;   // rows per thread
    constexpr int TP = PF_KT + 4;                                // vt row pitch
    __shared__ __align__(16) float vt[HD * TP];
    __shared__ __align__(16) float ps[R * PF_KT];
    const int tid = threadIdx.x;
    const int G = a.n_heads / a.n_kv, g = blockIdx.y;
    const int b0 = blockIdx.x * QT;
    if (b0 >= a.n_tok) return;
    const int blast = min(a.n_tok, b0 + QT) - 1;
    const int tmax = a.pos_base + blast;                  // last key any row here needs
    const int d = tid % HD, set = tid / HD;
    const bool act = set < NSET;
    float acc[RS];
#pragma unroll
    for (int k = 0; k < RS; k++) acc[k] = 0.0f;
    const size_t hoff = (size_t)g * HD;
    for (int t0 = 0; t0 <= tmax; t0 += PF_KT) {
        __syncthreads();
        for (int f = tid; f < PF_KT * (HD / 4); f += WG) {     // V rows -> vt[d][t]
            const int t = f / (HD / 4), c = (f % (HD / 4)) * 4;
            const size_t off = (size_t)min(t0 + t, tmax) * a.kv_dim + hoff + c;
            float4 v;
            if (F16) {
                const uint2 u = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(a.vc) + off);
                v = make_float4(h2f(u.x & 0xffff), h2f(u.x >> 16), h2f(u.y & 0xffff), h2f(u.y >> 16));
            } else {
                v = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(a.vc) + off);
            }
            vt[(c + 0) * TP + t] = v.x; vt[(c + 1) * TP + t] = v.y;
            vt[(c + 2) * TP + t] = v.z; vt[(c + 3) * TP + t] = v.w;
        }
        for (int f = tid; f < R * (PF_KT / 4); f += WG) {   // p = e * (1/sum), model.c:62-63
            const int r = f / (PF_KT / 4), c = (f % (PF_KT / 4)) * 4;
            const int b = b0 + r / GM, h = r % GM;
            float4 p = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (b < a.n_tok && h < G) {
                const size_t row = (size_t)(g * G + h) * a.n_tok + b;
                const int len = a.pos_base + b + 1;
                if (t0 + c < len) {
                    const float inv = a.rowinv[row], mx = a.rowmax[row];
                    const float4 sv = *reinterpret_cast<const float4 *>(a.scores + row * a.ldk + t0 + c);
                    const int t = t0 + c;
                    p.x = expf(sv.x - mx) * inv;
                    p.y = t + 1 < len ? expf(sv.y - mx) * inv : 0.0f;
                    p.z = t + 2 < len ? expf(sv.z - mx) * inv : 0.0f;
                    p.w = t + 3 < len ? expf(sv.w - mx) * inv : 0.0f;
                }
            }
            *reinterpret_cast<float4 *>(&ps[r * PF_KT + c]) = p;
        }
        __syncthreads();
        if (!act) continue;
        const float *vrow = &vt[d * TP];
        for (int t = 0; t < PF_KT; t += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(vrow + t);
#pragma unroll
            for (int k = 0; k < RS; k++) {
                const int r = min(set * RS + k, R - 1);
                const float4 p = *reinterpret_cast<const float4 *>(&ps[r * PF_KT + t]);
                float o = acc[k];          // positions in order, multiply and add rounded apart
                o = o + p.x * v.x;
                o = o + p.y * v.y;
                o = o + p.z * v.z;
                o = o + p.w * v.w;
                acc[k] = o;
            }
        }
    }
    if (!act) return;
#pragma unroll
    for (int k = 0; k < RS; k++) {
        const int r = set * RS + k;
        const int b = b0 + r / GM, h = r % GM;
        if (r >= R || b >= a.n_tok || h >= G) continue;
        a.out[(size_t)b * a.n_heads * HD + (size_t)(g * G + h) * HD + d] = acc[k];
    }
}

// P.V for head_dim 64 / 128, register-blocked: thread (dg, rs) accumulates
// dims 4*dg .. 4*dg+3 (of the HD / DS dims blockIdx.z covers: DS > 1 splits
// a head over workgroups for short prompts) of the RPS rows rs*RPS .. of the workgroup's 64 rows
// (QT = 64 / GM tokens x GM heads), so each position costs one V float4 and
// RPS/4 probability float4 reads from LDS for 8 * RPS multiplies and adds.
// V is staged row-major (vs[t][d]); probabilities position-major
// (ps[t][row]), computed while staging as expf(s - max) * (1/sum); the next
// tile's global loads are issued before the current tile's products.  Every
// (row, dim) sums its positions in order, multiply and add rounded apart;
// positions past a row's length carry probability 0 (see k_pf_pv).
// PRE: the score rows already hold the probabilities (k_pf_softmax), which
// are staged as they are.
template <int HD, int GM, bool F16, int DS, bool PRE>
__global__ __launch_bounds__(WG) void k_pf_pv2(AttnArgs a) {
    constexpr int HDS = HD / DS;                    // this workgroup's dims: blockIdx.z * HDS ..
    constexpr int RW = 64, QT = RW / GM, DG = HDS / 4, RSETS = WG / DG, RPS = RW / RSETS;
    constexpr int VLD = PF_KT * HDS / 4 / WG;       // V float4 loads per thread per tile
    constexpr int SLD = RW * PF_KT / 4 / WG;        // score float4 loads per thread per tile
    constexpr int PP = RW + 4;                      // ps row pitch
    static_assert(RW % RSETS == 0 && (RPS == 1 || RPS % 2 == 0) && WG % DG == 0 && VLD >= 1, "layout");
    __shared__ __align__(16) float vs[PF_KT * HDS];
    __shared__ __align__(16) float ps[PF_KT * PP];
    const int tid = threadIdx.x, dg = tid % DG, rs = tid / DG;
    const int G = a.n_heads / a.n_kv, g = blockIdx.y;
    // causal rows get longer with the token: the upper half of the kv groups
    // takes the token tiles in reverse, so the two workgroups that share a CU
    // (linear ids w and w + 256 with 8 kv groups) pair a long tile with a short one
    const int xt = g >= (int)gridDim.y / 2 ? (int)gridDim.x - 1 - (int)blockIdx.x : (int)blockIdx.x;
    const int b0 = xt * QT;
    if (b0 >= a.n_tok) return;
    const int blast = min(a.n_tok, b0 + QT) - 1;
    const int tmax = a.pos_base + blast;                  // last key any row here needs
    const size_t hoff = (size_t)g * HD + (size_t)blockIdx.z * HDS;
    // the one score row this thread stages (row = tid % RW in every tile)
    const int srow = tid % RW, sb = b0 + srow / GM, sh = srow % GM;
    const bool sok = sb < a.n_tok && sh < G;
    const size_t sgrow = sok ? (size_t)(g * G + sh) * a.n_tok + sb : 0;
    const int slen = sok ? a.pos_base + sb + 1 : 0;
    const float smx = sok && !PRE ? a.rowmax[sgrow] : 0.0f, sinv = sok && !PRE ? a.rowinv[sgrow] : 0.0f;
    const float *srowp = a.scores + sgrow * a.ldk;
    const int last4 = a.ldk - 4;

    f32x4 vr[VLD], sr[SLD];
    auto load = [&](int t0) {
#pragma unroll
        for (int i = 0; i < VLD; i++) {
            const int f = tid + i * WG, t = f / DG, c = (f % DG) * 4;
            const size_t off = (size_t)min(t0 + t, tmax) * a.kv_dim + hoff + c;
            if (F16) {
                const uint2 u = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(a.vc) + off);
                vr[i] = f32x4{h2f(u.x & 0xffff), h2f(u.x >> 16), h2f(u.y & 0xffff), h2f(u.y >> 16)};
            } else {
                vr[i] = *reinterpret_cast<const f32x4 *>(reinterpret_cast<const float *>(a.vc) + off);
            }
        }
#pragma unroll
        for (int i = 0; i < SLD; i++) {
            const int c4 = (tid + i * WG) / RW;
            sr[i] = *reinterpret_cast<const f32x4 *>(srowp + min(t0 + 4 * c4, last4));
        }
    };
    auto stage = [&](int t0) {
#pragma unroll
        for (int i = 0; i < VLD; i++) {
            const int f = tid + i * WG;
            *reinterpret_cast<f32x4 *>(&vs[(f / DG) * HDS + (f % DG) * 4]) = vr[i];
        }
#pragma unroll
        for (int i = 0; i < SLD; i++) {   // p = e * (1/sum), model.c:62-63
            const int c4 = (tid + i * WG) / RW, t = t0 + 4 * c4;
            const f32x4 e = sr[i];
            if (PRE) {
                ps[(4 * c4 + 0) * PP + srow] = t < slen ? e.x : 0.0f;
                ps[(4 * c4 + 1) * PP + srow] = t + 1 < slen ? e.y : 0.0f;
                ps[(4 * c4 + 2) * PP + srow] = t + 2 < slen ? e.z : 0.0f;
                ps[(4 * c4 + 3) * PP + srow] = t + 3 < slen ? e.w : 0.0f;
            } else {
                ps[(4 * c4 + 0) * PP + srow] = t < slen ? expf(e.x - smx) * sinv : 0.0f;
                ps[(4 * c4 + 1) * PP + srow] = t + 1 < slen ? expf(e.y - smx) * sinv : 0.0f;
                ps[(4 * c4 + 2) * PP + srow] = t + 2 < slen ? expf(e.z - smx) * sinv : 0.0f;
                ps[(4 * c4 + 3) * PP + srow] = t + 3 < slen ? expf(e.w - smx) * sinv : 0.0f;
            }
        }
    };

    float acc[RPS][4];
#pragma unroll
    for (int k = 0; k < RPS; k++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[k][e] = 0.0f;
    load(0);
    for (int t0 = 0; t0 <= tmax; t0 += PF_KT) {
        __syncthreads();                   // the previous tile's products are done
        stage(t0);
        __syncthreads();
        if (t0 + PF_KT <= tmax) load(t0 + PF_KT);
        const float *vp = &vs[dg * 4];
        const float *pp = &ps[rs * RPS];
#pragma unroll 4
        for (int t = 0; t < PF_KT; t++) {
            const float4 v = *reinterpret_cast<const float4 *>(vp + t * HDS);
            float p[RPS];
            if constexpr (RPS == 1) {
                p[0] = pp[t * PP];
            } else if constexpr (RPS % 4 == 0) {
#pragma unroll
                for (int k = 0; k < RPS; k += 4) {
                    const float4 q = *reinterpret_cast<const float4 *>(pp + t * PP + k);
                    p[k] = q.x; p[k + 1] = q.y; p[k + 2] = q.z; p[k + 3] = q.w;
                }
            } else {
#pragma unroll
                for (int k = 0; k < RPS; k += 2) {
                    const float2 q = *reinterpret_cast<const float2 *>(pp + t * PP + k);
                    p[k] = q.x; p[k + 1] = q.y;
                }
            }
#pragma unroll
            for (int k = 0; k < RPS; k++) {   // positions in order, multiply and add rounded apart
                acc[k][0] = acc[k][0] + p[k] * v.x;
                acc[k][1] = acc[k][1] + p[k] * v.y;
                acc[k][2] = acc[k][2] + p[k] * v.z;
                acc[k][3] = acc[k][3] + p[k] * v.w;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < RPS; k++) {
        const int r = rs * RPS + k, b = b0 + r / GM, h = r % GM;
        if (b >= a.n_tok || h >= G) continue;
        *reinterpret_cast<float4 *>(a.out + (size_t)b * a.n_heads * HD + (size_t)(g * G + h) * HD + blockIdx.z * HDS + dg * 4) =
            make_float4(acc[k][0], acc[k][1], acc[k][2], acc[k][3]);
    }
}

// rotate pair i of one head vector (model.c:66-80) by the tabulated
// (cos, sin) of pos * freq_i, computed on the host with the reference's
// expression and libm
__device__ __forceinline__ void rope_pair(float *v, int i, int hd, float2 cs, int style) {
    const int ia = style == ROPE_NEOX ? i : 2 * i;
    const int ib = style == ROPE_NEOX ? i + hd / 2 : 2 * i + 1;
    const float v0 = v[ia], v1 = v[ib];
    v[ia] = v0 * cs.x - v1 * cs.y;
    v[ib] = v0 * cs.y + v1 * cs.x;
}

// ---- prefill QK-norm + RoPE + KV store -----------------------------------
// One wave per (token, head vector), QKP_W head vectors of a token per
// workgroup (fewer, fuller workgroups to dispatch).  Every global load (the
// vector, its norm weights, the RoPE table row, and for a key the value row)
// is issued at the start, so the wave waits for memory once.
constexpr int QKP_W = 4;
template <int HD, bool F16>
__global__ __launch_bounds__(64 * QKP_W) void k_qkpost(QkPostArgs a) {
    constexpr int ND = (HD + 63) / 64, NP = (HD / 2 + 63) / 64;   // elements / pairs per lane
    __shared__ float vsh[QKP_W][HD];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, b = blockIdx.x;
    const int vh = blockIdx.y * QKP_W + w;
    // (waves past the last head vector have nothing to do; every wave still
    // reaches the barriers)
    const bool live = vh < a.n_heads + a.n_kv;
    float *v = vsh[w];
    const int qd = a.n_heads * HD, pos = a.pos_base + b;
    const bool isq = vh < a.n_heads;
    const int g = vh - a.n_heads;
    float *row = a.qkv + (size_t)b * a.stride + (isq ? (size_t)vh * HD : (size_t)qd + (size_t)g * HD);
    const float *vrow = a.qkv + (size_t)b * a.stride + qd + a.kv_dim + (size_t)max(g, 0) * HD;
    const float *nw = isq ? a.q_norm : a.k_norm;
    float x[ND], nwv[ND], vv[ND];
    float2 cs[NP];
#pragma unroll
    for (int k = 0; k < ND; k++) {
        const int d = lane + 64 * k;
        if (live && d < HD) {
            x[k] = row[d];
            if (a.q_norm) nwv[k] = nw[d];
            if (!isq) vv[k] = vrow[d];
        }
    }
#pragma unroll
    for (int k = 0; k < NP; k++) {
        const int i = lane + 64 * k;
        if (live && i < HD / 2) cs[k] = a.rope[(size_t)pos * (HD / 2) + i];
    }
    if (a.q_norm) {   // RMSNorm of the head vector (model.c:50-55): lane sums d = lane, lane + 64
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < ND; k++)
            if (lane + 64 * k < HD) ss += x[k] * x[k];
        ss = wave_sum(ss);
        const float scale = 1.0f / sqrtf(ss / (float)HD + a.eps);
#pragma unroll
        for (int k = 0; k < ND; k++) x[k] = x[k] * scale * nwv[k];
    }
#pragma unroll
    for (int k = 0; k < ND; k++)
        if (lane + 64 * k < HD) v[lane + 64 * k] = x[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < NP; k++)
        if (lane + 64 * k < HD / 2) rope_pair(v, lane + 64 * k, HD, cs[k], a.rope_style);
    __syncthreads();
    if (!live) return;
    if (isq) {
        for (int d = lane; d < HD; d += 64) row[d] = v[d];
        return;
    }
    const size_t off = (size_t)pos * a.kv_dim + (size_t)g * HD;
#pragma unroll
    for (int k = 0; k < ND; k++) {
        const int d = lane + 64 * k;
        if (d >= HD) continue;
        if (F16) {
            reinterpret_cast<uint16_t *>(a.kc)[off + d] = f2h(v[d]);
            reinterpret_cast<uint16_t *>(a.vc)[off + d] = f2h(vv[k]);
        } else {
            reinterpret_cast<float *>(a.kc)[off + d] = v[d];
            reinterpret_cast<float *>(a.vc)[off + d] = vv[k];
        }
    }
}

// --------------------------------------------------------------------------
// k_pf_flash: the prefill attention on fp32 matrix cores, one pass over the
// keys with a running softmax (the default; the three kernels above keep the
// reference's summation order and are selected with EHIP_PF_ATTN=exact).
//
// Rows are (token, head) pairs of one kv group, row R = b * G + h, so every
// K/V tile staged in LDS serves the group's G heads.  A workgroup takes 64
// rows (16 per wave) and walks the key tiles [0, its last visible key] in
// tiles of 64 keys.  Per tile and wave, with v_mfma_f32_16x16x4f32 (lane l
// supplies A[l % 16][l / 16] and B[l / 16][l % 16] and receives
// D[4 (l / 16) + r][l % 16], r = 0..3):
//   S^T = K . Q^T  (16 keys x 16 rows per product, 4 products per tile):
//       A = K[key 16kk + l%16][dim], B = Q[row l%16][dim] with lane quarter
//       q = l/16 covering dims q*HD/4 .. +HD/4-1 over the HD/4 steps, so a
//       lane's K and Q fragments are contiguous (16-byte loads); the lane
//       receives S[row l%16][key 16kk + 4q + r];
//   O^T += V^T . P^T (16 dims x 16 rows per product, HD/16 products): the
//       contraction runs over the keys in the order the scores came out,
//       key 16kk + 4q + r at step (kk, r), so the lane's own probabilities
//       are the B operand and never leave registers; A = V^T[dim][key] is
//       one 16-byte LDS read from the transposed V tile.
// Each lane holds one row's running maximum (log2 units) and partial sum;
// the four lanes of a row see the same maximum, and their partial sums and
// output quarters are combined at the end.  Scores are q.k * (1/sqrt(hd)) *
// log2(e), probabilities 2^(s - m): one v_exp_f32 each (model.c:57-64 and
// 207-278 in another summation order: the products are fp32, the sums fp32
// in the matrix cores' order).
// Roofline: matrix-core bound, 4 * hd flops per visible (row, key) pair
// (q.k and p.v); 157.3 TFLOP/s dense fp32 on the MI355X.
// Grid (kv heads, row tiles), kv heads varying fastest, so a kv head's
// workgroups share an XCD and its L2 holds the head's K/V; row tiles in
// reverse order, so the longest (latest tokens) start first.

__device__ __forceinline__ float fl_quarter_max(float v) {   // max over lanes i, i^16, i^32, i^48
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float fl_quarter_sum(float v) { return xor32_add(xor16_add(v)); }

template <int HD, bool F16>
__global__ __launch_bounds__(WG) void k_pf_flash(AttnArgs a) {
    constexpr int NS = HD / 4;       // score product steps; lane quarter q holds dims NS*q .. NS*q + NS - 1
    constexpr int ND = HD / 16;      // 16-dim output products
    constexpr int KP = HD + 4;       // K tile pitch (floats): a 16-lane quarter's 16-byte reads hit 64 banks
    constexpr int VP = FL_BK + 4;    // transposed V tile pitch
    static_assert(NS % 4 == 0, "head_dim must be a multiple of 16");
    __shared__ __align__(16) float ks[FL_BK * KP];
    __shared__ __align__(16) float vt[HD * VP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int i = lane & 15, q = lane >> 4;
    const int g = blockIdx.x;
    const int G = a.n_heads / a.n_kv, nrows = a.n_tok * G;
    const int r0 = (gridDim.y - 1 - blockIdx.y) * FL_BR;
    const int R = min(r0 + wave * 16 + i, nrows - 1);   // this lane's row (padding rows repeat the last)
    const int b = R / G, h = R % G;
    const int pos = a.pos_base + b;                       // keys [0, pos] are visible to the row
    const int kend = a.pos_base + (min(r0 + FL_BR, nrows) - 1) / G;   // the workgroup's last visible key
    const size_t hoff = (size_t)g * HD;

    float qf[NS];
    {
        const float *qr = a.q + (size_t)b * a.q_stride + (size_t)(g * G + h) * HD + NS * q;
#pragma unroll
        for (int s = 0; s < NS; s += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(qr + s);
            qf[s] = v.x; qf[s + 1] = v.y; qf[s + 2] = v.z; qf[s + 3] = v.w;
        }
    }
    const float sscale = a.inv_sqrt * 1.4426950408889634f;
    float m = -INFINITY, lsum = 0.0f;
    f32x4 o[ND];
#pragma unroll
    for (int d = 0; d < ND; d++) o[d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // K rows [k0, k0 + 64) staged as ks[key][dim] and V rows as vt[dim][key]
    // (keys past kend repeat row kend; no row sees them).  (Loading the next
    // tile into registers during the current one's products measured no
    // faster and cost the second wave per SIMD.)
    const int nkt = kend / FL_BK + 1;
    for (int kt = 0; kt < nkt; kt++) {
        const int k0 = kt * FL_BK;
        __syncthreads();   // the previous tile has been read
        // SCH chunks of K and V per thread are loaded before any is stored,
        // so the tile costs NST / SCH memory round trips rather than NST
        constexpr int NST = FL_BK * (HD / 4) / WG, SCH = NST < 4 ? NST : 4;
        static_assert(FL_BK * (HD / 4) % WG == 0 && NST % SCH == 0, "whole chunks per thread");
#pragma unroll
        for (int c0 = 0; c0 < NST; c0 += SCH) {
            float4 kv[SCH], vv[SCH];
#pragma unroll
            for (int j = 0; j < SCH; j++) {
                const int f = tid + (c0 + j) * WG, key = f / (HD / 4), c = (f % (HD / 4)) * 4;
                const size_t off = (size_t)min(k0 + key, kend) * a.kv_dim + hoff + c;
                if (F16) {
                    const uint2 ku = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(a.kc) + off);
                    const uint2 vu = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(a.vc) + off);
                    kv[j] = make_float4(h2f(ku.x & 0xffff), h2f(ku.x >> 16), h2f(ku.y & 0xffff), h2f(ku.y >> 16));
                    vv[j] = make_float4(h2f(vu.x & 0xffff), h2f(vu.x >> 16), h2f(vu.y & 0xffff), h2f(vu.y >> 16));
                } else {
                    kv[j] = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(a.kc) + off);
                    vv[j] = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(a.vc) + off);
                }
            }
#pragma unroll
            for (int j = 0; j < SCH; j++) {
                const int f = tid + (c0 + j) * WG, key = f / (HD / 4), c = (f % (HD / 4)) * 4;
                *reinterpret_cast<float4 *>(&ks[key * KP + c]) = kv[j];
                vt[(c + 0) * VP + key] = vv[j].x;
                vt[(c + 1) * VP + key] = vv[j].y;
                vt[(c + 2) * VP + key] = vv[j].z;
                vt[(c + 3) * VP + key] = vv[j].w;
            }
        }
        __syncthreads();
        // S^T: this lane gets S[row i][key 16kk + 4q + r]
        // (the four products interleaved: consecutive MFMAs never wait on each other)
        f32x4 sc[4];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) sc[kk] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < NS; s += 4) {
            float4 kv[4];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) kv[kk] = *reinterpret_cast<const float4 *>(&ks[(16 * kk + i) * KP + NS * q + s]);
#pragma unroll
            for (int kk = 0; kk < 4; kk++) sc[kk] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[kk].x, qf[s], sc[kk], 0, 0, 0);
#pragma unroll
            for (int kk = 0; kk < 4; kk++) sc[kk] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[kk].y, qf[s + 1], sc[kk], 0, 0, 0);
#pragma unroll
            for (int kk = 0; kk < 4; kk++) sc[kk] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[kk].z, qf[s + 2], sc[kk], 0, 0, 0);
#pragma unroll
            for (int kk = 0; kk < 4; kk++) sc[kk] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[kk].w, qf[s + 3], sc[kk], 0, 0, 0);
        }
        // running softmax of the row (log2 units); keys past the row's position are masked
        float mx = -INFINITY;
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t = k0 + 16 * kk + 4 * q + r;
                const float v = t <= pos ? sc[kk][r] * sscale : -INFINITY;
                sc[kk][r] = v;
                mx = fmaxf(mx, v);
            }
        const float mn = fmaxf(m, fl_quarter_max(mx));   // finite: key 0 is in the first tile
        const float alpha = __builtin_amdgcn_exp2f(m - mn);   // 0 on the first tile (m = -inf)
        m = mn;
        lsum *= alpha;
#pragma unroll
        for (int d = 0; d < ND; d++) o[d] *= alpha;
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = __builtin_amdgcn_exp2f(sc[kk][r] - mn);   // masked: 2^-inf = 0
                sc[kk][r] = p;
                lsum += p;
            }
        // O^T += V^T . P^T over the tile's keys in the scores' order (the
        // output products interleaved)
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            float4 vv[ND];
#pragma unroll
            for (int d = 0; d < ND; d++) vv[d] = *reinterpret_cast<const float4 *>(&vt[(16 * d + i) * VP + 16 * kk + 4 * q]);
#pragma unroll
            for (int d = 0; d < ND; d++) o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[d].x, sc[kk][0], o[d], 0, 0, 0);
#pragma unroll
            for (int d = 0; d < ND; d++) o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[d].y, sc[kk][1], o[d], 0, 0, 0);
#pragma unroll
            for (int d = 0; d < ND; d++) o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[d].z, sc[kk][2], o[d], 0, 0, 0);
#pragma unroll
            for (int d = 0; d < ND; d++) o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[d].w, sc[kk][3], o[d], 0, 0, 0);
        }
    }
    // o[d][r] = O^T[dim 16d + 4q + r][row i]: four consecutive dims of the row
    const float inv = 1.0f / fl_quarter_sum(lsum);
    if (r0 + wave * 16 + i < nrows) {
        float *out = a.out + (size_t)b * a.n_heads * HD + (size_t)(g * G + h) * HD + 4 * q;
#pragma unroll
        for (int d = 0; d < ND; d++)
            *reinterpret_cast<float4 *>(out + 16 * d) = make_float4(o[d][0] * inv, o[d][1] * inv, o[d][2] * inv, o[d][3] * inv);
    }
}

// --------------------------------------------------------------------------
// k_pf_flash16: the same attention with every fp32 product carried by fp16
// matrix cores (v_mfma_f32_16x16x32_f16, eight times the fp32 products' work
// in half their cycles).  Each fp32 operand x is scaled by a power of two so
// that its group's largest magnitude lies in [2^14, 2^15), then split as
// hi = fp16(x), lo = fp16(x - hi) (|x - hi - lo| <= 2^-22 |x|); a product is
// lo.hi + hi.lo + hi.hi, the dropped lo.lo term below 2^-22 of it.  Products
// and sums are fp32 in the matrix cores, and the power-of-two scales are
// removed exactly (ldexp), so the scores and outputs carry about four times
// the fp32 rounding of k_pf_flash.  Scales: one per Q row (its four lanes'
// maximum), one per K row and per V row; a row's probabilities p <= 1 of a
// tile are multiplied by 2^(14 + E - e_v) with E the smallest V-row
// exponent among the keys the row sees in that tile, so the row's output
// accumulator holds 2^(14 + E) sum p v and is rescaled by 2^(E - E') with
// the running softmax when E changes.  An fp16 cache needs neither the K/V
// scales nor lo planes: its values are fp16 already.
//
// k_pf_kvsplit converts the pass's keys once per layer: per (kv head, 64-key
// tile) it writes the tile's image (below) to HBM, and every row tile of
// k_pf_flash16 copies it into LDS as it lies, with direct-to-LDS loads
// (global_load_lds_dwordx4: a wave moves 1 KB of contiguous bytes without
// passing them through registers), instead of converting the tile again (at
// pp4096 each K/V row was otherwise converted by up to 32 workgroups).  The
// image, per tile, unpadded: 16-byte pieces are XOR-swizzled within their row
// by the row index, so the 16 rows a matrix-core operand read touches hit
// distinct banks:
//   K planes [plane][row][dim], key 32t + 8a + 4b + r at row
//   32t + 16b + 4a + r (fl_krow), so score product kk = 2t + b reads 16
//   consecutive rows and lane quarter q receives keys 32t + 8q + 4b + r:
//   eight consecutive keys per lane and 32-key half tile;
//   the per-key exponents of K and V (fp32 cache), int kex[64], vex[64];
//   V^T planes [plane][dim][key] (rows of 64 keys): the P.V product over keys
//   32t + 8q .. +7 (lane quarter q, element 4b + r) reads them as one 16-byte
//   row piece, and the lane's own probabilities are its B operand.
// k_pf_flash16 stages the first two parts (K and exponents) and the V part
// separately, each while the other is in use, so a tile's loads overlap the
// previous tile's products.
// Conversion: wave w takes key pairs 8w .. 8w + 7, lane l key pair
// 8w + (l & 7) and dim quads (l >> 3) + 8c; a row's maximum is a reduction
// over the eight lanes of its pair.  Keys past the pass's last repeat it.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));   // 16-byte image piece (kept in registers)

// maximum over lanes i, i ^ 8, i ^ 16, ... (the lanes of one key pair)
__device__ __forceinline__ float fl_pair_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, false)));   // row_ror:8
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}


size_t attn_kvimg_bytes(int hd, bool f16kv, int ctx, int n_kv) {
    const size_t tiles = (size_t)(ctx + FL_BK - 1) / FL_BK * (size_t)n_kv;
    switch (hd) {
        case 64: return tiles * (f16kv ? FlImg<64, true>::HBYTES : FlImg<64, false>::HBYTES);
        case 128: return tiles * (f16kv ? FlImg<128, true>::HBYTES : FlImg<128, false>::HBYTES);
    }
    return 0;
}

// grid (kv heads, tiles of the pass's keys [0, pos_base + n_tok))
template <int HD, bool F16>
__global__ __launch_bounds__(WG) void k_pf_kvsplit(AttnArgs a) {
    using I = FlImg<HD, F16>;
    constexpr int NC = HD / 32;         // dim quads per lane and key
    __shared__ __align__(16) uint8_t img[I::HBYTES];   // the image as it goes to HBM
    uint8_t *vimg = img + I::KE;
    int *kex = reinterpret_cast<int *>(img + I::KBYTES), *vex = kex + FL_BK;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = blockIdx.x, kt = blockIdx.y;
    const int klast = a.pos_base + a.n_tok - 1;
    const size_t hoff = (size_t)g * HD;
    const int k0 = kt * FL_BK;
    const int kp = 8 * wave + (lane & 7), dq0 = lane >> 3;
    if constexpr (F16) {
        uint2 kr[2][NC], vr[2][NC];
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const size_t off = (size_t)min(k0 + 2 * kp + j, klast) * a.kv_dim + hoff + 4 * (dq0 + 8 * c);
                kr[j][c] = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(a.kc) + off);
                vr[j][c] = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(a.vc) + off);
            }
        // dim quad dq = dq0 + 8c is half (dq & 1) of piece dq >> 1 of its K row;
        // keys 2kp, 2kp + 1 are word kp & 3 of piece kp >> 2 of a V^T row
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const int dq = dq0 + 8 * c;
                *reinterpret_cast<uint2 *>(img + I::k_at(fl_krow(2 * kp + j), dq >> 1) + 8 * (dq & 1)) = kr[j][c];
            }
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int d0 = 4 * (dq0 + 8 * c), w = 4 * (kp & 3);
            const uint32_t r4[4] = { (vr[0][c].x & 0xffffu) | (vr[1][c].x << 16),
                                     (vr[0][c].x >> 16) | (vr[1][c].x & 0xffff0000u),
                                     (vr[0][c].y & 0xffffu) | (vr[1][c].y << 16),
                                     (vr[0][c].y >> 16) | (vr[1][c].y & 0xffff0000u) };
#pragma unroll
            for (int e = 0; e < 4; e++)
                *reinterpret_cast<uint32_t *>(vimg + I::v_at(d0 + e, kp >> 2) + w) = r4[e];
        }
    } else {
        f32x4 kr[2][NC], vr[2][NC];
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const size_t off = (size_t)min(k0 + 2 * kp + j, klast) * a.kv_dim + hoff + 4 * (dq0 + 8 * c);
                kr[j][c] = *reinterpret_cast<const f32x4 *>(reinterpret_cast<const float *>(a.kc) + off);
                vr[j][c] = *reinterpret_cast<const f32x4 *>(reinterpret_cast<const float *>(a.vc) + off);
            }
        int ek[2], ev[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            float km = 0.0f, vm = 0.0f;
#pragma unroll
            for (int c = 0; c < NC; c++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    km = fmaxf(km, fabsf(kr[j][c][e]));
                    vm = fmaxf(vm, fabsf(vr[j][c][e]));
                }
            ek[j] = fl_exp(fl_pair_max(km));
            ev[j] = fl_exp(fl_pair_max(vm));
        }
        if (dq0 == 0) {
            kex[2 * kp] = ek[0]; kex[2 * kp + 1] = ek[1];
            vex[2 * kp] = ev[0]; vex[2 * kp + 1] = ev[1];
        }
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int c = 0; c < NC; c++) {
                _Float16 hi[4], lo[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float x = __builtin_amdgcn_ldexpf(kr[j][c][e], ek[j]);
                    hi[e] = (_Float16)x;
                    lo[e] = (_Float16)(x - (float)hi[e]);
                }
                const int dq = dq0 + 8 * c, rk = fl_krow(2 * kp + j);
                *reinterpret_cast<uint2 *>(img + I::k_at(rk, dq >> 1) + 8 * (dq & 1)) =
                    make_uint2(fl_pack(hi[0], hi[1]), fl_pack(hi[2], hi[3]));
                *reinterpret_cast<uint2 *>(img + I::k_at(FL_BK + rk, dq >> 1) + 8 * (dq & 1)) =
                    make_uint2(fl_pack(lo[0], lo[1]), fl_pack(lo[2], lo[3]));
            }
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float x0 = __builtin_amdgcn_ldexpf(vr[0][c][e], ev[0]);
                const float x1 = __builtin_amdgcn_ldexpf(vr[1][c][e], ev[1]);
                const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
                const _Float16 l0 = (_Float16)(x0 - (float)h0), l1 = (_Float16)(x1 - (float)h1);
                const int d = 4 * (dq0 + 8 * c) + e, w = 4 * (kp & 3);
                *reinterpret_cast<uint32_t *>(vimg + I::v_at(d, kp >> 2) + w) = fl_pack(h0, h1);
                *reinterpret_cast<uint32_t *>(vimg + I::v_at(HD + d, kp >> 2) + w) = fl_pack(l0, l1);
            }
    }
    __syncthreads();
    // the image to HBM as it lies
    u32x4 *dst = reinterpret_cast<u32x4 *>(a.kvimg + ((size_t)g * a.kvimg_tiles + kt) * I::HBYTES);
    for (int p = tid; p < I::HBYTES / 16; p += WG) dst[p] = *reinterpret_cast<const u32x4 *>(img + 16 * p);
}

template <bool B> struct FlMask { static constexpr bool value = B; };

// s_waitcnt immediate that waits until at most n vector memory operations of
// the wave are outstanding (expcnt and lgkmcnt left alone)
constexpr int fl_vmcnt(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }
// Workgroup barrier for the staging loop: this wave's LDS reads are done,
// then s_barrier, with no fence (a workgroup fence would wait for every
// vector memory operation, the next part's loads included; the loop waits for
// the loads it needs with explicit vmcnt counts).  The empty asm statements
// keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void fl_sync() {
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));   // lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}
// one 16-byte piece per lane from src into LDS at the wave-uniform base dst,
// lane l's piece at dst + 16 l (global_load_lds_dwordx4)
__device__ __forceinline__ void fl_load_lds(const uint8_t *src, uint8_t *dst) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
}

// 64 rows per workgroup, two workgroups per CU: one's barriers overlap the
// other's products (128 rows per workgroup, one per CU, measured slower).
// Per key tile, with its K part and exponents (kimg) and its V part (vimg)
// staged separately by direct-to-LDS loads:
//   scores from kimg, the exponents read; barrier; the next tile's K part
//   issued into kimg; softmax; wait for this tile's V part; barrier; P.V from
//   vimg; wait for the next K part; barrier; the next tile's V part issued.
// Each part's loads land while the other part's products run.
// KS = 2 (grids of fewer workgroups than CUs: short passes): two groups of
// RW waves per workgroup take the same 16 RW rows over alternate key tiles
// (group g tiles g, g + 2, ...), each with its own staging buffers and
// running softmax, and group 0 merges group 1's state (maximum, sums,
// accumulators through LDS) before the output; the barriers stay uniform.
// RW = 2 halves the rows per workgroup, so the grid doubles onto idle CUs.
template <int HD, bool F16, int KS, int RW>
__global__ __launch_bounds__(64 * RW * KS) void k_pf_flash16(AttnArgs a) {
    using I = FlImg<HD, F16>;
    constexpr int NQ = HD / 32;         // 32-dim steps of a score product
    constexpr int ND = HD / 16;         // 16-dim output products
    constexpr int GT = 64 * RW;                          // threads per key-tile group
    constexpr int BR = 16 * RW;                          // rows per workgroup
    constexpr int KE_N = (I::KE_SLABS + RW - 1) / RW, KE_MIN = I::KE_SLABS / RW;   // K-part slabs per wave
    constexpr int V_N = I::V_SLABS / RW;
    static_assert(HD % 32 == 0 && FL_BK == 64 && FL_BR == 64 && I::V_SLABS % RW == 0 && (RW == 4 || KS == 2),
                  "tile shape");
    static_assert(KS == 1 || KS == 2, "one or two key-tile groups");
    __shared__ __align__(16) uint8_t kimgs[KS][I::KE_SLABS * I::SLAB];   // K planes, exponents, slab padding
    __shared__ __align__(16) uint8_t vimgs[KS][I::VBYTES];
    const int grp = KS == 1 ? 0 : (int)threadIdx.x / GT;   // key-tile group
    uint8_t *kimg = kimgs[grp], *vimg = vimgs[grp];
    const int *kex = reinterpret_cast<const int *>(kimg + I::KBYTES), *vex = kex + FL_BK;
    const int tid = KS == 1 ? (int)threadIdx.x : (int)threadIdx.x % GT, lane = tid & 63, wave = tid >> 6;
    const int i = lane & 15, q = lane >> 4;
    const int g = blockIdx.x;
    const int G = a.n_heads / a.n_kv, nrows = a.n_tok * G;
    const int r0 = (gridDim.y - 1 - blockIdx.y) * BR;
    const int R = min(r0 + wave * 16 + i, nrows - 1);   // this lane's row (padding rows repeat the last)
    const int b = R / G, h = R % G;
    const int pos = a.pos_base + b;                       // keys [0, pos] are visible to the row
    const int kend = a.pos_base + (min(r0 + BR, nrows) - 1) / G;   // the workgroup's last visible key
    const int kfirst = a.pos_base + r0 / G;   // keys [0, kfirst] are visible to every row of the workgroup

    // the Q row: lane quarter q holds dims 32s + 8q .. + 7 of step s
    f16x8 qh[NQ], ql[NQ];
    int eq;
    {
        const float *qr = a.q + (size_t)b * a.q_stride + (size_t)(g * G + h) * HD + 8 * q;
        f32x4 qv[NQ][2];
        float mx = 0.0f;
#pragma unroll
        for (int s = 0; s < NQ; s++)
#pragma unroll
            for (int u = 0; u < 2; u++) {
                qv[s][u] = *reinterpret_cast<const f32x4 *>(qr + 32 * s + 4 * u);
#pragma unroll
                for (int e = 0; e < 4; e++) mx = fmaxf(mx, fabsf(qv[s][u][e]));
            }
        eq = fl_exp(fl_quarter_max(mx));
#pragma unroll
        for (int s = 0; s < NQ; s++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float x = __builtin_amdgcn_ldexpf(qv[s][e >> 2][e & 3], eq);
                qh[s][e] = (_Float16)x;
                ql[s][e] = (_Float16)(x - (float)qh[s][e]);
            }
    }
    const float sscale = a.inv_sqrt * 1.4426950408889634f;
    float m = -INFINITY, lsum = 0.0f;
    int ecur = 0;   // the row's accumulator holds 2^(14 + ecur) * sum p v
    f32x4 o[ND];
#pragma unroll
    for (int d = 0; d < ND; d++) o[d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // wave w moves slabs w, w + 4, ... of a part; the K part's last slab is
    // partly past the image, and its lanes there re-read the last piece into
    // kimg's padding
    const uint8_t *gimg = a.kvimg + (size_t)g * a.kvimg_tiles * I::HBYTES;
    auto stage_ke = [&](int kt) {
        const uint8_t *src = gimg + (size_t)kt * I::HBYTES;
#pragma unroll
        for (int u = 0; u < KE_N; u++) {
            const int sl = wave + RW * u;
            if (u < KE_MIN || sl < I::KE_SLABS)
                fl_load_lds(src + min(sl * I::SLAB + 16 * lane, I::KE - 16), kimg + sl * I::SLAB);
        }
    };
    auto stage_v = [&](int kt) {
        const uint8_t *src = gimg + (size_t)kt * I::HBYTES + I::KE;
#pragma unroll
        for (int u = 0; u < V_N; u++) {
            const int sl = wave + RW * u;
            fl_load_lds(src + sl * I::SLAB + 16 * lane, vimg + sl * I::SLAB);
        }
    };
    const int nkt = kend / FL_BK + 1, nit = (nkt + KS - 1) / KS;
    if (grp < nkt) {
        stage_ke(grp);
        stage_v(grp);
    }
    __builtin_amdgcn_s_waitcnt(fl_vmcnt(0));
    __syncthreads();

    for (int it = 0; it < nit; it++) {
        // this group's tile kt (act: it has one); `more`: another iteration
        // follows (uniform: the barriers); gmore: this group has a tile in it
        const int kt = it * KS + grp, k0 = kt * FL_BK;
        const bool act = KS == 1 || kt < nkt, more = it + 1 < nit, gmore = KS == 1 ? more : kt + KS < nkt;
        // ---- S'^T: sc[2t + b][r] = S'[row i][key k0 + 32t + 8q + 4b + r]
        f32x4 sc[4];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) sc[kk] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        int kx[2][8], vx[2][8];   // the per-key exponents of this lane's 16 keys
        if (act) {
#pragma unroll
        for (int s = 0; s < NQ; s++) {
            f16x8 kh[4], kl[4];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                kh[kk] = *reinterpret_cast<const f16x8 *>(kimg + I::k_at(16 * kk + i, 4 * s + q));
                if constexpr (!F16) kl[kk] = *reinterpret_cast<const f16x8 *>(kimg + I::k_at(FL_BK + 16 * kk + i, 4 * s + q));
            }
            if constexpr (!F16) {
#pragma unroll
                for (int kk = 0; kk < 4; kk++) sc[kk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl[kk], qh[s], sc[kk], 0, 0, 0);
            }
#pragma unroll
            for (int kk = 0; kk < 4; kk++) sc[kk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[kk], ql[s], sc[kk], 0, 0, 0);
#pragma unroll
            for (int kk = 0; kk < 4; kk++) sc[kk] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[kk], qh[s], sc[kk], 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int u = 0; u < 2; u++) {
                if constexpr (F16) {
#pragma unroll
                    for (int e = 0; e < 4; e++) kx[t][4 * u + e] = vx[t][4 * u + e] = 0;
                } else {
                    const int4 ka = *reinterpret_cast<const int4 *>(&kex[32 * t + 8 * q + 4 * u]);
                    const int4 va = *reinterpret_cast<const int4 *>(&vex[32 * t + 8 * q + 4 * u]);
                    kx[t][4 * u] = ka.x; kx[t][4 * u + 1] = ka.y; kx[t][4 * u + 2] = ka.z; kx[t][4 * u + 3] = ka.w;
                    vx[t][4 * u] = va.x; vx[t][4 * u + 1] = va.y; vx[t][4 * u + 2] = va.z; vx[t][4 * u + 3] = va.w;
                }
            }
        }
        if (more) {   // every wave is past its kimg reads: the next tile's K part may land
            fl_sync();
            if (gmore) stage_ke(kt + KS);
        }
        f16x8 ph[2], pl[2];
        if (act) {
        // running softmax of the row (log2 units); keys past the row's position
        // are masked (only in tiles that reach past the workgroup's first row)
        float mx = -INFINITY;
        int el = 1 << 20;   // the smallest V-row exponent among the row's visible keys of the tile
        auto scores = [&](auto masked) {
#pragma unroll
            for (int kk = 0; kk < 4; kk++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int t = kk >> 1, jj = 4 * (kk & 1) + r;
                    float v = __builtin_amdgcn_ldexpf(sc[kk][r], -(eq + kx[t][jj])) * sscale;
                    if constexpr (decltype(masked)::value) {
                        const bool vis = k0 + 32 * t + 8 * q + jj <= pos;
                        v = vis ? v : -INFINITY;
                        if (vis) el = min(el, vx[t][jj]);
                    } else {
                        el = min(el, vx[t][jj]);
                    }
                    sc[kk][r] = v;
                    mx = fmaxf(mx, v);
                }
        };
        if (k0 + FL_BK - 1 <= kfirst) scores(FlMask<false>{});
        else scores(FlMask<true>{});
        // finite: key 0 is in the first tile (KS = 2: group 1's first tile can
        // hide every key from a row; its maximum stays -inf and mz stands in)
        const float mn = fmaxf(m, fl_quarter_max(mx));
        const float mz = KS == 1 || mn != -INFINITY ? mn : 0.0f;
        const float alpha = __builtin_amdgcn_exp2f(m - mz);   // 0 on the first tile (m = -inf)
        m = mn;
        lsum *= alpha;
        int emin = -(int)fl_quarter_max(-(float)el);
        if (emin == (1 << 20)) emin = ecur;   // no visible key in this tile
        const float of = __builtin_amdgcn_ldexpf(alpha, emin - ecur);
        ecur = emin;
#pragma unroll
        for (int d = 0; d < ND; d++) o[d] *= of;
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t = kk >> 1, jj = 4 * (kk & 1) + r;
                const float p = __builtin_amdgcn_exp2f(sc[kk][r] - mz);   // masked: 2^-inf = 0
                lsum += p;
                const float x = __builtin_amdgcn_ldexpf(p, 14 + emin - vx[t][jj]);
                ph[t][jj] = (_Float16)x;
                pl[t][jj] = (_Float16)(x - (float)ph[t][jj]);
            }
        }
        if (it > 0) {   // this tile's V part, issued before the next tile's K part
            if (gmore) __builtin_amdgcn_s_waitcnt(fl_vmcnt(KE_MIN));
            else __builtin_amdgcn_s_waitcnt(fl_vmcnt(0));
            fl_sync();
        }
        // ---- O''^T += V'^T . P''^T over keys 32t + 8q + jj
        if (act)
#pragma unroll
        for (int t = 0; t < 2; t++) {
            f16x8 vh[ND], vl[ND];
#pragma unroll
            for (int d = 0; d < ND; d++) {
                vh[d] = *reinterpret_cast<const f16x8 *>(vimg + I::v_at(16 * d + i, 4 * t + q));
                if constexpr (!F16) vl[d] = *reinterpret_cast<const f16x8 *>(vimg + I::v_at(HD + 16 * d + i, 4 * t + q));
            }
            if constexpr (!F16) {
#pragma unroll
                for (int d = 0; d < ND; d++) o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl[d], ph[t], o[d], 0, 0, 0);
            }
#pragma unroll
            for (int d = 0; d < ND; d++) o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh[d], pl[t], o[d], 0, 0, 0);
#pragma unroll
            for (int d = 0; d < ND; d++) o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh[d], ph[t], o[d], 0, 0, 0);
        }
        if (more) {   // the next K part has landed and every wave is past its vimg reads
            __builtin_amdgcn_s_waitcnt(fl_vmcnt(0));
            fl_sync();
            if (gmore) stage_v(kt + KS);
        }
    }
    // o[d][r] = 2^(14 + ecur) O^T[dim 16d + 4q + r][row i]
    if constexpr (KS == 2) {
        // group 1's state into group 0's: with M the larger maximum, each
        // group's sums and accumulators (unscaled) weighted by 2^(m - M)
        __syncthreads();   // every wave is past its last image reads
        float *mo = reinterpret_cast<float *>(&vimgs[0][0]), *ms = reinterpret_cast<float *>(kimgs[1]);
        static_assert(ND * 4 * GT * 4 <= KS * I::VBYTES && 3 * GT * 4 <= I::KE_SLABS * I::SLAB, "merge fits the images");
        if (grp == 1) {
#pragma unroll
            for (int d = 0; d < ND; d++)
#pragma unroll
                for (int r = 0; r < 4; r++) mo[(4 * d + r) * GT + tid] = o[d][r];
            ms[tid] = m;
            ms[GT + tid] = lsum;
            ms[2 * GT + tid] = __int_as_float(ecur);
        }
        __syncthreads();
        if (grp == 1) return;
        const float m1 = ms[tid], l1 = ms[GT + tid];
        const int e1 = __float_as_int(ms[2 * GT + tid]);
        const float mm = fmaxf(m, m1);   // finite: group 0 holds key 0
        const float a0 = __builtin_amdgcn_exp2f(m - mm), a1 = __builtin_amdgcn_exp2f(m1 - mm);
        const float inv = 1.0f / fl_quarter_sum(lsum * a0 + l1 * a1);
#pragma unroll
        for (int d = 0; d < ND; d++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                o[d][r] = (__builtin_amdgcn_ldexpf(o[d][r], -(14 + ecur)) * a0 +
                           __builtin_amdgcn_ldexpf(mo[(4 * d + r) * GT + tid], -(14 + e1)) * a1) * inv;
    } else {
        const float inv = 1.0f / fl_quarter_sum(lsum);
        const int un = -(14 + ecur);
#pragma unroll
        for (int d = 0; d < ND; d++)
#pragma unroll
            for (int r = 0; r < 4; r++) o[d][r] = __builtin_amdgcn_ldexpf(o[d][r], un) * inv;
    }
    const bool live = r0 + wave * 16 + i < nrows;
    const size_t col = (size_t)(g * G + h) * HD + 4 * q;
    const size_t row = (size_t)b * a.n_heads * HD;
    if (live) {
#pragma unroll
        for (int d = 0; d < ND; d++)
            *reinterpret_cast<float4 *>(a.out + row + col + 16 * d) = make_float4(o[d][0], o[d][1], o[d][2], o[d][3]);
    }
    if (!a.qx) return;
    // the output's Q8_0 blocks for wo, with k_quant_rows's arithmetic: block
    // bk (dims 32bk ..) is o[2bk], o[2bk + 1] of the row's four lanes
    const int nbk = a.n_heads * HD / QB;
#pragma unroll
    for (int bk = 0; bk < ND / 2; bk++) {
        float mx = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int r = 0; r < 4; r++) mx = fmaxf(mx, fabsf(o[2 * bk + u][r]));
        mx = fl_quarter_max(mx);
        const float dsc = mx / 127.0f;
        const float id = dsc > 0.0f ? 1.0f / dsc : 0.0f;
        int cs = 0;
        uint32_t pk[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            pk[u] = 0;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int cq = (int)fminf(fmaxf(roundf(o[2 * bk + u][r] * id), -127.0f), 127.0f);
                cs += cq;
                pk[u] |= ((uint32_t)cq & 0xffu) << (8 * r);
            }
        }
        cs = (int)fl_quarter_sum((float)cs);   // exact: |sum| <= 32 * 127
        if (live) {
#pragma unroll
            for (int u = 0; u < 2; u++)
                *reinterpret_cast<uint32_t *>(a.qx + row + col + 16 * (2 * bk + u)) = pk[u];
            if (q == 0) {
                const size_t blk = (size_t)b * nbk + ((size_t)(g * G + h) * HD) / QB + bk;
                a.qdx[blk] = h2f(f2h(dsc));
                a.qxs[blk] = cs;
            }
        }
    }
}

// (host) integer environment switch, dflt when unset
static int env_int_attn(const char *name, int dflt) {
    const char *v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

int launch_attention_mfma(hipStream_t st, bool f16kv, const AttnArgs &a, bool *quantized) {
    if (quantized) *quantized = false;
    if (a.n_kv <= 0 || a.n_heads % a.n_kv != 0 || a.n_tok <= 0 || a.q_stride % 4) return -1;
    if (a.qx && (!a.qdx || !a.qxs)) return -1;
    const int G = a.n_heads / a.n_kv;
    const dim3 grid(a.n_kv, (a.n_tok * G + FL_BR - 1) / FL_BR);
    if (a.hd == 64 || a.hd == 128) {
        const int nkt = (a.pos_base + a.n_tok + FL_BK - 1) / FL_BK;
        if (!a.kvimg || a.kvimg_tiles < nkt) return -1;
        if (a.kvimg_fused && a.pos_base % FL_BK != 0) return -1;
        // tiles to convert here: all, or those before the pass (the q|k|v
        // product wrote the pass's own)
        const int nks = a.kvimg_fused ? a.pos_base / FL_BK : nkt;
        if (quantized) *quantized = a.qx != nullptr;
        const dim3 sgrid(a.n_kv, nks);
        // grids of up to one 64-row workgroup per CU (two for 64-dim heads,
        // whose images take half the LDS): 32-row workgroups of two key-tile
        // groups, twice the grid (Qwen3-0.6B shape pp512 3.17 -> 3.00 ms,
        // pp1024 4.67 -> 4.52; SmolLM2-135M shape pp1024 2.87 -> 2.63,
        // pp3072 6.25 -> 5.91; pp1536 with 128-dim heads, 384 workgroups,
        // 6.63 -> 6.95 ms: there the one-group tiles stay).  Measured and
        // dropped: 8-wave workgroups of two groups over the same 64 rows
        // (3.11 ms at pp512: the grid still covered half the CUs).
        // EHIP_PF_FLASH_KS=1 keeps the one-group kernel.
        const long gmax = a.hd == 64 ? 512 : 256;
        const bool ks2 = (long)grid.x * grid.y <= gmax && env_int_attn("EHIP_PF_FLASH_KS", 2) == 2;
        const dim3 grid2(a.n_kv, (a.n_tok * G + 31) / 32);
#define FL16(H, F)                                                                         \
    if (nks > 0) hipLaunchKernelGGL((k_pf_kvsplit<H, F>), sgrid, dim3(WG), 0, st, a);     \
    if (ks2) hipLaunchKernelGGL((k_pf_flash16<H, F, 2, 2>), grid2, dim3(WG), 0, st, a);   \
    else hipLaunchKernelGGL((k_pf_flash16<H, F, 1, 4>), grid, dim3(WG), 0, st, a);
        if (a.hd == 64) {
            if (f16kv) { FL16(64, true) } else { FL16(64, false) }
        } else {
            if (f16kv) { FL16(128, true) } else { FL16(128, false) }
        }
#undef FL16
        return 0;
    }
    switch (a.hd) {
#define FLL(H)                                                                                  \
    case H:                                                                                     \
        if (f16kv) hipLaunchKernelGGL((k_pf_flash<H, true>), grid, dim3(WG), 0, st, a);         \
        else hipLaunchKernelGGL((k_pf_flash<H, false>), grid, dim3(WG), 0, st, a);              \
        return 0;
        FLL(48) FLL(64) FLL(128)
#undef FLL
    }
    return -1;
}

// --------------------------------------------------------------------------
template <int HD, int GM, bool F16>
static void pf_go(hipStream_t st, const AttnArgs &a, bool *quantized) {
    constexpr int QT = 4 * PfRows<GM>::QW;
    const int ktiles = (a.pos_base + a.n_tok + PF_KT - 1) / PF_KT;
    const int qtiles = (a.n_tok + QT - 1) / QT;
    if constexpr (HD == 64 || HD == 128) {
        if (a.pos_base + a.n_tok <= PF_FUSE_KEYS) {
            // the whole attention in one kernel (and the output's quantization)
            hipLaunchKernelGGL((k_pf_softmax<HD, GM, F16, true>), dim3((a.n_tok + 3) / 4, a.n_kv), dim3(WG), 0, st, a);
            if (quantized) *quantized = a.qx != nullptr;
            return;
        }
        if (a.pos_base + a.n_tok <= PF_SM_KEYS) {
            // scores and softmax in one kernel, then P.V over the stored
            // probabilities with the head dims split 16 per workgroup
            hipLaunchKernelGGL((k_pf_softmax<HD, GM, F16, false>), dim3((a.n_tok + 3) / 4, a.n_kv), dim3(WG), 0, st, a);
            constexpr int QT2 = 64 / GM, DSPLIT = HD / 16;
            hipLaunchKernelGGL((k_pf_pv2<HD, GM, F16, DSPLIT, true>), dim3((a.n_tok + QT2 - 1) / QT2, a.n_kv, DSPLIT),
                               dim3(WG), 0, st, a);
            return;
        }
    }
    // short prompts: one token row per wave for four times the workgroups
    if (PfRows<GM>::QW > 1 && (long)ktiles * qtiles * a.n_kv < 1024)
        hipLaunchKernelGGL((k_pf_scores<HD, GM, F16, 1>), dim3(ktiles, (a.n_tok + 3) / 4, a.n_kv), dim3(WG), 0, st, a);
    else
        hipLaunchKernelGGL((k_pf_scores<HD, GM, F16, PfRows<GM>::QW>), dim3(ktiles, qtiles, a.n_kv), dim3(WG), 0, st, a);
    hipLaunchKernelGGL(k_pf_rowsum, dim3((a.n_heads * a.n_tok + 63) / 64), dim3(WG), 0, st, a);
    if constexpr (HD == 64 || HD == 128) {
        // short prompts: split the head dims over workgroups (32 per
        // workgroup) so the grid covers more CUs; each (row, dim) still sums
        // its positions in order
        constexpr int QT2 = 64 / GM, DSPLIT = HD / 32;
        const dim3 g2((a.n_tok + QT2 - 1) / QT2, a.n_kv);
        if ((long)g2.x * g2.y < 1024)   // measured: up to pp2048 for 8 kv heads
            hipLaunchKernelGGL((k_pf_pv2<HD, GM, F16, DSPLIT, false>), dim3(g2.x, g2.y, DSPLIT), dim3(WG), 0, st, a);
        else
            hipLaunchKernelGGL((k_pf_pv2<HD, GM, F16, 1, false>), g2, dim3(WG), 0, st, a);
    } else {
        hipLaunchKernelGGL((k_pf_pv<HD, GM, F16>), dim3(qtiles, a.n_kv), dim3(WG), 0, st, a);
    }
}

template <int HD, bool F16>
static int pf_pick_g(hipStream_t st, const AttnArgs &a, bool *quantized) {
    const int G = a.n_heads / a.n_kv;
    if (G <= 1) pf_go<HD, 1, F16>(st, a, quantized);
    else if (G <= 2) pf_go<HD, 2, F16>(st, a, quantized);
    else if (G <= 4) pf_go<HD, 4, F16>(st, a, quantized);
    else if (G <= 8) pf_go<HD, 8, F16>(st, a, quantized);
    else return -1;
    return 0;
}

int launch_attention(hipStream_t st, bool f16kv, const AttnArgs &a, bool *quantized) {
    if (quantized) *quantized = false;
    if (a.n_kv <= 0 || a.n_heads % a.n_kv != 0 || a.n_tok <= 0 || !a.scores || !a.tmax || !a.rowmax || !a.rowinv)
        return -1;
    if (a.ldk < a.pos_base + a.n_tok || a.ldk % 4) return -1;
    if (a.qx && (!a.qdx || !a.qxs || (a.n_heads * a.hd) % QB)) return -1;
    switch (a.hd) {
        case 48: return f16kv ? pf_pick_g<48, true>(st, a, quantized) : pf_pick_g<48, false>(st, a, quantized);
        case 64: return f16kv ? pf_pick_g<64, true>(st, a, quantized) : pf_pick_g<64, false>(st, a, quantized);
        case 128: return f16kv ? pf_pick_g<128, true>(st, a, quantized) : pf_pick_g<128, false>(st, a, quantized);
    }
    return -1;
}

int launch_qkpost(hipStream_t st, bool f16kv, const QkPostArgs &a) {
    dim3 grid(a.n_tok, (a.n_heads + a.n_kv + QKP_W - 1) / QKP_W);
    switch (a.hd) {
#define QKP(H)                                                                              \
    case H:                                                                                 \
        if (f16kv) hipLaunchKernelGGL((k_qkpost<H, true>), grid, dim3(64 * QKP_W), 0, st, a); \
        else hipLaunchKernelGGL((k_qkpost<H, false>), grid, dim3(64 * QKP_W), 0, st, a);    \
        return 0;
        QKP(48) QKP(64) QKP(128)
#undef QKP
    }
    return -1;
}

}  // namespace ehip
