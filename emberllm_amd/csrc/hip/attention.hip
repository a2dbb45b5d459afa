// attention.hip — prefill GQA attention over the HBM-resident KV cache (gfx950).
//
// Replaces the per-token attention calls of ember_prefill (src/model.c:335-337
// -> attention -> attn_heads + softmax, model.c:57-64, 207-278) and its
// QK-norm / RoPE / kv_store loop (model.c:323-333, k_qkpost).  The decode
// form lives in attn_decode.hip.
//
// Roofline: HBM-bound.  Algorithmic bytes per decode step and layer =
// 2 * (pos+1) * kv_dim * esize (K and V read once) + 2 * kv_dim * esize (the
// new position written).
//
// Grid = (chunks, kv heads, tokens).  A workgroup owns one kv head and one
// chunk of positions, and computes all kv_mul query heads of that group from
// the same K/V rows, so each cache row is read once per step.  Lanes are laid
// out LPR per cache row (4 elements each): a wave load covers 64/LPR whole
// rows.  Scores for the chunk stay in LDS; each chunk produces (max, sum,
// unnormalised output) and the last workgroup of the (token, kv head) to
// finish — detected with an agent-scope atomic counter — merges them.  The
// split keeps >= 256 workgroups busy at long context with only 8 kv heads.
#include "kernels.h"

namespace ehip {

template <int HD> struct Lay {
    static constexpr int P = HD / 4;                        // 4-element pieces per row
    static constexpr int LPR = P <= 8 ? 8 : (P <= 16 ? 16 : (P <= 32 ? 32 : 64));
    static constexpr int RPL = 64 / LPR;                    // rows per wave load
};

template <bool F16>
__device__ __forceinline__ float4 load4(const void *base, size_t idx) {
    if (F16) {
        const uint2 u = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(base) + idx);
        return make_float4(h2f((uint16_t)(u.x & 0xffff)), h2f((uint16_t)(u.x >> 16)),
                           h2f((uint16_t)(u.y & 0xffff)), h2f((uint16_t)(u.y >> 16)));
    } else {
        return *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(base) + idx);
    }
}

// RMSNorm of one head vector held in LDS by one wave (model.c:50-55)
template <int HD>
__device__ __forceinline__ void head_norm(float *v, const float *w, float eps, int lane) {
    float ss = 0.0f;
    for (int d = lane; d < HD; d += 64) ss += v[d] * v[d];
    ss = wave_sum(ss);
    const float scale = 1.0f / sqrtf(ss / (float)HD + eps);
    for (int d = lane; d < HD; d += 64) v[d] = v[d] * scale * w[d];
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

template <int HD, int GM, bool F16>
__global__ __launch_bounds__(WG) void k_attn(AttnArgs a) {
    using L = Lay<HD>;
    __shared__ __align__(16) float qs[GM][HD];
    __shared__ float sc[GM][ATT_CHUNK_MAX];
    __shared__ __align__(16) float vacc[NWAVE][GM][HD];
    __shared__ float ml[GM][2];
    __shared__ int is_last;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int G = a.n_heads / a.n_kv;
    const int pos = a.pos_base + b;
    const int npos = pos + 1;

    // chunking, identical in every workgroup of this (token, kv head)
    int nc = (npos + a.min_chunk - 1) / a.min_chunk;
    if (nc > a.max_chunks) nc = a.max_chunks;
    const int need = (npos + ATT_CHUNK_MAX - 1) / ATT_CHUNK_MAX;
    if (nc < need) nc = need;
    const int clen = (npos + nc - 1) / nc;
    nc = (npos + clen - 1) / clen;
    if (c >= nc) return;
    const int t0 = c * clen, t1 = min(npos, t0 + clen), len = t1 - t0;
    const size_t hoff = (size_t)g * HD;

    // ---- prologue: q rows of the group --------------------------------------
    {
        const float *qrow = a.q + (size_t)b * a.q_stride + (size_t)g * G * HD;
        for (int i = tid; i < G * HD; i += WG) qs[i / HD][i % HD] = qrow[i];
        __syncthreads();
    }

    const int j = lane % L::LPR, rw = lane / L::LPR;
    const bool pj = j < L::P;
    float4 qr[GM];
#pragma unroll
    for (int h = 0; h < GM; h++)
        qr[h] = (h < G && pj) ? *reinterpret_cast<const float4 *>(&qs[h][4 * j]) : make_float4(0, 0, 0, 0);

    // ---- scores --------------------------------------------------------
    for (int t = t0 + wave * L::RPL + rw; t < t1; t += NWAVE * L::RPL) {
        float4 k4 = make_float4(0, 0, 0, 0);
        if (pj) k4 = load4<F16>(a.kc, (size_t)t * a.kv_dim + hoff + 4 * j);
        float p[GM];
#pragma unroll
        for (int h = 0; h < GM; h++) {
            p[h] = qr[h].x * k4.x + qr[h].y * k4.y + qr[h].z * k4.z + qr[h].w * k4.w;
#pragma unroll
            for (int off = 1; off < L::LPR; off <<= 1) p[h] += __shfl_xor(p[h], off);
        }
        if (j == 0) {
#pragma unroll
            for (int h = 0; h < GM; h++)
                if (h < G) sc[h][t - t0] = p[h] * a.inv_sqrt;
        }
    }
    __syncthreads();

    // ---- softmax statistics of the chunk -------------------------------
    for (int h = wave; h < G; h += NWAVE) {
        float m = -INFINITY;
        for (int i = lane; i < len; i += 64) m = fmaxf(m, sc[h][i]);
        m = wave_max(m);
        float l = 0.0f;
        for (int i = lane; i < len; i += 64) { const float e = expf(sc[h][i] - m); sc[h][i] = e; l += e; }
        l = wave_sum(l);
        if (nc == 1) {  // whole row here: normalise first, as model.c:62-63
            const float inv = 1.0f / l;
            for (int i = lane; i < len; i += 64) sc[h][i] *= inv;
        }
        if (lane == 0) { ml[h][0] = m; ml[h][1] = l; }
    }
    __syncthreads();

    // ---- p . V ----------------------------------------------------------
    float4 acc[GM];
#pragma unroll
    for (int h = 0; h < GM; h++) acc[h] = make_float4(0, 0, 0, 0);
    for (int t = t0 + wave * L::RPL + rw; t < t1; t += NWAVE * L::RPL) {
        float4 v4 = make_float4(0, 0, 0, 0);
        if (pj) v4 = load4<F16>(a.vc, (size_t)t * a.kv_dim + hoff + 4 * j);
#pragma unroll
        for (int h = 0; h < GM; h++) {
            if (h < G) {
                const float pr = sc[h][t - t0];
                acc[h].x += pr * v4.x; acc[h].y += pr * v4.y;
                acc[h].z += pr * v4.z; acc[h].w += pr * v4.w;
            }
        }
    }
#pragma unroll
    for (int h = 0; h < GM; h++) {
#pragma unroll
        for (int off = L::LPR; off < 64; off <<= 1) {
            acc[h].x += __shfl_xor(acc[h].x, off); acc[h].y += __shfl_xor(acc[h].y, off);
            acc[h].z += __shfl_xor(acc[h].z, off); acc[h].w += __shfl_xor(acc[h].w, off);
        }
        if (rw == 0 && pj && h < G) *reinterpret_cast<float4 *>(&vacc[wave][h][4 * j]) = acc[h];
    }
    __syncthreads();

    const size_t head0 = (size_t)b * a.n_heads + (size_t)g * G;   // first query head row
    if (nc == 1) {
        for (int i = tid; i < G * HD; i += WG) {
            const int h = i / HD, d = i % HD;
            float o = 0.0f;
#pragma unroll
            for (int w = 0; w < NWAVE; w++) o += vacc[w][h][d];
            a.out[(head0 + h) * HD + d] = o;
        }
        return;
    }

    // ---- split: publish the partial, last workgroup merges --------------
    const int stride = HD + 2;
    for (int i = tid; i < G * HD; i += WG) {
        const int h = i / HD, d = i % HD;
        float o = 0.0f;
#pragma unroll
        for (int w = 0; w < NWAVE; w++) o += vacc[w][h][d];
        a.part[((head0 + h) * a.max_chunks + c) * stride + d] = o;
    }
    if (tid < G) {
        float *pm = a.part + ((head0 + tid) * a.max_chunks + c) * stride + HD;
        pm[0] = ml[tid][0]; pm[1] = ml[tid][1];
    }
    __threadfence();
    __syncthreads();
    unsigned *ctr = a.counters + (size_t)b * a.n_kv + g;
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        is_last = prev == (unsigned)(nc - 1);
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    for (int i = tid; i < G * HD; i += WG) {
        const int h = i / HD, d = i % HD;
        const float *ph = a.part + (head0 + h) * a.max_chunks * stride;
        float M = -INFINITY;
        for (int k = 0; k < nc; k++) M = fmaxf(M, ph[k * stride + HD]);
        float Ls = 0.0f, O = 0.0f;
        for (int k = 0; k < nc; k++) {
            const float f = expf(ph[k * stride + HD] - M);
            Ls += ph[k * stride + HD + 1] * f;
            O += ph[k * stride + d] * f;
        }
        a.out[(head0 + h) * HD + d] = O * (1.0f / Ls);
    }
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- prefill QK-norm + RoPE + KV store -----------------------------------
template <int HD, bool F16>
__global__ __launch_bounds__(64) void k_qkpost(QkPostArgs a) {
    __shared__ float v[HD];
    const int lane = threadIdx.x, b = blockIdx.x, vh = blockIdx.y;
    const int qd = a.n_heads * HD, pos = a.pos_base + b;
    const bool isq = vh < a.n_heads;
    const int g = vh - a.n_heads;
    float *row = a.qkv + (size_t)b * a.stride + (isq ? (size_t)vh * HD : (size_t)qd + (size_t)g * HD);
    for (int d = lane; d < HD; d += 64) v[d] = row[d];
    __syncthreads();
    if (a.q_norm) { head_norm<HD>(v, isq ? a.q_norm : a.k_norm, a.eps, lane); __syncthreads(); }
    for (int i = lane; i < HD / 2; i += 64) rope_pair(v, i, HD, a.rope[(size_t)pos * (HD / 2) + i], a.rope_style);
    __syncthreads();
    if (isq) {
        for (int d = lane; d < HD; d += 64) row[d] = v[d];
        return;
    }
    const float *vrow = a.qkv + (size_t)b * a.stride + qd + a.kv_dim + (size_t)g * HD;
    const size_t off = (size_t)pos * a.kv_dim + (size_t)g * HD;
    for (int d = lane; d < HD; d += 64) {
        if (F16) {
            reinterpret_cast<uint16_t *>(a.kc)[off + d] = f2h(v[d]);
            reinterpret_cast<uint16_t *>(a.vc)[off + d] = f2h(vrow[d]);
        } else {
            reinterpret_cast<float *>(a.kc)[off + d] = v[d];
            reinterpret_cast<float *>(a.vc)[off + d] = vrow[d];
        }
    }
}

// --------------------------------------------------------------------------
template <int HD, int GM, bool F16>
static void go_attn(hipStream_t st, const AttnArgs &a) {
    dim3 grid(a.max_chunks, a.n_kv, a.n_tok);
    hipLaunchKernelGGL((k_attn<HD, GM, F16>), grid, dim3(WG), 0, st, a);
}

template <int HD, bool F16>
static int pick_g(hipStream_t st, const AttnArgs &a) {
    const int G = a.n_heads / a.n_kv;
    if (G <= 1) go_attn<HD, 1, F16>(st, a);
    else if (G <= 2) go_attn<HD, 2, F16>(st, a);
    else if (G <= 4) go_attn<HD, 4, F16>(st, a);
    else if (G <= 8) go_attn<HD, 8, F16>(st, a);
    else return -1;
    return 0;
}

int launch_attention(hipStream_t st, bool f16kv, const AttnArgs &a) {
    if (a.n_kv <= 0 || a.n_heads % a.n_kv != 0) return -1;
    if ((a.ctx + ATT_CHUNK_MAX - 1) / ATT_CHUNK_MAX > a.max_chunks) return -1;
    switch (a.hd) {
        case 48: return f16kv ? pick_g<48, true>(st, a) : pick_g<48, false>(st, a);
        case 64: return f16kv ? pick_g<64, true>(st, a) : pick_g<64, false>(st, a);
        case 128: return f16kv ? pick_g<128, true>(st, a) : pick_g<128, false>(st, a);
    }
    return -1;
}

int launch_qkpost(hipStream_t st, bool f16kv, const QkPostArgs &a) {
    dim3 grid(a.n_tok, a.n_heads + a.n_kv);
    switch (a.hd) {
#define QKP(H)                                                                              \
    case H:                                                                                 \
        if (f16kv) hipLaunchKernelGGL((k_qkpost<H, true>), grid, dim3(64), 0, st, a);       \
        else hipLaunchKernelGGL((k_qkpost<H, false>), grid, dim3(64), 0, st, a);            \
        return 0;
        QKP(48) QKP(64) QKP(128)
#undef QKP
    }
    return -1;
}

}  // namespace ehip
