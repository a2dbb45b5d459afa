// attn_decode.hip — decode-step GQA attention over the HBM KV cache (gfx950).
//
// Replaces, for one token, the QK-norm / RoPE / kv_store steps of
// ember_forward (src/model.c:386-393) and attention -> attn_heads + softmax
// (src/model.c:57-64, 207-278).
//
// Roofline: HBM-bound.  Algorithmic bytes per launch (one layer) =
// 2 * (pos+1) * kv_dim * esize (K and V rows read once) + 2 * kv_dim * esize
// (the new row written) + the q|k|v input and the output (a few KB).
//
// Grid = (chunks, kv heads).  A workgroup owns CR consecutive positions of
// one kv head and serves all kv_mul query heads of that group from the same
// K/V rows, so each cache row is read once per step.  CR is sized so that
// each thread holds exactly NL = 8 sixteen-byte pieces of K and 8 of V:
//   1. every K/V load of the chunk is issued first, into registers (the rows
//      before `pos` are already in the cache);
//   2. while they are in flight, the token's q heads and k/v are read from the
//      QKV matvec output, QK-normed and rotated, and the chunk that owns
//      `pos` stores the new k/v row;
//   3. scores (LPR lanes per row, cross-lane sums), the chunk's softmax
//      statistics, then p.V, reduced over rows in registers and over waves in
//      LDS.
// With one chunk the normalised output is written directly (model.c:57-64
// order: max, exp, 1/sum).  Otherwise each chunk publishes (o, m, l) and
// k_attn_merge (one workgroup per query head, the next kernel on the stream)
// rescales and sums them.  A kernel boundary orders the two; a per-workgroup
// release fence and counter would cost more than the extra launch here.
#include "kernels.h"

namespace ehip {

template <int HD, bool F16> struct DecLay {
    static constexpr int PE = F16 ? 8 : 4;                 // elements per 16-byte piece
    static constexpr int P = HD / PE;                      // pieces per row
    static constexpr int LPR = P <= 4 ? 4 : (P <= 8 ? 8 : (P <= 16 ? 16 : (P <= 32 ? 32 : 64)));
    static constexpr int RPL = 64 / LPR;                   // rows per wave load
    static constexpr int RPB = NWAVE * RPL;                // rows per workgroup load
    static constexpr int NL = 8;                           // loads per thread, K and V each
    static constexpr int CR = NL * RPB;                    // positions per chunk
    static_assert(HD % PE == 0, "head_dim must be a multiple of the piece size");
};

// Sum over aligned groups of N lanes (N = 8 .. 64), every lane of the group
// receiving it: DPP moves within rows of 16, lane swaps across rows.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    v = dpp_add<0xb1, 0xf>(v);                            // quad_perm [1,0,3,2]
    v = dpp_add<0x4e, 0xf>(v);                            // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xf>(v);                           // row_half_mirror
    if constexpr (N >= 16) v = dpp_add<0x140, 0xf>(v);    // row_mirror
    if constexpr (N >= 32) v = xor16_add(v);
    if constexpr (N >= 64) v = xor32_add(v);
    return v;
}

// Sum over the lanes i, i + N, i + 2N, ... of the wave (N = 8 .. 64)
template <int N>
__device__ __forceinline__ float stride_sum(float v) {
    if constexpr (N <= 8) v = xor8_add(v);
    if constexpr (N <= 16) v = xor16_add(v);
    if constexpr (N <= 32) v = xor32_add(v);
    return v;
}

template <bool F16>
__device__ __forceinline__ void piece_to_float(const uint4 &u, float *f) {
    if (F16) {
        const uint32_t w[4] = { u.x, u.y, u.z, u.w };
#pragma unroll
        for (int k = 0; k < 4; k++) {
            f[2 * k] = h2f((uint16_t)(w[k] & 0xffff));
            f[2 * k + 1] = h2f((uint16_t)(w[k] >> 16));
        }
    } else {
        f[0] = __uint_as_float(u.x); f[1] = __uint_as_float(u.y);
        f[2] = __uint_as_float(u.z); f[3] = __uint_as_float(u.w);
    }
}

// RMSNorm of one head vector held in LDS by one wave (model.c:50-55)
template <int HD>
__device__ __forceinline__ void dec_head_norm(float *v, const float *w, float eps, int lane) {
    float ss = 0.0f;
    for (int d = lane; d < HD; d += 64) ss += v[d] * v[d];
    ss = wave_sum(ss);
    const float scale = 1.0f / sqrtf(ss / (float)HD + eps);
    for (int d = lane; d < HD; d += 64) v[d] = v[d] * scale * w[d];
}

template <int HD, int GM, bool F16>
__global__ __launch_bounds__(WG) void k_attn_dec(AttnArgs a) {
    using L = DecLay<HD, F16>;
    constexpr int PE = L::PE, CR = L::CR, NL = L::NL;
    __shared__ __align__(16) float qs[GM][HD];
    __shared__ __align__(16) float kn[HD], vn[HD];
    __shared__ float cs[HD / 2], sn[HD / 2];
    __shared__ float sc[GM][CR];
    __shared__ __align__(16) float vacc[NWAVE][GM][HD];
    __shared__ float ml[GM][2];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = blockIdx.x, g = blockIdx.y;
    const int G = a.n_heads / a.n_kv;
    const int pos = a.tokpos[1];
    const int npos = pos + 1;
    const int nc = (npos + CR - 1) / CR;
    if (c >= nc) return;
    const int t0 = c * CR, t1 = min(npos, t0 + CR);
    const size_t hoff = (size_t)g * HD;
    const int j = lane % L::LPR, rw = lane / L::LPR;
    const bool pj = j < L::P;

    // ---- 1. loads: this token's q heads, k, v and (cos, sin) first, then
    // every cached K/V row of the chunk (rows before `pos`), all in flight --
    constexpr int QPT = (GM * HD + WG - 1) / WG;
    const int qd = a.n_heads * HD;
    float qv[QPT];
#pragma unroll
    for (int r = 0; r < QPT; r++) qv[r] = a.q[(size_t)g * G * HD + min(tid + r * WG, G * HD - 1)];
    const int dt = min(tid, HD - 1);
    const float kv0 = a.q[qd + hoff + dt];
    const float vv0 = a.q[qd + a.kv_dim + hoff + dt];
    const float2 rp = a.rope[(size_t)pos * (HD / 2) + min(tid, HD / 2 - 1)];
    uint4 kr[NL], vr[NL];
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int t = t0 + i * L::RPB + wave * L::RPL + rw;
        const size_t off = (size_t)min(t, pos) * a.kv_dim + hoff + (size_t)min(j, L::P - 1) * PE;
        if (F16) {
            kr[i] = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(a.kc) + off);
            vr[i] = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(a.vc) + off);
        } else {
            kr[i] = *reinterpret_cast<const uint4 *>(reinterpret_cast<const float *>(a.kc) + off);
            vr[i] = *reinterpret_cast<const uint4 *>(reinterpret_cast<const float *>(a.vc) + off);
        }
    }

    // ---- 2. QK-norm, RoPE and the cache store of this token ----------------
    {
#pragma unroll
        for (int r = 0; r < QPT; r++) {
            const int i = tid + r * WG;
            if (i < G * HD) qs[i / HD][i % HD] = qv[r];
        }
        if (tid < HD) { kn[tid] = kv0; vn[tid] = vv0; }
        if (tid < HD / 2) { cs[tid] = rp.x; sn[tid] = rp.y; }
        __syncthreads();
        if (a.q_norm) {   // model.c:386-389, after bias, before RoPE
            for (int h = wave; h <= G; h += NWAVE)
                dec_head_norm<HD>(h < G ? qs[h] : kn, h < G ? a.q_norm : a.k_norm, a.eps, lane);
            __syncthreads();
        }
        for (int i = tid; i < (G + 1) * (HD / 2); i += WG) {   // model.c:66-80
            const int h = i / (HD / 2), p = i % (HD / 2);
            float *v = h < G ? qs[h] : kn;
            const int ia = a.rope_style == ROPE_NEOX ? p : 2 * p;
            const int ib = a.rope_style == ROPE_NEOX ? p + HD / 2 : 2 * p + 1;
            const float v0 = v[ia], v1 = v[ib];
            v[ia] = v0 * cs[p] - v1 * sn[p];
            v[ib] = v0 * sn[p] + v1 * cs[p];
        }
        __syncthreads();
        if (F16) {   // the cache holds fp16 (model.c:39-48): attend to the rounded values
            for (int d = tid; d < HD; d += WG) { kn[d] = h2f(f2h(kn[d])); vn[d] = h2f(f2h(vn[d])); }
        }
        if (c == nc - 1) {   // the chunk holding `pos` stores its row
            const size_t off = (size_t)pos * a.kv_dim + hoff;
            for (int d = tid; d < HD; d += WG) {
                if (F16) {
                    reinterpret_cast<uint16_t *>(a.kc)[off + d] = f2h(kn[d]);
                    reinterpret_cast<uint16_t *>(a.vc)[off + d] = f2h(vn[d]);
                } else {
                    reinterpret_cast<float *>(a.kc)[off + d] = kn[d];
                    reinterpret_cast<float *>(a.vc)[off + d] = vn[d];
                }
            }
        }
        __syncthreads();
    }

    // ---- 3. scores -----------------------------------------------------------
    float qr[GM][PE];
#pragma unroll
    for (int h = 0; h < GM; h++)
#pragma unroll
        for (int e = 0; e < PE; e++) qr[h][e] = (h < G && pj) ? qs[h][j * PE + e] : 0.0f;
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int t = t0 + i * L::RPB + wave * L::RPL + rw;
        float kf[PE];
        if (t == pos) {
#pragma unroll
            for (int e = 0; e < PE; e++) kf[e] = pj ? kn[j * PE + e] : 0.0f;
        } else {
            piece_to_float<F16>(kr[i], kf);
        }
        float p[GM];
#pragma unroll
        for (int h = 0; h < GM; h++) {
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < PE; e++) s += qr[h][e] * kf[e];
            p[h] = group_sum<L::LPR>(s);
        }
        if (j == L::LPR - 1 && t < t1) {
#pragma unroll
            for (int h = 0; h < GM; h++)
                if (h < G) sc[h][t - t0] = p[h] * a.inv_sqrt;
        }
    }
    __syncthreads();

    // ---- 4. softmax statistics of the chunk --------------------------------
    const int len = t1 - t0;
    for (int h = wave; h < G; h += NWAVE) {
        float m = -INFINITY;
        for (int i = lane; i < len; i += 64) m = fmaxf(m, sc[h][i]);
        m = wave_max(m);
        float l = 0.0f;
        for (int i = lane; i < len; i += 64) { const float e = expf(sc[h][i] - m); sc[h][i] = e; l += e; }
        l = wave_sum(l);
        if (nc == 1) {   // whole row here: normalise the weights, as model.c:62-63
            const float inv = 1.0f / l;
            for (int i = lane; i < len; i += 64) sc[h][i] *= inv;
        }
        if (lane == 0) { ml[h][0] = m; ml[h][1] = l; }
    }
    __syncthreads();

    // ---- 5. p . V -------------------------------------------------------------
    float acc[GM][PE];
#pragma unroll
    for (int h = 0; h < GM; h++)
#pragma unroll
        for (int e = 0; e < PE; e++) acc[h][e] = 0.0f;
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int t = t0 + i * L::RPB + wave * L::RPL + rw;
        if (t >= t1) continue;
        float vf[PE];
        if (t == pos) {
#pragma unroll
            for (int e = 0; e < PE; e++) vf[e] = pj ? vn[j * PE + e] : 0.0f;
        } else {
            piece_to_float<F16>(vr[i], vf);
        }
#pragma unroll
        for (int h = 0; h < GM; h++) {
            if (h < G) {
                const float pr = sc[h][t - t0];
#pragma unroll
                for (int e = 0; e < PE; e++) acc[h][e] += pr * vf[e];
            }
        }
    }
#pragma unroll
    for (int h = 0; h < GM; h++) {
#pragma unroll
        for (int e = 0; e < PE; e++) acc[h][e] = stride_sum<L::LPR>(acc[h][e]);
        if (rw == 0 && pj && h < G)
#pragma unroll
            for (int e = 0; e < PE; e++) vacc[wave][h][j * PE + e] = acc[h][e];
    }
    __syncthreads();

    const size_t head0 = (size_t)g * G;   // first query head of the group
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

    // ---- 6. split: publish (o, m, l) for k_attn_merge ------------------------
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
        pm[0] = ml[tid][0];
        pm[1] = ml[tid][1];
    }
}

// One workgroup per query head: o = sum_k o_k exp(m_k - M) / sum_k l_k exp(m_k - M)
// over the chunk partials.  Thread (s, d) owns output dim d and the chunks
// k = s, s + S, ...; its partial loads are issued before the statistics are
// reduced.  With a single chunk the attention kernel wrote the output.
constexpr int MERGE_MAX_CHUNKS = 2048;
constexpr int MERGE_BATCH = 64;

template <int HD>
__global__ __launch_bounds__(WG) void k_attn_merge(AttnArgs a, int chunk) {
    constexpr int S = WG / HD;                 // chunk slices
    __shared__ float fs[MERGE_MAX_CHUNKS];
    __shared__ float red[NWAVE];
    __shared__ float osum[S][HD];
    const int tid = threadIdx.x, h = blockIdx.x;
    const int pos = a.tokpos[1];
    const int nc = (pos + 1 + chunk - 1) / chunk;
    if (nc == 1) return;
    const int stride = HD + 2;
    const float *ph = a.part + (size_t)h * a.max_chunks * stride;
    const int d = tid % HD, sl = tid / HD;
    const bool act = sl < S;
    // loads first: this thread's chunk statistics, then its first batch of
    // partial outputs
    const int k0s = min(tid, nc - 1);
    const float m0 = ph[(size_t)k0s * stride + HD], l0 = ph[(size_t)k0s * stride + HD + 1];
    float po[MERGE_BATCH];
#pragma unroll
    for (int b = 0; b < MERGE_BATCH; b++) {
        const int k = min(sl + b * S, nc - 1);
        po[b] = act ? ph[(size_t)k * stride + d] : 0.0f;
    }
    // statistics: chunk maxima, then weights f_k and the denominator
    float mloc = tid < nc ? m0 : -INFINITY;
    for (int k = tid + WG; k < nc; k += WG) mloc = fmaxf(mloc, ph[(size_t)k * stride + HD]);
    mloc = wave_max(mloc);
    if ((tid & 63) == 0) red[tid >> 6] = mloc;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < NWAVE; w++) M = fmaxf(M, red[w]);
    __syncthreads();
    float lloc = 0.0f;
    if (tid < nc) {
        const float f = expf(m0 - M);
        fs[tid] = f;
        lloc = l0 * f;
    }
    for (int k = tid + WG; k < nc; k += WG) {
        const float f = expf(ph[(size_t)k * stride + HD] - M);
        fs[k] = f;
        lloc += ph[(size_t)k * stride + HD + 1] * f;
    }
    const float L = block_sum(lloc, red);
    __syncthreads();
    float o = 0.0f;
#pragma unroll
    for (int b = 0; b < MERGE_BATCH; b++) {
        const int k = sl + b * S;
        if (act && k < nc) o += po[b] * fs[k];
    }
    for (int k0 = MERGE_BATCH * S; k0 < nc; k0 += MERGE_BATCH * S) {   // beyond the first batch
#pragma unroll
        for (int b = 0; b < MERGE_BATCH; b++) {
            const int k = min(k0 + sl + b * S, nc - 1);
            po[b] = act ? ph[(size_t)k * stride + d] : 0.0f;
        }
#pragma unroll
        for (int b = 0; b < MERGE_BATCH; b++) {
            const int k = k0 + sl + b * S;
            if (act && k < nc) o += po[b] * fs[k];
        }
    }
    if (act) osum[sl][d] = o;
    __syncthreads();
    if (tid < HD) {
        float t = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < S; s2++) t += osum[s2][tid];
        a.out[(size_t)h * HD + tid] = t * (1.0f / L);
    }
}

// --------------------------------------------------------------------------
int attn_decode_chunk(int hd, bool f16kv) {
    switch (hd) {
        case 48: return f16kv ? DecLay<48, true>::CR : DecLay<48, false>::CR;
        case 64: return f16kv ? DecLay<64, true>::CR : DecLay<64, false>::CR;
        case 128: return f16kv ? DecLay<128, true>::CR : DecLay<128, false>::CR;
    }
    return 0;
}

template <int HD, bool F16>
static int dec_pick_g(hipStream_t st, const AttnArgs &a) {
    const int G = a.n_heads / a.n_kv;
    dim3 grid(a.max_chunks, a.n_kv);
    if (G <= 1) hipLaunchKernelGGL((k_attn_dec<HD, 1, F16>), grid, dim3(WG), 0, st, a);
    else if (G <= 2) hipLaunchKernelGGL((k_attn_dec<HD, 2, F16>), grid, dim3(WG), 0, st, a);
    else if (G <= 4) hipLaunchKernelGGL((k_attn_dec<HD, 4, F16>), grid, dim3(WG), 0, st, a);
    else if (G <= 8) hipLaunchKernelGGL((k_attn_dec<HD, 8, F16>), grid, dim3(WG), 0, st, a);
    else return -1;
    hipLaunchKernelGGL((k_attn_merge<HD>), dim3(a.n_heads), dim3(WG), 0, st, a, DecLay<HD, F16>::CR);
    return 0;
}

int launch_attn_decode(hipStream_t st, bool f16kv, const AttnArgs &a) {
    if (a.n_kv <= 0 || a.n_heads % a.n_kv != 0) return -1;
    const int cr = attn_decode_chunk(a.hd, f16kv);
    if (cr <= 0 || (a.ctx + cr - 1) / cr > a.max_chunks || a.max_chunks > MERGE_MAX_CHUNKS) return -1;
    switch (a.hd) {
        case 48: return f16kv ? dec_pick_g<48, true>(st, a) : dec_pick_g<48, false>(st, a);
        case 64: return f16kv ? dec_pick_g<64, true>(st, a) : dec_pick_g<64, false>(st, a);
        case 128: return f16kv ? dec_pick_g<128, true>(st, a) : dec_pick_g<128, false>(st, a);
    }
    return -1;
}

}  // namespace ehip
