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
// Grid = (kv heads, chunks), kv heads varying fastest so that neighbouring
// workgroups read whole cache rows.  A workgroup owns CR = IT * NL * RPB
// consecutive positions of one kv head and serves all kv_mul query heads of
// that group from the same K/V rows, so each cache row is read once per step.
// Lane (rw, j) of a wave holds 16-byte piece j of row rw of each wave load:
//   1. loads: the token's q heads / k / v pieces (straight out of the QKV
//      matvec), the QK-norm weights and the RoPE (cos, sin) of its piece, then
//      the first batch of NL K pieces and NL V pieces per thread;
//   2. QK-norm and RoPE in registers: a head's sum of squares is a reduction
//      over the LPR lanes of its row, a NEOX partner element sits P/2 lanes
//      away, an interleaved partner in the same lane; the chunk holding
//      `pos` stores the new k/v row;
//   3. IT batches, each issuing the next batch's loads before its own scores
//      (cross-lane sums over the row's lanes), with a running softmax
//      (max, sum of exp, sum of exp * V) per wave;
//   4. the four waves' partials combine in LDS.  With one chunk that is the
//      output (model.c:57-64: max, exp, 1/sum); otherwise the chunk's
//      (o, m, l) is stored and k_attn_merge, the next kernel, combines them.
// Measured on the MI355X, the kernel boundary is the cheapest way to order
// the partials before the merge: a last-arriver merge inside this kernel
// needs device-scope stores, a wait for their completion and an atomic,
// three memory round trips on the critical path while the HBM queues are
// full, and cost more than the extra launch.
#include <algorithm>

#include "kernels.h"

namespace ehip {

template <int HD, bool F16> struct DecLay {
    static constexpr int PE = F16 ? 8 : 4;                 // elements per 16-byte piece
    static constexpr int P = HD / PE;                      // pieces per row
    static constexpr int LPR = P <= 8 ? 8 : (P <= 16 ? 16 : (P <= 32 ? 32 : 64));
    static constexpr int RPL = 64 / LPR;                   // rows per wave load
    static constexpr int RPB = NWAVE * RPL;                // rows per workgroup load
    static_assert(HD % PE == 0 && P % 2 == 0, "head_dim must split into an even number of pieces");
};

template <int HD, bool F16, int NL, int IT>
constexpr int dec_chunk() { return NL * DecLay<HD, F16>::RPB * IT; }

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

// Sum / maximum over the lanes i, i + N, i + 2N, ... of the wave (N = 8 .. 64)
template <int N>
__device__ __forceinline__ float stride_sum(float v) {
    if constexpr (N <= 8) v = xor8_add(v);
    if constexpr (N <= 16) v = xor16_add(v);
    if constexpr (N <= 32) v = xor32_add(v);
    return v;
}
template <int N>
__device__ __forceinline__ float stride_max(float v) {
    if constexpr (N <= 8)
        v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, false)));
    if constexpr (N <= 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    if constexpr (N <= 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
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

template <int PE>
__device__ __forceinline__ void load_floats(float (&v)[PE], const float *p) {
#pragma unroll
    for (int e = 0; e < PE; e += 4) {
        const float4 f = *reinterpret_cast<const float4 *>(p + e);
        v[e] = f.x; v[e + 1] = f.y; v[e + 2] = f.z; v[e + 3] = f.w;
    }
}

template <int HD, int GM, bool F16, int NL, int IT>
__global__ __launch_bounds__(WG) void k_attn_dec(AttnArgs a) {
    using L = DecLay<HD, F16>;
    constexpr int PE = L::PE, P = L::P, LPR = L::LPR, RPL = L::RPL, RPB = L::RPB;
    constexpr int BR = NL * RPB;      // rows per batch
    constexpr int CR = BR * IT;       // rows per chunk
    __shared__ float sm_m[NWAVE][GM], sm_l[NWAVE][GM];
    __shared__ __align__(16) float sm_o[NWAVE][GM][HD];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = blockIdx.x, c = blockIdx.y;   // kv heads vary fastest: neighbours read whole cache rows
    const int G = a.n_heads / a.n_kv;
    const int pos = a.tokpos[1];
    const int nc = (pos + 1 + CR - 1) / CR;
    if (c >= nc) return;
    const int t0 = c * CR, t1 = min(pos + 1, t0 + CR);
    const int j = lane % LPR, rw = lane / LPR;
    const bool pj = j < P;
    const int jc = pj ? j : P - 1;   // clamped piece index for loads
    const int qd = a.n_heads * HD;
    const size_t hoff = (size_t)g * HD;
    const bool neox = a.rope_style == ROPE_NEOX;

    // ---- 1. loads --------------------------------------------------------
    float qv[GM][PE], kn[PE], vn[PE], qw[PE], kw[PE];
    float2 cs[PE];
#pragma unroll
    for (int h = 0; h < GM; h++)
        load_floats<PE>(qv[h], a.q + ((size_t)g * G + min(h, G - 1)) * HD + jc * PE);
    load_floats<PE>(kn, a.q + qd + hoff + jc * PE);
    load_floats<PE>(vn, a.q + qd + a.kv_dim + hoff + jc * PE);
    if (a.q_norm) {
        load_floats<PE>(qw, a.q_norm + jc * PE);
        load_floats<PE>(kw, a.k_norm + jc * PE);
    }
    {
        const float2 *rp = a.rope + (size_t)pos * (HD / 2);
        const int i0 = neox ? (jc % (P / 2)) * PE : jc * (PE / 2);
#pragma unroll
        for (int e = 0; e < PE; e += 2) {
            const float4 f = *reinterpret_cast<const float4 *>(rp + i0 + min(e, neox ? PE - 2 : PE / 2 - 2));
            cs[e] = make_float2(f.x, f.y);
            cs[e + 1] = make_float2(f.z, f.w);
        }
    }
    uint4 kr[NL], vr[NL];
    auto load_batch = [&](int tb) {   // K rows first, then V rows
#pragma unroll
        for (int i = 0; i < NL; i++) {
            const int t = min(tb + i * RPB + wave * RPL + rw, pos);
            const size_t off = (size_t)t * a.kv_dim + hoff + (size_t)jc * PE;
            kr[i] = F16 ? *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(a.kc) + off)
                        : *reinterpret_cast<const uint4 *>(reinterpret_cast<const float *>(a.kc) + off);
        }
#pragma unroll
        for (int i = 0; i < NL; i++) {
            const int t = min(tb + i * RPB + wave * RPL + rw, pos);
            const size_t off = (size_t)t * a.kv_dim + hoff + (size_t)jc * PE;
            vr[i] = F16 ? *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(a.vc) + off)
                        : *reinterpret_cast<const uint4 *>(reinterpret_cast<const float *>(a.vc) + off);
        }
    };
    load_batch(t0);

    // ---- 2. QK-norm (model.c:386-389, after bias, before RoPE) and RoPE
    // (model.c:66-80) of the group's q heads and of k, in registers --------
    auto head_norm = [&](float (&v)[PE], const float (&w)[PE]) {
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < PE; e++) ss += v[e] * v[e];
        ss = group_sum<LPR>(pj ? ss : 0.0f);
        const float scale = 1.0f / sqrtf(ss / (float)HD + a.eps);
#pragma unroll
        for (int e = 0; e < PE; e++) v[e] = v[e] * scale * w[e];
    };
    const int partner = lane - j + (jc + P / 2) % P;
    const bool low = j < P / 2;
    auto rope = [&](float (&v)[PE]) {
        if (neox) {   // pairs (i, i + hd/2): the partner piece is P/2 lanes away
#pragma unroll
            for (int e = 0; e < PE; e++) {
                const float pv = __shfl(v[e], partner);
                v[e] = low ? v[e] * cs[e].x - pv * cs[e].y : pv * cs[e].y + v[e] * cs[e].x;
            }
        } else {      // pairs (2i, 2i + 1) inside the piece
#pragma unroll
            for (int e = 0; e < PE; e += 2) {
                const float v0 = v[e], v1 = v[e + 1];
                const float2 r = cs[e / 2];
                v[e] = v0 * r.x - v1 * r.y;
                v[e + 1] = v0 * r.y + v1 * r.x;
            }
        }
    };
    if (a.q_norm) {
#pragma unroll
        for (int h = 0; h < GM; h++) head_norm(qv[h], qw);
        head_norm(kn, kw);
    }
#pragma unroll
    for (int h = 0; h < GM; h++) rope(qv[h]);
    rope(kn);
    if (F16) {   // the cache holds fp16 (model.c:39-48): attend to the rounded values
#pragma unroll
        for (int e = 0; e < PE; e++) { kn[e] = h2f(f2h(kn[e])); vn[e] = h2f(f2h(vn[e])); }
    }
    if (c == nc - 1 && wave == 0 && rw == 0 && pj) {   // the chunk holding `pos` stores its row
        const size_t off = (size_t)pos * a.kv_dim + hoff + (size_t)j * PE;
        if constexpr (F16) {
            uint32_t pk[PE / 2], pv[PE / 2];
#pragma unroll
            for (int e = 0; e < PE / 2; e++) {
                pk[e] = (uint32_t)f2h(kn[2 * e]) | ((uint32_t)f2h(kn[2 * e + 1]) << 16);
                pv[e] = (uint32_t)f2h(vn[2 * e]) | ((uint32_t)f2h(vn[2 * e + 1]) << 16);
            }
            *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(a.kc) + off) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(a.vc) + off) = make_uint4(pv[0], pv[1], pv[2], pv[3]);
        } else {
            *reinterpret_cast<float4 *>(reinterpret_cast<float *>(a.kc) + off) = make_float4(kn[0], kn[1], kn[2], kn[3]);
            *reinterpret_cast<float4 *>(reinterpret_cast<float *>(a.vc) + off) = make_float4(vn[0], vn[1], vn[2], vn[3]);
        }
    }

    // ---- 3. batches of BR rows: the next batch's loads are issued before the
    // current batch's scores; a running (max, sum, output) per wave --------
    float m[GM], l[GM], o[GM][PE];
#pragma unroll
    for (int h = 0; h < GM; h++) {
        m[h] = -INFINITY;
        l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < PE; e++) o[h][e] = 0.0f;
    }
    for (int it = 0; it < IT; it++) {
        const int tb = t0 + it * BR;
        if (tb >= t1) break;
        uint4 kc[NL], vc[NL];
#pragma unroll
        for (int i = 0; i < NL; i++) { kc[i] = kr[i]; vc[i] = vr[i]; }
        if (it + 1 < IT && tb + BR < t1) load_batch(tb + BR);
        float sc[NL][GM];
#pragma unroll
        for (int i = 0; i < NL; i++) {
            const int t = tb + i * RPB + wave * RPL + rw;
            float kf[PE];
            if (t == pos) {
#pragma unroll
                for (int e = 0; e < PE; e++) kf[e] = kn[e];
            } else {
                piece_to_float<F16>(kc[i], kf);
            }
#pragma unroll
            for (int h = 0; h < GM; h++) {
                float sv = 0.0f;
#pragma unroll
                for (int e = 0; e < PE; e++) sv += qv[h][e] * kf[e];
                sc[i][h] = group_sum<LPR>(pj ? sv : 0.0f) * a.inv_sqrt;
            }
        }
        float mn[GM];
#pragma unroll
        for (int h = 0; h < GM; h++) {
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < NL; i++)
                if (tb + i * RPB + wave * RPL + rw < t1) mx = fmaxf(mx, sc[i][h]);
            mn[h] = fmaxf(m[h], stride_max<LPR>(mx));
            const float r = m[h] == -INFINITY ? 0.0f : expf(m[h] - mn[h]);
            l[h] *= r;
#pragma unroll
            for (int e = 0; e < PE; e++) o[h][e] *= r;
            m[h] = mn[h];
        }
#pragma unroll
        for (int i = 0; i < NL; i++) {
            const int t = tb + i * RPB + wave * RPL + rw;
            if (t >= t1) continue;
            float vf[PE];
            if (t == pos) {
#pragma unroll
                for (int e = 0; e < PE; e++) vf[e] = vn[e];
            } else {
                piece_to_float<F16>(vc[i], vf);
            }
#pragma unroll
            for (int h = 0; h < GM; h++) {
                const float p = expf(sc[i][h] - m[h]);
                l[h] += p;
#pragma unroll
                for (int e = 0; e < PE; e++) o[h][e] += p * vf[e];
            }
        }
    }
#pragma unroll
    for (int h = 0; h < GM; h++) {
        l[h] = stride_sum<LPR>(l[h]);
#pragma unroll
        for (int e = 0; e < PE; e++) o[h][e] = stride_sum<LPR>(o[h][e]);
        if (rw == 0 && pj && h < G)
#pragma unroll
            for (int e = 0; e < PE; e++) sm_o[wave][h][j * PE + e] = o[h][e];
        if (lane == 0 && h < G) { sm_m[wave][h] = m[h]; sm_l[wave][h] = l[h]; }
    }
    __syncthreads();

    // ---- 4. combine the waves; publish or write ----------------------------
    // Partials: o at part[head][chunk][HD], (m, l) at part_ml[head][chunk][2].
    const size_t head0 = (size_t)g * G;   // first query head of the group
    float *part_ml = a.part + (size_t)a.n_heads * a.max_chunks * HD;
    for (int i = tid; i < G * HD; i += WG) {
        const int h = i / HD, d = i % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NWAVE; w++) M = fmaxf(M, sm_m[w][h]);
        float O = 0.0f, S = 0.0f;
#pragma unroll
        for (int w = 0; w < NWAVE; w++) {
            const float mw = sm_m[w][h];
            const float f = mw == -INFINITY ? 0.0f : expf(mw - M);
            O += f * sm_o[w][h][d];
            S += f * sm_l[w][h];
        }
        if (nc == 1) {
            a.out[(head0 + h) * HD + d] = O * (1.0f / S);
        } else {
            const size_t slot = (head0 + h) * a.max_chunks + c;
            a.part[slot * HD + d] = O;
            if (d == 0) { part_ml[2 * slot] = M; part_ml[2 * slot + 1] = S; }
        }
    }
}

// Split-K merge, one workgroup per query head (the next kernel on the
// stream, so the partials written above are visible without fences):
//   o = sum_k o_k e^(m_k - M) / sum_k l_k e^(m_k - M),  M = max_k m_k.
// Thread (s, q) owns float4 quad q of the head row and chunks k = s, s + NS,
// ...; every partial it needs is loaded in one batch, issued together with
// the chunk statistics, before any reduction.
template <int HD>
__global__ __launch_bounds__(WG) void k_attn_merge(AttnArgs a, int chunk) {
    constexpr int QPR = HD / 4, NS = WG / QPR, KB = 16;
    extern __shared__ __align__(16) float dyn[];   // [max_chunks] float2, then [NS][HD]
    __shared__ float red[NWAVE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = blockIdx.x;
    const int pos = a.tokpos[1];
    const int nc = (pos + 1 + chunk - 1) / chunk;
    if (nc == 1) return;   // the attention kernel wrote the output
    float2 *sml = reinterpret_cast<float2 *>(dyn);
    float *slice = dyn + 2 * a.max_chunks;
    const float *po = a.part + (size_t)h * a.max_chunks * HD;
    const float2 *pml = reinterpret_cast<const float2 *>(a.part + (size_t)a.n_heads * a.max_chunks * HD) +
                        (size_t)h * a.max_chunks;
    const int q = tid % QPR, sl = tid / QPR;
    const bool act = sl < NS;
    float4 ov[KB];
    auto load_round = [&](int r) {
#pragma unroll
        for (int b = 0; b < KB; b++)
            ov[b] = *reinterpret_cast<const float4 *>(po + (size_t)min(sl + NS * (r * KB + b), nc - 1) * HD + 4 * q);
    };
    load_round(0);
    float mx = -INFINITY;
    for (int k = tid; k < nc; k += WG) {
        const float2 v = pml[k];
        sml[k] = v;
        mx = fmaxf(mx, v.x);
    }
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < NWAVE; w++) M = fmaxf(M, red[w]);
    float sp = 0.0f;
    for (int k = tid; k < nc; k += WG) {
        const float f = expf(sml[k].x - M);
        sml[k].x = f;
        sp += sml[k].y * f;
    }
    const float S = block_sum(sp, red);   // its barriers also publish the weights f_k
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const int rounds = (nc + NS * KB - 1) / (NS * KB);
    for (int r = 0; r < rounds; r++) {
        if (r > 0) load_round(r);
#pragma unroll
        for (int b = 0; b < KB; b++) {
            const int k = sl + NS * (r * KB + b);
            const float f = (act && k < nc) ? sml[k].x : 0.0f;
            acc.x += f * ov[b].x; acc.y += f * ov[b].y; acc.z += f * ov[b].z; acc.w += f * ov[b].w;
        }
    }
    if (act) *reinterpret_cast<float4 *>(slice + (size_t)sl * HD + 4 * q) = acc;
    __syncthreads();
    for (int d = tid; d < HD; d += WG) {
        float O = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < NS; s2++) O += slice[(size_t)s2 * HD + d];
        a.out[(size_t)h * HD + d] = O * (1.0f / S);
    }
}

// --------------------------------------------------------------------------
int attn_decode_chunk(int hd, bool f16kv) {
    switch (hd) {
        case 48: return f16kv ? dec_chunk<48, true, ATT_DEC_NL, ATT_DEC_IT>() : dec_chunk<48, false, ATT_DEC_NL, ATT_DEC_IT>();
        case 64: return f16kv ? dec_chunk<64, true, ATT_DEC_NL, ATT_DEC_IT>() : dec_chunk<64, false, ATT_DEC_NL, ATT_DEC_IT>();
        case 128: return f16kv ? dec_chunk<128, true, ATT_DEC_NL, ATT_DEC_IT>() : dec_chunk<128, false, ATT_DEC_NL, ATT_DEC_IT>();
    }
    return 0;
}

template <int HD, bool F16>
static int dec_pick_g(hipStream_t st, const AttnArgs &a, bool with_merge) {
    const int G = a.n_heads / a.n_kv;
    dim3 grid(a.n_kv, a.max_chunks);
    constexpr int NL = ATT_DEC_NL, IT = ATT_DEC_IT;
    if (G <= 1) hipLaunchKernelGGL((k_attn_dec<HD, 1, F16, NL, IT>), grid, dim3(WG), 0, st, a);
    else if (G <= 2) hipLaunchKernelGGL((k_attn_dec<HD, 2, F16, NL, IT>), grid, dim3(WG), 0, st, a);
    else if (G <= 4) hipLaunchKernelGGL((k_attn_dec<HD, 4, F16, NL, IT>), grid, dim3(WG), 0, st, a);
    else if (G <= 8) hipLaunchKernelGGL((k_attn_dec<HD, 8, F16, NL, IT>), grid, dim3(WG), 0, st, a);
    else return -1;
    if (!with_merge) return 0;
    const size_t lds = 8 * (size_t)a.max_chunks + 4 * (size_t)(WG / (HD / 4)) * HD;
    hipLaunchKernelGGL((k_attn_merge<HD>), dim3(a.n_heads), dim3(WG), lds, st, a, dec_chunk<HD, F16, NL, IT>());
    return 0;
}

int launch_attn_decode(hipStream_t st, bool f16kv, const AttnArgs &a, bool with_merge) {
    if (a.n_kv <= 0 || a.n_heads % a.n_kv != 0 || !a.part) return -1;
    const int cr = attn_decode_chunk(a.hd, f16kv);
    if (cr <= 0 || (a.ctx + cr - 1) / cr > a.max_chunks) return -1;
    switch (a.hd) {
        case 48: return f16kv ? dec_pick_g<48, true>(st, a, with_merge) : dec_pick_g<48, false>(st, a, with_merge);
        case 64: return f16kv ? dec_pick_g<64, true>(st, a, with_merge) : dec_pick_g<64, false>(st, a, with_merge);
        case 128: return f16kv ? dec_pick_g<128, true>(st, a, with_merge) : dec_pick_g<128, false>(st, a, with_merge);
    }
    return -1;
}

}  // namespace ehip
