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
// Grid = (kv heads, max_chunks), kv heads varying fastest, so neighbouring
// workgroups read whole cache rows.  Rows [0, pos] of each kv head are split
// into equal chunks, one per workgroup of that head; with max_chunks =
// ATT_DEC_WPC * #CUs / n_kv every CU streams the same share whatever the position (a CU
// holding one more chunk than the others would set the kernel's length).
// With the in-kernel merge the grid is 1-D instead: 8 * xm_slots workgroups,
// workgroup L on XCD L % 8 (round-robin dispatch) taking slot L / 8 there;
// the kv heads g = x, x + 8, ... of XCD x share its slots as chunks, so every
// chunk of a kv head runs on one XCD whatever the number of kv heads (with 8
// kv heads this is the 2-D grid above, slot for chunk).
// Chunks hold at least ATT_DEC_RMIN rows: at short contexts a few chunks
// (and a short merge) beat many chunks of two or three rows.  A
// workgroup serves all kv_mul query heads of its kv head from the same K/V
// rows, so each cache row is read once per step.  Lane (rw, j) of a wave holds
// 16-byte piece j of row rw of each wave load:
//   1. loads: the token's q heads / k / v pieces (straight out of the QKV
//      matvec), the QK-norm weights and the RoPE (cos, sin) of its piece, then
//      the first batch of NL K pieces and NL V pieces per thread;
//   2. QK-norm and RoPE in registers: a head's sum of squares is a reduction
//      over the LPR lanes of its row, a NEOX partner element sits P/2 lanes
//      away, an interleaved partner in the same lane; the chunk holding `pos`
//      stores the new k/v row;
//   3. batches, each issuing the next batch's loads before its own scores
//      (cross-lane sums over the row's lanes), with a running softmax (max,
//      sum of exp, sum of exp * V) per wave.  Scores are kept in log2 units
//      (scaled by log2(e)/sqrt(hd)), so each probability is one v_exp_f32;
//   4. the four waves' partials combine in LDS.  With one chunk that is the
//      output (model.c:57-64: max, exp, 1/sum); otherwise the chunk's
//      (o, m, l) partial is stored.
// Merging the chunks of a kv head: when all workgroups of each kv head run on
// one XCD (checked at state creation by k_xcc_probe and again by every
// workgroup), the last workgroup of the head to finish merges them through
// that XCD's L2: partial stores complete in L2, an L2 atomic counts arrivals,
// and the last arriver reads the partials back from L2 — no device-scope
// round trip and no second kernel.  Otherwise k_attn_merge, the next kernel
// on the stream, merges them.
#include <algorithm>

#include "kernels.h"

namespace ehip {

constexpr float LOG2E = 1.4426950408889634f;

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

__device__ __forceinline__ int xcc_id() {
    unsigned x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return (int)x;
}

template <int HD, bool F16> struct DecLay {
    static constexpr int PE = F16 ? 8 : 4;                 // elements per 16-byte piece
    static constexpr int P = HD / PE;                      // pieces per row
    static constexpr int LPR = P <= 8 ? 8 : (P <= 16 ? 16 : (P <= 32 ? 32 : 64));
    static constexpr int RPL = 64 / LPR;                   // rows per wave load
    static_assert(HD % PE == 0 && P % 2 == 0, "head_dim must split into an even number of pieces");
};

// XMODE: 0 = chunk partials for k_attn_merge; 1 = in-kernel merge on the
// 2-D grid (n_kv a multiple of 8: chunk c of kv head g is workgroup
// g + n_kv c, max_chunks = 8 xm_slots / n_kv); 2 = in-kernel merge on the
// 1-D grid of 8 * xm_slots; 3 = mode 1 with the wo product folded in (every
// workgroup of kv head g, on g's XCD, waits for the merged o_g and computes
// its wo_rows rows of the group's wo partial: see AttnArgs::wo); 4 = mode 2
// with the wo product folded in the same way, each kv head's rows shared
// over its own chunk count, G * HD / 16 of the CPR lanes per row in use and
// (CPR >= 32) two rounds of rows per workgroup; 5 = mode 3 with a Q4_0 wo
// (one whole 32-weight block per lane: GM * HD / 32 lanes per row).
template <int HD, int GM, bool F16, int NL, int NW, int XMODE>
__global__ __launch_bounds__(NW * 64) void k_attn_dec(AttnArgs a) {
    constexpr bool XM = XMODE != 0, FW = XMODE >= 3, FW1 = XMODE == 4, FWQ4 = XMODE == 5;
    using L = DecLay<HD, F16>;
    constexpr int PE = L::PE, P = L::P, LPR = L::LPR, RPL = L::RPL;
    constexpr int NT = NW * 64, RPB = NW * RPL;   // threads, rows per workgroup load
    constexpr int BR = NL * RPB;      // rows per batch
    constexpr int QPR = HD / 4;                                   // float4s per head row (merge)
    constexpr int NSL = GM * QPR >= NT ? 1 : NT / (GM * QPR);     // chunk slices in the merge
    __shared__ float sm_m[NW][GM], sm_l[NW][GM];
    __shared__ __align__(16) float sm_o[NW][GM][HD];
    __shared__ float sm_xm[NSL][GM], sm_xl[NSL][GM];
    __shared__ __align__(16) float4 sm_acc[NT];
    __shared__ int sm_last;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int g, c, nchunk;   // kv head, chunk, chunks of the kv head
    if constexpr (XMODE == 2 || XMODE == 4) {
        // the mapping's arguments are read before anything depends on them,
        // so their scalar loads are in flight together
        asm volatile("" ::"s"(a.n_kv), "s"(a.xm_slots), "s"(a.q), "s"(a.tokpos), "s"(a.xm_xcc));
        const int L = blockIdx.x, x = L & 7, s = L >> 3;
        const int H = x < a.n_kv ? (a.n_kv - 1 - x) / 8 + 1 : 0;   // kv heads on this XCD
        if (H == 0) return;
        nchunk = a.xm_slots / H;
        g = x + 8 * (s % H);
        c = s / H;
        if (c >= nchunk) return;
    } else {
        g = blockIdx.x; c = blockIdx.y;   // kv heads vary fastest: neighbours read whole cache rows
        nchunk = a.max_chunks;
    }
    const int G = a.n_heads / a.n_kv;
    const int xcc_want = XM ? a.xm_xcc[g] : 0;
    // FW: this thread's 16 wo codes (row fw_r of the workgroup's wo_rows,
    // 16-byte chunk fw_j of the group's G * HD columns) and their block
    // scale, loaded before anything else (they depend on nothing)
    constexpr int CPR = GM * HD / 16;   // chunk lanes per wo row (G * HD / 16 in use; all with G == GM)
    constexpr int RPR = NT / CPR;       // wo rows per round
    constexpr int FWR = FW1 && CPR >= 32 ? 2 : 1;   // rounds of rows
    const int fw_r = tid / CPR, fw_j = tid % CPR;
    const int fw_row = c * a.wo_rows + fw_r;
    int4 fw_q = make_int4(0, 0, 0, 0);
    uint16_t fw_d = 0;
    if constexpr (FW && !FW1 && !FWQ4) {
        const int rc = min(c * a.wo_rows + min(fw_r, a.wo_rows - 1), a.wo.rows - 1);
        const int col0 = g * G * HD;
        fw_q = *reinterpret_cast<const int4 *>(a.wo.q + (size_t)rc * a.wo.cols + col0 + 16 * fw_j);
        fw_d = a.wo.d[(size_t)rc * (a.wo.cols / QB) + col0 / QB + fw_j / 2];
    }
    // mode 5: the lane's Q4_0 block (16 bytes of nibbles) and scale of row
    // fw_r5 of the workgroup's wo_rows
    constexpr int CPR5 = GM * HD / 32;
    const int fw_r5 = tid / CPR5, fw_j5 = tid % CPR5;
    int4 fw_q5 = make_int4(0, 0, 0, 0);
    uint16_t fw_d5 = 0;
    if constexpr (FWQ4) {
        const int rc = min(c * a.wo_rows + min(fw_r5, a.wo_rows - 1), a.wo.rows - 1);
        const int blk = g * G * HD / QB + fw_j5;
        fw_q5 = *reinterpret_cast<const int4 *>(a.wo.q + (size_t)rc * (a.wo.cols / 2) + 16 * blk);
        fw_d5 = a.wo.d[(size_t)rc * (a.wo.cols / QB) + blk];
    }
    int4 fw_q4[FWR];      // mode 4: rows fw_r + k RPR of the kv head's own wo_rows
    uint16_t fw_d4[FWR];
    if constexpr (FW1) {
        const int wo_rows = (a.wo.rows + nchunk - 1) / nchunk;
        const int fw_jc = min(fw_j, G * HD / 16 - 1);
        const int col0 = g * G * HD;
#pragma unroll
        for (int k = 0; k < FWR; k++) {
            const int rc = min(c * wo_rows + min(fw_r + k * RPR, wo_rows - 1), a.wo.rows - 1);
            fw_q4[k] = *reinterpret_cast<const int4 *>(a.wo.q + (size_t)rc * a.wo.cols + col0 + 16 * fw_jc);
            fw_d4[k] = a.wo.d[(size_t)rc * (a.wo.cols / QB) + col0 / QB + fw_jc / 2];
        }
    }
    // FW: o_g is complete in this XCD's L2: raise the group's flag
    auto raise = [&]() {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            if (xcc_id() != xcc_want) __hip_atomic_fetch_or(a.xm_err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.wo_flag + g * XM_CNT_STRIDE, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };

    if constexpr (FW) {
        auto attend = [&]() {
#include "attn_decode_body.inc"
        };
        attend();
    } else {
#include "attn_decode_body.inc"
        return;
    }

    // ---- 6. (FW) the group's wo partial ------------------------------------
    // Wait for the flag (a bounded wait: on time-out the error flag sends the
    // host to the two-kernel schedule), then quantize o_g as k_matvec's
    // PRO_PLAIN prologue does (the same codes and fp16-rounded scales) and
    // take this workgroup's rows in k_matvec's block order per lane:
    // ((float)isum * dw) * dx, summed over the row's lanes.
    __shared__ int sm_go;
    __shared__ __align__(16) int sm_qx[GM * HD / 4];
    __shared__ float sm_dx[GM * HD / QB];
    __shared__ int sm_xs[GM * HD / QB];   // mode 5: the blocks' code sums
    if (tid == 0) {
        if (xcc_id() != xcc_want) __hip_atomic_fetch_or(a.xm_err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int ok = 1;
        for (int n = 0; __hip_atomic_load(a.wo_flag + g * XM_CNT_STRIDE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0; n++) {
            if (n >= a.wo_spin) {
                ok = 0;
                __hip_atomic_fetch_or(a.xm_err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        sm_go = ok;
    }
    __syncthreads();
    if (!sm_go) return;
    if (tid < (FW1 ? G : GM) * HD / 4) {
        const float4 x = *reinterpret_cast<const float4 *>(a.out + (size_t)g * G * HD + 4 * tid);
        float m = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
        m = max8(m);
        const float d = m / 127.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        const int q0 = (int)fminf(fmaxf(roundf(x.x * id), -127.0f), 127.0f);
        const int q1 = (int)fminf(fmaxf(roundf(x.y * id), -127.0f), 127.0f);
        const int q2 = (int)fminf(fmaxf(roundf(x.z * id), -127.0f), 127.0f);
        const int q3 = (int)fminf(fmaxf(roundf(x.w * id), -127.0f), 127.0f);
        sm_qx[tid] = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | (q3 << 24);
        if ((tid & 7) == 0) sm_dx[tid >> 3] = h2f(f2h(d));
        if constexpr (FWQ4) {
            const int xs = sum8(q0 + q1 + q2 + q3);
            if ((tid & 7) == 0) sm_xs[tid >> 3] = xs;
        }
    }
    __syncthreads();
    if constexpr (FWQ4) {   // k_matvec's Q4_0 block: low nibbles x codes 0-15, high x 16-31, minus 8 x code sum
        const int4 xl = *reinterpret_cast<const int4 *>(&sm_qx[8 * fw_j5]);
        const int4 xh = *reinterpret_cast<const int4 *>(&sm_qx[8 * fw_j5 + 4]);
        const int m = 0x0f0f0f0f;
        int isum = sdot4(fw_q5.x & m, xl.x, 0);
        isum = sdot4(fw_q5.y & m, xl.y, isum);
        isum = sdot4(fw_q5.z & m, xl.z, isum);
        isum = sdot4(fw_q5.w & m, xl.w, isum);
        isum = sdot4((fw_q5.x >> 4) & m, xh.x, isum);
        isum = sdot4((fw_q5.y >> 4) & m, xh.y, isum);
        isum = sdot4((fw_q5.z >> 4) & m, xh.z, isum);
        isum = sdot4((fw_q5.w >> 4) & m, xh.w, isum);
        isum -= 8 * sm_xs[fw_j5];
        float v = ((float)isum * h2f(fw_d5)) * sm_dx[fw_j5];
        v = group_sum<CPR5>(v);
        const int row = c * a.wo_rows + fw_r5;
        if (fw_j5 == 0 && fw_r5 < a.wo_rows && row < a.wo.rows) a.wo_part[(size_t)g * a.wo.rows + row] = v;
        return;
    }
    if constexpr (FW1) {
        const int wo_rows = (a.wo.rows + nchunk - 1) / nchunk, cpr_g = G * HD / 16;
        const int fw_jc = min(fw_j, cpr_g - 1);
        const int4 xq = *reinterpret_cast<const int4 *>(&sm_qx[4 * fw_jc]);
        const float dx = sm_dx[fw_jc >> 1];
#pragma unroll
        for (int k = 0; k < FWR; k++) {
            int isum = sdot4(fw_q4[k].x, xq.x, 0);
            isum = sdot4(fw_q4[k].y, xq.y, isum);
            isum = sdot4(fw_q4[k].z, xq.z, isum);
            isum = sdot4(fw_q4[k].w, xq.w, isum);
            isum += __builtin_amdgcn_mov_dpp(isum, 0xb1, 0xf, 0xf, false);   // quad_perm [1,0,3,2]
            float v = (fw_j & 1) || fw_j >= cpr_g ? 0.0f : ((float)isum * h2f(fw_d4[k])) * dx;
            v = group_sum<CPR>(v);
            const int r = fw_r + k * RPR, row = c * wo_rows + r;
            if (fw_j == 0 && r < wo_rows && row < a.wo.rows) a.wo_part[(size_t)g * a.wo.rows + row] = v;
        }
        return;
    }
    const int4 xq = *reinterpret_cast<const int4 *>(&sm_qx[4 * fw_j]);
    int isum = sdot4(fw_q.x, xq.x, 0);
    isum = sdot4(fw_q.y, xq.y, isum);
    isum = sdot4(fw_q.z, xq.z, isum);
    isum = sdot4(fw_q.w, xq.w, isum);
    // lanes 2k, 2k + 1 hold the two halves of block k
    isum += __builtin_amdgcn_mov_dpp(isum, 0xb1, 0xf, 0xf, false);   // quad_perm [1,0,3,2]
    float v = (fw_j & 1) ? 0.0f : ((float)isum * h2f(fw_d)) * sm_dx[fw_j >> 1];
    v = group_sum<CPR>(v);
    if (fw_j == 0 && fw_r < a.wo_rows && fw_row < a.wo.rows) a.wo_part[(size_t)g * a.wo.rows + fw_row] = v;
}

// Split-K merge, one workgroup per query head, when the chunks of a kv head
// do not all run on one XCD (the next kernel on the stream, so the partials
// written above are visible without fences):
//   o = sum_k o_k 2^(m_k - M) / sum_k l_k 2^(m_k - M),  M = max_k m_k
// (chunk maxima are in log2 units).  Thread (s, q) owns float4 quad q of the
// head row and chunks k = s, s + NS, ...; every partial it needs is loaded in
// one batch, issued together with the chunk statistics, before any reduction.
template <int HD, bool F16>   // F16: the cache type, which sets the chunk rows
__global__ __launch_bounds__(WG) void k_attn_merge(AttnArgs a) {
    constexpr int QPR = HD / 4, NS = WG / QPR, KB = 16;
    extern __shared__ __align__(16) float dyn[];   // [max_chunks] float2, then [NS][HD]
    __shared__ float red[NWAVE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = blockIdx.x;
    const int pos = a.tokpos[1];
    const int R = dec_chunk_rows(pos, a.max_chunks, F16);
    const int nc = (pos + 1 + R - 1) / R;
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
        const float f = __builtin_amdgcn_exp2f(sml[k].x - M);
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

// Records the XCD of every workgroup of a (gx, gy) grid: out[y * gx + x].
__global__ void k_xcc_probe(int *out) {
    if (threadIdx.x == 0) out[blockIdx.y * gridDim.x + blockIdx.x] = xcc_id();
}

int launch_xcc_probe(hipStream_t st, int gx, int gy, int *out) {
    if (gx <= 0 || gy <= 0) return -1;
    hipLaunchKernelGGL(k_xcc_probe, dim3(gx, gy), dim3(64), 0, st, out);
    return 0;
}

// --------------------------------------------------------------------------
int attn_decode_chunks(int ctx, int n_kv, int hd, int n_cu) {
    if (hd != 48 && hd != 64 && hd != 128) return 0;
    const int by_rows = (ctx + ATT_DEC_CR - 1) / ATT_DEC_CR;
    const int by_cus = n_kv > 0 ? ATT_DEC_WPC * n_cu / n_kv : 1;
    return std::max(1, std::max(by_rows, by_cus));
}

int attn_decode_slots(int ctx, int n_kv, int n_cu) {
    const int hmax = (n_kv + 7) / 8;   // kv heads on the busiest XCD
    const int by_rows = hmax * ((ctx + ATT_DEC_CR - 1) / ATT_DEC_CR);
    return std::max(hmax, std::max(by_rows, ATT_DEC_WPC * n_cu / 8));
}

template <int HD, bool F16, int GM>
static void dec_launch(hipStream_t st, const AttnArgs &a, dim3 grid) {
    constexpr int NL = ATT_DEC_NL, NW = ATT_DEC_NW;
    if (!a.xm_cnt) hipLaunchKernelGGL((k_attn_dec<HD, GM, F16, NL, NW, 0>), grid, dim3(NW * 64), 0, st, a);
    else if (grid.y > 1 && a.wo_part && a.wo.dtype == DT_Q4) {
        if constexpr (HD != 48 && GM * HD >= 256) hipLaunchKernelGGL((k_attn_dec<HD, GM, F16, NL, NW, 5>), grid, dim3(NW * 64), 0, st, a);
    }
    else if (grid.y > 1 && a.wo_part) {
        if constexpr (HD != 48 && GM * HD >= 128) hipLaunchKernelGGL((k_attn_dec<HD, GM, F16, NL, NW, 3>), grid, dim3(NW * 64), 0, st, a);
    }
    else if (grid.y > 1) hipLaunchKernelGGL((k_attn_dec<HD, GM, F16, NL, NW, 1>), grid, dim3(NW * 64), 0, st, a);
    else if (a.wo_part) {
        if constexpr (HD != 48 && GM * HD >= 128) hipLaunchKernelGGL((k_attn_dec<HD, GM, F16, NL, NW, 4>), grid, dim3(NW * 64), 0, st, a);
    }
    else hipLaunchKernelGGL((k_attn_dec<HD, GM, F16, NL, NW, 2>), grid, dim3(NW * 64), 0, st, a);
}

template <int HD, bool F16>
static int dec_pick_g(hipStream_t st, const AttnArgs &a, bool with_merge) {
    const int G = a.n_heads / a.n_kv;
    // the in-kernel merge's 1-D grid is the 2-D one, chunk for slot, when n_kv
    // is a multiple of 8 (whose prologue needs no mapping)
    const dim3 grid = !a.xm_cnt || a.n_kv % 8 == 0 ? dim3(a.n_kv, a.max_chunks) : dim3(8 * a.xm_slots);
    if (G <= 1) dec_launch<HD, F16, 1>(st, a, grid);
    else if (G <= 2) dec_launch<HD, F16, 2>(st, a, grid);
    else if (G <= 4) dec_launch<HD, F16, 4>(st, a, grid);
    else if (G <= 8) dec_launch<HD, F16, 8>(st, a, grid);
    else return -1;
    if (!with_merge || a.xm_cnt) return 0;
    const size_t lds = 8 * (size_t)a.max_chunks + 4 * (size_t)(WG / (HD / 4)) * HD;
    hipLaunchKernelGGL((k_attn_merge<HD, F16>), dim3(a.n_heads), dim3(WG), lds, st, a);
    return 0;
}

int launch_attn_decode(hipStream_t st, bool f16kv, const AttnArgs &a, bool with_merge) {
    if (a.n_kv <= 0 || a.n_heads % a.n_kv != 0 || !a.part) return -1;
    if (a.xm_cnt) {
        // every kv head gets xm_slots / (its XCD's kv heads) chunks of at most
        // ATT_DEC_CR rows; with n_kv a multiple of 8 that is the 2-D grid's
        // max_chunks = 8 xm_slots / n_kv
        const int per_head = a.xm_slots / ((a.n_kv + 7) / 8);
        if (!a.xm_err || !a.xm_xcc || a.xm_slots <= 0) return -1;
        if (a.n_kv % 8 == 0 ? a.max_chunks != 8 * a.xm_slots / a.n_kv : a.max_chunks < a.xm_slots) return -1;
        if ((long)per_head * ATT_DEC_CR < a.ctx) return -1;
    } else if ((long)a.max_chunks * ATT_DEC_CR < a.ctx) {
        return -1;
    }
    if (a.wo_part) {   // the folded wo product: whole 32-weight blocks per kv group, 8-64 chunk lanes per row
        const int G = a.n_heads / a.n_kv, GM = G <= 1 ? 1 : (G <= 2 ? 2 : (G <= 4 ? 4 : 8));
        const bool q4 = a.wo.dtype == DT_Q4;   // mode 5: one block per lane
        const int cpr = GM * a.hd / (q4 ? 32 : 16), rpr = ATT_DEC_NW * 64 / cpr;
        if (!a.xm_cnt || !a.wo_flag || (a.wo.dtype != DT_Q8 && !(q4 && a.n_kv % 8 == 0)) || !a.wo.q || !a.wo.d) return -1;
        if ((a.hd != 64 && a.hd != 128) || (G * a.hd) % QB || cpr < 8 || cpr > 64) return -1;
        if (a.wo.cols != a.n_heads * a.hd || a.wo.rows <= 0 || a.wo_spin < 0) return -1;
        if (a.n_kv % 8 == 0) {   // mode 3: G == GM, the host's wo_rows in one round
            if (G != GM || a.wo_rows <= 0 || (long)a.wo_rows * a.max_chunks < a.wo.rows || a.wo_rows > rpr) return -1;
        } else {                 // mode 4: each kv head's chunk count, up to two rounds of rows
            if (a.n_kv > 8) return -1;
            const int nchunk = a.xm_slots, rounds = cpr >= 32 ? 2 : 1;
            if ((a.wo.rows + nchunk - 1) / nchunk > rounds * rpr) return -1;
        }
    }
    switch (a.hd) {
        case 48: return f16kv ? dec_pick_g<48, true>(st, a, with_merge) : dec_pick_g<48, false>(st, a, with_merge);
        case 64: return f16kv ? dec_pick_g<64, true>(st, a, with_merge) : dec_pick_g<64, false>(st, a, with_merge);
        case 128: return f16kv ? dec_pick_g<128, true>(st, a, with_merge) : dec_pick_g<128, false>(st, a, with_merge);
    }
    return -1;
}

}  // namespace ehip
