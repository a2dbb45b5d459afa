// matvec.hip — decode-step matrix-vector products for gfx950.
//
// Replaces ember_matmul -> mm_rows -> vecdot_q8 / vecdot_q4 / dot_f32
// (src/kernels.c:120-220) together with the RMSNorm, activation quantization,
// bias, residual and SwiGLU work around each call in ember_forward
// (src/model.c:375-412); with argmax outputs set, also the greedy branch of
// ember_sample (src/sample.c:114-127) over the logits it produces.
//
// Roofline: HBM-bound.  Algorithmic bytes per output row = cols (Q8_0 codes)
// or cols/2 (Q4_0 nibbles) + 2*cols/32 (fp16 scales): the 34 / 18 bytes per
// 32 weights of the file.
//
// A decode matvec is a single short pass over the weights, so its time is
// set by how many HBM round trips lie on each wave's critical path.  The
// kernel therefore:
//   1. issues the weight loads of its first row group before anything else
//      (they do not depend on the activation);
//   2. while those are in flight, loads the activation as float4s (all of a
//      thread's loads issued together), applies the RMSNorm and quantizes to
//      Q8_0 in registers: a 32-element block spans 8 consecutive lanes, so
//      its absolute maximum is three cross-lane steps;
//   3. walks further row groups with the next group's loads issued before
//      the current group's arithmetic.
// Lane l owns 16-byte chunks l, l+64, ... of a row, so one wave load moves
// 1 KB of contiguous row bytes.  A Q8_0 chunk is half a block: the two halves
// of block j sit in lanes 2j and 2j+1 and are paired with one cross-lane add
// before the block scale is applied, so the integer block sum is exact as in
// the reference.  A Q4_0 chunk is one whole block (16 bytes of nibbles); the
// nibble bias of 8 is removed through the block sum of the activation codes.
#include <climits>

#include "kernels.h"

namespace ehip {

template <int DT>
__device__ __forceinline__ int chunk_count(int K) {
    return DT == DT_Q8 ? K / 16 : (DT == DT_Q4 ? K / QB : K / 4);
}

__device__ __forceinline__ void am_take(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
}

// block-wide (value, index) maximum, ties to the smaller index
__device__ __forceinline__ void am_block(float &v, int &i, float *sv, int *si) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float v2 = __shfl_xor(v, off);
        const int i2 = __shfl_xor(i, off);
        am_take(v, i, v2, i2);
    }
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) { sv[w] = v; si[w] = i; }
    __syncthreads();
    v = sv[0]; i = si[0];
#pragma unroll
    for (int k = 1; k < NWAVE; k++) am_take(v, i, sv[k], si[k]);
}

// One wave's group of UPW output rows (NR weight rows each): the payload
// chunks this lane owns, their raw fp16 block scales and, for the epilogue,
// the bias (EPI_STORE) or the residual being added to (EPI_RESID).  Every
// load is unconditional — rows past the end re-read the last row and lanes
// past the row's chunks re-read its last chunk — so the loads issue back to
// back with no branch or wait between them; validity is applied afterwards.
template <int DT, int EPI, int NCH, int UPW>
struct RowGroup {
    static constexpr int NR = EPI == EPI_SWIGLU ? 2 : 1;
    int4 w[UPW][NR][NCH];
    uint16_t d[UPW][NR][NCH];
    float pre[UPW];

    __device__ __forceinline__ void load(const MatvecArgs &a, int u0, int lane, int nch, int nb) {
        const int rb = DT == DT_Q8 ? a.W.cols : a.W.cols / 2;
#pragma unroll
        for (int j = 0; j < UPW; j++) {
            const int uc = min(u0 + j, a.units - 1);
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const size_t row = (size_t)(uc + r * a.pair_off);
                const int4 *wrow = reinterpret_cast<const int4 *>(a.W.q + row * rb);
                const uint16_t *drow = a.W.d + row * nb;
#pragma unroll
                for (int i = 0; i < NCH; i++) {
                    const int c = min(lane + 64 * i, nch - 1);
                    w[j][r][i] = wrow[c];
                    d[j][r][i] = drow[DT == DT_Q8 ? (c >> 1) : c];
                }
            }
            if (EPI == EPI_STORE) pre[j] = a.bias ? a.bias[uc] : 0.0f;
            else if (EPI == EPI_RESID) pre[j] = a.out[uc];
            else pre[j] = 0.0f;
        }
    }
};

template <int DT, int PRO, int EPI, int NCH, int UPW>
__global__ __launch_bounds__(WG) void k_matvec(MatvecArgs a) {
    // XPT float4 slots of the activation per thread: K <= 1024*NCH (Q8_0)
    // or 2048*NCH (Q4_0)
    constexpr int XPT = DT == DT_Q8 ? NCH : 2 * NCH;
    constexpr int NR = EPI == EPI_SWIGLU ? 2 : 1;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float red[NWAVE];
    __shared__ float am_v[NWAVE];
    __shared__ int am_i[NWAVE];
    const int K = a.W.cols, nb = K / QB, nslot = K / 4;
    int8_t *qx = reinterpret_cast<int8_t *>(smem);           // [K] codes
    float *dx = reinterpret_cast<float *>(smem + K);         // [nb] scales
    int *xsum = reinterpret_cast<int *>(dx + nb);            // [nb] code sums (Q4_0)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nch = chunk_count<DT>(K);
    const int gw = blockIdx.x * NWAVE + wave, nw = gridDim.x * NWAVE;

    // ---- 1. activation loads, then the first row group's weights ----------
    // (issued in this order, the activation can be used while the weights
    // are still in flight)
    float4 xv[XPT], nw4[XPT];
#pragma unroll
    for (int i = 0; i < XPT; i++) xv[i] = nw4[i] = make_float4(0, 0, 0, 0);
    int qv[XPT];
    float dv[XPT];
    if (PRO == PRO_EMBED_NORM) {
        const int tok = a.tokpos[0];
        const int8_t *row = reinterpret_cast<const int8_t *>(a.emb.q) + (size_t)tok * K;
        const uint16_t *drow = a.emb.d + (size_t)tok * nb;
        const float4 *frow = reinterpret_cast<const float4 *>(a.emb.q) + (size_t)tok * nslot;
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int s = min(tid + WG * i, nslot - 1);
            if (a.emb.dtype == DT_F32) {
                xv[i] = frow[s];
            } else {
                qv[i] = reinterpret_cast<const int *>(row)[s];
                dv[i] = h2f(drow[s >> 3]);
            }
        }
    } else {
        const float4 *in4 = reinterpret_cast<const float4 *>(a.in);
#pragma unroll
        for (int i = 0; i < XPT; i++) xv[i] = in4[min(tid + WG * i, nslot - 1)];
    }
    // PRO_NORM_PARTS: the partial vectors, loaded with the input (every load
    // unconditional: parts past n_parts re-read the last one and are dropped)
    constexpr int NPV = PRO == PRO_NORM_PARTS ? MATVEC_MAX_PARTS : 1;
    float4 pv[PRO == PRO_NORM_PARTS ? XPT : 1][NPV];
    if constexpr (PRO == PRO_NORM_PARTS) {
        const float4 *p4 = reinterpret_cast<const float4 *>(a.parts);
#pragma unroll
        for (int i = 0; i < XPT; i++)
#pragma unroll
            for (int p = 0; p < NPV; p++)
                pv[i][p] = p4[(size_t)min(p, a.n_parts - 1) * nslot + min(tid + WG * i, nslot - 1)];
        if (blockIdx.x == 0 && tid < a.n_parts)
            __hip_atomic_store(a.flag_reset + tid * XM_CNT_STRIDE, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (PRO != PRO_PLAIN) {
        const float4 *w4 = reinterpret_cast<const float4 *>(a.norm_w);
#pragma unroll
        for (int i = 0; i < XPT; i++) nw4[i] = w4[min(tid + WG * i, nslot - 1)];
    }
    RowGroup<DT, EPI, NCH, UPW> cur;
    int u0 = gw * UPW;
    cur.load(a, u0, lane, nch, nb);

    // ---- 2. RMSNorm and Q8_0 quantization of the activation, in registers --
    if constexpr (PRO == PRO_NORM_PARTS) {   // x + (p_0 + p_1 + ...), parts in order
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            float4 t = pv[i][0];
#pragma unroll
            for (int p = 1; p < NPV; p++)
                if (p < a.n_parts) { t.x += pv[i][p].x; t.y += pv[i][p].y; t.z += pv[i][p].z; t.w += pv[i][p].w; }
            xv[i].x += t.x; xv[i].y += t.y; xv[i].z += t.z; xv[i].w += t.w;
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const bool live = tid + WG * i < nslot;
        if (PRO == PRO_EMBED_NORM && a.emb.dtype != DT_F32) {   // Q8_0 embedding (model.c:83-100)
            const int q = qv[i];
            xv[i] = make_float4((float)(int8_t)(q & 0xff) * dv[i], (float)(int8_t)((q >> 8) & 0xff) * dv[i],
                                (float)(int8_t)((q >> 16) & 0xff) * dv[i], (float)(int8_t)(q >> 24) * dv[i]);
        }
        if (!live) xv[i] = make_float4(0, 0, 0, 0);
        if (PRO != PRO_PLAIN) ss += xv[i].x * xv[i].x + xv[i].y * xv[i].y + xv[i].z * xv[i].z + xv[i].w * xv[i].w;
    }
    if ((PRO == PRO_EMBED_NORM || PRO == PRO_NORM_PARTS) && blockIdx.x == 0) {
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int s = tid + WG * i;
            if (s < nslot) reinterpret_cast<float4 *>(a.x_out)[s] = xv[i];
        }
    }
    if (PRO != PRO_PLAIN) {
        const float tot = block_sum(ss, red);
        const float scale = 1.0f / sqrtf(tot / (float)K + a.eps);   // model.c:50-55
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            xv[i].x = xv[i].x * scale * nw4[i].x; xv[i].y = xv[i].y * scale * nw4[i].y;
            xv[i].z = xv[i].z * scale * nw4[i].z; xv[i].w = xv[i].w * scale * nw4[i].w;
        }
    }
    // kernels.c:73-92: d = amax/127, inverse of the unrounded d, round half
    // away from zero, clamp to +-127; the fp16-rounded d is what the dot uses
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int s = tid + WG * i;
        float m = fmaxf(fmaxf(fabsf(xv[i].x), fabsf(xv[i].y)), fmaxf(fabsf(xv[i].z), fabsf(xv[i].w)));
        m = max8(m);
        const float d = m / 127.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        const int q0 = (int)fminf(fmaxf(roundf(xv[i].x * id), -127.0f), 127.0f);
        const int q1 = (int)fminf(fmaxf(roundf(xv[i].y * id), -127.0f), 127.0f);
        const int q2 = (int)fminf(fmaxf(roundf(xv[i].z * id), -127.0f), 127.0f);
        const int q3 = (int)fminf(fmaxf(roundf(xv[i].w * id), -127.0f), 127.0f);
        int qs = q0 + q1 + q2 + q3;
        if (DT == DT_Q4) qs = sum8(qs);
        if (s < nslot) {
            reinterpret_cast<int *>(qx)[s] = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | (q3 << 24);
            if ((tid & 7) == 0) {
                dx[s >> 3] = h2f(f2h(d));
                if (DT == DT_Q4) xsum[s >> 3] = qs;
            }
        }
    }
    __syncthreads();

    // ---- 3. this lane's activation chunks ---------------------------------
    int4 xr[NCH], xr2[NCH];
    float dxr[NCH];
    int xsr[NCH];
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const int c = lane + 64 * i;
        xr[i] = make_int4(0, 0, 0, 0); xr2[i] = xr[i]; dxr[i] = 0.0f; xsr[i] = 0;
        if (DT == DT_Q8 && c < nch) {
            xr[i] = reinterpret_cast<const int4 *>(qx)[c];
            dxr[i] = dx[c >> 1];
        } else if (DT == DT_Q4 && c < nch) {
            xr[i] = reinterpret_cast<const int4 *>(qx)[2 * c];
            xr2[i] = reinterpret_cast<const int4 *>(qx)[2 * c + 1];
            dxr[i] = dx[c];
            xsr[i] = xsum[c];
        }
    }

    // the error-flag word behind the outputs, for the host's copy
    if (EPI == EPI_STORE && a.out_host && blockIdx.x == 0 && tid == 0)
        reinterpret_cast<int *>(a.out_host)[a.units] = reinterpret_cast<const int *>(a.out)[a.units];

    // ---- 4. row groups: prefetch the next, compute the current ------------
    float best_v = -INFINITY;
    int best_i = INT_MAX;
    for (; u0 < a.units; u0 += nw * UPW) {
        RowGroup<DT, EPI, NCH, UPW> nxt;
        const bool more = u0 + nw * UPW < a.units;
        if (more) nxt.load(a, u0 + nw * UPW, lane, nch, nb);
        // every row's lane partials first, then all the cross-lane sums
        // together (independent chains the scheduler interleaves), then one
        // epilogue in which lane j finishes row j
        float v[UPW][NR];
#pragma unroll
        for (int j = 0; j < UPW; j++) {
#pragma unroll
            for (int r = 0; r < NR; r++) {
                float s = 0.0f;
#pragma unroll
                for (int i = 0; i < NCH; i++) {
                    const int4 w = cur.w[j][r][i];
                    int d;
                    if (DT == DT_Q8) {
                        d = sdot4(w.x, xr[i].x, 0);
                        d = sdot4(w.y, xr[i].y, d);
                        d = sdot4(w.z, xr[i].z, d);
                        d = sdot4(w.w, xr[i].w, d);
                        // lanes 2j, 2j+1 hold the two halves of block j
                        d += __builtin_amdgcn_mov_dpp(d, 0xb1, 0xf, 0xf, false);   // quad_perm [1,0,3,2]
                        if (lane & 1) d = 0;
                    } else {
                        const int m = 0x0f0f0f0f;
                        d = sdot4(w.x & m, xr[i].x, 0);
                        d = sdot4(w.y & m, xr[i].y, d);
                        d = sdot4(w.z & m, xr[i].z, d);
                        d = sdot4(w.w & m, xr[i].w, d);
                        d = sdot4((w.x >> 4) & m, xr2[i].x, d);
                        d = sdot4((w.y >> 4) & m, xr2[i].y, d);
                        d = sdot4((w.z >> 4) & m, xr2[i].z, d);
                        d = sdot4((w.w >> 4) & m, xr2[i].w, d);
                        d -= 8 * xsr[i];
                    }
                    // block product in the reference's order: (acc * dw) * dx
                    const float dw = lane + 64 * i < nch ? h2f(cur.d[j][r][i]) : 0.0f;
                    s += ((float)d * dw) * dxr[i];
                }
                v[j][r] = s;
            }
        }
#pragma unroll
        for (int j = 0; j < UPW; j++)
#pragma unroll
            for (int r = 0; r < NR; r++) v[j][r] = wave_sum(v[j][r]);
        // lane j < UPW: row u0 + j
        float mine[NR], pre = 0.0f;
#pragma unroll
        for (int r = 0; r < NR; r++) mine[r] = v[0][r];
        pre = cur.pre[0];
#pragma unroll
        for (int j = 1; j < UPW; j++)
            if (lane == j) {
#pragma unroll
                for (int r = 0; r < NR; r++) mine[r] = v[j][r];
                pre = cur.pre[j];
            }
        const int u = u0 + lane;
        if (lane < UPW && u < a.units) {
            if (EPI == EPI_STORE) {
                const float o = a.bias ? mine[0] + pre : mine[0];
                a.out[u] = o;
                if (a.out_host) a.out_host[u] = o;
                am_take(best_v, best_i, o, u);
            } else if (EPI == EPI_RESID) {
                a.out[u] = pre + mine[0];
            } else {
                const float g = mine[0];
                a.out[u] = g / (1.0f + expf(-g)) * mine[NR - 1];
            }
        }
        if (more) cur = nxt;
    }

    // ---- 5. greedy selection over the logits (optional): this workgroup's
    // winner; argmax_merge picks the first maximum over the winners ---------
    if (EPI != EPI_STORE || !a.am_val) return;
    am_block(best_v, best_i, am_v, am_i);
    if (tid == 0) {
        a.am_val[blockIdx.x] = best_v;
        a.am_idx[blockIdx.x] = best_i;
    }
}

// F32 weights (files the reference leaves unquantized, quant.c:26-57): plain
// fp32 dot products in the reference's order (dot_f32, kernels.c:120-135),
// the activation kept in LDS.
template <int PRO, int EPI>
__global__ __launch_bounds__(WG) void k_matvec_f32(MatvecArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float red[NWAVE];
    const int K = a.W.cols;
    float *xs = reinterpret_cast<float *>(smem);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float ss = 0.0f;
    for (int i = tid; i < K; i += WG) {
        float v;
        if (PRO == PRO_EMBED_NORM) {
            const int tok = a.tokpos[0];
            v = a.emb.dtype == DT_F32 ? reinterpret_cast<const float *>(a.emb.q)[(size_t)tok * K + i]
                                      : (float)reinterpret_cast<const int8_t *>(a.emb.q)[(size_t)tok * K + i] *
                                            h2f(a.emb.d[(size_t)tok * (K / QB) + i / QB]);
            if (blockIdx.x == 0) a.x_out[i] = v;
        } else {
            v = a.in[i];
        }
        xs[i] = v;
        ss += v * v;
    }
    if (PRO != PRO_PLAIN) {
        const float tot = block_sum(ss, red);
        const float scale = 1.0f / sqrtf(tot / (float)K + a.eps);
        for (int i = tid; i < K; i += WG) xs[i] = xs[i] * scale * a.norm_w[i];
    }
    __syncthreads();
    constexpr int NR = EPI == EPI_SWIGLU ? 2 : 1;
    const int gw = blockIdx.x * NWAVE + wave, nw = gridDim.x * NWAVE;
    const float4 *x4 = reinterpret_cast<const float4 *>(xs);
    for (int u = gw; u < a.units; u += nw) {
        float v[NR];
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const float4 *wrow = reinterpret_cast<const float4 *>(a.W.q) + (size_t)(u + r * a.pair_off) * (K / 4);
            float s = 0.0f;
            for (int c = lane; c < K / 4; c += 64) {
                const float4 w = wrow[c], x = x4[c];
                s += w.x * x.x + w.y * x.y + w.z * x.z + w.w * x.w;
            }
            v[r] = wave_sum(s);
        }
        if (lane == 0) {
            if (EPI == EPI_STORE) a.out[u] = a.bias ? v[0] + a.bias[u] : v[0];
            else if (EPI == EPI_RESID) a.out[u] += v[0];
            else { const float g = v[0]; a.out[u] = g / (1.0f + expf(-g)) * v[NR - 1]; }
        }
    }
}

// --------------------------------------------------------------------------
static int grid_for(int units, int upw) {
    long waves = (units + upw - 1) / upw;
    long grid = (waves + NWAVE - 1) / NWAVE;
    if (grid > MATVEC_MAX_GRID) grid = MATVEC_MAX_GRID;
    return grid < 1 ? 1 : (int)grid;
}

template <int DT, int PRO, int EPI, int NCH, int UPW>
static int go(hipStream_t st, const MatvecArgs &a, size_t lds) {
    const int grid = grid_for(a.units, UPW);
    hipLaunchKernelGGL((k_matvec<DT, PRO, EPI, NCH, UPW>), dim3(grid), dim3(WG), lds, st, a);
    return grid;
}

// rows per wave: the largest of 4, 3, 2, 1 that still gives every CU a
// workgroup, within a register budget (wide rows keep fewer rows in flight).
// 3 keeps 3072-row products (Qwen3's w1|w3) at one workgroup per CU instead
// of 1.5 (some CUs working twice as long as the others).
template <int DT, int PRO, int EPI, int NCH>
static int pick_upw(hipStream_t st, const MatvecArgs &a, size_t lds) {
    if constexpr (NCH <= 2) {
        if (a.units >= 4 * NWAVE * 256) return go<DT, PRO, EPI, NCH, 4>(st, a, lds);
        if (a.units >= 3 * NWAVE * 256) return go<DT, PRO, EPI, NCH, 3>(st, a, lds);
    }
    if constexpr (NCH <= 3) {
        if (a.units >= 2 * NWAVE * 256) return go<DT, PRO, EPI, NCH, 2>(st, a, lds);
    }
    return go<DT, PRO, EPI, NCH, 1>(st, a, lds);
}

template <int DT, int PRO, int EPI>
static int pick_nch(hipStream_t st, const MatvecArgs &a, size_t lds) {
    const int K = a.W.cols;
    const int per_lane = DT == DT_Q8 ? (K / 16 + 63) / 64 : (K / QB + 63) / 64;
    if (per_lane <= 1) return pick_upw<DT, PRO, EPI, 1>(st, a, lds);
    if (per_lane <= 2) return pick_upw<DT, PRO, EPI, 2>(st, a, lds);
    if (per_lane <= 3) return pick_upw<DT, PRO, EPI, 3>(st, a, lds);
    if (per_lane <= 5) return pick_upw<DT, PRO, EPI, 5>(st, a, lds);
    if constexpr (DT == DT_Q8) {
        if (per_lane <= 8) return pick_upw<DT, PRO, EPI, 8>(st, a, lds);
    }
    return -1;
}

template <int PRO, int EPI>
static int pick_dt(hipStream_t st, const MatvecArgs &a) {
    const int K = a.W.cols;
    switch (a.W.dtype) {
        case DT_Q8: return pick_nch<DT_Q8, PRO, EPI>(st, a, (size_t)K + (size_t)(K / QB) * 8);
        case DT_Q4: return pick_nch<DT_Q4, PRO, EPI>(st, a, (size_t)K + (size_t)(K / QB) * 8);
        case DT_F32: {
            if constexpr (PRO == PRO_NORM_PARTS) return -1;
            if ((size_t)K * 4 > 64 * 1024) return -1;
            long grid = ((long)a.units + NWAVE - 1) / NWAVE;
            if (grid > MATVEC_MAX_GRID) grid = MATVEC_MAX_GRID;
            hipLaunchKernelGGL((k_matvec_f32<PRO, EPI>), dim3(grid), dim3(WG), (size_t)K * 4, st, a);
            return (int)grid;
        }
    }
    return -1;
}

int launch_matvec(hipStream_t st, int pro, int epi, const MatvecArgs &a) {
    const int K = a.W.cols;
    if (K % QB != 0 || K <= 0 || a.units <= 0) return -1;
    if (a.am_val && (epi != EPI_STORE || a.W.dtype == DT_F32)) return -1;
    if (a.out_host && (epi != EPI_STORE || a.W.dtype == DT_F32)) return -1;
    int grid = -1;
    if (pro == PRO_NORM && epi == EPI_STORE) grid = pick_dt<PRO_NORM, EPI_STORE>(st, a);
    else if (pro == PRO_EMBED_NORM && epi == EPI_STORE) grid = pick_dt<PRO_EMBED_NORM, EPI_STORE>(st, a);
    else if (pro == PRO_NORM && epi == EPI_SWIGLU) grid = pick_dt<PRO_NORM, EPI_SWIGLU>(st, a);
    else if (pro == PRO_PLAIN && epi == EPI_RESID) grid = pick_dt<PRO_PLAIN, EPI_RESID>(st, a);
    else if (pro == PRO_NORM_PARTS && epi == EPI_SWIGLU) {
        if (!a.parts || !a.x_out || !a.flag_reset || a.n_parts < 1 || a.n_parts > MATVEC_MAX_PARTS) return -1;
        if (a.W.dtype != DT_Q8 && a.W.dtype != DT_Q4) return -1;
        grid = pick_dt<PRO_NORM_PARTS, EPI_SWIGLU>(st, a);
    }
    if (grid <= 0) return -1;
    if (a.am_val) return launch_argmax_merge(st, a.am_val, a.am_idx, grid, a.units, a.am_tokpos, a.am_out, a.am_cap);
    return 0;
}

int launch_matvec_parts(hipStream_t st, int pro, const MatvecArgs &a) {
    const int K = a.W.cols;
    if (K % QB != 0 || K <= 0 || a.units <= 0 || !a.am_val || a.W.dtype == DT_F32) return -1;
    if (pro == PRO_NORM) return pick_dt<PRO_NORM, EPI_STORE>(st, a);
    if (pro == PRO_EMBED_NORM) return pick_dt<PRO_EMBED_NORM, EPI_STORE>(st, a);
    return -1;
}

}  // namespace ehip
