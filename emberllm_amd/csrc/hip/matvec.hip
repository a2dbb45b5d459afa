// matvec.hip — decode-step matrix-vector products for gfx950.
//
// Replaces ember_matmul -> mm_rows -> vecdot_q8 / vecdot_q4 / dot_f32
// (src/kernels.c:120-220) together with the RMSNorm, activation quantization,
// bias, residual and SwiGLU work around each call in ember_forward
// (src/model.c:375-412).
//
// Roofline: HBM-bound.  Algorithmic bytes per output row = cols (Q8_0 codes)
// + 2*cols/32 (fp16 scales), i.e. the 34 bytes per 32 weights of the file.
//
// Work split: every workgroup first builds the quantized activation in LDS
// (each one redundantly: the input is a few KB and L2-resident), then each
// wave64 streams whole rows.  Lane l owns 16-byte chunks l, l+64, ... of a
// row, so one wave load instruction moves 1 KB of contiguous row bytes.  A
// Q8_0 chunk is half a block: the two halves of block j live in lanes 2j and
// 2j+1 and are paired with one cross-lane add before the block scale is
// applied, so the integer block sum is exact as in the reference.  A Q4_0
// chunk is one whole block (16 bytes of nibbles); the nibble bias of 8 is
// removed through the precomputed block sum of the activation codes.
#include "kernels.h"

namespace ehip {

template <int DT>
__device__ __forceinline__ int chunk_count(int K) {
    return DT == DT_Q8 ? K / 16 : (DT == DT_Q4 ? K / QB : K / 4);
}

template <int DT, int PRO, int EPI, int NCH, int UPW>
__global__ __launch_bounds__(WG) void k_matvec(MatvecArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int K = a.W.cols, nb = K / QB;
    float *xs = reinterpret_cast<float *>(smem);
    int8_t *qx = reinterpret_cast<int8_t *>(xs + K);
    float *dx = reinterpret_cast<float *>(qx + K);
    int *xsum = reinterpret_cast<int *>(dx + nb);
    float *red = reinterpret_cast<float *>(xsum + nb);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // ---- prologue: input (optionally the embedding row), RMSNorm --------
    float ss = 0.0f;
    if (PRO == PRO_EMBED_NORM) {
        const int tok = a.tokpos[0];
        if (a.emb.dtype == DT_F32) {
            const float *row = reinterpret_cast<const float *>(a.emb.q) + (size_t)tok * K;
            for (int i = tid; i < K; i += WG) { float v = row[i]; xs[i] = v; ss += v * v; }
        } else {  // Q8_0 embedding (model.c:83-100)
            const int8_t *row = reinterpret_cast<const int8_t *>(a.emb.q) + (size_t)tok * K;
            const uint16_t *drow = a.emb.d + (size_t)tok * nb;
            for (int i = tid; i < K; i += WG) {
                float v = (float)row[i] * h2f(drow[i / QB]);
                xs[i] = v; ss += v * v;
            }
        }
        if (blockIdx.x == 0)
            for (int i = tid; i < K; i += WG) a.x_out[i] = xs[i];
    } else {
        for (int i = tid; i < K; i += WG) { float v = a.in[i]; xs[i] = v; ss += v * v; }
    }
    if (PRO != PRO_PLAIN) {
        const float tot = block_sum(ss, red);
        const float scale = 1.0f / sqrtf(tot / (float)K + a.eps);
        for (int i = tid; i < K; i += WG) xs[i] = xs[i] * scale * a.norm_w[i];
    }
    __syncthreads();

    // ---- activation quantization (kernels.c:73-92) -----------------------
    if (DT != DT_F32) {
        for (int blk = wave * 2 + (lane >> 5); blk < nb; blk += NWAVE * 2) {
            float dq;
            const int q = quant_q8_lane(xs[blk * QB + (lane & 31)], &dq);
            qx[blk * QB + (lane & 31)] = (int8_t)q;
            if (DT == DT_Q4) {
                int s = q;
#pragma unroll
                for (int off = 16; off > 0; off >>= 1) s += __shfl_xor(s, off);
                if ((lane & 31) == 0) xsum[blk] = s;
            }
            if ((lane & 31) == 0) dx[blk] = dq;
        }
        __syncthreads();
    }

    const int nch = chunk_count<DT>(K);
    const int gw = blockIdx.x * NWAVE + wave, nw = gridDim.x * NWAVE;
    constexpr int NR = EPI == EPI_SWIGLU ? 2 : 1;

    // ---- activation chunks this lane owns, in registers -------------------
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

    for (int u0 = gw * UPW; u0 < a.units; u0 += nw * UPW) {
        float acc[UPW][NR];
        if (DT == DT_F32) {
#pragma unroll
            for (int j = 0; j < UPW; j++)
#pragma unroll
                for (int r = 0; r < NR; r++) {
                    acc[j][r] = 0.0f;
                    const int u = u0 + j;
                    if (u >= a.units) continue;
                    const float4 *wrow = reinterpret_cast<const float4 *>(a.W.q) +
                                         (size_t)(u + r * a.pair_off) * (K / 4);
                    const float4 *x4 = reinterpret_cast<const float4 *>(xs);
                    for (int c = lane; c < nch; c += 64) {
                        const float4 w = wrow[c], x = x4[c];
                        acc[j][r] += w.x * x.x + w.y * x.y + w.z * x.z + w.w * x.w;
                    }
                }
        } else {
            int4 wv[UPW][NR][NCH];
            float wd[UPW][NR][NCH];
            // issue every load of this group of rows before any arithmetic
#pragma unroll
            for (int j = 0; j < UPW; j++)
#pragma unroll
                for (int r = 0; r < NR; r++) {
                    const int u = u0 + j;
                    const size_t row = (size_t)(u + r * a.pair_off);
                    const bool live = u < a.units;
                    const int rb = DT == DT_Q8 ? K : K / 2;
                    const int4 *wrow = reinterpret_cast<const int4 *>(a.W.q + row * rb);
                    const uint16_t *drow = a.W.d + row * nb;
#pragma unroll
                    for (int i = 0; i < NCH; i++) {
                        const int c = lane + 64 * i;
                        const bool ok = live && c < nch;
                        wv[j][r][i] = ok ? wrow[c] : make_int4(0, 0, 0, 0);
                        wd[j][r][i] = ok ? h2f(drow[DT == DT_Q8 ? (c >> 1) : c]) : 0.0f;
                    }
                }
#pragma unroll
            for (int j = 0; j < UPW; j++)
#pragma unroll
                for (int r = 0; r < NR; r++) {
                    float s = 0.0f;
#pragma unroll
                    for (int i = 0; i < NCH; i++) {
                        const int4 w = wv[j][r][i];
                        int d;
                        if (DT == DT_Q8) {
                            d = sdot4(w.x, xr[i].x, 0);
                            d = sdot4(w.y, xr[i].y, d);
                            d = sdot4(w.z, xr[i].z, d);
                            d = sdot4(w.w, xr[i].w, d);
                            d += __shfl_xor(d, 1);   // lanes 2j, 2j+1: both halves of block j
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
                        s += ((float)d * wd[j][r][i]) * dxr[i];
                    }
                    acc[j][r] = s;
                }
        }
        // ---- reduce and epilogue ----------------------------------------
#pragma unroll
        for (int j = 0; j < UPW; j++) {
            float v[NR];
#pragma unroll
            for (int r = 0; r < NR; r++) v[r] = wave_sum(acc[j][r]);
            const int u = u0 + j;
            if (lane == 0 && u < a.units) {
                if (EPI == EPI_STORE) {
                    a.out[u] = a.bias ? v[0] + a.bias[u] : v[0];
                } else if (EPI == EPI_RESID) {
                    a.out[u] += v[0];
                } else {
                    const float g = v[0];
                    a.out[u] = g / (1.0f + expf(-g)) * v[NR - 1];
                }
            }
        }
    }
}

// --------------------------------------------------------------------------
template <int DT, int PRO, int EPI, int NCH>
static void go(hipStream_t st, const MatvecArgs &a, int grid, size_t lds) {
    constexpr int UPW = (EPI == EPI_SWIGLU || NCH > 2) ? 2 : 4;
    hipLaunchKernelGGL((k_matvec<DT, PRO, EPI, NCH, UPW>), dim3(grid), dim3(WG), lds, st, a);
}

template <int DT, int PRO, int EPI>
static int pick_nch(hipStream_t st, const MatvecArgs &a, int grid, size_t lds) {
    const int K = a.W.cols;
    const int per_lane = DT == DT_Q8 ? (K / 16 + 63) / 64 : (K / QB + 63) / 64;
    if (DT == DT_F32) { go<DT, PRO, EPI, 1>(st, a, grid, lds); return 0; }
    if (per_lane <= 1) go<DT, PRO, EPI, 1>(st, a, grid, lds);
    else if (per_lane <= 2) go<DT, PRO, EPI, 2>(st, a, grid, lds);
    else if (per_lane <= 3) go<DT, PRO, EPI, 3>(st, a, grid, lds);
    else if (per_lane <= 5) go<DT, PRO, EPI, 5>(st, a, grid, lds);
    else if (DT == DT_Q8 && per_lane <= 8) go<DT, PRO, EPI, 8>(st, a, grid, lds);
    else return -1;
    return 0;
}

template <int PRO, int EPI>
static int pick_dt(hipStream_t st, const MatvecArgs &a, int grid, size_t lds) {
    switch (a.W.dtype) {
        case DT_Q8: return pick_nch<DT_Q8, PRO, EPI>(st, a, grid, lds);
        case DT_Q4: return pick_nch<DT_Q4, PRO, EPI>(st, a, grid, lds);
        case DT_F32: return pick_nch<DT_F32, PRO, EPI>(st, a, grid, lds);
    }
    return -1;
}

int launch_matvec(hipStream_t st, int pro, int epi, const MatvecArgs &a) {
    const int K = a.W.cols;
    if (K % QB != 0 || K <= 0) return -1;
    const size_t lds = (size_t)K * 4 + K + (size_t)(K / QB) * 8 + NWAVE * 4;
    if (lds > 64 * 1024) return -1;
    // enough waves to give every row group its own wave, capped at 8 WGs/CU
    const int upw = (epi == EPI_SWIGLU) ? 2 : 4;
    long waves = (a.units + upw - 1) / upw;
    long grid = (waves + NWAVE - 1) / NWAVE;
    if (grid > 2048) grid = 2048;
    if (grid < 1) grid = 1;
    int rc = -1;
    if (pro == PRO_NORM && epi == EPI_STORE) rc = pick_dt<PRO_NORM, EPI_STORE>(st, a, (int)grid, lds);
    else if (pro == PRO_EMBED_NORM && epi == EPI_STORE) rc = pick_dt<PRO_EMBED_NORM, EPI_STORE>(st, a, (int)grid, lds);
    else if (pro == PRO_NORM && epi == EPI_SWIGLU) rc = pick_dt<PRO_NORM, EPI_SWIGLU>(st, a, (int)grid, lds);
    else if (pro == PRO_PLAIN && epi == EPI_RESID) rc = pick_dt<PRO_PLAIN, EPI_RESID>(st, a, (int)grid, lds);
    return rc;
}

}  // namespace ehip
