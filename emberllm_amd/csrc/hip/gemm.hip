// gemm.hip — batched prefill products for gfx950.
//
// Replaces ember_matmul_batch -> mmb_rows (src/kernels.c:223-264) and the
// per-token RMSNorm / SwiGLU / embedding loops of ember_prefill
// (src/model.c:305-351).
//
// k_quant_rows: one workgroup per token row builds the Q8_0 activation codes
// (optionally after the embedding lookup, an RMSNorm or the SwiGLU gate),
// eight lanes per 32-element block.
// k_gemm_mfma (Q8_0 / Q4_0 weights): int8 matrix cores, one
// v_mfma_i32_32x32x32_i8 per 32-weight quant block, so each block's integer
// dot product is exact and separately available; the fp32 epilogue of every
// block applies the reference's order sum += ((float)isum * dw) * dx
// (vecdot_q8 / vecdot_q4, kernels.c:151-183), or for products over at least
// GEMM_SPLIT_MIN_K inputs (FUSED) sum = fma((float)isum, dw * dx, sum): one
// rounding and one VALU operation fewer per output and block, and with the
// scale products dw * dx of a tile taken from one fp16 matrix instruction
// (exact: both are fp16 values) a second VALU operation fewer.  Those
// products already split their block sums over pipelines elsewhere (the
// short-prompt and decode products), so the models they belong to run at the
// reference builds' own noise floor; the others keep the reference's order.
// Roofline: the epilogue's VALU operations per output element and block
// bound it, not the MFMA rate.
// k_gemm (F32 weights): a 64 x 64 tile per workgroup, 4 x 4 micro-tiles per
// thread, dot_f32 order.
#include "kernels.h"
#include "flimg.h"

namespace ehip {

// The row is staged in LDS with each 32-element block padded to QP floats,
// so that the quantizing lanes' 16-byte reads of consecutive blocks spread
// over the banks.  Element i lives at xs[lds_at(i)].
constexpr int QP = 36;
__device__ __forceinline__ int lds_at(int i) { return i + (i / QB) * (QP - QB); }

__global__ __launch_bounds__(WG) void k_quant_rows(QuantRowsArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    float *xs = reinterpret_cast<float *>(smem);
    __shared__ float red[NWAVE];
    const int K = a.cols, nb = K / QB, b = blockIdx.x;
    const int tid = threadIdx.x;
    // the row loops are unrolled so a thread's global loads are issued together;
    // thread tid sums the squares of elements tid, tid + WG, ... in that order
    float ss = 0.0f;
    if (a.ids) {
        const int tok = a.ids[b];
#pragma unroll 4
        for (int i = tid; i < K; i += WG) {
            float v;
            if (a.emb.dtype == DT_F32) v = reinterpret_cast<const float *>(a.emb.q)[(size_t)tok * K + i];
            else v = (float)reinterpret_cast<const int8_t *>(a.emb.q)[(size_t)tok * K + i] *
                     h2f(a.emb.d[(size_t)tok * nb + i / QB]);
            xs[lds_at(i)] = v; ss += v * v;
            a.x_out[(size_t)b * K + i] = v;
        }
    } else if (a.swiglu) {
        const float *row = a.x + (size_t)b * a.x_stride;
#pragma unroll 4
        for (int i = tid; i < K; i += WG) {
            const float g = row[i];
            const float v = g / (1.0f + expf(-g)) * row[K + i];
            xs[lds_at(i)] = v; ss += v * v;
        }
    } else {
        const float *row = a.x + (size_t)b * a.x_stride;
#pragma unroll 4
        for (int i = tid; i < K; i += WG) { const float v = row[i]; xs[lds_at(i)] = v; ss += v * v; }
    }
    if (a.norm_w) {
        const float tot = block_sum(ss, red);
        const float scale = 1.0f / sqrtf(tot / (float)K + a.eps);
#pragma unroll 4
        for (int i = tid; i < K; i += WG) xs[lds_at(i)] = xs[lds_at(i)] * scale * a.norm_w[i];
    }
    __syncthreads();
    if (a.xf)
        for (int i = tid; i < K; i += WG) a.xf[(size_t)b * K + i] = xs[lds_at(i)];
    if (a.qx) {
        // eight lanes per block, four elements each: the quant_q8_lane
        // arithmetic (d = amax/127, the inverse of the unrounded d, round half
        // away from zero, clamp), the block's maximum and code sum as 8-lane
        // DPP reductions
        const int part = tid & 7;
        for (int blk = tid >> 3; blk < nb; blk += WG / 8) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(xs + blk * QP + 4 * part);
            float mx = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
            mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0xb1, 0xf, 0xf, false)));
            mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0x4e, 0xf, 0xf, false)));
            mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0x141, 0xf, 0xf, false)));
            const float d = mx / 127.0f;
            const float id = d > 0.0f ? 1.0f / d : 0.0f;
            const int c0 = (int)fminf(fmaxf(roundf(v.x * id), -127.0f), 127.0f);
            const int c1 = (int)fminf(fmaxf(roundf(v.y * id), -127.0f), 127.0f);
            const int c2 = (int)fminf(fmaxf(roundf(v.z * id), -127.0f), 127.0f);
            const int c3 = (int)fminf(fmaxf(roundf(v.w * id), -127.0f), 127.0f);
            int sum = c0 + c1 + c2 + c3;
            sum += __builtin_amdgcn_mov_dpp(sum, 0xb1, 0xf, 0xf, false);
            sum += __builtin_amdgcn_mov_dpp(sum, 0x4e, 0xf, 0xf, false);
            sum += __builtin_amdgcn_mov_dpp(sum, 0x141, 0xf, 0xf, false);
            *reinterpret_cast<uint32_t *>(a.qx + (size_t)b * K + (size_t)blk * QB + 4 * part) =
                ((uint32_t)c0 & 0xffu) | (((uint32_t)c1 & 0xffu) << 8) | (((uint32_t)c2 & 0xffu) << 16) |
                (((uint32_t)c3 & 0xffu) << 24);
            if (part == 0) {
                a.dx[(size_t)b * nb + blk] = h2f(f2h(d));
                a.xs[(size_t)b * nb + blk] = sum;
            }
        }
    }
}

int launch_quant_rows(hipStream_t st, const QuantRowsArgs &a) {
    const size_t lds = (size_t)(a.cols / QB) * QP * 4;
    if (a.cols % QB != 0 || lds > 64 * 1024 || a.n <= 0) return -1;
    hipLaunchKernelGGL(k_quant_rows, dim3(a.n), dim3(WG), lds, st, a);
    return 0;
}

// --------------------------------------------------------------------------
constexpr int TM = 64, TN = 64;

template <int DT, int EPI>
__global__ __launch_bounds__(WG) void k_gemm(GemmArgs a) {
    // one K-block of the tile: weights, activations, their scales
    __shared__ __align__(16) uint8_t ws[TM * (DT == DT_F32 ? 128 : 32)];
    __shared__ __align__(16) uint8_t xsm[TN * (DT == DT_F32 ? 128 : 32)];
    __shared__ float dws[TM], dxs[TN];
    __shared__ int sums[TN];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int u0 = blockIdx.x * TM, b0 = blockIdx.y * TN;
    const int K = a.W.cols, nb = K / QB;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;

    for (int blk = 0; blk < nb; blk++) {
        if (DT == DT_F32) {
            // 64 rows x 32 floats each for W and X: 512 float4 apiece
            for (int i = tid; i < TM * 8; i += WG) {
                const int r = i >> 3, p = i & 7;
                const int u = u0 + r;
                float4 w = make_float4(0, 0, 0, 0);
                if (u < a.units)
                    w = reinterpret_cast<const float4 *>(a.W.q)[((size_t)u * K + blk * QB) / 4 + p];
                reinterpret_cast<float4 *>(ws)[i] = w;
                const int t = b0 + r;
                float4 x = make_float4(0, 0, 0, 0);
                if (t < a.n) x = reinterpret_cast<const float4 *>(a.xf)[((size_t)t * K + blk * QB) / 4 + p];
                reinterpret_cast<float4 *>(xsm)[i] = x;
            }
        } else {
            if (tid < 128) {
                const int r = tid >> 1, h = tid & 1;
                const int u = u0 + r, t = b0 + r;
                int4 w = make_int4(0, 0, 0, 0), x = make_int4(0, 0, 0, 0);
                if (DT == DT_Q8) {
                    if (u < a.units) w = *reinterpret_cast<const int4 *>(a.W.q + (size_t)u * K + blk * QB + h * 16);
                    reinterpret_cast<int4 *>(ws)[tid] = w;
                } else if (h == 0) {
                    if (u < a.units) w = *reinterpret_cast<const int4 *>(a.W.q + (size_t)u * (K / 2) + blk * 16);
                    reinterpret_cast<int4 *>(ws)[r] = w;
                }
                if (t < a.n) x = *reinterpret_cast<const int4 *>(a.qx + (size_t)t * K + blk * QB + h * 16);
                reinterpret_cast<int4 *>(xsm)[tid] = x;
            } else if (tid < 192) {
                const int u = u0 + tid - 128;
                dws[tid - 128] = u < a.units ? h2f(a.W.d[(size_t)u * nb + blk]) : 0.0f;
            } else {
                const int t = b0 + tid - 192;
                dxs[tid - 192] = t < a.n ? a.dx[(size_t)t * nb + blk] : 0.0f;
                sums[tid - 192] = (DT == DT_Q4 && t < a.n) ? a.xs[(size_t)t * nb + blk] : 0;
            }
        }
        __syncthreads();
        if (DT == DT_F32) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float *w = reinterpret_cast<const float *>(ws) + (tx * 4 + i) * QB;
                    const float *x = reinterpret_cast<const float *>(xsm) + (ty * 4 + j) * QB;
                    float s = acc[i][j];
                    for (int k = 0; k < QB; k++) s += w[k] * x[k];  // dot_f32 order
                    acc[i][j] = s;
                }
        } else {
            int xv[4][8];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int4 *xp = reinterpret_cast<const int4 *>(xsm) + (ty * 4 + j) * 2;
                const int4 lo = xp[0], hi = xp[1];
                xv[j][0] = lo.x; xv[j][1] = lo.y; xv[j][2] = lo.z; xv[j][3] = lo.w;
                xv[j][4] = hi.x; xv[j][5] = hi.y; xv[j][6] = hi.z; xv[j][7] = hi.w;
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = tx * 4 + i;
                int wv[8];
                if (DT == DT_Q8) {
                    const int4 *wp = reinterpret_cast<const int4 *>(ws) + r * 2;
                    const int4 lo = wp[0], hi = wp[1];
                    wv[0] = lo.x; wv[1] = lo.y; wv[2] = lo.z; wv[3] = lo.w;
                    wv[4] = hi.x; wv[5] = hi.y; wv[6] = hi.z; wv[7] = hi.w;
                } else {
                    const int4 p = reinterpret_cast<const int4 *>(ws)[r];
                    const int m = 0x0f0f0f0f;
                    wv[0] = p.x & m; wv[1] = p.y & m; wv[2] = p.z & m; wv[3] = p.w & m;
                    wv[4] = (p.x >> 4) & m; wv[5] = (p.y >> 4) & m; wv[6] = (p.z >> 4) & m; wv[7] = (p.w >> 4) & m;
                }
                const float dw = dws[r];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    int d = 0;
#pragma unroll
                    for (int k = 0; k < 8; k++) d = sdot4(wv[k], xv[j][k], d);
                    if (DT == DT_Q4) d -= 8 * sums[ty * 4 + j];
                    acc[i][j] += ((float)d * dw) * dxs[ty * 4 + j];
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int u = u0 + tx * 4 + i;
        if (u >= a.units) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int t = b0 + ty * 4 + j;
            if (t >= a.n) continue;
            float *o = a.out + (size_t)t * a.out_stride + u;
            if (EPI == EPI_STORE) *o = a.bias ? acc[i][j] + a.bias[u] : acc[i][j];
            else *o += acc[i][j];
        }
    }
}

// --------------------------------------------------------------------------
// int8 MFMA GEMM.  Workgroup tile GM_U (units) x TT (tokens, 128 or 64), four
// waves in a 2 x 2 arrangement, each owning 2 x (TT / 64) MFMA tiles of
// 32 x 32 (64-token tiles when 128 would leave CUs idle: the 1024-output wo
// and w2 products of a 2048-token pass).  K advances KB quant blocks per
// stage; stages are double-buffered in LDS (the next stage's global loads are
// issued before the current stage's products).  KB = 2 (measured against 8,
// which was slower at every prompt length once no stage registers sat in
// scratch memory).
// Output (i, j) of an MFMA tile sits in lane j + 32*((i/4)%2), accumulator
// (i%4) + 4*(i/8); A fragments hold W[u][16h .. 16h+15] of one block, B
// fragments X[t][16h .. 16h+15], h = lane / 32.
// SP = 2 (fused block scaling, Q8_0, 64-token tiles): two such pipelines of
// 256 threads side by side in one workgroup, pipeline p over the p-th half of
// the blocks, their sums added in pipeline order at the end (through LDS):
// twice the waves per SIMD for grids of at most two workgroups per CU.
constexpr int GM_U = 128;
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int mrow(int r, int h) { return (r & 3) + 4 * h + 8 * (r >> 2); }

// One k or v head's 64-key tile image for k_pf_flash16, with k_pf_kvsplit's
// bytes (flimg.h): the lane (j, h) of wave pair half lw holds key kl's dims
// 32 lw + mrow(r, h) in v0[r] and the dims 64 above them in v1[r], as stored
// in the cache.  An fp32 cache's keys take the power-of-two scale of their
// largest |value| over the 128 dims (the two waves' maxima meet in xmx) and
// split into hi and lo fp16 planes; an fp16 cache's are copied.  Every wave
// of the workgroup calls it (a barrier).
template <bool F16>
__device__ __forceinline__ void qk_image(uint8_t *im, bool isk, const float *v0, const float *v1, int kl, int lw,
                                         int h, float *xmx) {
    using I = FlImg<128, F16>;
    int ex = 0;
    if constexpr (!F16) {
        float mx = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r++) mx = fmaxf(mx, fmaxf(fabsf(v0[r]), fabsf(v1[r])));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        if (h == 0) xmx[64 * lw + kl] = mx;
        __syncthreads();
        ex = fl_exp(fmaxf(xmx[kl], xmx[64 + kl]));
        if (lw == 0 && h == 0) reinterpret_cast<int *>(im + I::KBYTES)[(isk ? 0 : FL_BK) + kl] = ex;
    }
    const int rk = fl_krow(kl);
#pragma unroll
    for (int q4 = 0; q4 < 4; q4++)
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const float *v = u ? v1 : v0;
            const int d = 32 * lw + 4 * h + 8 * q4 + 64 * u;   // dims d .. d + 3
            _Float16 hi[4], lo[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float x = F16 ? v[4 * q4 + e] : __builtin_amdgcn_ldexpf(v[4 * q4 + e], ex);
                hi[e] = (_Float16)x;
                lo[e] = (_Float16)(x - (float)hi[e]);
            }
            if (isk) {   // K planes: 4 dims = half of a 16-byte piece of row rk
                const int dq = d / 4;
                *reinterpret_cast<uint2 *>(im + I::k_at(rk, dq >> 1) + 8 * (dq & 1)) =
                    make_uint2(fl_pack(hi[0], hi[1]), fl_pack(hi[2], hi[3]));
                if constexpr (!F16)
                    *reinterpret_cast<uint2 *>(im + I::k_at(FL_BK + rk, dq >> 1) + 8 * (dq & 1)) =
                        make_uint2(fl_pack(lo[0], lo[1]), fl_pack(lo[2], lo[3]));
            } else {     // V^T planes: key kl of rows d .. d + 3
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    *reinterpret_cast<uint16_t *>(im + I::KE + I::v_at(d + e, kl >> 3) + 2 * (kl & 7)) =
                        __builtin_bit_cast(uint16_t, hi[e]);
                    if constexpr (!F16)
                        *reinterpret_cast<uint16_t *>(im + I::KE + I::v_at(128 + d + e, kl >> 3) + 2 * (kl & 7)) =
                            __builtin_bit_cast(uint16_t, lo[e]);
                }
            }
        }
}

template <int DT, int EPI, int TT, int KB, bool FUSED, int SP>
__global__ __launch_bounds__(WG * SP) void k_gemm_mfma(GemmArgs a, QkPostArgs p) {
    constexpr int GM_KB = KB;
    constexpr int GM_T = TT, NY = TT / 64;            // tokens per tile, MFMA tiles per wave along tokens
    constexpr int WB = DT == DT_Q8 ? 32 : 16;          // weight bytes per row and block
    constexpr int WROW = GM_KB * WB, XROW = GM_KB * 32; // stage bytes per row
    // LDS row pitches: 16 bytes of padding, so the fragment reads (lanes j
    // at rows j, 16 bytes each) spread over the banks; at the bare 64-byte
    // (Q4_0 weights: 32-byte) pitch every eight lanes of a read met on the
    // same banks, and the LDS spent as many cycles stalled on bank conflicts
    // as serving reads
    constexpr int WP = WROW + 16, XP = XROW + 16;
    static_assert(TT == 64 || TT == 128, "token tile of 64 or 128");
    static_assert(SP == 1 || (SP == 2 && FUSED && TT == 64 && DT == DT_Q8), "split pipelines: fused Q8_0, 64-token tiles");
    __shared__ __align__(16) uint8_t wsp[SP][2][GM_U * WP];
    __shared__ __align__(16) int8_t xsp[SP][2][GM_T * XP];
    // fp32 scales, or with FUSED the fp16 scale bits (the first half of each
    // array: [buf][kb][row] packed at the same strides in uint16 units)
    __shared__ float dwp[SP][2][GM_KB][GM_U], dxp[SP][2][GM_KB][GM_T];
    __shared__ int sxp[SP][2][GM_KB][GM_T];
    const int tid = SP == 1 ? (int)threadIdx.x : (int)threadIdx.x % WG, pl = SP == 1 ? 0 : (int)threadIdx.x / WG;
    const int lane = tid & 63, wave = tid >> 6;
    auto &ws = wsp[pl]; auto &xsm = xsp[pl]; auto &dws = dwp[pl]; auto &dxs = dxp[pl]; auto &sxs = sxp[pl];
    uint16_t (*dwh)[GM_KB][GM_U] = reinterpret_cast<uint16_t (*)[GM_KB][GM_U]>(&dwp[pl][0][0][0]);
    uint16_t (*dxh)[GM_KB][GM_T] = reinterpret_cast<uint16_t (*)[GM_KB][GM_T]>(&dxp[pl][0][0][0]);
    const int j = lane & 31, h = lane >> 5;
    const int u0 = blockIdx.x * GM_U, t0 = blockIdx.y * GM_T;
    // pipeline pl: blocks [bp0, bp0 + nbp); pipeline 0 has the most stages
    const int K = a.W.cols, nb = K / QB, nbh = SP == 1 ? nb : ((nb + 1) / 2 + GM_KB - 1) / GM_KB * GM_KB;
    const int bp0 = pl * nbh, nbp = min(nb, bp0 + nbh) - bp0, nst = (nbh + GM_KB - 1) / GM_KB;
    const int wu = (wave & 1) * 64, wt = (wave >> 1) * (TT / 2);   // this wave's 64 x TT/2 corner
    // the weight row of tile row r: u0 + r, or with EPI_SWIGLU the (gate, up)
    // pair of hidden unit c0 + r / 2 (gate rows first in W, up rows at
    // pair_off), so that a gate and its up product land in neighbouring
    // accumulators of one lane and a wave's 64 rows are one 32-unit block of h
    const int c0 = blockIdx.x * (GM_U / 2);
    auto wrow_of = [&](int r) __attribute__((always_inline)) {
        if constexpr (EPI == EPI_SWIGLU) return min(c0 + (r >> 1), a.units - 1) + ((r & 1) ? a.pair_off : 0);
        else return min(u0 + r, a.units - 1);
    };
    // the tile rows of fragment x: wu + 32 x .. + 31, or with EPI_QKPOST (the
    // tile one 128-dim head vector) 32 (wave & 1) + 64 x .., so that a lane
    // holds each dimension d < 64 of its rows in fragment 0 and its rotary
    // partner d + 64 at the same accumulator of fragment 1
    auto arow = [&](int x) __attribute__((always_inline)) {
        if constexpr (EPI == EPI_QKPOST) return (wave & 1) * 32 + 64 * x;
        else return wu + 32 * x;
    };

    // global -> registers for one stage: weights (WROW bytes per row), codes, scales
    constexpr int WLD = GM_U * WROW / 16 / WG, XLD = GM_T * XROW / 16 / WG;
    constexpr int NDW = GM_KB * GM_U / WG, NDX = (GM_KB * GM_T + WG - 1) / WG;   // scales per thread
    static_assert(GM_KB * GM_U % WG == 0, "weight scales per thread");
    // Staging registers hold the loaded values untouched: a use of any of
    // them here (such as converting a scale) would make the compiler wait for
    // every load issued before it, exposing a memory round trip per stage.
    i32x4 wr[WLD], xr[XLD];   // native vectors: HIP's int4 struct kept these in scratch
    uint16_t dwr[NDW]; float dxr[NDX]; int xsr[NDX];
    auto load = [&](int st) __attribute__((always_inline)) {
        const int b0 = bp0 + st * GM_KB;
#pragma unroll
        for (int i = 0; i < WLD; i++) {
            const int f = tid + i * WG, row = f / (WROW / 16), c = (f % (WROW / 16)) * 16;
            const int u = wrow_of(row), blk = min(b0 + c / WB, nb - 1);
            wr[i] = *reinterpret_cast<const i32x4 *>(a.W.q + (size_t)u * (nb * WB) + (size_t)blk * WB + c % WB);
        }
#pragma unroll
        for (int i = 0; i < XLD; i++) {
            const int f = tid + i * WG, row = f / (XROW / 16), c = (f % (XROW / 16)) * 16;
            const int t = min(t0 + row, a.n - 1), blk = min(b0 + c / 32, nb - 1);
            xr[i] = *reinterpret_cast<const i32x4 *>(a.qx + (size_t)t * K + (size_t)blk * 32 + c % 32);
        }
        // GM_KB * GM_U weight scales and GM_KB * GM_T activation scales
#pragma unroll
        for (int i = 0; i < NDW; i++) {
            const int f = tid + i * WG, kb = f / GM_U, r = f % GM_U;
            dwr[i] = a.W.d[(size_t)wrow_of(r) * nb + min(b0 + kb, nb - 1)];
        }
#pragma unroll
        for (int i = 0; i < NDX; i++) {
            const int f = min(tid + i * WG, GM_KB * GM_T - 1), kb = f / GM_T, r = f % GM_T;
            const int t = min(t0 + r, a.n - 1), blk = min(b0 + kb, nb - 1);
            dxr[i] = a.dx[(size_t)t * nb + blk];
            xsr[i] = DT == DT_Q4 ? a.xs[(size_t)t * nb + blk] : 0;
        }
    };
    auto store = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < WLD; i++) {
            const int f = tid + i * WG;
            *reinterpret_cast<i32x4 *>(ws[buf] + (f / (WROW / 16)) * WP + (f % (WROW / 16)) * 16) = wr[i];
        }
#pragma unroll
        for (int i = 0; i < XLD; i++) {
            const int f = tid + i * WG;
            *reinterpret_cast<i32x4 *>(xsm[buf] + (f / (XROW / 16)) * XP + (f % (XROW / 16)) * 16) = xr[i];
        }
#pragma unroll
        for (int i = 0; i < NDW; i++) {
            const int f = tid + i * WG;
            if constexpr (FUSED) dwh[buf][f / GM_U][f % GM_U] = dwr[i];
            else dws[buf][f / GM_U][f % GM_U] = h2f(dwr[i]);
        }
#pragma unroll
        for (int i = 0; i < NDX; i++) {
            const int f = tid + i * WG;
            if (f < GM_KB * GM_T) {
                // activation scales are fp16 values held as fp32: exact both ways
                if constexpr (FUSED) dxh[buf][f / GM_T][f % GM_T] = f2h(dxr[i]);
                else dxs[buf][f / GM_T][f % GM_T] = dxr[i];
                sxs[buf][f / GM_T][f % GM_T] = xsr[i];
            }
        }
    };

    float acc[2][NY][16];
#pragma unroll
    for (int x = 0; x < 2; x++)
#pragma unroll
        for (int y = 0; y < NY; y++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[x][y][r] = 0.0f;

    load(0);
    store(0);
    __syncthreads();
    for (int st = 0; st < nst; st++) {
        const int buf = st & 1;
        if (st + 1 < nst) load(st + 1);
#pragma unroll
        for (int kb = 0; kb < GM_KB; kb++) {
            if (st * GM_KB + kb >= nbp) break;
            i32x4 af[2], bf[NY];
#pragma unroll
            for (int x = 0; x < 2; x++) {      // weight rows wu + 32x + j, k-half h
                const uint8_t *src = ws[buf] + (size_t)(arow(x) + j) * WP + kb * WB;
                if (DT == DT_Q8) {
                    af[x] = *reinterpret_cast<const i32x4 *>(src + 16 * h);
                } else {                       // nibbles: low = weights 0..15, high = 16..31
                    const i32x4 raw = *reinterpret_cast<const i32x4 *>(src);
                    const int sh = 4 * h, m = 0x0f0f0f0f;
                    af[x] = i32x4{(raw[0] >> sh) & m, (raw[1] >> sh) & m, (raw[2] >> sh) & m, (raw[3] >> sh) & m};
                }
            }
#pragma unroll
            for (int y = 0; y < NY; y++)
                bf[y] = *reinterpret_cast<const i32x4 *>(xsm[buf] + (size_t)(wt + 32 * y + j) * XP + kb * 32 + 16 * h);
            // FUSED: the block's scale products dw * dx of a 32 x 32 tile as
            // one fp16 matrix instruction, an outer product (weight scales in
            // element 0 of A's lanes 0..31, activation scales in element 0 of
            // B's, every other element zero, so no scale meets another
            // block's).  A product of two fp16 values is exact in fp32, so
            // these are the bits of the fp32 multiply, and the epilogue keeps
            // a conversion and an fma per output.
            f16x4 sa[2], sb[NY];
            if constexpr (FUSED) {
#pragma unroll
                for (int x = 0; x < 2; x++) {
                    sa[x] = f16x4{};
                    sa[x][0] = __builtin_bit_cast(_Float16, (uint16_t)(h ? 0 : dwh[buf][kb][arow(x) + j]));
                }
#pragma unroll
                for (int y = 0; y < NY; y++) {
                    sb[y] = f16x4{};
                    sb[y][0] = __builtin_bit_cast(_Float16, (uint16_t)(h ? 0 : dxh[buf][kb][wt + 32 * y + j]));
                }
            }
#pragma unroll
            for (int x = 0; x < 2; x++)
#pragma unroll
                for (int y = 0; y < NY; y++) {
                    i32x16 d = {};
                    d = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[x], bf[y], d, 0, 0, 0);
                    const int xsum = DT == DT_Q4 ? sxs[buf][kb][wt + 32 * y + j] : 0;
                    if constexpr (FUSED) {
                        const f32x16 sc = __builtin_amdgcn_mfma_f32_32x32x8f16(sa[x], sb[y], f32x16{}, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int isum = DT == DT_Q4 ? d[r] - 8 * xsum : d[r];
                            acc[x][y][r] = fmaf((float)isum, sc[r], acc[x][y][r]);
                        }
                        // 128-token tiles: each tile's products and epilogue
                        // stay together (the compiler otherwise hoists the
                        // scale products: 176 VGPRs, two waves per SIMD
                        // instead of three; 114.6 -> 102.8 us per 4096-token
                        // w1|w3 product with the barrier)
                        if constexpr (TT == 128) __builtin_amdgcn_sched_barrier(0);
                    } else {
                        const float dx = dxs[buf][kb][wt + 32 * y + j];
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int isum = DT == DT_Q4 ? d[r] - 8 * xsum : d[r];
                            const float dw = dws[buf][kb][arow(x) + mrow(r, h)];
                            acc[x][y][r] += ((float)isum * dw) * dx;
                        }
                    }
                }
        }
        __syncthreads();
        if (st + 1 < nst) {
            store(buf ^ 1);
            __syncthreads();
        }
    }
    if constexpr (SP == 2) {   // pipeline 1's sums through the (now free) weight stages
        static_assert(2 * NY * 16 * WG * 4 <= (int)sizeof(wsp), "exchange fits the stages");
        float *xch = reinterpret_cast<float *>(&wsp[0][0][0]);
        if (pl == 1) {
#pragma unroll
            for (int x = 0; x < 2; x++)
#pragma unroll
                for (int y = 0; y < NY; y++)
#pragma unroll
                    for (int r = 0; r < 16; r++) xch[((x * NY + y) * 16 + r) * WG + tid] = acc[x][y][r];
        }
        __syncthreads();
        if (pl == 1) return;
#pragma unroll
        for (int x = 0; x < 2; x++)
#pragma unroll
            for (int y = 0; y < NY; y++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[x][y][r] += xch[((x * NY + y) * 16 + r) * WG + tid];
    }
    if constexpr (EPI == EPI_QKPOST) {
        // k_qkpost's work on the tile, one 128-dim head vector x TT tokens
        // (attention.hip; model.c:323-333): the bias (EPI_STORE's order), the
        // head's RMSNorm for q and k heads (model.c:50-55) in k_qkpost's
        // order (the squares of dims l and l + 64 added, then wave_sum over
        // l = 0..63; the pair sums meet in LDS by token), neox RoPE from the
        // host table (model.c:66-80), then q back into its q|k|v row and k
        // and v into the cache.  a.out, when set, receives the raw product.
        // Rounds of 64 tokens (y; two rounds of 32, one per wave pair, where
        // the pair sums of 64 tokens do not fit the stages): pair sums, one
        // wave_sum per token, apply.
        constexpr int PSS = 65;   // pair sums per token, padded
        constexpr int H2 = (64 * PSS + 64) * 4 <= (int)sizeof(wsp) ? 1 : 2, NTR = 64 / H2;
        static_assert(GM_U == 128 && SP == 1 && TT == 64 && (NTR * PSS + NTR + 128 + 128) * 4 <= (int)sizeof(wsp),
                      "one head vector x 64 tokens; sums fit the stages");
        float *pss = reinterpret_cast<float *>(&wsp[0][0][0]), *scl = pss + NTR * PSS, *nws = scl + NTR;
        const int vh = blockIdx.x, lw = wave & 1;   // lane dims 32 lw + mrow(r, h), and + 64
        const bool isq = vh < p.n_heads, isk = !isq && vh < p.n_heads + p.n_kv;
        const int g = isq ? 0 : vh - p.n_heads - (isk ? 0 : p.n_kv);
        const bool norm = p.q_norm && (isq || isk), rot = isq || isk;
        const float *nwp = isq ? p.q_norm : p.k_norm;
        // the head's norm weights, read from LDS after the first barrier
        if (norm && tid < 128) nws[tid] = nwp[tid];
        // p.kvimg: the k and v heads also write their 64-key tile's image for
        // k_pf_flash16 (pos_base a multiple of FL_BK: the tile is the pass's
        // tokens t0 ..), with the keys' maxima meeting in LDS (xmx)
        const bool img = p.kvimg && !isq;
        float *xmx = nws + 128;
        uint8_t *im = p.kvimg ? p.kvimg + ((size_t)g * p.kvimg_tiles + (p.pos_base + t0) / FL_BK) *
                                              (p.kv_f16 ? FlImg<128, true>::HBYTES : FlImg<128, false>::HBYTES)
                              : nullptr;
#pragma unroll
        for (int y = 0; y < NY; y++)
#pragma unroll
        for (int hh = 0; hh < H2; hh++) {
            const bool live = H2 == 1 || (wave >> 1) == hh;   // this round's token columns
            const int lt = (H2 == 1 ? (wave >> 1) * 32 : 0) + j;        // the round's token
            const int t = t0 + wt + 32 * y + j, tc = min(t, a.n - 1);
            if (live) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int d = 32 * lw + mrow(r, h);
                    if (a.bias) {
                        acc[0][y][r] = acc[0][y][r] + a.bias[u0 + d];
                        acc[1][y][r] = acc[1][y][r] + a.bias[u0 + d + 64];
                    }
                    if (a.out && t < a.n) {
                        a.out[(size_t)t * a.out_stride + u0 + d] = acc[0][y][r];
                        a.out[(size_t)t * a.out_stride + u0 + d + 64] = acc[1][y][r];
                    }
                    if (norm) pss[lt * PSS + d] = acc[0][y][r] * acc[0][y][r] + acc[1][y][r] * acc[1][y][r];
                }
            }
            if (norm) {
                __syncthreads();
#pragma unroll 1
                for (int k = 0; k < NTR / 4; k++) {   // wave w: the round's tokens NTR / 4 * w ..
                    const int tk = NTR / 4 * wave + k;
                    const float ss = wave_sum(pss[tk * PSS + lane]);
                    if (lane == 0) scl[tk] = 1.0f / sqrtf(ss / 128.0f + p.eps);
                }
                __syncthreads();
            }
            // every column (those past the pass's last token repeat it: the
            // tile image wants them) in place: normed and rotated q and k,
            // v as it is
            const int pos = p.pos_base + tc;
            if (live && rot) {
                const float sc = norm ? scl[lt] : 1.0f;
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) {   // accumulators 4 q4 .. + 3: dims d0 .. d0 + 3
                    const int d0 = 32 * lw + 4 * h + 8 * q4;
                    const f32x4 ca = *reinterpret_cast<const f32x4 *>(p.rope + (size_t)pos * 64 + d0);
                    const f32x4 cb = *reinterpret_cast<const f32x4 *>(p.rope + (size_t)pos * 64 + d0 + 2);
                    f32x4 n0 = f32x4{1.0f, 1.0f, 1.0f, 1.0f}, n1 = n0;
                    if (norm) {
                        n0 = *reinterpret_cast<const f32x4 *>(nws + d0);
                        n1 = *reinterpret_cast<const f32x4 *>(nws + d0 + 64);
                    }
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        float x0 = acc[0][y][4 * q4 + e], x1 = acc[1][y][4 * q4 + e];
                        if (norm) {
                            x0 = x0 * sc * n0[e];
                            x1 = x1 * sc * n1[e];
                        }
                        const float c = e < 2 ? ca[2 * e] : cb[2 * e - 4];
                        const float sn = e < 2 ? ca[2 * e + 1] : cb[2 * e - 3];
                        acc[0][y][4 * q4 + e] = x0 * c - x1 * sn;
                        acc[1][y][4 * q4 + e] = x0 * sn + x1 * c;
                    }
                }
            }
            if (live && t < a.n) {
                const size_t kvo = (size_t)pos * p.kv_dim + (size_t)g * 128;
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) {
                    const int d0 = 32 * lw + 4 * h + 8 * q4;
                    f32x4 y0, y1;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        y0[e] = acc[0][y][4 * q4 + e];
                        y1[e] = acc[1][y][4 * q4 + e];
                    }
                    if (isq) {
                        float *qo = p.qkv + (size_t)t * p.stride + u0 + d0;
                        *reinterpret_cast<f32x4 *>(qo) = y0;
                        *reinterpret_cast<f32x4 *>(qo + 64) = y1;
                    } else {
                        void *dst = isk ? p.kc : p.vc;
                        if (p.kv_f16) {
                            uint16_t *o = reinterpret_cast<uint16_t *>(dst) + kvo + d0;
                            *reinterpret_cast<uint2 *>(o) = make_uint2(f2h(y0[0]) | ((uint32_t)f2h(y0[1]) << 16),
                                                                       f2h(y0[2]) | ((uint32_t)f2h(y0[3]) << 16));
                            *reinterpret_cast<uint2 *>(o + 64) = make_uint2(f2h(y1[0]) | ((uint32_t)f2h(y1[1]) << 16),
                                                                            f2h(y1[2]) | ((uint32_t)f2h(y1[3]) << 16));
                        } else {
                            float *o = reinterpret_cast<float *>(dst) + kvo + d0;
                            *reinterpret_cast<f32x4 *>(o) = y0;
                            *reinterpret_cast<f32x4 *>(o + 64) = y1;
                        }
                    }
                }
            }
            if (norm && (y + 1 < NY || hh + 1 < H2)) __syncthreads();   // the next round's sums reuse pss
        }
        if (img) {   // the pass's tile image of this k or v head (k_pf_kvsplit's bytes)
            const int kl = (wave >> 1) * 32 + j;   // key within the tile
            if (p.kv_f16)
                qk_image<true>(im, isk, acc[0][0], acc[1][0], kl, lw, h, xmx);
            else
                qk_image<false>(im, isk, acc[0][0], acc[1][0], kl, lw, h, xmx);
        }
        return;
    }
    if constexpr (EPI == EPI_SWIGLU) {
        // h = silu(gate) * up for the wave's block of 32 hidden units (lane j
        // holds 16 of them for token column j, lane j + 32 the other 16), then
        // the Q8_0 codes, fp16-rounded scale and code sum of k_quant_rows'
        // SwiGLU rows: the same values (the block maximum and the code sum do
        // not depend on their order)
        const int hb0 = c0 + wu / 2, nbo = a.units / QB;
#pragma unroll
        for (int y = 0; y < NY; y++) {
            const int t = t0 + wt + 32 * y + j;
            float v[2][8];
            float mx = 0.0f;
#pragma unroll
            for (int x = 0; x < 2; x++)
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const float g = acc[x][y][2 * k], u = acc[x][y][2 * k + 1];
                    v[x][k] = g / (1.0f + expf(-g)) * u;
                    mx = fmaxf(mx, fabsf(v[x][k]));
                }
            if (a.out && t < a.n)   // the gate | up products themselves, where asked for
#pragma unroll
                for (int x = 0; x < 2; x++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int hu = hb0 + (32 * x + mrow(r, h)) / 2;
                        a.out[(size_t)t * a.out_stride + ((r & 1) ? a.pair_off : 0) + hu] = acc[x][y][r];
                    }
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float dq = mx / 127.0f;
            const float id = dq > 0.0f ? 1.0f / dq : 0.0f;
            int cs = 0;
            int cq[2][8];
#pragma unroll
            for (int x = 0; x < 2; x++)
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    cq[x][k] = (int)fminf(fmaxf(roundf(v[x][k] * id), -127.0f), 127.0f);
                    cs += cq[x][k];
                }
            cs += __shfl_xor(cs, 32);
            if (t >= a.n) continue;
            // accumulators 4kk, 4kk + 2 hold hidden units 16x + 2h + 4kk and the next one
#pragma unroll
            for (int x = 0; x < 2; x++)
#pragma unroll
                for (int kk = 0; kk < 4; kk++)
                    *reinterpret_cast<uint16_t *>(a.oq + (size_t)t * a.units + hb0 + 16 * x + 2 * h + 4 * kk) =
                        (uint16_t)(((uint32_t)cq[x][2 * kk] & 0xffu) | (((uint32_t)cq[x][2 * kk + 1] & 0xffu) << 8));
            if (h == 0) {
                a.odx[(size_t)t * nbo + hb0 / QB] = h2f(f2h(dq));
                a.oxs[(size_t)t * nbo + hb0 / QB] = cs;
            }
        }
        return;
    }
#pragma unroll
    for (int x = 0; x < 2; x++)
#pragma unroll
        for (int y = 0; y < NY; y++) {
            const int t = t0 + wt + 32 * y + j;
            if (t >= a.n) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int u = u0 + wu + 32 * x + mrow(r, h);
                if (u >= a.units) continue;
                float *o = a.out + (size_t)t * a.out_stride + u;
                if (EPI == EPI_STORE) *o = a.bias ? acc[x][y][r] + a.bias[u] : acc[x][y][r];
                else *o += acc[x][y][r];
            }
        }
}

// --------------------------------------------------------------------------
// Short prompts: the 128-unit tiles above leave most CUs idle (a 128-token
// wo or w2 product is 16 workgroups), and the reference's block order keeps
// K in one workgroup.  This variant takes 32 units x 32 tokens per workgroup,
// one 16 x 16 v_mfma_i32_16x16x32_i8 tile per wave and quant block.  K is
// consumed in stages of GS_KB = 4 blocks, and the loads of the next
// GS_P - 1 stages are in flight in a ring of registers while a stage is
// stored to LDS and computed: with a short K the kernel's time is the
// global round trip, which one stage of prefetch exposed once per stage.
// Loads land in registers, so the compiler's in-order wait for the oldest
// stage lets the younger ones stay in flight.  Fragments of the 16 x 16 x 32
// product: lane l holds A[l % 16][8 (l / 16) .. +7] (eight int8 of a weight
// row), B[8 (l / 16) .. +7][l % 16] (of a token row), and outputs
// D[4 (l / 16) + r][l % 16], r = 0..3.  The epilogue is the same
// sum += ((float)isum * dw) * dx in block order.
constexpr int GS_T = 32, GS_KB = 4;

// SPLIT > 1 (K of at least 1024): the workgroup runs SPLIT of the pipelines
// above side by side, pipeline q over the q-th contiguous part of the
// blocks, and adds their sums in pipeline order at the end.  The waves'
// serial walk over K (each block's product feeds the next block's sum) is
// then a SPLIT-th as long, and SPLIT times as many waves share each SIMD.
// The split products also apply each block as one fma (as k_gemm_mfma's
// FUSED form): sum = fma((float)isum, dw * dx, sum).
// FULL: every pipeline's block range is a whole number of stages (nb a
// multiple of 4 * SPLIT), so no load needs clamping and no stage is partial:
// the loads walk precomputed pointers and the epilogue has no tail test.
// U: units per workgroup, 32 (four waves per pipeline, 2 x 2 tiles) or 16
// (two waves, the tokens' two tiles): 16-unit tiles give the narrow products
// twice the workgroups, so they spread over every CU instead of doubling the
// waves, LDS traffic and epilogues of half of them.
// Register ring depth (stages) of a pipeline.
__host__ __device__ constexpr int gs_ring(int split, int u) { return split > 1 && u == 32 ? 4 : 8; }
// ONE: the pipeline's stages fit the ring (nst <= gs_ring), so all of them
// are loaded at the start and the stages run as straight-line code; a loop
// header would merge the ring's states and make the compiler wait for every
// load there, and the two forms in one kernel cost both their registers.
// Two-pipeline 32-unit workgroups run two or three per CU: at most 128
// VGPRs (four waves per SIMD).
template <int DT, int EPI, int SPLIT, bool FULL, int U, bool ONE>
__global__ __launch_bounds__(64 * (U / 16) * (GS_T / 16) * SPLIT, SPLIT == 2 && U == 32 ? 4 : 1)
void k_gemm_small(GemmArgs a) {
    constexpr int NWP = (U / 16) * (GS_T / 16), NTP = 64 * NWP;   // waves, threads per pipeline
    constexpr int P = gs_ring(SPLIT, U);
    constexpr int WB = DT == DT_Q8 ? 32 : 16;                 // weight bytes per row and block
    constexpr int WROW = GS_KB * WB, XROW = GS_KB * 32;        // stage bytes per row
    constexpr int WP = WROW + 16, XP = XROW + 16;              // LDS row pitches
    constexpr int WCH = U * WROW / 16, XCH = GS_T * XROW / 16; // 16-byte chunks per stage
    constexpr int XPT = XCH / NTP;                             // X chunks per thread and stage
    constexpr int NSW = GS_KB * U, NSX = GS_KB * GS_T;         // weight / token scales per stage
    static_assert(WCH <= NTP && XCH % NTP == 0 && NSW <= NTP && NSX <= NTP, "chunks and scales per thread");
    __shared__ __align__(16) uint8_t ws[SPLIT][2][U * WP];
    __shared__ __align__(16) int8_t xsm[SPLIT][2][GS_T * XP];
    __shared__ __align__(16) float dws[SPLIT][2][GS_KB][U], dxs[SPLIT][2][GS_KB][GS_T];
    __shared__ int sxs[SPLIT][2][GS_KB][GS_T];
    __shared__ __align__(16) float red[SPLIT > 1 ? SPLIT - 1 : 1][NWP][64][4];
    const int tid = threadIdx.x % NTP, q = threadIdx.x / NTP;   // thread of pipeline q
    const int lane = tid & 63, wave = tid >> 6;
    const int fr = lane & 15, fg = lane >> 4;
    const int u0 = blockIdx.x * U, t0 = blockIdx.y * GS_T;
    const int K = a.W.cols, nb = K / QB;
    const int nbq = (nb + SPLIT - 1) / SPLIT, kb0 = q * nbq, kb1 = min(nb, kb0 + nbq);   // this pipeline's blocks
    const int nst = (nbq + GS_KB - 1) / GS_KB;                // stages, the same in every pipeline
    const int wu = U == 32 ? (wave & 1) * 16 : 0, wt = U == 32 ? (wave >> 1) * 16 : wave * 16;
    uint8_t (&wsq)[2][U * WP] = ws[q];
    int8_t (&xsq)[2][GS_T * XP] = xsm[q];
    float (&dwq)[2][GS_KB][U] = dws[q];
    float (&dxq)[2][GS_KB][GS_T] = dxs[q];
    int (&sxq)[2][GS_KB][GS_T] = sxs[q];
    // SPLIT > 1: the scales as fp16 bits (the first half of each array)
    uint16_t (&dwhq)[2][GS_KB][U] = *reinterpret_cast<uint16_t (*)[2][GS_KB][U]>(&dws[q][0][0][0]);
    uint16_t (&dxhq)[2][GS_KB][GS_T] = *reinterpret_cast<uint16_t (*)[2][GS_KB][GS_T]>(&dxs[q][0][0][0]);

    // the epilogue's residual (or bias) values: their loads go out first, so
    // the stores at the end do not wait for a round trip (not in the
    // two-pipeline 32-unit kernel, whose registers are spoken for)
    constexpr bool PRE = !(SPLIT == 2 && U == 32);
    const int to = t0 + wt + fr;
    float pre[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (PRE)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int u = min(u0 + wu + 4 * fg + r, a.units - 1);
            if (EPI == EPI_RESID) pre[r] = a.out[(size_t)min(to, a.n - 1) * a.out_stride + u];
            else pre[r] = a.bias ? a.bias[u] : 0.0f;
        }

    // register ring: slot j holds a stage s with s % P == j
    i32x4 wr[P], xr[P][XPT];
    uint16_t dwr[P];
    float dxr[P];
    int xsr[P];
    // FULL: this thread's first-stage addresses; stage st adds st * GS_KB blocks
    // ONE: threads past the last W chunk or scale repeat the last one (the
    // same value to the same LDS word), so neither a load nor a store is
    // conditional: the compiler would otherwise move a load next to its
    // conditional store and wait for it there.  The looped form (whose header
    // waits for every load anyway) skips them.
    const bool ldw = ONE || tid < WCH, lsw = ONE || tid < NSW, lsx = ONE || tid < NSX;
    const int wch = min(tid, WCH - 1);
    const int wrow = wch / (WROW / 16), wc = (wch % (WROW / 16)) * 16;
    const int skw = min(tid, NSW - 1) / U, srw = min(tid, NSW - 1) % U;
    const int skx = min(tid, NSX - 1) / GS_T, srx = min(tid, NSX - 1) % GS_T;
    // (the pipeline's base is uniform; the thread's part is a 32-bit offset,
    // one register instead of a 64-bit address per stream)
    const uint32_t wo0 = (uint32_t)(min(u0 + wrow, a.units - 1) * (nb * WB) + wc);
    uint32_t xo0[XPT];
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int c = tid + i * NTP, xrow = c / (XROW / 16), xc = (c % (XROW / 16)) * 16;
        xo0[i] = (uint32_t)(min(t0 + xrow, a.n - 1) * K + xc);
    }
    const uint32_t dwo0 = (uint32_t)(min(u0 + srw, a.units - 1) * nb + skw);
    const uint32_t dxo0 = (uint32_t)(min(t0 + srx, a.n - 1) * nb + skx);
    auto load = [&](int j, int st) {
        if constexpr (FULL) {
            const int b0 = kb0 + st * GS_KB;
            if (ldw) wr[j] = *reinterpret_cast<const i32x4 *>(a.W.q + (size_t)b0 * WB + wo0);
#pragma unroll
            for (int i = 0; i < XPT; i++) xr[j][i] = *reinterpret_cast<const i32x4 *>(a.qx + (size_t)b0 * 32 + xo0[i]);
            if (lsw) dwr[j] = (a.W.d + b0)[dwo0];
            if (lsx) {
                dxr[j] = (a.dx + b0)[dxo0];
                if (DT == DT_Q4) xsr[j] = (a.xs + b0)[dxo0];
            }
            return;
        }
        const int b0 = kb0 + st * GS_KB;
        if (ldw) {
            const int u = min(u0 + wrow, a.units - 1), blk = min(b0 + wc / WB, nb - 1);
            wr[j] = *reinterpret_cast<const i32x4 *>(a.W.q + (size_t)u * (nb * WB) + (size_t)blk * WB + wc % WB);
        }
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int cc = tid + i * NTP, row = cc / (XROW / 16), c = (cc % (XROW / 16)) * 16;
            const int t = min(t0 + row, a.n - 1), blk = min(b0 + c / 32, nb - 1);
            xr[j][i] = *reinterpret_cast<const i32x4 *>(a.qx + (size_t)t * K + (size_t)blk * 32 + c % 32);
        }
        if (lsw) dwr[j] = a.W.d[(size_t)min(u0 + srw, a.units - 1) * nb + min(b0 + skw, nb - 1)];
        if (lsx) {
            const int t = min(t0 + srx, a.n - 1), blk = min(b0 + skx, nb - 1);
            dxr[j] = a.dx[(size_t)t * nb + blk];
            if (DT == DT_Q4) xsr[j] = a.xs[(size_t)t * nb + blk];
        }
    };
    auto store = [&](int j, int buf) {
        if (ldw) *reinterpret_cast<i32x4 *>(wsq[buf] + wrow * WP + wc) = wr[j];
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int c = tid + i * NTP;
            *reinterpret_cast<i32x4 *>(xsq[buf] + (c / (XROW / 16)) * XP + (c % (XROW / 16)) * 16) = xr[j][i];
        }
        if (lsw) {
            if constexpr (SPLIT > 1) dwhq[buf][skw][srw] = dwr[j];
            else dwq[buf][skw][srw] = h2f(dwr[j]);
        }
        if (lsx) {
            // activation scales are fp16 values held as fp32: exact both ways
            if constexpr (SPLIT > 1) dxhq[buf][skx][srx] = f2h(dxr[j]);
            else dxq[buf][skx][srx] = dxr[j];
            if (DT == DT_Q4) sxq[buf][skx][srx] = xsr[j];
        }
    };

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // one stage: its registers to LDS, the ring's next load, its fragments
    // and scales, then its products, then the epilogues in block order
    // (blocks past the pipeline's end contribute nothing)
    auto stage = [&](int j, int st, bool refill) {
        const int buf = st & 1;
        // every wave has finished the stage that last used this buffer
        store(j, buf);
        __syncthreads();
        if (refill && st + P - 1 < nst) load((j + P - 1) % P, st + P - 1);
        const int nkb = FULL ? GS_KB : min(GS_KB, kb1 - (kb0 + st * GS_KB));
        long af[GS_KB], bf[GS_KB];
        float dx[GS_KB];
        f32x4 dw[GS_KB];
        f16x4 sa[GS_KB], sb[GS_KB];
        int xsum[GS_KB];
#pragma unroll
        for (int kb = 0; kb < GS_KB; kb++) {
            const uint8_t *wp = wsq[buf] + (wu + fr) * WP + kb * WB;
            if (DT == DT_Q8) {
                af[kb] = *reinterpret_cast<const long *>(wp + 8 * fg);
            } else {   // nibbles: low = weights 0..15, high = 16..31 of the block
                const unsigned long long raw = *reinterpret_cast<const unsigned long long *>(wp + 8 * (fg & 1));
                af[kb] = (long)((raw >> (4 * (fg >> 1))) & 0x0f0f0f0f0f0f0f0full);
            }
            bf[kb] = *reinterpret_cast<const long *>(xsq[buf] + (wt + fr) * XP + kb * 32 + 8 * fg);
            if constexpr (SPLIT > 1) {
                // the scale products as a 16 x 16 x 16 fp16 outer product
                // (k_gemm_mfma's FUSED form): weight scale of row wu + fr and
                // token scale of column wt + fr in element 0 of lanes 0..15
                sa[kb] = f16x4{};
                sb[kb] = f16x4{};
                sa[kb][0] = __builtin_bit_cast(_Float16, (uint16_t)(fg ? 0 : dwhq[buf][kb][wu + fr]));
                sb[kb][0] = __builtin_bit_cast(_Float16, (uint16_t)(fg ? 0 : dxhq[buf][kb][wt + fr]));
            } else {
                dx[kb] = dxq[buf][kb][wt + fr];
                dw[kb] = *reinterpret_cast<const f32x4 *>(&dwq[buf][kb][wu + 4 * fg]);
            }
            xsum[kb] = DT == DT_Q4 ? sxq[buf][kb][wt + fr] : 0;
        }
        i32x4 d[GS_KB];
#pragma unroll
        for (int kb = 0; kb < GS_KB; kb++)
            d[kb] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af[kb], bf[kb], i32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int kb = 0; kb < GS_KB; kb++) {
            if (kb >= nkb) break;
            if constexpr (SPLIT > 1) {
                const f32x4 sc = __builtin_amdgcn_mfma_f32_16x16x16f16(sa[kb], sb[kb], f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int isum = DT == DT_Q4 ? d[kb][r] - 8 * xsum[kb] : d[kb][r];
                    acc[r] = fmaf((float)isum, sc[r], acc[r]);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int isum = DT == DT_Q4 ? d[kb][r] - 8 * xsum[kb] : d[kb][r];
                    acc[r] += ((float)isum * dw[kb][r]) * dx[kb];
                }
            }
        }
    };
    if constexpr (ONE) {
        // every stage in flight from the start; stages past the last one
        // reload it (nothing reads them), so no load is conditional and the
        // compiler's waits count exactly the loads issued after the stage
        // being stored
#pragma unroll
        for (int j = 0; j < P; j++) load(j, min(j, nst - 1));
#pragma unroll
        for (int j = 0; j < P; j++) {
            if (j >= nst) break;
            stage(j, j, false);
        }
    } else {
#pragma unroll
        for (int j = 0; j < P - 1; j++) load(j, j);
        for (int s0 = 0; s0 < nst; s0 += P) {
#pragma unroll
            for (int j = 0; j < P; j++) {
                const int st = s0 + j;
                if (st >= nst) break;
                stage(j, st, true);
            }
        }
    }
    if constexpr (SPLIT > 1) {   // the pipelines' sums, added in pipeline order
        if (q > 0)
#pragma unroll
            for (int r = 0; r < 4; r++) red[q - 1][wave][lane][r] = acc[r];
        __syncthreads();
        if (q > 0) return;
#pragma unroll
        for (int p = 0; p < SPLIT - 1; p++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[r] += red[p][wave][lane][r];
    }
    if (to >= a.n) return;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int u = u0 + wu + 4 * fg + r;
        if (u >= a.units) continue;
        float *o = a.out + (size_t)to * a.out_stride + u;
        if (EPI == EPI_STORE) *o = a.bias ? acc[r] + (PRE ? pre[r] : a.bias[u]) : acc[r];
        else *o = (PRE ? pre[r] : *o) + acc[r];
    }
}

// k_gemm_swq: the w1|w3 product of a short prompt with the SwiGLU and the
// Q8_0 quantization of its rows in the epilogue (replacing k_quant_rows's
// SwiGLU pass and its launch).  A workgroup takes SW_U = 32 hidden units
// (their 32 gate and 32 up weight rows) x SW_T = 16 tokens, so each token's
// 32 SwiGLU values of the tile are one Q8_0 block; wave w computes the 16 x 16
// tile of rows 32 (w / 2) + 16 (w % 2) with the stage machinery of
// k_gemm_small's straight-line form (every stage in flight from the start;
// SPLIT pipelines over K added in pipeline order).  The gate and up sums meet
// in LDS; then eight lanes per token apply g / (1 + expf(-g)) * u
// (model.c:403-406) and quantize the block with k_quant_rows's arithmetic.
constexpr int SW_U = 32, SW_T = 16;
__host__ __device__ constexpr int sw_ring(int split) { return split > 1 ? 4 : 8; }
template <int DT, int SPLIT, bool FULL>
__global__ __launch_bounds__(256 * SPLIT, SPLIT == 2 ? 4 : 1) void k_gemm_swq(GemmArgs a) {
    constexpr int NTP = 256, P = sw_ring(SPLIT), RW = 2 * SW_U;   // threads per pipeline, ring, weight rows
    constexpr int WB = DT == DT_Q8 ? 32 : 16;
    constexpr int WROW = GS_KB * WB, XROW = GS_KB * 32, WP = WROW + 16, XP = XROW + 16;
    constexpr int WCH = RW * WROW / 16, WPT = (WCH + NTP - 1) / NTP;   // weight chunks (per thread)
    constexpr int XCH = SW_T * XROW / 16;                      // token chunks (threads past them repeat the last)
    constexpr int NSW = GS_KB * RW, NSX = GS_KB * SW_T;        // weight / token scales per stage
    static_assert(WCH % NTP == 0 || WCH < NTP, "weight chunks per thread");
    static_assert(XCH <= NTP && NSW <= NTP && NSX <= NTP, "one token chunk and scale per thread");
    __shared__ __align__(16) uint8_t ws[SPLIT][2][RW * WP];
    __shared__ __align__(16) int8_t xsm[SPLIT][2][SW_T * XP];
    __shared__ __align__(16) float dws[SPLIT][2][GS_KB][RW], dxs[SPLIT][2][GS_KB][SW_T];
    __shared__ int sxs[SPLIT][2][GS_KB][SW_T];
    __shared__ __align__(16) float red[SPLIT > 1 ? SPLIT - 1 : 1][4][64][4];
    __shared__ float hs[SW_T][RW + 1];                         // [token][gate 0..31 | up 32..63]
    const int tid = threadIdx.x % NTP, q = threadIdx.x / NTP;
    const int lane = tid & 63, wave = tid >> 6, fr = lane & 15, fg = lane >> 4;
    const int wr0 = (wave >> 1) * SW_U + (wave & 1) * 16;     // the wave's first tile row
    const int u0 = blockIdx.x * SW_U, t0 = blockIdx.y * SW_T;
    const int K = a.W.cols, nb = K / QB;
    const int nbq = (nb + SPLIT - 1) / SPLIT, kb0 = q * nbq, kb1 = min(nb, kb0 + nbq);
    const int nst = (nbq + GS_KB - 1) / GS_KB;                // <= P (checked by the launcher)
    uint8_t (&wsq)[2][RW * WP] = ws[q];
    int8_t (&xsq)[2][SW_T * XP] = xsm[q];
    float (&dwq)[2][GS_KB][RW] = dws[q];
    float (&dxq)[2][GS_KB][SW_T] = dxs[q];
    int (&sxq)[2][GS_KB][SW_T] = sxs[q];
    // weight row of tile row r: gate rows u0.., then up rows pair_off + u0..
    auto wrow_of = [&](int r) { return (r < SW_U ? 0 : a.pair_off) + min(u0 + r % SW_U, a.units - 1); };

    i32x4 wr[P][WPT], xr[P];
    uint16_t dwr[P];
    float dxr[P];
    int xsr[P];
    // every load and store is unconditional: threads past the last chunk or
    // scale repeat it (the same value to the same LDS word)
    int wrow[WPT], wc[WPT];
#pragma unroll
    for (int i = 0; i < WPT; i++) {
        const int c = min(tid + i * NTP, WCH - 1);
        wrow[i] = c / (WROW / 16);
        wc[i] = (c % (WROW / 16)) * 16;
    }
    const int xcn = min(tid, XCH - 1), xrow = xcn / (XROW / 16), xc = (xcn % (XROW / 16)) * 16;
    const int skw = min(tid, NSW - 1) / RW, srw = min(tid, NSW - 1) % RW;
    const int skx = min(tid, NSX - 1) / SW_T, srx = min(tid, NSX - 1) % SW_T;
    auto load = [&](int j, int st) {
        const int b0 = kb0 + st * GS_KB;
#pragma unroll
        for (int i = 0; i < WPT; i++) {
            const int blk = FULL ? b0 + wc[i] / WB : min(b0 + wc[i] / WB, nb - 1);
            wr[j][i] = *reinterpret_cast<const i32x4 *>(a.W.q + (size_t)wrow_of(wrow[i]) * (nb * WB) +
                                                        (size_t)blk * WB + wc[i] % WB);
        }
        {
            const int t = min(t0 + xrow, a.n - 1), blk = FULL ? b0 + xc / 32 : min(b0 + xc / 32, nb - 1);
            xr[j] = *reinterpret_cast<const i32x4 *>(a.qx + (size_t)t * K + (size_t)blk * 32 + xc % 32);
        }
        dwr[j] = a.W.d[(size_t)wrow_of(srw) * nb + (FULL ? b0 + skw : min(b0 + skw, nb - 1))];
        {
            const int t = min(t0 + srx, a.n - 1), blk = FULL ? b0 + skx : min(b0 + skx, nb - 1);
            dxr[j] = a.dx[(size_t)t * nb + blk];
            if (DT == DT_Q4) xsr[j] = a.xs[(size_t)t * nb + blk];
        }
    };
    auto store = [&](int j, int buf) {
#pragma unroll
        for (int i = 0; i < WPT; i++) *reinterpret_cast<i32x4 *>(wsq[buf] + wrow[i] * WP + wc[i]) = wr[j][i];
        *reinterpret_cast<i32x4 *>(xsq[buf] + xrow * XP + xc) = xr[j];
        dwq[buf][skw][srw] = h2f(dwr[j]);
        dxq[buf][skx][srx] = dxr[j];
        if (DT == DT_Q4) sxq[buf][skx][srx] = xsr[j];
    };
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < P; j++) load(j, min(j, nst - 1));
#pragma unroll
    for (int j = 0; j < P; j++) {
        if (j >= nst) break;
        const int buf = j & 1;
        store(j, buf);
        __syncthreads();
        const int nkb = FULL ? GS_KB : min(GS_KB, kb1 - (kb0 + j * GS_KB));
        long af[GS_KB], bf[GS_KB];
        float dx[GS_KB];
        f32x4 dw[GS_KB];
        int xsum[GS_KB];
#pragma unroll
        for (int kb = 0; kb < GS_KB; kb++) {
            const uint8_t *wp = wsq[buf] + (wr0 + fr) * WP + kb * WB;
            if (DT == DT_Q8) {
                af[kb] = *reinterpret_cast<const long *>(wp + 8 * fg);
            } else {   // nibbles: low = weights 0..15, high = 16..31 of the block
                const unsigned long long raw = *reinterpret_cast<const unsigned long long *>(wp + 8 * (fg & 1));
                af[kb] = (long)((raw >> (4 * (fg >> 1))) & 0x0f0f0f0f0f0f0f0full);
            }
            bf[kb] = *reinterpret_cast<const long *>(xsq[buf] + fr * XP + kb * 32 + 8 * fg);
            dx[kb] = dxq[buf][kb][fr];
            dw[kb] = *reinterpret_cast<const f32x4 *>(&dwq[buf][kb][wr0 + 4 * fg]);
            xsum[kb] = DT == DT_Q4 ? sxq[buf][kb][fr] : 0;
        }
        i32x4 d[GS_KB];
#pragma unroll
        for (int kb = 0; kb < GS_KB; kb++)
            d[kb] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af[kb], bf[kb], i32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int kb = 0; kb < GS_KB; kb++) {
            if (kb >= nkb) break;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int isum = DT == DT_Q4 ? d[kb][r] - 8 * xsum[kb] : d[kb][r];
                acc[r] += ((float)isum * dw[kb][r]) * dx[kb];
            }
        }
    }
    if constexpr (SPLIT > 1) {   // the pipelines' sums, added in pipeline order
        if (q > 0)
#pragma unroll
            for (int r = 0; r < 4; r++) red[q - 1][wave][lane][r] = acc[r];
        __syncthreads();
        if (q == 0)
#pragma unroll
            for (int p = 0; p < SPLIT - 1; p++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[r] += red[p][wave][lane][r];
    }
    if (q == 0) {
#pragma unroll
        for (int r = 0; r < 4; r++) hs[fr][wr0 + 4 * fg + r] = acc[r];
        if (a.out && t0 + fr < a.n)   // the gate | up products themselves, where asked for
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int tr = wr0 + 4 * fg + r, u = u0 + tr % SW_U;
                if (u < a.units) a.out[(size_t)(t0 + fr) * a.out_stride + (tr < SW_U ? 0 : a.pair_off) + u] = acc[r];
            }
    }
    __syncthreads();
    if (q > 0 || tid >= SW_T * 8) return;
    // token tid / 8, hidden units 4 (tid % 8) .. + 3 of the tile
    const int tt = tid >> 3, hp = (tid & 7) * 4;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float g = hs[tt][hp + i], u = hs[tt][SW_U + hp + i];
        v[i] = g / (1.0f + expf(-g)) * u;
    }
    const float mx = max8(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    const float dq = mx / 127.0f;
    const float id = dq > 0.0f ? 1.0f / dq : 0.0f;
    int c[4];
#pragma unroll
    for (int i = 0; i < 4; i++) c[i] = (int)fminf(fmaxf(roundf(v[i] * id), -127.0f), 127.0f);
    const int cs = sum8(c[0] + c[1] + c[2] + c[3]);
    const int t = t0 + tt;
    if (t >= a.n || u0 + hp >= a.units) return;
    const int nbo = a.units / QB;
    *reinterpret_cast<uint32_t *>(a.oq + (size_t)t * a.units + u0 + hp) =
        ((uint32_t)c[0] & 0xffu) | (((uint32_t)c[1] & 0xffu) << 8) | (((uint32_t)c[2] & 0xffu) << 16) |
        (((uint32_t)c[3] & 0xffu) << 24);
    if (hp == 0) {
        a.odx[(size_t)t * nbo + u0 / QB] = h2f(f2h(dq));
        a.oxs[(size_t)t * nbo + u0 / QB] = cs;
    }
}

// One key's K rows in its 64-key tile image for k_pf_flash16 (k_pf_kvsplit's
// layout, flimg.h), for k_gemm_qkv's wave-per-token epilogue: lane l holds
// dims l + 64 k of the key's cache values v[k]; ex is the key's power-of-two
// scale (fp32 cache: from its largest |value|).
template <int HD, bool F16>
__device__ __forceinline__ void qkv_key_image(uint8_t *im, const float *v, int kl, int ex, int lane) {
    using I = FlImg<HD, F16>;
    const int rk = fl_krow(kl);
#pragma unroll
    for (int k = 0; k < HD / 64; k++) {
        const int d = lane + 64 * k;
        const float x = F16 ? v[k] : __builtin_amdgcn_ldexpf(v[k], ex);
        const _Float16 hi = (_Float16)x, lo = (_Float16)(x - (float)hi);
        *reinterpret_cast<uint16_t *>(im + I::k_at(rk, d >> 3) + 2 * (d & 7)) = __builtin_bit_cast(uint16_t, hi);
        if constexpr (!F16)
            *reinterpret_cast<uint16_t *>(im + I::k_at(FL_BK + rk, d >> 3) + 2 * (d & 7)) = __builtin_bit_cast(uint16_t, lo);
    }
    if (!F16 && lane == 0) reinterpret_cast<int *>(im + I::KBYTES)[kl] = ex;
}
// A k head's key at position pos and, when it is the pass's last, the rest
// of its tile (k_pf_kvsplit repeats the last key there).
template <int HD, bool F16>
__device__ __forceinline__ void qkv_tile_image(const QkPostArgs &p, int g, const float *v, int pos, bool last,
                                               int lane) {
    using I = FlImg<HD, F16>;
    uint8_t *im = p.kvimg + ((size_t)g * p.kvimg_tiles + pos / FL_BK) * I::HBYTES;
    int ex = 0;
    if constexpr (!F16) {
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < HD / 64; k++) m = fmaxf(m, fabsf(v[k]));
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        ex = fl_exp(m);
    }
    qkv_key_image<HD, F16>(im, v, pos % FL_BK, ex, lane);
    if (last)
        for (int kp = pos % FL_BK + 1; kp < FL_BK; kp++) qkv_key_image<HD, F16>(im, v, kp, ex, lane);
}

// k_gemm_qkv: the q|k|v product of a short prompt with k_qkpost's work in
// the epilogue (replacing that kernel and its launch).  A workgroup takes one
// head vector (HD units: a q, k or v head) x QV_T = 16 tokens, wave w the
// 16 x 16 tile of units 16 w, with the stage machinery of k_gemm_small's
// straight-line form.  The tile (with the bias) meets in LDS; then a wave
// per token does what k_qkpost does for it, with the same lane layout (lane
// l holds elements l, l + 64) and so the same sums: the RMSNorm of q and k
// heads (model.c:386-389), RoPE from the host table (model.c:66-80), q back
// into its q|k|v row, k and v into the cache (model.c:39-48); with
// p.kvimg also the keys' bytes in the K/V tile images of the matrix-core
// attention (qkv_tile_image).
constexpr int QV_T = 16;
__host__ __device__ constexpr int qv_ring(int split) { return split > 1 ? 4 : 8; }
template <int DT, int SPLIT, bool FULL, int HD, bool F16>
__global__ __launch_bounds__(64 * (HD / 16) * SPLIT) void k_gemm_qkv(GemmArgs a, QkPostArgs p, float *raw) {
    constexpr int NWP = HD / 16, NTP = 64 * NWP, P = qv_ring(SPLIT);
    constexpr int WB = DT == DT_Q8 ? 32 : 16;
    constexpr int WROW = GS_KB * WB, XROW = GS_KB * 32, WP = WROW + 16, XP = XROW + 16;
    constexpr int WCH = HD * WROW / 16, WPT = (WCH + NTP - 1) / NTP;
    constexpr int XCH = QV_T * XROW / 16;
    constexpr int NSW = GS_KB * HD, NSX = GS_KB * QV_T;
    constexpr int ND = HD / 64, TPW = QV_T / NWP;             // elements per lane, tokens per wave
    static_assert(WCH % NTP == 0 || WCH < NTP, "weight chunks per thread");
    static_assert(XCH <= NTP && NSW <= NTP && NSX <= NTP && HD % 64 == 0, "one token chunk and scale per thread");
    __shared__ __align__(16) uint8_t ws[SPLIT][2][HD * WP];
    __shared__ __align__(16) int8_t xsm[SPLIT][2][QV_T * XP];
    __shared__ __align__(16) float dws[SPLIT][2][GS_KB][HD], dxs[SPLIT][2][GS_KB][QV_T];
    __shared__ int sxs[SPLIT][2][GS_KB][QV_T];
    __shared__ __align__(16) float red[SPLIT > 1 ? SPLIT - 1 : 1][NWP][64][4];
    __shared__ float hs[QV_T][HD + 1];
    __shared__ int exs[QV_T];   // (p.kvimg, fp32 cache) the v head's per-key scales
    const int tid = threadIdx.x % NTP, q = threadIdx.x / NTP;
    const int lane = tid & 63, wave = tid >> 6, fr = lane & 15, fg = lane >> 4;
    const int vh = blockIdx.x, u0 = vh * HD, t0 = blockIdx.y * QV_T, wu = wave * 16;
    const int K = a.W.cols, nb = K / QB;
    const int nbq = (nb + SPLIT - 1) / SPLIT, kb0 = q * nbq, kb1 = min(nb, kb0 + nbq);
    const int nst = (nbq + GS_KB - 1) / GS_KB;                // <= P (checked by the launcher)
    uint8_t (&wsq)[2][HD * WP] = ws[q];
    int8_t (&xsq)[2][QV_T * XP] = xsm[q];
    float (&dwq)[2][GS_KB][HD] = dws[q];
    float (&dxq)[2][GS_KB][QV_T] = dxs[q];
    int (&sxq)[2][GS_KB][QV_T] = sxs[q];

    // the epilogue's per-head inputs, loaded first: head kind, norm weights,
    // bias and the RoPE rows of the wave's tokens
    const bool isq = vh < p.n_heads, isk = !isq && vh < p.n_heads + p.n_kv;
    const int g = vh - p.n_heads - (isk || isq ? 0 : p.n_kv);  // kv head of a k or v head
    const bool neox = p.rope_style == ROPE_NEOX;
    const float *nwp = isq ? p.q_norm : p.k_norm;
    float nwv[ND];
    float2 cs[TPW][ND];
#pragma unroll
    for (int k = 0; k < ND; k++) {
        const int d = lane + 64 * k, i = neox ? d % (HD / 2) : d / 2;
        nwv[k] = p.q_norm && (isq || isk) ? nwp[d] : 1.0f;
#pragma unroll
        for (int j = 0; j < TPW; j++) {
            const int t = min(t0 + wave * TPW + j, a.n - 1);
            cs[j][k] = p.rope[(size_t)(p.pos_base + t) * (HD / 2) + i];
        }
    }
    float bias[4];
#pragma unroll
    for (int r = 0; r < 4; r++) bias[r] = a.bias ? a.bias[u0 + wu + 4 * fg + r] : 0.0f;

    i32x4 wr[P][WPT], xr[P];
    uint16_t dwr[P];
    float dxr[P];
    int xsr[P];
    // every load and store is unconditional: threads past the last chunk or
    // scale repeat it (the same value to the same LDS word)
    int wrow[WPT], wc[WPT];
#pragma unroll
    for (int i = 0; i < WPT; i++) {
        const int c = min(tid + i * NTP, WCH - 1);
        wrow[i] = c / (WROW / 16);
        wc[i] = (c % (WROW / 16)) * 16;
    }
    const int xcn = min(tid, XCH - 1), xrow = xcn / (XROW / 16), xc = (xcn % (XROW / 16)) * 16;
    const int skw = min(tid, NSW - 1) / HD, srw = min(tid, NSW - 1) % HD;
    const int skx = min(tid, NSX - 1) / QV_T, srx = min(tid, NSX - 1) % QV_T;
    auto load = [&](int j, int st) {
        const int b0 = kb0 + st * GS_KB;
#pragma unroll
        for (int i = 0; i < WPT; i++) {
            const int blk = FULL ? b0 + wc[i] / WB : min(b0 + wc[i] / WB, nb - 1);
            wr[j][i] = *reinterpret_cast<const i32x4 *>(a.W.q + (size_t)(u0 + wrow[i]) * (nb * WB) +
                                                        (size_t)blk * WB + wc[i] % WB);
        }
        {
            const int t = min(t0 + xrow, a.n - 1), blk = FULL ? b0 + xc / 32 : min(b0 + xc / 32, nb - 1);
            xr[j] = *reinterpret_cast<const i32x4 *>(a.qx + (size_t)t * K + (size_t)blk * 32 + xc % 32);
        }
        dwr[j] = a.W.d[(size_t)(u0 + srw) * nb + (FULL ? b0 + skw : min(b0 + skw, nb - 1))];
        {
            const int t = min(t0 + srx, a.n - 1), blk = FULL ? b0 + skx : min(b0 + skx, nb - 1);
            dxr[j] = a.dx[(size_t)t * nb + blk];
            if (DT == DT_Q4) xsr[j] = a.xs[(size_t)t * nb + blk];
        }
    };
    auto store = [&](int j, int buf) {
#pragma unroll
        for (int i = 0; i < WPT; i++) *reinterpret_cast<i32x4 *>(wsq[buf] + wrow[i] * WP + wc[i]) = wr[j][i];
        *reinterpret_cast<i32x4 *>(xsq[buf] + xrow * XP + xc) = xr[j];
        dwq[buf][skw][srw] = h2f(dwr[j]);
        dxq[buf][skx][srx] = dxr[j];
        if (DT == DT_Q4) sxq[buf][skx][srx] = xsr[j];
    };
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < P; j++) load(j, min(j, nst - 1));
#pragma unroll
    for (int j = 0; j < P; j++) {
        if (j >= nst) break;
        const int buf = j & 1;
        store(j, buf);
        __syncthreads();
        const int nkb = FULL ? GS_KB : min(GS_KB, kb1 - (kb0 + j * GS_KB));
        long af[GS_KB], bf[GS_KB];
        float dx[GS_KB];
        f32x4 dw[GS_KB];
        int xsum[GS_KB];
#pragma unroll
        for (int kb = 0; kb < GS_KB; kb++) {
            const uint8_t *wp = wsq[buf] + (wu + fr) * WP + kb * WB;
            if (DT == DT_Q8) {
                af[kb] = *reinterpret_cast<const long *>(wp + 8 * fg);
            } else {   // nibbles: low = weights 0..15, high = 16..31 of the block
                const unsigned long long rw = *reinterpret_cast<const unsigned long long *>(wp + 8 * (fg & 1));
                af[kb] = (long)((rw >> (4 * (fg >> 1))) & 0x0f0f0f0f0f0f0f0full);
            }
            bf[kb] = *reinterpret_cast<const long *>(xsq[buf] + fr * XP + kb * 32 + 8 * fg);
            dx[kb] = dxq[buf][kb][fr];
            dw[kb] = *reinterpret_cast<const f32x4 *>(&dwq[buf][kb][wu + 4 * fg]);
            xsum[kb] = DT == DT_Q4 ? sxq[buf][kb][fr] : 0;
        }
        i32x4 d[GS_KB];
#pragma unroll
        for (int kb = 0; kb < GS_KB; kb++)
            d[kb] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af[kb], bf[kb], i32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int kb = 0; kb < GS_KB; kb++) {
            if (kb >= nkb) break;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int isum = DT == DT_Q4 ? d[kb][r] - 8 * xsum[kb] : d[kb][r];
                acc[r] += ((float)isum * dw[kb][r]) * dx[kb];
            }
        }
    }
    if constexpr (SPLIT > 1) {   // the pipelines' sums, added in pipeline order
        if (q > 0)
#pragma unroll
            for (int r = 0; r < 4; r++) red[q - 1][wave][lane][r] = acc[r];
        __syncthreads();
        if (q == 0)
#pragma unroll
            for (int s2 = 0; s2 < SPLIT - 1; s2++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[r] += red[s2][wave][lane][r];
    }
    if (q == 0) {   // the product with its bias (EPI_STORE's order: sum, then + bias)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float v = a.bias ? acc[r] + bias[r] : acc[r];
            hs[fr][wu + 4 * fg + r] = v;
            if (raw && t0 + fr < a.n) raw[(size_t)(t0 + fr) * p.stride + u0 + wu + 4 * fg + r] = v;
        }
    }
    __syncthreads();
    // a v head writing the tile image keeps every wave for the transposed
    // V rows at the end (a barrier)
    const bool vimg = p.kvimg && !isq && !isk;
    if (q > 0 && !vimg) return;
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        if (q > 0) break;
        const int tt = wave * TPW + j, t = t0 + tt;              // uniform over the wave
        if (t >= a.n) break;
        const int pos = p.pos_base + t;
        float x[ND];
#pragma unroll
        for (int k = 0; k < ND; k++) x[k] = hs[tt][lane + 64 * k];
        if (!isq && !isk) {   // a v head: to the cache as it is
            const size_t off = (size_t)pos * p.kv_dim + (size_t)g * HD;
#pragma unroll
            for (int k = 0; k < ND; k++) {
                if (F16) reinterpret_cast<uint16_t *>(p.vc)[off + lane + 64 * k] = f2h(x[k]);
                else reinterpret_cast<float *>(p.vc)[off + lane + 64 * k] = x[k];
            }
            if (vimg && !F16) {   // the key's scale from its largest |value|
                float m = 0.0f;
#pragma unroll
                for (int k = 0; k < ND; k++) m = fmaxf(m, fabsf(x[k]));
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
                if (lane == 0) exs[tt] = fl_exp(m);
            }
            continue;
        }
        if (p.q_norm) {   // RMSNorm of the head vector (model.c:50-55)
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < ND; k++) ss += x[k] * x[k];
            ss = wave_sum(ss);
            const float scale = 1.0f / sqrtf(ss / (float)HD + p.eps);
#pragma unroll
            for (int k = 0; k < ND; k++) x[k] = x[k] * scale * nwv[k];
        }
        // RoPE: the first element of a pair becomes v0 * cos - v1 * sin, the
        // second v0 * sin + v1 * cos
        float y[ND];
#pragma unroll
        for (int k = 0; k < ND; k++) {
            const int d = lane + 64 * k;
            const bool first = neox ? d < HD / 2 : (d & 1) == 0;
            float xp;
            if (HD == 128 && neox) xp = x[k ^ 1];
            else xp = __shfl(x[k], (neox ? (d < HD / 2 ? d + HD / 2 : d - HD / 2) : d ^ 1) % 64);
            y[k] = first ? x[k] * cs[j][k].x - xp * cs[j][k].y : xp * cs[j][k].y + x[k] * cs[j][k].x;
        }
        if (isq) {
#pragma unroll
            for (int k = 0; k < ND; k++) p.qkv[(size_t)t * p.stride + u0 + lane + 64 * k] = y[k];
        } else {
            const size_t off = (size_t)pos * p.kv_dim + (size_t)g * HD;
#pragma unroll
            for (int k = 0; k < ND; k++) {
                if (F16) reinterpret_cast<uint16_t *>(p.kc)[off + lane + 64 * k] = f2h(y[k]);
                else reinterpret_cast<float *>(p.kc)[off + lane + 64 * k] = y[k];
            }
            if (p.kvimg) qkv_tile_image<HD, F16>(p, g, y, pos, t == a.n - 1, lane);
        }
    }
    if (vimg) {
        // V^T rows of the image (k_pf_kvsplit's bytes): 16-byte pieces of 8
        // keys for every dim, the workgroup's 16 keys and, in the workgroup
        // of the pass's last token, the rest of its tile (the last key
        // repeated), from the tile in LDS
        using I = FlImg<HD, F16>;
        __syncthreads();   // every key's scale in exs
        const int n_t = min(QV_T, a.n - t0), kl0 = (p.pos_base + t0) % FL_BK;
        const int pc0 = kl0 / 8, pc1 = t0 + QV_T >= a.n ? FL_BK / 8 : (kl0 + QV_T) / 8;
        uint8_t *im = p.kvimg + ((size_t)g * p.kvimg_tiles + (p.pos_base + t0) / FL_BK) * I::HBYTES;
        for (int w = threadIdx.x; w < HD * (pc1 - pc0); w += NTP * SPLIT) {
            const int d = w % HD, pc = pc0 + w / HD;
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                _Float16 hi[2], lo[2];
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const int tt = min(8 * pc + e + u - kl0, n_t - 1);
                    const float x = F16 ? hs[tt][d] : __builtin_amdgcn_ldexpf(hs[tt][d], exs[tt]);
                    hi[u] = (_Float16)x;
                    lo[u] = (_Float16)(x - (float)hi[u]);
                }
                hw[e / 2] = fl_pack(hi[0], hi[1]);
                lw[e / 2] = fl_pack(lo[0], lo[1]);
            }
            *reinterpret_cast<u32x4 *>(im + I::KE + I::v_at(d, pc)) = u32x4{hw[0], hw[1], hw[2], hw[3]};
            if constexpr (!F16) {
                *reinterpret_cast<u32x4 *>(im + I::KE + I::v_at(HD + d, pc)) = u32x4{lw[0], lw[1], lw[2], lw[3]};
                if (d == 0)
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        reinterpret_cast<int *>(im + I::KBYTES)[FL_BK + 8 * pc + e] = exs[min(8 * pc + e - kl0, n_t - 1)];
            }
        }
    }
}

// K of at least 1024 (32 blocks) splits into 4 pipelines when the grid fits
// the GPU at one 1024-thread workgroup per CU (the split's LDS); shorter K
// keeps the blocks of every output in one sequential sum, and a larger grid
// keeps 256-thread workgroups (two rounds of split workgroups measured
// slower: q|k|v 12.7 against 11.1 us, w1|w3 17.8 against 13.2 at 128 tokens)
constexpr int GS_SPLIT = 4, GS_SPLIT_MIN_BLOCKS = GEMM_SPLIT_MIN_K / QB, GS_SPLIT_MAX_GRID = 256;
// Grids of up to GS_SPLIT2_MAX_GRID workgroups split K in two (512-thread
// workgroups, two or three per CU): half the serial walk per output for two
// pipelines' instructions per SIMD.
constexpr int GS_SPLIT2_MAX_GRID = 1024;
// 32-unit grids of up to GS_U16_MAX_GRID workgroups (at most half the CUs)
// take 16-unit tiles instead.
constexpr int GS_U16_MAX_GRID = 128;

// k_gemm_mfma's tiles for gu 128-row tiles of units and n tokens: 64-token
// tiles while 128-token tiles give fewer than two workgroups per CU (the
// epilogue's dependent chains want the waves: Qwen3-0.6B-shape pp1024 6.64
// -> 6.23 ms; from 512 workgroups on the 128-token tiles are as fast or
// faster), and when they fill whole rounds of the GPU's workgroup slots where
// 128-token tiles would not: a 256-CU part holds 3 of those per CU (166
// VGPRs) and 4 of these (110), so a 4096-token q|k|v product (1,024 or 2,048
// workgroups) runs two full rounds of 64-token tiles instead of one and a
// third (pp4096 19.95 -> 19.55 ms).  Products over at least GEMM_SPLIT_MIN_K
// inputs take the fused block scaling (see k_gemm_mfma), and Q8_0 64-token
// grids of fewer than two workgroups per CU split K over two pipelines
// (Qwen3-0.6B shape: pp512 3.93 -> 3.78 ms, pp1024 5.85 -> 5.78; with the
// matrix-core scale products the 512-workgroup wo and w2 of pp4096 no
// longer gain from it, 15.68 -> 15.56 ms without, while pp2048's 256 still
// do, 8.11 -> 7.76 ms).
static void mfma_shape(long gu, int n, int cols, bool *t64, bool *fused, bool *sp2) {
    const long g128 = gu * ((n + 127) / 128), gt64 = gu * ((n + 63) / 64);
    auto fill = [](long g, long slots) { return (double)g / (double)(((g + slots - 1) / slots) * slots); };
    *t64 = g128 < 512 || fill(gt64, 4 * 256) > fill(g128, 3 * 256) + 0.1;
    *fused = cols >= GEMM_SPLIT_MIN_K;
    *sp2 = *fused && *t64 && gt64 < 2 * 256;
}

int launch_gemm(hipStream_t st, int epi, const GemmArgs &a) {
    if (a.W.cols % QB != 0 || a.n <= 0) return -1;
    if (a.W.dtype == DT_Q8 || a.W.dtype == DT_Q4) {
        // 128-token tiles unless that leaves fewer workgroups than CUs
        // (a 256-CU part); 64-token tiles then double the grid
        const int gu = (a.units + GM_U - 1) / GM_U;
        // 32 x 32 tiles for short prompts, and for the narrow (<= 1024-output)
        // wo / w2 products over fewer than GEMM_SPLIT_MIN_K inputs up to twice
        // that grid (at 2048 tokens +2% over the 64-token tiles below).  The
        // longer narrow products take the tiles below from 256 workgroups on:
        // with the fused block scaling's matrix-core scale products they are
        // faster there (Qwen3-0.6B shape, 2048 tokens: 55.6 -> 42.1 us per wo
        // or w2 product; 4096 tokens: pp4096 22.9 -> 21.2 ms)
        const long g64 = (long)gu * ((a.n + 63) / 64);
        if (g64 < 256 || (a.units <= 1024 && g64 < 512 && a.W.cols < GEMM_SPLIT_MIN_K)) {
            // 16-unit tiles when 32-unit ones would leave half the CUs idle
            const int ty = (a.n + GS_T - 1) / GS_T;
            const bool u16 = (long)((a.units + 31) / 32) * ty <= GS_U16_MAX_GRID;
            const dim3 gs((a.units + (u16 ? 15 : 31)) / (u16 ? 16 : 32), ty);
            const int nb = a.W.cols / QB;
            const bool split = nb >= GS_SPLIT_MIN_BLOCKS && (long)gs.x * gs.y <= GS_SPLIT_MAX_GRID;
            const bool split2 = !split && nb >= GS_SPLIT_MIN_BLOCKS && (long)gs.x * gs.y <= GS_SPLIT2_MAX_GRID;
            const int sp = split ? GS_SPLIT : split2 ? 2 : 1;
            const bool full = nb % (GS_KB * sp) == 0;
            const int nst = ((nb + sp - 1) / sp + GS_KB - 1) / GS_KB;   // stages per pipeline
            const bool one = nst <= gs_ring(sp, u16 ? 16 : 32);
#define GSK(DT, E, SP, FL, UU) \
            if (one) hipLaunchKernelGGL((k_gemm_small<DT, E, SP, FL, UU, true>), gs, dim3(UU * 8 * SP), 0, st, a); \
            else hipLaunchKernelGGL((k_gemm_small<DT, E, SP, FL, UU, false>), gs, dim3(UU * 8 * SP), 0, st, a);
#define GSL(DT, SP, FL, UU)                                                                              \
            if (epi == EPI_STORE) { GSK(DT, EPI_STORE, SP, FL, UU) }                                        \
            else if (epi == EPI_RESID) { GSK(DT, EPI_RESID, SP, FL, UU) }                                   \
            else return -1;                                                                              \
            return 0;
#define GSU(DT, SP, FL) if (u16) { GSL(DT, SP, FL, 16) } else { GSL(DT, SP, FL, 32) }
#define GSF(DT)                                                                                          \
            if (split) { if (full) { GSU(DT, GS_SPLIT, true) } else { GSU(DT, GS_SPLIT, false) } }      \
            if (split2) { if (full) { GSU(DT, 2, true) } else { GSU(DT, 2, false) } }                    \
            if (full) { GSU(DT, 1, true) } else { GSU(DT, 1, false) }
            if (a.W.dtype == DT_Q8) { GSF(DT_Q8) }
            GSF(DT_Q4)
#undef GSF
#undef GSU
#undef GSL
#undef GSK
        }
        bool t64, fused, sp2;   // (mfma_shape)
        mfma_shape(gu, a.n, a.W.cols, &t64, &fused, &sp2);
        dim3 g(gu, t64 ? (a.n + 63) / 64 : (a.n + 127) / 128);
#define GMK(DT, TT, FU, SP)                                                                             \
        if (epi == EPI_STORE) hipLaunchKernelGGL((k_gemm_mfma<DT, EPI_STORE, TT, 2, FU, SP>), g, dim3(WG * SP), 0, st, a, QkPostArgs{}); \
        else if (epi == EPI_RESID) hipLaunchKernelGGL((k_gemm_mfma<DT, EPI_RESID, TT, 2, FU, SP>), g, dim3(WG * SP), 0, st, a, QkPostArgs{}); \
        else return -1;                                                                                 \
        return 0;
#define GMF(DT, TT) if (fused) { GMK(DT, TT, true, 1) } else { GMK(DT, TT, false, 1) }
        if (a.W.dtype == DT_Q8 && sp2) { GMK(DT_Q8, 64, true, 2) }
        if (a.W.dtype == DT_Q8) { if (t64) { GMF(DT_Q8, 64) } else { GMF(DT_Q8, 128) } }
        if (t64) { GMF(DT_Q4, 64) } else { GMF(DT_Q4, 128) }
#undef GMK
#undef GMF
    }
    dim3 grid((a.units + TM - 1) / TM, (a.n + TN - 1) / TN);
#define G(DT)                                                                              \
    if (a.W.dtype == DT) {                                                                 \
        if (epi == EPI_STORE) hipLaunchKernelGGL((k_gemm<DT, EPI_STORE>), grid, dim3(WG), 0, st, a); \
        else if (epi == EPI_RESID) hipLaunchKernelGGL((k_gemm<DT, EPI_RESID>), grid, dim3(WG), 0, st, a); \
        else return -1;                                                                    \
        return 0;                                                                          \
    }
    G(DT_Q8) G(DT_Q4) G(DT_F32)
#undef G
    return -1;
}


bool gemm_swiglu_fits(const GemmArgs &a) {
    if ((a.W.dtype != DT_Q8 && a.W.dtype != DT_Q4) || a.n <= 0 || a.units % SW_U != 0 || a.W.cols % QB != 0)
        return false;
    if (!a.oq || !a.odx || !a.oxs || a.pair_off < a.units) return false;
    // the shapes whose w1|w3 product launch_gemm gives the short-prompt kernel
    const long g64 = (long)((2 * a.units + GM_U - 1) / GM_U) * ((a.n + 63) / 64);
    if (!(g64 < 256 || (2 * a.units <= 1024 && g64 < 512))) return false;
    const int nb = a.W.cols / QB, sp = nb >= GS_SPLIT_MIN_BLOCKS ? 2 : 1;
    return ((nb + sp - 1) / sp + GS_KB - 1) / GS_KB <= sw_ring(sp);
}

// longer passes: k_gemm_mfma's EPI_SWIGLU form over hidden-unit pairs, on the
// tiles launch_gemm would give the w1|w3 product
bool gemm_swiglu_long_fits(const GemmArgs &a) {
    if ((a.W.dtype != DT_Q8 && a.W.dtype != DT_Q4) || a.n <= 0 || a.W.cols % QB != 0) return false;
    if (!a.oq || !a.odx || !a.oxs || a.pair_off < a.units || a.units % (GM_U / 2) != 0) return false;
    const long g64 = (long)(2 * a.units / GM_U) * ((a.n + 63) / 64);
    return !(g64 < 256 || (2 * a.units <= 1024 && g64 < 512));
}

int launch_gemm_swiglu(hipStream_t st, const GemmArgs &a) {
    if (gemm_swiglu_long_fits(a)) {
        const long gu = 2 * a.units / GM_U;
        bool t64, fused, sp2;
        mfma_shape(gu, a.n, a.W.cols, &t64, &fused, &sp2);
        const dim3 g((unsigned)gu, t64 ? (a.n + 63) / 64 : (a.n + 127) / 128);
#define GMS(DT, TT, FU, SP) { hipLaunchKernelGGL((k_gemm_mfma<DT, EPI_SWIGLU, TT, 2, FU, SP>), g, dim3(WG * SP), 0, st, a, QkPostArgs{}); return 0; }
#define GMSF(DT, TT) if (fused) GMS(DT, TT, true, 1) else GMS(DT, TT, false, 1)
        if (a.W.dtype == DT_Q8 && sp2) GMS(DT_Q8, 64, true, 2)
        if (a.W.dtype == DT_Q8) { if (t64) { GMSF(DT_Q8, 64) } else { GMSF(DT_Q8, 128) } }
        if (t64) { GMSF(DT_Q4, 64) } else { GMSF(DT_Q4, 128) }
#undef GMSF
#undef GMS
    }
    if (!gemm_swiglu_fits(a)) return -1;
    const int nb = a.W.cols / QB, sp = nb >= GS_SPLIT_MIN_BLOCKS ? 2 : 1;
    const bool full = nb % (GS_KB * sp) == 0;
    const dim3 g(a.units / SW_U, (a.n + SW_T - 1) / SW_T), b(256 * sp);
#define SWL(DT)                                                                            \
    if (sp == 2) { if (full) hipLaunchKernelGGL((k_gemm_swq<DT, 2, true>), g, b, 0, st, a); \
                   else hipLaunchKernelGGL((k_gemm_swq<DT, 2, false>), g, b, 0, st, a); }   \
    else if (full) hipLaunchKernelGGL((k_gemm_swq<DT, 1, true>), g, b, 0, st, a);           \
    else hipLaunchKernelGGL((k_gemm_swq<DT, 1, false>), g, b, 0, st, a);
    if (a.W.dtype == DT_Q8) { SWL(DT_Q8) } else { SWL(DT_Q4) }
#undef SWL
    return 0;
}


bool gemm_qkpost_fits(const GemmArgs &g, const QkPostArgs &p) {
    if ((g.W.dtype != DT_Q8 && g.W.dtype != DT_Q4) || g.n <= 0 || g.W.cols % QB != 0 || g.xf) return false;
    if (p.hd != GM_U || p.rope_style != ROPE_NEOX || g.units != (p.n_heads + 2 * p.n_kv) * p.hd || p.n_tok != g.n)
        return false;
    // the shapes whose product launch_gemm gives k_gemm_mfma; they run on
    // 64-token tiles with one pipeline, where the epilogue keeps the kernel
    // at 128 VGPRs (four waves per SIMD; the two-pipeline and 128-token tiles
    // would lose a wave per SIMD to it).  Against those tiles with k_qkpost
    // (Qwen3-0.6B shape): pp1024 5.05 -> 4.80 ms, pp3072 12.36 -> 11.52.
    const long g64 = (long)(g.units / GM_U) * ((g.n + 63) / 64);
    return !(g64 < 256 || (g.units <= 1024 && g64 < 512 && g.W.cols < GEMM_SPLIT_MIN_K));
}

int launch_gemm_qkpost(hipStream_t st, bool f16kv, const GemmArgs &a, const QkPostArgs &p0) {
    if (!gemm_qkpost_fits(a, p0)) return -1;
    QkPostArgs p = p0;
    p.kv_f16 = f16kv ? 1 : 0;
    const long gu = a.units / GM_U;
    const bool fused = a.W.cols >= GEMM_SPLIT_MIN_K;   // (mfma_shape)
    const dim3 g((unsigned)gu, (a.n + 63) / 64);
#define GMQ(DT, FU) { hipLaunchKernelGGL((k_gemm_mfma<DT, EPI_QKPOST, 64, 2, FU, 1>), g, dim3(WG), 0, st, a, p); return 0; }
    if (a.W.dtype == DT_Q8) { if (fused) GMQ(DT_Q8, true) else GMQ(DT_Q8, false) }
    if (fused) GMQ(DT_Q4, true) else GMQ(DT_Q4, false)
#undef GMQ
}

bool gemm_qkv_fits(const GemmArgs &g, const QkPostArgs &p) {
    if ((g.W.dtype != DT_Q8 && g.W.dtype != DT_Q4) || g.n <= 0 || g.W.cols % QB != 0) return false;
    if ((p.hd != 64 && p.hd != 128) || g.units != (p.n_heads + 2 * p.n_kv) * p.hd || p.n_tok != g.n) return false;
    // the shapes whose q|k|v product launch_gemm gives the short-prompt kernel
    const long g64 = (long)((g.units + GM_U - 1) / GM_U) * ((g.n + 63) / 64);
    if (!(g64 < 256 || (g.units <= 1024 && g64 < 512))) return false;
    const int nb = g.W.cols / QB, sp = nb >= GS_SPLIT_MIN_BLOCKS ? 2 : 1;
    return ((nb + sp - 1) / sp + GS_KB - 1) / GS_KB <= qv_ring(sp);
}

int launch_gemm_qkv(hipStream_t st, bool f16kv, const GemmArgs &g, const QkPostArgs &p, float *raw) {
    if (!gemm_qkv_fits(g, p)) return -1;
    const int nb = g.W.cols / QB, sp = nb >= GS_SPLIT_MIN_BLOCKS ? 2 : 1;
    const bool full = nb % (GS_KB * sp) == 0;
    const dim3 grid(p.n_heads + 2 * p.n_kv, (g.n + QV_T - 1) / QV_T), blk(4 * p.hd * sp);
#define QVK(DT, SP, FL, H)                                                                                         \
    if (f16kv) hipLaunchKernelGGL((k_gemm_qkv<DT, SP, FL, H, true>), grid, blk, 0, st, g, p, raw);              \
    else hipLaunchKernelGGL((k_gemm_qkv<DT, SP, FL, H, false>), grid, blk, 0, st, g, p, raw);
#define QVH(DT, SP, FL) if (p.hd == 128) { QVK(DT, SP, FL, 128) } else { QVK(DT, SP, FL, 64) }
#define QVD(DT)                                                                                                    \
    if (sp == 2) { if (full) { QVH(DT, 2, true) } else { QVH(DT, 2, false) } }                                    \
    else if (full) { QVH(DT, 1, true) } else { QVH(DT, 1, false) }
    if (g.W.dtype == DT_Q8) { QVD(DT_Q8) } else { QVD(DT_Q4) }
#undef QVD
#undef QVH
#undef QVK
    return 0;
}

}  // namespace ehip
