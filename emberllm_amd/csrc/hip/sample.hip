// sample.hip — on-device token selection for gfx950.
//
// Replaces argmax (src/sample.c:114-118), the whole of ember_sample when
// temperature <= 0 (sample.c:123-127): the chosen token is the FIRST index
// holding the maximum logit.  It also advances the decode loop held in
// device memory: tokpos = {argmax, pos + 1, n + 1}, so the next replay of
// the decode graph consumes the chosen token without a host round trip.
//
// Roofline: HBM-bound, 4 bytes per logit read once (608 KB at vocab 151936).
// Two kernels: each workgroup of k_argmax_part reduces one contiguous slice
// to its (value, index) winner; k_argmax_merge (one workgroup) picks the
// first maximum over the winners.  The kernel boundary orders the two
// instead of a per-workgroup fence and counter, which cost tens of ns per
// workgroup on this GPU.  Ties resolve to the smaller index at every level,
// which reproduces the reference's strict `>` scan from index 0.  The lm_head
// matvec can write the per-workgroup winners itself (matvec.hip), leaving
// only the merge.
#include <climits>

#include "kernels.h"

namespace ehip {

__device__ __forceinline__ void take_better(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
}

__device__ __forceinline__ void block_argmax(float &v, int &i, float *sv, int *si) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float v2 = __shfl_xor(v, off);
        const int i2 = __shfl_xor(i, off);
        take_better(v, i, v2, i2);
    }
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) { sv[w] = v; si[w] = i; }
    __syncthreads();
    v = sv[0]; i = si[0];
#pragma unroll
    for (int k = 1; k < NWAVE; k++) take_better(v, i, sv[k], si[k]);
}

constexpr int ARGMAX_PER_THREAD = 4;   // a slice is at most 4 * WG logits

__global__ __launch_bounds__(WG) void k_argmax_part(ArgmaxArgs a) {
    __shared__ float sv[NWAVE];
    __shared__ int si[NWAVE];
    const int per = (a.n + gridDim.x - 1) / gridDim.x;
    const int i0 = blockIdx.x * per, i1 = min(a.n, i0 + per);
    float lv[ARGMAX_PER_THREAD];
#pragma unroll
    for (int k = 0; k < ARGMAX_PER_THREAD; k++)   // every load issued before any compare
        lv[k] = a.logits[min(i0 + (int)threadIdx.x + k * WG, a.n - 1)];
    float v = -INFINITY;
    int idx = INT_MAX;
#pragma unroll
    for (int k = 0; k < ARGMAX_PER_THREAD; k++) {
        const int i = i0 + (int)threadIdx.x + k * WG;
        if (i < i1) take_better(v, idx, lv[k], i);
    }
    block_argmax(v, idx, sv, si);
    if (threadIdx.x == 0) { a.pval[blockIdx.x] = v; a.pidx[blockIdx.x] = idx; }
}

constexpr int MERGE_PER_THREAD = (MATVEC_MAX_GRID + WG - 1) / WG;

__global__ __launch_bounds__(WG) void k_argmax_merge(const float *pval, const int *pidx, int nparts, int n,
                                                     int *tokpos, int *out, int cap) {
    __shared__ float sv[NWAVE];
    __shared__ int si[NWAVE];
    float lv[MERGE_PER_THREAD];
    int li[MERGE_PER_THREAD];
#pragma unroll
    for (int k = 0; k < MERGE_PER_THREAD; k++) {
        const int b = min((int)threadIdx.x + k * WG, nparts - 1);
        lv[k] = pval[b];
        li[k] = pidx[b];
    }
    float v = -INFINITY;
    int idx = INT_MAX;
#pragma unroll
    for (int k = 0; k < MERGE_PER_THREAD; k++)
        if ((int)threadIdx.x + k * WG < nparts) take_better(v, idx, lv[k], li[k]);
    block_argmax(v, idx, sv, si);
    if (threadIdx.x == 0) {
        // all-NaN logits leave idx unset; the reference's scan then returns 0
        const int tok = (idx >= 0 && idx < n) ? idx : 0;
        tokpos[0] = tok;
        tokpos[1] += 1;
        const int k = tokpos[2];
        if (k < cap) out[k] = tok;
        tokpos[2] = k + 1;
    }
}

int launch_argmax_merge(hipStream_t st, const float *pval, const int *pidx, int nparts, int n,
                        int *tokpos, int *out, int cap) {
    if (nparts <= 0 || nparts > MATVEC_MAX_GRID || n <= 0) return -1;
    hipLaunchKernelGGL(k_argmax_merge, dim3(1), dim3(WG), 0, st, pval, pidx, nparts, n, tokpos, out, cap);
    return 0;
}

int launch_argmax(hipStream_t st, const ArgmaxArgs &a) {
    if (a.n <= 0) return -1;
    int nb = (a.n + ARGMAX_PER_THREAD * WG - 1) / (ARGMAX_PER_THREAD * WG);
    if (nb > ARGMAX_MAX_BLOCKS) return -1;   // larger vocabularies need a wider first pass
    hipLaunchKernelGGL(k_argmax_part, dim3(nb), dim3(WG), 0, st, a);
    return launch_argmax_merge(st, a.pval, a.pidx, nb, a.n, a.tokpos, a.out, a.cap);
}

}  // namespace ehip
