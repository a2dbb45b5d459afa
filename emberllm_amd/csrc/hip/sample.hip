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

// --------------------------------------------------------------------------
// Full sampler.  The per-token ordering work is exact: penalties in history
// order, division by the temperature, expf, division by the sum, candidates
// ordered by (probability descending, index ascending) — what the reference's
// stable qsort yields — and the cumulative sums of top-p and of the draw in
// that order.  Only the softmax sum is taken in a fixed tree order instead
// of index order, so a probability can differ from the reference's in its
// last bit; a draw could then differ only when it lands within that of a
// cumulative boundary.

// penalties (sample.c:76-96): one lane, history in array order
__global__ void k_samp_pen(SampleArgs a) {
    if (threadIdx.x != 0 || !a.hist || a.hist_cap <= 0) return;
    const int len = a.hist_meta[0];
    const bool rep = a.p.repeat_penalty != 1.0f, freq = a.p.frequency_penalty != 0.0f,
               pres = a.p.presence_penalty != 0.0f;
    if (len == 0 || (!rep && !freq && !pres)) return;
    for (int i = 0; i < len; i++) {
        const int t = a.hist[i];
        if (t < 0 || t >= a.n) continue;
        bool first = true;
        for (int j = 0; j < i; j++) if (a.hist[j] == t) { first = false; break; }
        float l = a.logits[t];
        if (first) {
            if (rep) l = l > 0.0f ? l / a.p.repeat_penalty : l * a.p.repeat_penalty;
            if (pres) l -= a.p.presence_penalty;
        }
        if (freq) l -= a.p.frequency_penalty;
        a.logits[t] = l;
    }
}

__device__ __forceinline__ void samp_slice(int n, int &lo, int &hi) {
    const int per = (n + SAMPLE_GRID - 1) / SAMPLE_GRID;
    lo = min(n, (int)blockIdx.x * per);
    hi = min(n, lo + per);
}

// logits /= T, slice maximum
__global__ __launch_bounds__(WG) void k_samp_a(SampleArgs a) {
    __shared__ float red[NWAVE];
    int lo, hi;
    samp_slice(a.n, lo, hi);
    float mx = -INFINITY;
    for (int i = lo + threadIdx.x; i < hi; i += WG) {
        const float l = a.logits[i] / a.p.temperature;
        a.logits[i] = l;
        mx = fmaxf(mx, l);
    }
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = red[0];
        for (int w = 1; w < NWAVE; w++) m = fmaxf(m, red[w]);
        a.pmax[blockIdx.x] = m;
    }
}

// e = expf(l - max) in place, slice sum
__global__ __launch_bounds__(WG) void k_samp_b(SampleArgs a) {
    __shared__ float red[NWAVE];
    float M = -INFINITY;
    for (int w = 0; w < SAMPLE_GRID; w++) M = fmaxf(M, a.pmax[w]);
    int lo, hi;
    samp_slice(a.n, lo, hi);
    float s = 0.0f;
    for (int i = lo + threadIdx.x; i < hi; i += WG) {
        const float e = expf(a.logits[i] - M);
        a.logits[i] = e;
        s += e;
    }
    const float t = block_sum(s, red);
    if (threadIdx.x == 0) a.psum[blockIdx.x] = t;
}

// (p desc, index asc): the order of the reference's stable sort
__device__ __forceinline__ bool samp_before(float pa, int ia, float pb, int ib) {
    return pa > pb || (pa == pb && ia < ib);
}

// bitonic sort of N (p, idx) pairs in LDS into samp_before order
template <int N>
__device__ __forceinline__ void samp_sort(float *sp, int *si) {
    for (int k = 2; k <= N; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            __syncthreads();
            for (int i = threadIdx.x; i < N; i += blockDim.x) {
                const int l = i ^ j;
                if (l > i) {
                    const bool up = (i & k) == 0;   // this block ascends in samp_before order
                    const bool sw = up ? samp_before(sp[l], si[l], sp[i], si[i])
                                       : samp_before(sp[i], si[i], sp[l], si[l]);
                    if (sw) {
                        const float tp = sp[i]; sp[i] = sp[l]; sp[l] = tp;
                        const int ti = si[i]; si[i] = si[l]; si[l] = ti;
                    }
                }
            }
        }
    __syncthreads();
}

// p = e / sum; the slice's first SAMPLE_TOPK_MAX candidates
__global__ __launch_bounds__(WG) void k_samp_c(SampleArgs a) {
    __shared__ float sp[SAMPLE_SLICE_MAX];
    __shared__ int si[SAMPLE_SLICE_MAX];
    __shared__ float S;
    if (threadIdx.x == 0) {
        float t = 0.0f;
        for (int w = 0; w < SAMPLE_GRID; w++) t += a.psum[w];
        S = t;
    }
    __syncthreads();
    int lo, hi;
    samp_slice(a.n, lo, hi);
    for (int i = threadIdx.x; i < SAMPLE_SLICE_MAX; i += WG) {
        const bool in = lo + i < hi;
        sp[i] = in ? a.logits[lo + i] / S : -1.0f;
        si[i] = in ? lo + i : INT_MAX;
    }
    samp_sort<SAMPLE_SLICE_MAX>(sp, si);
    for (int i = threadIdx.x; i < SAMPLE_TOPK_MAX; i += WG) {
        a.cval[blockIdx.x * SAMPLE_TOPK_MAX + i] = sp[i];
        a.cidx[blockIdx.x * SAMPLE_TOPK_MAX + i] = si[i];
    }
}

__device__ __forceinline__ void samp_emit(const SampleArgs &a, int tok) {
    if (a.hist && a.hist_cap > 0) {   // ember_sampler_accept
        const int pos = a.hist_meta[1];
        a.hist[pos] = tok;
        a.hist_meta[1] = (pos + 1) % a.hist_cap;
        if (a.hist_meta[0] < a.hist_cap) a.hist_meta[0] += 1;
    }
    a.tokpos[0] = tok;
    a.tokpos[1] += 1;
    const int k = a.tokpos[2];
    if (k < a.cap) a.out[k] = tok;
    a.tokpos[2] = k + 1;
}

// merge the candidates, then top-k / min-p / top-p and the draw (sample.c:136-175)
__global__ __launch_bounds__(WG) void k_samp_d(SampleArgs a) {
    constexpr int NC = SAMPLE_GRID * SAMPLE_TOPK_MAX;
    __shared__ float sp[NC];
    __shared__ int si[NC];
    for (int i = threadIdx.x; i < NC; i += WG) { sp[i] = a.cval[i]; si[i] = a.cidx[i]; }
    samp_sort<NC>(sp, si);
    if (threadIdx.x != 0) return;
    int m = min(a.n, a.p.top_k);
    if (a.p.min_p > 0.0f && a.p.min_p < 1.0f) {
        const float thresh = a.p.min_p * sp[0];
        int keep = 1;
        while (keep < m && sp[keep] >= thresh) keep++;
        m = keep;
    }
    float cutoff;
    if (a.p.top_p > 0.0f && a.p.top_p < 1.0f) {
        float cum = 0.0f;
        int last = m - 1;
        for (int i = 0; i < m; i++) { cum += sp[i]; if (cum >= a.p.top_p) { last = i; break; } }
        m = last + 1;
        cutoff = cum;
    } else {
        cutoff = 0.0f;
        for (int i = 0; i < m; i++) cutoff += sp[i];
    }
    unsigned long long x = a.rng[0];   // xorshift64* (sample.c:98-105)
    x ^= x >> 12; x ^= x << 25; x ^= x >> 27;
    a.rng[0] = x;
    const unsigned int u = (unsigned int)((x * 0x2545F4914F6CDD1DULL) >> 32);
    const float r = (float)(u >> 8) / 16777216.0f * cutoff;
    float cum = 0.0f;
    int chosen = si[m - 1];
    for (int i = 0; i < m; i++) { cum += sp[i]; if (r < cum) { chosen = si[i]; break; } }
    samp_emit(a, chosen);
}

// greedy with penalties: first maximum over the penalized logits
__global__ void k_samp_greedy_emit(SampleArgs a) {
    if (threadIdx.x == 0) {
        const int tok = a.tokpos[0];   // written by the argmax merge
        // the argmax merge already advanced tokpos and out; only the ring is left
        if (a.hist && a.hist_cap > 0) {
            const int pos = a.hist_meta[1];
            a.hist[pos] = tok;
            a.hist_meta[1] = (pos + 1) % a.hist_cap;
            if (a.hist_meta[0] < a.hist_cap) a.hist_meta[0] += 1;
        }
    }
}

int launch_sample(hipStream_t st, const SampleArgs &a) {
    if (a.n <= 0 || (a.n + SAMPLE_GRID - 1) / SAMPLE_GRID > SAMPLE_SLICE_MAX) return -1;
    hipLaunchKernelGGL(k_samp_pen, dim3(1), dim3(64), 0, st, a);
    if (a.p.temperature <= 0.0f) {
        ArgmaxArgs g{};
        g.logits = a.logits; g.n = a.n; g.pval = a.am_val; g.pidx = a.am_idx;
        g.tokpos = a.tokpos; g.out = a.out; g.cap = a.cap;
        if (launch_argmax(st, g)) return -1;
        hipLaunchKernelGGL(k_samp_greedy_emit, dim3(1), dim3(64), 0, st, a);
        return 0;
    }
    if (a.p.top_k < 1 || a.p.top_k > SAMPLE_TOPK_MAX) return -1;
    hipLaunchKernelGGL(k_samp_a, dim3(SAMPLE_GRID), dim3(WG), 0, st, a);
    hipLaunchKernelGGL(k_samp_b, dim3(SAMPLE_GRID), dim3(WG), 0, st, a);
    hipLaunchKernelGGL(k_samp_c, dim3(SAMPLE_GRID), dim3(WG), 0, st, a);
    hipLaunchKernelGGL(k_samp_d, dim3(1), dim3(WG), 0, st, a);
    return 0;
}

}  // namespace ehip
