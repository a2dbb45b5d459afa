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

// penalties (sample.c:76-96).  Each token's updates depend only on its own
// occurrences, so the lane holding a token's first occurrence in history
// order applies all of them, in that order: the repetition and presence
// penalties once, then the frequency penalty once per occurrence.
__global__ __launch_bounds__(WG) void k_samp_pen(SampleArgs a) {
    if (!a.hist || a.hist_cap <= 0) return;
    const int len = a.hist_meta[0];
    const bool rep = a.p.repeat_penalty != 1.0f, freq = a.p.frequency_penalty != 0.0f,
               pres = a.p.presence_penalty != 0.0f;
    for (int i = threadIdx.x; i < len; i += WG) {
        const int t = a.hist[i];
        if (t < 0 || t >= a.n) continue;
        bool first = true;
        for (int j = 0; j < i; j++) if (a.hist[j] == t) { first = false; break; }
        if (!first) continue;
        int occ = 1;
        for (int j = i + 1; j < len; j++) occ += a.hist[j] == t;
        float l = a.logits[t];
        if (rep) l = l > 0.0f ? l / a.p.repeat_penalty : l * a.p.repeat_penalty;
        if (pres) l -= a.p.presence_penalty;
        if (freq) for (int k = 0; k < occ; k++) l -= a.p.frequency_penalty;
        a.logits[t] = l;
    }
}

constexpr int SAMP_E = SAMPLE_SLICE_MAX / WG;   // slice elements per thread

__device__ __forceinline__ void samp_slice(int n, int &lo, int &hi) {
    const int per = (n + SAMPLE_GRID - 1) / SAMPLE_GRID;
    lo = min(n, (int)blockIdx.x * per);
    hi = min(n, lo + per);
}

// logits /= T, slice maximum.  Every load is issued before the first use.
__global__ __launch_bounds__(WG) void k_samp_a(SampleArgs a) {
    __shared__ float red[NWAVE];
    int lo, hi;
    samp_slice(a.n, lo, hi);
    float l[SAMP_E];
#pragma unroll
    for (int k = 0; k < SAMP_E; k++) {
        const int i = lo + (int)threadIdx.x + k * WG;
        l[k] = i < hi ? a.logits[i] : 0.0f;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < SAMP_E; k++) {
        const int i = lo + (int)threadIdx.x + k * WG;
        if (i < hi) {
            const float v = l[k] / a.p.temperature;
            a.logits[i] = v;
            mx = fmaxf(mx, v);
        }
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
    int lo, hi;
    samp_slice(a.n, lo, hi);
    float l[SAMP_E];
#pragma unroll
    for (int k = 0; k < SAMP_E; k++) {
        const int i = lo + (int)threadIdx.x + k * WG;
        l[k] = i < hi ? a.logits[i] : 0.0f;
    }
    float M = -INFINITY;
    for (int w = 0; w < SAMPLE_GRID; w++) M = fmaxf(M, a.pmax[w]);
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < SAMP_E; k++) {
        const int i = lo + (int)threadIdx.x + k * WG;
        if (i < hi) {
            const float e = expf(l[k] - M);
            a.logits[i] = e;
            s += e;
        }
    }
    const float t = block_sum(s, red);
    if (threadIdx.x == 0) a.psum[blockIdx.x] = t;
}

// (p desc, index asc): the order of the reference's stable sort
__device__ __forceinline__ bool samp_before(float pa, int ia, float pb, int ib) {
    return pa > pb || (pa == pb && ia < ib);
}

// Unsigned key with the order of the float (for the non-NaN values here).
__device__ __forceinline__ unsigned samp_key(float p) {
    const unsigned b = __float_as_uint(p);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

struct SelLds {
    alignas(16) unsigned hist[512];
    int cnt[SAMP_E * NWAVE];
    int sel[3];
};

// Radix selection of the K-th largest key among the valid ones (1 <= K <=
// their count), from the top in digits of 9 (sign and exponent), 8, 8 and 7
// bits, stopping once the bin holding the K-th key is taken whole.  On
// return the keys with (key & M) > P are taken (K - R of them) and R of the
// C keys with (key & M) == P complete the K: all of them when C == R, else
// (M == ~0, exactly equal keys) the first R in index order.
__device__ __forceinline__ void radix_select(const unsigned (&key)[SAMP_E], const bool (&val)[SAMP_E], int K,
                                             SelLds &s, unsigned &P, unsigned &M, int &R, int &C) {
    P = 0; M = 0; R = K; C = 0;
#pragma unroll 1
    for (int pass = 0; pass < 4; pass++) {
        const int shift = pass == 0 ? 23 : pass == 1 ? 15 : pass == 2 ? 7 : 0;
        const int bits = pass == 0 ? 9 : pass == 3 ? 7 : 8;
        const unsigned dmask = (1u << bits) - 1u;
        s.hist[threadIdx.x] = 0;
        s.hist[threadIdx.x + WG] = 0;
        __syncthreads();
#pragma unroll
        for (int k = 0; k < SAMP_E; k++)
            if (val[k] && (key[k] & M) == P) atomicAdd(&s.hist[(key[k] >> shift) & dmask], 1u);
        __syncthreads();
        if (threadIdx.x < 64) {
            // lane l holds bins 8l..8l+7; find the bin where the count from the top reaches R
            const int l = threadIdx.x;
            const uint4 h0 = reinterpret_cast<const uint4 *>(s.hist)[2 * l];
            const uint4 h1 = reinterpret_cast<const uint4 *>(s.hist)[2 * l + 1];
            const unsigned hb[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
            unsigned own = 0;
#pragma unroll
            for (int b = 0; b < 8; b++) own += hb[b];
            unsigned suf = own;   // count in lanes >= l
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const unsigned t = __shfl_down(suf, off);
                if (l + off < 64) suf += t;
            }
            const unsigned r = (unsigned)R;
            unsigned c = suf - own;   // count above this lane's bins
            if (c < r && r <= suf) {
                int sb = 0;
                unsigned sc = 0, sh = 0;
                bool found = false;
#pragma unroll
                for (int b = 7; b >= 0; b--) {
                    if (!found && c + hb[b] >= r) { found = true; sb = b; sc = c; sh = hb[b]; }
                    c += hb[b];
                }
                s.sel[0] = 8 * l + sb;
                s.sel[1] = (int)sc;
                s.sel[2] = (int)sh;
            }
        }
        __syncthreads();
        P |= (unsigned)s.sel[0] << shift;
        M |= dmask << shift;
        R -= s.sel[1];
        C = s.sel[2];
        if (C == R) break;   // the whole bin is taken: no further digits needed
    }
}

// Rank of each flagged element among the flagged ones in index order, where
// thread t holds elements t + k*WG (k = 0..SAMP_E-1); *total gets their count.
__device__ __forceinline__ void block_rank(const bool (&f)[SAMP_E], int (&rank)[SAMP_E], int &total, SelLds &s) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const unsigned long long below = (1ull << lane) - 1ull;
    __syncthreads();   // s.cnt may still be read by a previous call
#pragma unroll
    for (int k = 0; k < SAMP_E; k++) {
        const unsigned long long b = __ballot(f[k]);
        rank[k] = __popcll(b & below);
        if (lane == 0) s.cnt[k * NWAVE + w] = __popcll(b);
    }
    __syncthreads();
    int base = 0;
#pragma unroll
    for (int k = 0; k < SAMP_E; k++) {
        int row = 0, pre = 0;
#pragma unroll
        for (int v = 0; v < NWAVE; v++) {
            const int c = s.cnt[k * NWAVE + v];
            pre += v < w ? c : 0;
            row += c;
        }
        rank[k] += base + pre;
        base += row;
    }
    total = base;
}

// Which of the held elements belong to the first K in samp_before order
// (keys from samp_key, distinct indices increasing with position).
__device__ __forceinline__ void samp_top(const unsigned (&key)[SAMP_E], const bool (&val)[SAMP_E], int K,
                                         bool (&take)[SAMP_E], SelLds &s) {
    unsigned P, M;
    int R, C;
    radix_select(key, val, K, s, P, M, R, C);
    bool tie[SAMP_E];
#pragma unroll
    for (int k = 0; k < SAMP_E; k++) {
        take[k] = val[k] && (key[k] & M) > P;
        tie[k] = val[k] && (key[k] & M) == P;
    }
    if (C == R) {
#pragma unroll
        for (int k = 0; k < SAMP_E; k++) take[k] = take[k] || tie[k];
    } else {   // equal probabilities: the smaller indices come first
        int rk[SAMP_E], nt;
        block_rank(tie, rk, nt, s);
#pragma unroll
        for (int k = 0; k < SAMP_E; k++) take[k] = take[k] || (tie[k] && rk[k] < R);
    }
}

// p = e / sum; the slice's first SAMPLE_TOPK_MAX candidates in samp_before
// order, written in index order (which k_samp_d's tie ranking relies on).
__global__ __launch_bounds__(WG) void k_samp_c(SampleArgs a) {
    __shared__ SelLds s;
    __shared__ float S;
    int lo, hi;
    samp_slice(a.n, lo, hi);
    float e[SAMP_E];
#pragma unroll
    for (int k = 0; k < SAMP_E; k++) {
        const int i = lo + (int)threadIdx.x + k * WG;
        e[k] = i < hi ? a.logits[i] : 0.0f;
    }
    if (threadIdx.x == 0) {
        float t = 0.0f;
        for (int w = 0; w < SAMPLE_GRID; w++) t += a.psum[w];
        S = t;
    }
    __syncthreads();
    float p[SAMP_E];
    unsigned key[SAMP_E];
    bool val[SAMP_E], take[SAMP_E];
#pragma unroll
    for (int k = 0; k < SAMP_E; k++) {
        val[k] = lo + (int)threadIdx.x + k * WG < hi;
        p[k] = e[k] / S;
        key[k] = samp_key(p[k]);
        take[k] = false;
    }
    const int K = min(hi - lo, SAMPLE_TOPK_MAX);
    if (K > 0) samp_top(key, val, K, take, s);
    int pos[SAMP_E], nt;
    block_rank(take, pos, nt, s);
    float *cv = a.cval + blockIdx.x * SAMPLE_TOPK_MAX;
    int *ci = a.cidx + blockIdx.x * SAMPLE_TOPK_MAX;
#pragma unroll
    for (int k = 0; k < SAMP_E; k++)
        if (take[k] && pos[k] < SAMPLE_TOPK_MAX) {
            cv[pos[k]] = p[k];
            ci[pos[k]] = lo + (int)threadIdx.x + k * WG;
        }
    for (int j = nt + (int)threadIdx.x; j < SAMPLE_TOPK_MAX; j += WG) { cv[j] = -1.0f; ci[j] = INT_MAX; }
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

__device__ __forceinline__ float lane_f(float v, int i) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}

// The first min(n, top_k) of all candidates, then top-k / min-p / top-p and
// the draw (sample.c:136-175).  Candidate position order is index order.
// The final 64 are sorted by one wave (bitonic network over lanes); the
// cumulative sums are taken sequentially in sorted order as the reference's
// loops take them.
__global__ __launch_bounds__(WG) void k_samp_d(SampleArgs a) {
    constexpr int NC = SAMPLE_GRID * SAMPLE_TOPK_MAX;
    static_assert(NC == SAMP_E * WG, "candidate count");
    __shared__ SelLds s;
    __shared__ float tp[SAMPLE_TOPK_MAX];
    __shared__ int ti[SAMPLE_TOPK_MAX];
    float p[SAMP_E];
    int id[SAMP_E];
    unsigned key[SAMP_E];
    bool val[SAMP_E], take[SAMP_E];
#pragma unroll
    for (int k = 0; k < SAMP_E; k++) {
        p[k] = a.cval[threadIdx.x + k * WG];
        id[k] = a.cidx[threadIdx.x + k * WG];
    }
#pragma unroll
    for (int k = 0; k < SAMP_E; k++) {
        val[k] = id[k] >= 0 && id[k] < a.n;
        key[k] = samp_key(p[k]);
    }
    const int K = min(a.n, a.p.top_k);   // 1..SAMPLE_TOPK_MAX, checked at launch
    samp_top(key, val, K, take, s);
    int pos[SAMP_E], nt;
    block_rank(take, pos, nt, s);
#pragma unroll
    for (int k = 0; k < SAMP_E; k++)
        if (take[k] && pos[k] < SAMPLE_TOPK_MAX) { tp[pos[k]] = p[k]; ti[pos[k]] = id[k]; }
    for (int j = nt + (int)threadIdx.x; j < SAMPLE_TOPK_MAX; j += WG) { tp[j] = -1.0f; ti[j] = INT_MAX; }
    __syncthreads();
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    float v = tp[lane];
    int ix = ti[lane];
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const float pv = __shfl_xor(v, j);
            const int pi = __shfl_xor(ix, j);
            const bool want_first = ((lane & j) == 0) == ((lane & k) == 0);
            if (want_first ? samp_before(pv, pi, v, ix) : samp_before(v, ix, pv, pi)) { v = pv; ix = pi; }
        }
    int m = min(nt, K);
    if (a.p.min_p > 0.0f && a.p.min_p < 1.0f) {
        const float thresh = a.p.min_p * lane_f(v, 0);
        const unsigned long long drop = __ballot(lane >= 1 && lane < m && !(v >= thresh));
        if (drop) m = __builtin_ctzll(drop);
    }
    float cum = 0.0f, c = 0.0f;   // cum = sum of the sorted p[0..lane], in order
#pragma unroll
    for (int i = 0; i < 64; i++) {
        c += lane_f(v, i);
        if (lane == i) cum = c;
    }
    if (a.p.top_p > 0.0f && a.p.top_p < 1.0f) {
        const unsigned long long hit = __ballot(lane < m && cum >= a.p.top_p);
        if (hit) m = __builtin_ctzll(hit) + 1;
    }
    const float cutoff = __shfl(cum, m - 1);
    unsigned long long x = a.rng[0];   // xorshift64* (sample.c:98-105)
    x ^= x >> 12; x ^= x << 25; x ^= x >> 27;
    const unsigned int u = (unsigned int)((x * 0x2545F4914F6CDD1DULL) >> 32);
    const float r = (float)(u >> 8) / 16777216.0f * cutoff;
    const unsigned long long in = __ballot(lane < m && r < cum);
    const int chosen = __shfl(ix, in ? __builtin_ctzll(in) : m - 1);
    if (lane == 0) {
        a.rng[0] = x;
        samp_emit(a, chosen);
    }
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
    const bool pen = a.hist && a.hist_cap > 0 &&
        (a.p.repeat_penalty != 1.0f || a.p.frequency_penalty != 0.0f || a.p.presence_penalty != 0.0f);
    if (pen) hipLaunchKernelGGL(k_samp_pen, dim3(1), dim3(WG), 0, st, a);
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
