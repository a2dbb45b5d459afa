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
#include <utility>

#include "kernels.h"
#include "libm_expf.h"

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
//
// After the logits (and the penalties), one kernel of SAMPLE_GRID workgroups,
// one slice of the vocabulary each (k_samp_fused):
//   1. M = max logit / T, from per-part maxima that come with the logits (the
//      lm_head's per-workgroup winners, or k_argmax_part's); e = expf(l/T - M)
//      over the slice and the slice's sum of e in a fixed order;
//   2. a bound e_lo from K = min(n, top_k) distinct tokens (the K largest of
//      128 group maxima of those winners) that every token among the first K
//      of the final order reaches (samp_bound); the slice passes on only its
//      tokens with e >= e_lo, typically a few, at most SAMP_CAP;
//   3. the last workgroup to arrive (an arrival counter) forms S = the sum of
//      the slice sums in a fixed tree order, p = e / S for the passed tokens,
//      ranks them by (p desc, index asc) — by counting when there are at
//      most WG of them, else with a bitonic network — and draws.  If a slice
//      had more than SAMP_CAP tokens to pass (flat or degenerate logits), it
//      streams the whole vocabulary through the network instead, keeping the
//      running first 64: exact, and slower.

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
constexpr int SAMP_CAP = 4 * WG / SAMPLE_GRID;   // tokens a slice may pass on
constexpr int SAMP_PARTS = 8;                    // per-part maxima per thread
static_assert(SAMPLE_GRID % 64 == 0 && SAMPLE_GRID <= WG, "one thread per slice in the final workgroup");
static_assert(SAMP_CAP % 4 == 0 && SAMP_CAP <= SAMPLE_TOPK_MAX && SAMPLE_GRID * SAMP_CAP == 4 * WG,
              "passed-on slots: 4 per thread");
static_assert(MATVEC_MAX_GRID <= SAMP_PARTS * WG && ARGMAX_MAX_BLOCKS <= SAMP_PARTS * WG, "per-part maxima");

__device__ __forceinline__ void samp_slice(int n, int &lo, int &hi) {
    const int per = (n + SAMPLE_GRID - 1) / SAMPLE_GRID;
    lo = min(n, (int)blockIdx.x * per);
    hi = min(n, lo + per);
}

// e of a logit: the reference's division by the temperature, then its C
// library's expf of the difference to the maximum (sample.c:129-134;
// libm_expf.h)
__device__ __forceinline__ float samp_e(float l, float T, float M) { return libm_expf(l / T - M); }

// (p desc, index asc): the order of the reference's stable sort
__device__ __forceinline__ bool samp_before(float pa, int ia, float pb, int ib) {
    return pa > pb || (pa == pb && ia < ib);
}

// 64-bit key whose unsigned order is samp_before's for p >= 0 (p = e / S,
// never negative): p's bits above, the complement of the index below.
__device__ __forceinline__ unsigned long long samp_key(float p, int ix) {
    return ((unsigned long long)__float_as_uint(p) << 32) | (unsigned)~ix;
}

__device__ __forceinline__ float lane_f(float v, int i) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}

// Why e_lo bounds the first K.  Let C be K distinct tokens and eps the least
// e among them.  p = fl(e / S) is monotone in e, so at least K tokens have
// p >= fl(eps / S): the K-th largest p is >= fl(eps / S), and so is the p of
// every token x among the first K.  Either e_x >= eps, or fl(e_x / S) ==
// fl(eps / S), i.e. e_x / S and eps / S round to the same float: then
// eps - e_x <= S ulp(fl(eps / S)) < eps 2^-22 + S 2^-149, with S <= n <= 2^18
// (every e <= 1).  e_lo = eps - eps 2^-20 - 2^-128 lies below both cases.
// C is the K largest (in e) of the 128 group maxima, group j holding the
// per-part maxima j, j + 128, ...: distinct parts, distinct tokens.  A part
// with no finite winner contributes -inf (e = 0), which only lowers eps.
// eps, the K-th largest of the 128 e values, is the largest e that at least
// K of them reach.  Thread t < 128 holds group t's e.  Every thread returns
// e_lo (0 when NaNs leave no such e).
__device__ __forceinline__ float samp_bound(float g, int K, float T, float M, float *ge, float *red) {
    const int t = threadIdx.x;
    const float e = samp_e(g, T, M);
    if (t < 128) ge[t] = e;
    __syncthreads();
    float x = 0.0f;
    if (t < 128) {
        int cnt = 0;
#pragma unroll
        for (int q = 0; q < 128; q += 4) {
            const float4 o = *reinterpret_cast<const float4 *>(ge + q);
            cnt += (o.x >= e ? 1 : 0) + (o.y >= e ? 1 : 0) + (o.z >= e ? 1 : 0) + (o.w >= e ? 1 : 0);
        }
        x = cnt >= K ? e : 0.0f;
    }
    x = wave_max(x);
    if ((t & 63) == 0) red[t >> 6] = x;
    __syncthreads();
    x = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    return x - x * 0x1p-20f - 0x1p-128f;
}

// One compare-exchange of the bitonic network at position e (partner e ^ j):
// keep the earlier of the pair in samp_before order where the k-block runs
// forward and e is the lower position, or runs backward and e is the upper.
__device__ __forceinline__ void bit_cx(float &v, int &ix, float pv, int pi, int e, int j, int k) {
    const bool first = ((e & j) == 0) == ((e & k) == 0);
    if (first ? samp_before(pv, pi, v, ix) : samp_before(v, ix, pv, pi)) { v = pv; ix = pi; }
}

// The in-thread stage j = J of the network: pairs (i, i | J) with (i & J) == 0.
template <int PER, int J>
__device__ __forceinline__ void bit_local(float (&v)[PER], int (&ix)[PER], int k) {
    if constexpr (J < PER) {
        const int e0 = PER * (int)threadIdx.x;
#pragma unroll
        for (int i = 0; i < PER; i++) {
            if (i & J) continue;
            const float va = v[i], vb = v[i | J];
            const int ia = ix[i], ib = ix[i | J];
            bit_cx(v[i], ix[i], vb, ib, e0 + i, J, k);
            bit_cx(v[i | J], ix[i | J], va, ia, e0 + (i | J), J, k);
        }
    }
}

// Sorts the PER * WG (p, index) pairs held by the workgroup, pair PER*t + i in
// thread t, into samp_before order.  Partners in the same thread exchange in
// registers, in the same wave through lane shuffles, otherwise through LDS
// (lp, li: PER * WG entries).  The network is fixed: NaNs cannot stall it.
template <int PER>
__device__ __forceinline__ void bitonic_sort(float (&v)[PER], int (&ix)[PER], float *lp, int *li) {
    constexpr int N = PER * WG;
    const int t = threadIdx.x;
#pragma unroll 1
    for (int k = 2; k <= N; k <<= 1) {
#pragma unroll 1
        for (int j = k >> 1; j > 0; j >>= 1) {
            if (j < PER) {
                if (j == 1) bit_local<PER, 1>(v, ix, k);
                else bit_local<PER, 2>(v, ix, k);
            } else if (j < 64 * PER) {
                const int lm = j / PER;
#pragma unroll
                for (int i = 0; i < PER; i++) {
                    const float pv = __shfl_xor(v[i], lm);
                    const int pi = __shfl_xor(ix[i], lm);
                    bit_cx(v[i], ix[i], pv, pi, PER * t + i, j, k);
                }
            } else {
                __syncthreads();   // earlier readers of lp/li are done
#pragma unroll
                for (int i = 0; i < PER; i++) { lp[PER * t + i] = v[i]; li[PER * t + i] = ix[i]; }
                __syncthreads();
#pragma unroll
                for (int i = 0; i < PER; i++) {
                    const int e = PER * t + i;
                    bit_cx(v[i], ix[i], lp[e ^ j], li[e ^ j], e, j, k);
                }
            }
        }
    }
}

// The device state the draw reads and advances, loaded early by one thread.
struct SampState {
    unsigned long long rng;
    int pos, ngen, hlen, hpos;
};

__device__ __forceinline__ SampState samp_state_load(const SampleArgs &a) {
    SampState q;
    q.rng = a.rng[0];
    q.pos = a.tokpos[1];
    q.ngen = a.tokpos[2];
    const bool h = a.hist && a.hist_cap > 0;
    q.hlen = h ? a.hist_meta[0] : 0;
    q.hpos = h ? a.hist_meta[1] : 0;
    return q;
}

// ember_sampler_accept and the decode loop's {token, pos + 1, n + 1}
__device__ __forceinline__ void samp_emit(const SampleArgs &a, const SampState &q, int tok) {
    if (a.hist && a.hist_cap > 0) {
        a.hist[q.hpos] = tok;
        a.hist_meta[1] = (q.hpos + 1) % a.hist_cap;
        if (q.hlen < a.hist_cap) a.hist_meta[0] = q.hlen + 1;
    }
    a.tokpos[0] = tok;
    a.tokpos[1] = q.pos + 1;
    if (q.ngen < a.cap) a.out[q.ngen] = tok;
    a.tokpos[2] = q.ngen + 1;
}

// Kernel arguments are loaded where first used; pinning them at the start
// issues all their scalar loads together instead of one miss per phase.
#define SAMP_PIN(x) asm volatile("" ::"s"(x))

// Launched with SAMPLE_GRID workgroups; a.nparts per-part maxima in a.am_val.
__global__ __launch_bounds__(WG) void k_samp_fused(SampleArgs a) {
    __shared__ float red[NWAVE], red2[NWAVE];
    __shared__ float gm[NWAVE][64];
    __shared__ int sh_nk;
    __shared__ float lp[4 * WG];
    __shared__ int li[4 * WG];
    __shared__ unsigned long long lk[WG];
    __shared__ float fp[SAMPLE_TOPK_MAX];
    __shared__ int fi[SAMPLE_TOPK_MAX];
    __shared__ int sh_last;
    __shared__ int scn[SAMPLE_GRID], pre[SAMPLE_GRID];
    __shared__ float wsum[SAMPLE_GRID / 64];
    __shared__ int wcnt[SAMPLE_GRID / 64];
    __shared__ bool wovf[SAMPLE_GRID / 64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    SAMP_PIN(a.logits); SAMP_PIN(a.am_val); SAMP_PIN(a.cval); SAMP_PIN(a.cidx); SAMP_PIN(a.psum);
    SAMP_PIN(a.scnt); SAMP_PIN(a.rng); SAMP_PIN(a.tokpos); SAMP_PIN(a.out); SAMP_PIN(a.hist);
    SAMP_PIN(a.hist_meta); SAMP_PIN(a.n); SAMP_PIN(a.nparts); SAMP_PIN(a.cap); SAMP_PIN(a.hist_cap);
    SAMP_PIN(a.p.temperature); SAMP_PIN(a.p.top_k); SAMP_PIN(a.p.top_p); SAMP_PIN(a.p.min_p);
    const float T = a.p.temperature;
    const int K = min(a.n, a.p.top_k);   // 1..SAMPLE_TOPK_MAX, checked at launch
    int lo, hi;
    samp_slice(a.n, lo, hi);

    // ---- 1. loads: the per-part maxima and the slice's logits --------------
    // (indices clamped into range, so every load is unconditional)
    float pm[SAMP_PARTS], l[SAMP_E];
#pragma unroll
    for (int k = 0; k < SAMP_PARTS; k++) pm[k] = a.am_val[min(tid + k * WG, a.nparts - 1)];
#pragma unroll
    for (int k = 0; k < SAMP_E; k++) l[k] = a.logits[min(lo + tid + k * WG, a.n - 1)];
#pragma unroll
    for (int k = 0; k < SAMP_PARTS; k++)
        if (tid + k * WG >= a.nparts) pm[k] = -INFINITY;

    // ---- 2. M and the bound (every wave computes both) ---------------------
    float g = pm[0];   // this thread's parts all fall in group tid % 128
#pragma unroll
    for (int k = 1; k < SAMP_PARTS; k++) g = fmaxf(g, pm[k]);
    gm[w][lane] = g;
    __syncthreads();
    const float ga = fmaxf(gm[0][lane], gm[2][lane]), gb = fmaxf(gm[1][lane], gm[3][lane]);
    // max(l) / T == max(l / T): correctly rounded division is monotone
    const float M = wave_max(fmaxf(ga, gb)) / T;
    if (tid == 0) sh_nk = 0;   // samp_bound's barriers order this before the counting
    const float e_lo = samp_bound(w & 1 ? gb : ga, K, T, M, lp, red);   // thread t: group t % 128

    // ---- 3. e, the slice sum, the tokens passed on --------------------------
    // A token passed on takes the next slot of an LDS counter: the order
    // within a slice does not matter, the final ranking breaks ties by index.
    float *cv = a.cval + blockIdx.x * SAMP_CAP;
    int *ci = a.cidx + blockIdx.x * SAMP_CAP;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < SAMP_E; k++) {
        const int i = lo + tid + k * WG;
        if (k * WG < hi - lo && i < hi) {   // the first test is uniform
            const float e = samp_e(l[k], T, M);
            s += e;
            if (e >= e_lo) {
                const int slot = atomicAdd(&sh_nk, 1);
                if (slot < SAMP_CAP) { cv[slot] = e; ci[slot] = i; }
            }
        }
    }
    s = wave_sum(s);
    if (lane == 0) red2[w] = s;
    __syncthreads();
    if (tid == 0) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < NWAVE; i++) t += red2[i];
        a.psum[blockIdx.x] = t;
        a.scnt[blockIdx.x] = sh_nk;
    }

    // ---- 4. arrival: the last workgroup carries on --------------------------
    // Every wave's stores have completed before the release (which writes the
    // L2 back for the other XCDs); the acquire invalidates this CU's caches.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const int old = __hip_atomic_fetch_add(a.scnt + SAMPLE_GRID, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        sh_last = old == SAMPLE_GRID - 1;
    }
    __syncthreads();
    if (!sh_last) return;
    if (tid == 0) __hip_atomic_store(a.scnt + SAMPLE_GRID, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // ---- 5. one round trip: counts, sums and every passed-on slot ----------
    // thread t < SAMPLE_GRID: slice t's count and sum; slots 4 tid .. 4 tid + 3
    int c = 0;
    float ps = 0.0f;
    if (tid < SAMPLE_GRID) { c = a.scnt[tid]; ps = a.psum[tid]; }
    const float4 cv4 = reinterpret_cast<const float4 *>(a.cval)[tid];
    const int4 ci4 = reinterpret_cast<const int4 *>(a.cidx)[tid];
    SampState st{};
    if (tid == 0) st = samp_state_load(a);   // used by the draw only
    if (tid < SAMPLE_GRID) {
        const float ws = wave_sum(ps);
        int incl = c;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int u = __shfl_up(incl, off);
            if (lane >= off) incl += u;
        }
        scn[tid] = c;
        pre[tid] = incl - c;   // within this wave of slices
        const bool ovf = __ballot(c > SAMP_CAP) != 0;
        if (lane == 63) { wsum[w] = ws; wcnt[w] = incl; wovf[w] = ovf; }
    }
    if (tid < 64) { fp[tid] = -1.0f; fi[tid] = INT_MAX; }
    __syncthreads();
    float S = wsum[0];   // a fixed tree order over the slices
    int total = wcnt[0];
    bool ovf = wovf[0];
#pragma unroll
    for (int v = 1; v < SAMPLE_GRID / 64; v++) { S += wsum[v]; total += wcnt[v]; ovf = ovf || wovf[v]; }
    const int mode = (ovf || total < K) ? 2 : total <= WG ? 0 : total <= 4 * WG ? 1 : 2;

    // ---- 6. the first 64 in samp_before order into fp/fi --------------------
    if (mode != 2) {   // compact the passed tokens to [0, total)
        constexpr int TPS = SAMP_CAP / 4;   // threads per slice
        const int sl = tid / TPS, c = scn[sl];
        int b = pre[sl];
#pragma unroll
        for (int v = 0; v < SAMPLE_GRID / 64 - 1; v++) b += v < sl / 64 ? wcnt[v] : 0;
        const float cv[4] = { cv4.x, cv4.y, cv4.z, cv4.w };
        const int cx[4] = { ci4.x, ci4.y, ci4.z, ci4.w };
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 4 * (tid % TPS) + i;
            if (r < c) {
                const float pv = cv[i] / S;
                if (mode == 0) lk[b + r] = samp_key(pv, cx[i]);
                else { lp[b + r] = pv; li[b + r] = cx[i]; }
            }
        }
        __syncthreads();
    }
    if (mode == 0) {   // rank by counting: distinct indices make the ranks distinct
        if (tid < total) {
            const unsigned long long my = lk[tid];
            int rank = 0;
#pragma unroll 8
            for (int q = 0; q < total; q++) rank += lk[q] > my ? 1 : 0;
            if (rank < SAMPLE_TOPK_MAX) {
                fp[rank] = __uint_as_float((unsigned)(my >> 32));
                fi[rank] = (int)~(unsigned)my;
            }
        }
    } else if (mode == 1) {
        float v4[4];
        int i4[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = 4 * tid + i;
            v4[i] = q < total ? lp[q] : -1.0f;
            i4[i] = q < total ? li[q] : INT_MAX;
        }
        bitonic_sort<4>(v4, i4, lp, li);
        if (tid < SAMPLE_TOPK_MAX / 4) {
#pragma unroll
            for (int i = 0; i < 4; i++) { fp[4 * tid + i] = v4[i]; fi[4 * tid + i] = i4[i]; }
        }
    } else {
        // the whole vocabulary, 4 * WG - 64 logits at a time beside the running 64
        constexpr int STEP = 4 * WG - SAMPLE_TOPK_MAX;
#pragma unroll 1
        for (int base = 0; base < a.n; base += STEP) {
            float v4[4];
            int i4[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int q = 4 * tid + i;
                if (q < SAMPLE_TOPK_MAX) {
                    v4[i] = fp[q];
                    i4[i] = fi[q];
                } else {
                    const int x = base + q - SAMPLE_TOPK_MAX;
                    v4[i] = x < a.n ? samp_e(a.logits[x], T, M) / S : -1.0f;
                    i4[i] = x < a.n ? x : INT_MAX;
                }
            }
            bitonic_sort<4>(v4, i4, lp, li);
            __syncthreads();   // every read of fp/fi above is done
            if (tid < SAMPLE_TOPK_MAX / 4) {
#pragma unroll
                for (int i = 0; i < 4; i++) { fp[4 * tid + i] = v4[i]; fi[4 * tid + i] = i4[i]; }
            }
            __syncthreads();
        }
    }
    __syncthreads();
    if (tid >= 64) return;

    // ---- 7. min-p, top-p and the draw (sample.c:141-175) --------------------
    const float v = fp[lane];
    const int ix = fi[lane];
    int m = K;   // the first K are real tokens on every path above
    if (a.p.min_p > 0.0f && a.p.min_p < 1.0f) {
        const float thresh = a.p.min_p * lane_f(v, 0);
        const unsigned long long drop = __ballot(lane >= 1 && lane < m && !(v >= thresh));
        if (drop) m = __builtin_ctzll(drop);
    }
    float cum = 0.0f;   // sum of the sorted p[0..lane], in order (adding +0 after it changes nothing)
#pragma unroll
    for (int q = 0; q < 64; q += 4) {
        const float4 f = *reinterpret_cast<const float4 *>(fp + q);
        cum += q <= lane ? f.x : 0.0f;
        cum += q + 1 <= lane ? f.y : 0.0f;
        cum += q + 2 <= lane ? f.z : 0.0f;
        cum += q + 3 <= lane ? f.w : 0.0f;
    }
    if (a.p.top_p > 0.0f && a.p.top_p < 1.0f) {
        const unsigned long long hit = __ballot(lane < m && cum >= a.p.top_p);
        if (hit) m = __builtin_ctzll(hit) + 1;
    }
    const float cutoff = lane_f(cum, m - 1);
    // xorshift64* (sample.c:98-107) on the state lane 0 loaded
    const unsigned xh = (unsigned)__builtin_amdgcn_readlane((int)(st.rng >> 32), 0),
                   xl = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)st.rng, 0);
    unsigned long long x = ((unsigned long long)xh << 32) | xl;
    x ^= x >> 12; x ^= x << 25; x ^= x >> 27;
    const unsigned int u = (unsigned int)((x * 0x2545F4914F6CDD1DULL) >> 32);
    const float r = (float)(u >> 8) / 16777216.0f * cutoff;
    const unsigned long long in = __ballot(lane < m && r < cum);
    const int chosen = __builtin_amdgcn_readlane(ix, in ? __builtin_ctzll(in) : m - 1);
    if (lane == 0) {
        a.rng[0] = x;
        samp_emit(a, st, chosen);
    }
}

// --------------------------------------------------------------------------
// Any top_k (0 = no cap, or more than SAMPLE_TOPK_MAX): every token can be a
// candidate, so the whole (p desc, index asc) order is formed, and with it
// every token's probability exactly as the reference forms it: with a
// hundred thousand candidates the running sums are ~1e-5 apart, so a
// last-bit difference in the softmax sum would move a draw now and then.
// Five steps:
//   k_sw_e      e = expf(l/T - M) for every token, as the reference's C
//               library computes it (libm_expf.h);
//   k_sw_sum    one wave: S = the sum of e in index order, one addition at a
//               time (sample.c:131-133);
//   k_sw_tile   p = e / S and a 64-bit key per token, ~bits(p) above the
//               index, whose ascending order is the reference's stable
//               descending sort; 4096 keys per workgroup sorted in LDS
//               (bitonic network);
//   k_sw_merge  runs of L sorted keys merged pairwise by rank: each key's
//               place is its index in its run plus the number of keys of the
//               other run before it (a binary search), log2(n / 4096) passes;
//   k_sw_draw   one wave: top-k cap, min-p (a search of the sorted p), then
//               the running sum in sorted order, one addition at a time as
//               the reference does (sample.c:149-175), stopping where it
//               reaches top_p and keeping every partial sum; the draw is the
//               first partial sum above r, found by binary search (the sums
//               never decrease).
// The two sequential sums are the part that cannot be parallelized exactly;
// each costs about one dependent addition per token.

// e of a logit (the same expf as samp_e)
__device__ __forceinline__ float sw_e(float l, float T, float M) { return libm_expf(l / T - M); }

// The sum of the 64 lanes' v in lane order, added to acc one value at a time;
// lane q receives the running sum through its own value.
__device__ __forceinline__ float sw_chain(float &acc, float v) {
    float mine = 0.0f;
#pragma unroll
    for (int q = 0; q < 64; q++) {
        acc += lane_f(v, q);
        mine = (int)threadIdx.x == q ? acc : mine;
    }
    return mine;
}

__global__ __launch_bounds__(WG) void k_sw_e(SampleArgs a) {
    __shared__ float red[NWAVE];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float T = a.p.temperature;
    int lo, hi;
    samp_slice(a.n, lo, hi);
    float g = -INFINITY;
#pragma unroll
    for (int k = 0; k < SAMP_PARTS; k++)
        if (tid + k * WG < a.nparts) g = fmaxf(g, a.am_val[tid + k * WG]);
    g = wave_max(g);
    if (lane == 0) red[w] = g;
    __syncthreads();
    // max(l) / T == max(l / T): correctly rounded division is monotone
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) / T;
    float l[SAMP_E];
#pragma unroll
    for (int k = 0; k < SAMP_E; k++) l[k] = a.logits[min(lo + tid + k * WG, a.n - 1)];
#pragma unroll
    for (int k = 0; k < SAMP_E; k++) {
        const int i = lo + tid + k * WG;
        if (k * WG < hi - lo && i < hi) a.we[i] = sw_e(l[k], T, M);
    }
}

// one wave: S = e_0 + e_1 + ... in index order, into psum[0]
__global__ __launch_bounds__(64) void k_sw_sum(SampleArgs a) {
    const int lane = threadIdx.x;
    float acc = 0.0f;
    float nxt = a.we[min(lane, a.n - 1)];
    for (int c0 = 0; c0 < a.n; c0 += 64) {
        const float v = c0 + lane < a.n ? nxt : 0.0f;   // + 0 past the end changes nothing
        nxt = a.we[min(c0 + 64 + lane, a.n - 1)];      // the next chunk's load in flight
        (void)sw_chain(acc, v);
    }
    if (lane == 0) a.psum[0] = acc;
}

constexpr int SW_PER = SAMPLE_WIDE_TILE / WG;   // keys per thread in the tile sort

__global__ __launch_bounds__(WG) void k_sw_tile(SampleArgs a) {
    __shared__ unsigned long long ks[SAMPLE_WIDE_TILE];
    const int tid = threadIdx.x;
    const float S = a.psum[0];
    const int base = blockIdx.x * SAMPLE_WIDE_TILE;
#pragma unroll
    for (int k = 0; k < SW_PER; k++) {
        const int e = tid + k * WG, i = base + e;
        unsigned long long key = ~0ull;   // padding sorts last
        if (i < a.n) {
            const float p = a.we[i] / S;
            key = ((unsigned long long)~__float_as_uint(p) << 32) | (unsigned)i;
        }
        ks[e] = key;
    }
    for (int k = 2; k <= SAMPLE_WIDE_TILE; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            __syncthreads();
            for (int e = tid; e < SAMPLE_WIDE_TILE / 2; e += WG) {
                // pair (x, x + j), x with bit j clear; ascending where bit k of x is clear
                const int x = 2 * e - (e & (j - 1));
                const unsigned long long u = ks[x], v = ks[x + j];
                const bool up = (x & k) == 0;
                if ((u > v) == up) { ks[x] = v; ks[x + j] = u; }
            }
        }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < SW_PER; k++) a.wkeys[base + tid + k * WG] = ks[tid + k * WG];
}

// src runs of L keys, pairs (2r, 2r + 1) merged into dst runs of 2L.  A key of
// the first run goes after the other run's smaller keys, one of the second
// run after its smaller or equal ones (equal keys are padding), so every
// destination is distinct.
__global__ __launch_bounds__(WG) void k_sw_merge(const unsigned long long *src, unsigned long long *dst, int L) {
    const int i = blockIdx.x * WG + threadIdx.x;
    const unsigned long long key = src[i];
    const int r = i / L, j = i % L, b = (r & ~1) * L;
    const bool first = (r & 1) == 0;
    const unsigned long long *o = src + (first ? b + L : b);
    int lo = 0, hi = L;   // count of o[] before key
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        const unsigned long long v = o[mid];
        if (first ? v < key : v <= key) lo = mid + 1;
        else hi = mid;
    }
    dst[b + j + lo] = key;
}

__global__ __launch_bounds__(64) void k_sw_draw(SampleArgs a, const unsigned long long *keys) {
    const int lane = threadIdx.x;
    const SampState st = samp_state_load(a);
    auto pof = [](unsigned long long k) { return __uint_as_float(~(unsigned)(k >> 32)); };
    int m = a.p.top_k > 0 && a.p.top_k < a.n ? a.p.top_k : a.n;
    // min-p (sample.c:145-150): keep the first token, then while p >= min_p * p_0
    if (a.p.min_p > 0.0f && a.p.min_p < 1.0f) {
        const float thresh = a.p.min_p * pof(keys[0]);
        for (int c0 = 1; c0 < m; c0 += 64) {
            const int i = c0 + lane;
            const unsigned long long drop = __ballot(i < m && !(pof(keys[min(i, m - 1)]) >= thresh));
            if (drop) { m = c0 + __builtin_ctzll(drop); break; }
        }
    }
    // the running sum in sorted order; lane q keeps the sum through candidate c0 + q
    const bool tp = a.p.top_p > 0.0f && a.p.top_p < 1.0f;
    float cum = 0.0f, cutoff = 0.0f;
    bool done = false;
    for (int c0 = 0; c0 < m && !done; c0 += 64) {
        const int i = c0 + lane;
        const float pv = i < m ? pof(keys[i]) : 0.0f;   // + 0 past the end changes nothing
        const float mine = sw_chain(cum, pv);
        int last = m - 1;
        if (tp) {
            const unsigned long long hit = __ballot(i < m && mine >= a.p.top_p);
            if (hit) { last = c0 + __builtin_ctzll(hit); done = true; }
        }
        if (i < m && i <= last) a.wcum[i] = mine;
        if (done) { m = last + 1; cutoff = lane_f(mine, last - c0); }
    }
    if (!done) cutoff = cum;
    __builtin_amdgcn_s_waitcnt(0);   // this wave's partial sums are stored
    unsigned long long x = st.rng;
    x ^= x >> 12; x ^= x << 25; x ^= x >> 27;
    const unsigned int u = (unsigned int)((x * 0x2545F4914F6CDD1DULL) >> 32);
    const float r = (float)(u >> 8) / 16777216.0f * cutoff;
    int lo = 0, hi = m;   // first i < m with r < wcum[i]; none: the last candidate
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (r < a.wcum[mid]) hi = mid;
        else lo = mid + 1;
    }
    const int chosen = (int)(unsigned)keys[min(lo, m - 1)];
    if (lane == 0) {
        a.rng[0] = x;
        samp_emit(a, st, chosen);
    }
}

static int launch_sample_wide(hipStream_t st, const SampleArgs &b) {
    if (!b.we || !b.wkeys || !b.wcum) return -1;
    const int pad = sample_wide_pad(b.n);
    hipLaunchKernelGGL(k_sw_e, dim3(SAMPLE_GRID), dim3(WG), 0, st, b);
    hipLaunchKernelGGL(k_sw_sum, dim3(1), dim3(64), 0, st, b);
    hipLaunchKernelGGL(k_sw_tile, dim3(pad / SAMPLE_WIDE_TILE), dim3(WG), 0, st, b);
    unsigned long long *src = b.wkeys, *dst = b.wkeys + pad;
    for (int L = SAMPLE_WIDE_TILE; L < pad; L <<= 1) {
        hipLaunchKernelGGL(k_sw_merge, dim3(pad / WG), dim3(WG), 0, st, src, dst, L);
        std::swap(src, dst);
    }
    hipLaunchKernelGGL(k_sw_draw, dim3(1), dim3(64), 0, st, b, (const unsigned long long *)src);
    return 0;
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

bool sample_penalized(const SampleArgs &a) {
    return a.hist && a.hist_cap > 0 &&
        (a.p.repeat_penalty != 1.0f || a.p.frequency_penalty != 0.0f || a.p.presence_penalty != 0.0f);
}

int launch_sample(hipStream_t st, const SampleArgs &a) {
    if (a.n <= 0 || (a.n + SAMPLE_GRID - 1) / SAMPLE_GRID > SAMPLE_SLICE_MAX) return -1;
    const bool pen = sample_penalized(a);
    if (pen) hipLaunchKernelGGL(k_samp_pen, dim3(1), dim3(WG), 0, st, a);
    if (a.p.temperature <= 0.0f) {
        ArgmaxArgs g{};
        g.logits = a.logits; g.n = a.n; g.pval = a.am_val; g.pidx = a.am_idx;
        g.tokpos = a.tokpos; g.out = a.out; g.cap = a.cap;
        if (launch_argmax(st, g)) return -1;
        hipLaunchKernelGGL(k_samp_greedy_emit, dim3(1), dim3(64), 0, st, a);
        return 0;
    }
    const bool wide = a.exact || a.p.top_k < 1 || a.p.top_k > SAMPLE_TOPK_MAX;
    SampleArgs b = a;
    if (pen || b.nparts <= 0) {   // per-part maxima of the logits as they now are
        ArgmaxArgs g{};
        g.logits = a.logits; g.n = a.n; g.pval = a.am_val; g.pidx = a.am_idx;
        const int nb = (a.n + ARGMAX_PER_THREAD * WG - 1) / (ARGMAX_PER_THREAD * WG);
        if (nb > ARGMAX_MAX_BLOCKS) return -1;
        hipLaunchKernelGGL(k_argmax_part, dim3(nb), dim3(WG), 0, st, g);
        b.nparts = nb;
    }
    if (b.nparts > SAMP_PARTS * WG) return -1;
    if (wide) return launch_sample_wide(st, b);
    hipLaunchKernelGGL(k_samp_fused, dim3(SAMPLE_GRID), dim3(WG), 0, st, b);
    return 0;
}

}  // namespace ehip
