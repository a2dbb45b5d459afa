// noalloc.hip — ehip_sample_noalloc: the device sampler for callers that
// cannot allocate (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).
//
// It runs the kernels of ehip_sample (launch_sample, sample.hip: penalties,
// temperature, softmax, top-k <= 64, min-p, top-p, one xorshift64* draw, as
// src/sample.c:76-175) on logits the caller already holds in device memory,
// and keeps every intermediate the kernels need (slice sums, candidate
// lists, per-part maxima, the arrival counter, the token/position triple)
// in one file-scope device array, `scratch`, instead of state buffers.
//
// The array is SCRATCH_BYTES per GPU, held by each GPU the library runs on
// until the process ends.  Host code never passes the array's name to a
// kernel or copy (in host code it only names a host-side stand-in): the
// first call on a device (or ehip_state_create on it) looks up the device
// address with hipGetSymbolAddress, once per device with that device
// current, and every launch uses that address.  All calls on one GPU share
// its array and the last call's contents stay there; the parts that must
// start at zero (the counters and the token triple) are cleared by a small
// fill kernel at the start of every call, on the caller's stream.  Calls
// that overlap on one GPU (two streams, two threads) race on the array.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "../../../include/ehip.h"
#include "kernels.h"

namespace ehip {

// layout of the scratch array (byte offsets, 256-byte aligned pieces)
constexpr size_t SCR_TOKPOS = 0;                                                   // int[4]
constexpr size_t SCR_SCNT = 256;                                                   // int[2 * SAMPLE_GRID]
constexpr size_t SCR_PSUM = SCR_SCNT + 4 * 2 * SAMPLE_GRID;                        // float[SAMPLE_GRID]
constexpr size_t SCR_AMV = SCR_PSUM + 4 * SAMPLE_GRID;                             // float[ARGMAX_MAX_BLOCKS]
constexpr size_t SCR_AMI = SCR_AMV + 4 * ARGMAX_MAX_BLOCKS;                        // int[ARGMAX_MAX_BLOCKS]
constexpr size_t SCR_CVAL = SCR_AMI + 4 * ARGMAX_MAX_BLOCKS;                       // float[GRID][TOPK_MAX]
constexpr size_t SCR_CIDX = SCR_CVAL + 4 * (size_t)SAMPLE_GRID * SAMPLE_TOPK_MAX;  // int[GRID][TOPK_MAX]
constexpr size_t SCRATCH_BYTES = SCR_CIDX + 4 * (size_t)SAMPLE_GRID * SAMPLE_TOPK_MAX;
static_assert(SCR_SCNT % 256 == 0 && SCR_PSUM % 256 == 0 && SCR_AMV % 256 == 0 && SCR_CVAL % 256 == 0 &&
              SCR_CIDX % 256 == 0, "scratch pieces are 256-byte aligned");
// the largest vocabulary the array's per-part maxima and slices cover
constexpr int NOALLOC_MAX_LOGITS = ARGMAX_MAX_BLOCKS * 4 * WG;
static_assert(NOALLOC_MAX_LOGITS <= SAMPLE_GRID * SAMPLE_SLICE_MAX, "slices cover the parts");

static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

// zero the first `n` ints at p (graph-capture safe, unlike a memset node)
__global__ void k_zero_ints(int *p, int n) {
    if ((int)threadIdx.x < n) p[threadIdx.x] = 0;
}

constexpr int MAX_DEVICES = 64;
static void *g_ptr[MAX_DEVICES];
static std::mutex g_mu;

// The device address of `scratch` on the current device, looked up once
// per device; nullptr on failure (the HIP error is named in *why).
static unsigned char *scratch_ptr(hipError_t *why) {
    int dev = -1;
    *why = hipGetDevice(&dev);
    if (*why != hipSuccess) return nullptr;
    if (dev < 0 || dev >= MAX_DEVICES) { *why = hipErrorInvalidDevice; return nullptr; }
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[dev]) {
        void *p = nullptr;
        *why = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (*why != hipSuccess || !p) return nullptr;
        g_ptr[dev] = p;
    }
    return static_cast<unsigned char *>(g_ptr[dev]);
}

}  // namespace ehip

using namespace ehip;

static int fail(const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    set_error_text(buf);
    return -1;
}

// Set-up on the current device (called by ehip_state_create): resolves the
// scratch address before any caller captures a graph on the device.
extern "C" int ehip_noalloc_setup(void) {
    hipError_t e = hipSuccess;
    if (!scratch_ptr(&e)) return fail("ehip_sample_noalloc: scratch address lookup failed: %s", hipGetErrorString(e));
    return 0;
}

extern "C" int ehip_sample_noalloc(float *logits, int n, const EmberSampler *params, uint64_t *rng_state,
                                   int *history, int *hist_meta, int *token, void *stream) {
    if (!logits || !params || !rng_state || !token) return fail("ehip_sample_noalloc: null argument");
    if (n <= 0 || n > NOALLOC_MAX_LOGITS)
        return fail("ehip_sample_noalloc: %d logits; the scratch array covers 1..%d", n, NOALLOC_MAX_LOGITS);
    if (params->temperature > 0.0f && (params->top_k < 1 || params->top_k > SAMPLE_TOPK_MAX))
        return fail("ehip_sample_noalloc: top_k %d outside [1,%d]", params->top_k, SAMPLE_TOPK_MAX);
    const int cap = history && hist_meta ? params->hist_cap : 0;
    if (cap < 0) return fail("ehip_sample_noalloc: negative history capacity");
    hipError_t e = hipSuccess;
    unsigned char *base = scratch_ptr(&e);
    if (!base) return fail("ehip_sample_noalloc: scratch address lookup failed: %s", hipGetErrorString(e));
    hipStream_t st = static_cast<hipStream_t>(stream);

    SampleArgs a{};
    a.logits = logits; a.n = n;
    a.p.temperature = params->temperature; a.p.top_p = params->top_p; a.p.min_p = params->min_p;
    a.p.repeat_penalty = params->repeat_penalty; a.p.presence_penalty = params->presence_penalty;
    a.p.frequency_penalty = params->frequency_penalty; a.p.top_k = params->top_k;
    a.rng = reinterpret_cast<unsigned long long *>(rng_state);
    a.hist = cap > 0 ? history : nullptr;
    a.hist_meta = hist_meta;
    a.hist_cap = cap;
    a.tokpos = reinterpret_cast<int *>(base + SCR_TOKPOS);
    a.scnt = reinterpret_cast<int *>(base + SCR_SCNT);
    a.psum = reinterpret_cast<float *>(base + SCR_PSUM);
    a.am_val = reinterpret_cast<float *>(base + SCR_AMV);
    a.am_idx = reinterpret_cast<int *>(base + SCR_AMI);
    a.cval = reinterpret_cast<float *>(base + SCR_CVAL);
    a.cidx = reinterpret_cast<int *>(base + SCR_CIDX);
    a.nparts = 0;            // per-part maxima are computed from these logits
    a.out = token; a.cap = 1;
    // the token triple and the counters (per-slice counts, then the arrival
    // counter) start at zero
    hipLaunchKernelGGL(k_zero_ints, dim3(1), dim3(64), 0, st, a.tokpos, 4);
    hipLaunchKernelGGL(k_zero_ints, dim3(1), dim3(2 * SAMPLE_GRID), 0, st, a.scnt, 2 * SAMPLE_GRID);
    if (launch_sample(st, a)) return fail("ehip_sample_noalloc: sampler launch failed");
    e = hipGetLastError();
    if (e != hipSuccess) return fail("ehip_sample_noalloc: launch: %s", hipGetErrorString(e));
    return 0;
}
