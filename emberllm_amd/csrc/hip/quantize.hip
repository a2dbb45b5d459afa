// quantize.hip — the requantizer's block quantization on the GPU
// (ehip_quantize_rows), which replaces the per-row quantizer loops of
// quantize_tensor (src/quant.c:26-57) called by ember_quantize_file.
//
// fp32 rows stream from the caller's (mapped) host memory through a ring of
// pinned slots: host threads copy a slot's rows in, the slot's DMA, one
// quantize launch per tensor in it and the DMA of the encoded blocks back to
// a pinned output slot follow on one stream, and the encoded blocks are
// copied to the caller's buffers when the slot comes round again.  Each
// thread encodes one 32-weight block with the reference's arithmetic
// (src/kernels.c:73-115), so the blocks equal the host quantizers' byte for
// byte:
//   Q8_0: amax over |x| (first maximum), d = amax/127, inverse from the
//         unrounded d (0 when d is 0), codes round half away from zero,
//         clamped to +-127, d stored as fp16 (RNE).
//   Q4_0: v = the element of largest magnitude (first one), d = v/-8,
//         inverse 1/d (0 when d is 0), codes (int)(x*inv + 8.5) truncated
//         and clamped to 0..15, element i in the low and element i+16 in the
//         high nibble of byte i.
// When a block's largest magnitude is below about 3.7e-37 (Q8_0) or 2.4e-38
// (Q4_0), 1/d overflows to infinity and x*inv is infinite or NaN; a block
// holding an infinity has d infinite and inverse 0, so its infinite (and NaN)
// elements give NaN products.  The reference converts with (int)lroundf(p)
// (Q8_0) and (int)(p + 8.5f) (Q4_0); on x86-64 those give LONG_MIN and
// INT_MIN for such products, whose int values clamp to code 0 in both
// encodings whatever the sign.  The device's conversions would saturate
// instead, so such products take the host's result explicitly.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <vector>

#include "../../../include/ehip.h"
#include "kernels.h"
#include "staging.h"

namespace {

using namespace ehip;

// float -> fp16 bits, round to nearest even, with the host conversion's
// handling of every input: magnitudes that round past 65504, infinities and
// NaNs give a signed infinity; below 2^-14 the result is a multiple of 2^-24.
__device__ __forceinline__ uint16_t half_bits(float f) {
    uint32_t u = __float_as_uint(f);
    const uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) return (uint16_t)(sign | (uint32_t)rintf(__uint_as_float(a) * 16777216.0f));
    a += 0xfffu + ((a >> 13) & 1u);
    return (uint16_t)(sign | ((a - 0x38000000u) >> 13));
}

// One thread per block: x holds nblk * 32 floats (16-byte aligned), out
// receives nblk encoded blocks of 34 (Q8_0) or 18 (Q4_0) bytes.
template <int DT>
__global__ __launch_bounds__(256) void k_quant_blocks(const float *__restrict__ x, size_t nblk,
                                                      uint16_t *__restrict__ out) {
    constexpr int HALVES = DT == DT_Q8 ? 17 : 9;   // block size in 16-bit words
    for (size_t b = blockIdx.x * (size_t)blockDim.x + threadIdx.x; b < nblk; b += (size_t)gridDim.x * blockDim.x) {
        float v[32];
        const float4 *src = reinterpret_cast<const float4 *>(x + b * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 t = src[i];
            v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
        }
        uint16_t *o = out + b * HALVES;
        if (DT == DT_Q8) {
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; i++) amax = fabsf(v[i]) > amax ? fabsf(v[i]) : amax;
            const float d = amax / 127.0f;
            const float inv = d > 0.0f ? 1.0f / d : 0.0f;
            o[0] = half_bits(d);
            auto code = [inv](float x) {
                // (int)lroundf(p): the rounded value (half away from zero)
                // reduced to its low 32 bits, and 0 (the low bits of
                // LONG_MIN) for NaN, infinities and |p| >= 2^63
                const float r = roundf(__fmul_rn(x, inv));
                int q = fabsf(r) < 0x1p63f ? (int)(long long)r : 0;
                q = q > 127 ? 127 : q < -127 ? -127 : q;
                return (uint32_t)q & 0xffu;
            };
#pragma unroll
            for (int i = 0; i < 16; i++) o[1 + i] = (uint16_t)(code(v[2 * i]) | (code(v[2 * i + 1]) << 8));
        } else {
            float amax = 0.0f, vmax = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; i++)
                if (fabsf(v[i]) > amax) { amax = fabsf(v[i]); vmax = v[i]; }
            const float d = vmax / -8.0f;
            const float inv = d != 0.0f ? 1.0f / d : 0.0f;
            o[0] = half_bits(d);
            uint32_t byte[16];
            auto code = [inv](float x) {
                const float t = __fadd_rn(__fmul_rn(x, inv), 8.5f);
                const int q = fabsf(t) < 0x1p31f ? (int)t : 0;
                return (uint32_t)(q < 0 ? 0 : q > 15 ? 15 : q);
            };
#pragma unroll
            for (int i = 0; i < 16; i++) byte[i] = code(v[i]) | (code(v[i + 16]) << 4);
#pragma unroll
            for (int i = 0; i < 8; i++) o[1 + i] = (uint16_t)(byte[2 * i] | (byte[2 * i + 1] << 8));
        }
    }
}

struct QuantStager {
    static constexpr int SLOTS = 3;
    static constexpr size_t SLOT_MAX = (size_t)32 << 20;   // fp32 bytes per slot
    struct Seg { int job; int64_t r, n; size_t in_off, out_off; };
    size_t in_bytes, out_bytes;
    hipStream_t st = nullptr;
    uint8_t *pin_in[SLOTS] = {}, *dev_in[SLOTS] = {}, *dev_out[SLOTS] = {}, *pin_out[SLOTS] = {};
    hipEvent_t ev[SLOTS] = {};
    std::vector<Seg> pending[SLOTS];   // blocks waiting in pin_out[k] for their destinations
    int next = 0, threads = 1;
    bool ok = false;

    explicit QuantStager(size_t total) {
        in_bytes = std::min(SLOT_MAX, std::max<size_t>(total, 128));
        in_bytes = (in_bytes + 127) & ~(size_t)127;
        out_bytes = in_bytes / 128 * 34;   // 32 floats in, at most 34 bytes out
        if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) { st = nullptr; return; }
        for (int i = 0; i < SLOTS; i++) {
            if (hipHostMalloc(reinterpret_cast<void **>(&pin_in[i]), in_bytes, hipHostMallocDefault) != hipSuccess) {
                pin_in[i] = nullptr;
                return;
            }
            if (hipHostMalloc(reinterpret_cast<void **>(&pin_out[i]), out_bytes, hipHostMallocDefault) != hipSuccess) {
                pin_out[i] = nullptr;
                return;
            }
            if (hipMalloc(reinterpret_cast<void **>(&dev_in[i]), in_bytes) != hipSuccess) { dev_in[i] = nullptr; return; }
            if (hipMalloc(reinterpret_cast<void **>(&dev_out[i]), out_bytes) != hipSuccess) { dev_out[i] = nullptr; return; }
            if (hipEventCreateWithFlags(&ev[i], hipEventDisableTiming) != hipSuccess) { ev[i] = nullptr; return; }
        }
        threads = staging_threads();
        ok = true;
    }
    ~QuantStager() {
        if (st) (void)hipStreamSynchronize(st);
        for (int i = 0; i < SLOTS; i++) {
            if (ev[i]) (void)hipEventDestroy(ev[i]);
            if (dev_in[i]) (void)hipFree(dev_in[i]);
            if (dev_out[i]) (void)hipFree(dev_out[i]);
            if (pin_in[i]) (void)hipHostFree(pin_in[i]);
            if (pin_out[i]) (void)hipHostFree(pin_out[i]);
        }
        if (st) (void)hipStreamDestroy(st);
    }

    static size_t out_row(const EhipQuantJob &j) { return (size_t)(j.cols / 32) * (j.dtype == DT_Q8 ? 34 : 18); }

    // Wait for slot k's last round and copy its encoded blocks out.
    bool drain(int k, const EhipQuantJob *jobs) {
        if (hipEventSynchronize(ev[k]) != hipSuccess) { set_error_text("requantizer: waiting for a slot failed"); return false; }
        std::vector<CopySpan> spans;
        for (const Seg &g : pending[k]) {
            const size_t ob = out_row(jobs[g.job]);
            spans.push_back({ static_cast<uint8_t *>(jobs[g.job].dst) + g.r * ob, pin_out[k] + g.out_off, g.n * ob });
        }
        parallel_copy(spans, threads);
        pending[k].clear();
        return true;
    }

    bool flush(const EhipQuantJob *jobs, std::vector<Seg> &segs, size_t used_in, size_t used_out) {
        if (segs.empty()) return true;
        const int k = next;
        next = (next + 1) % SLOTS;
        if (!drain(k, jobs)) return false;
        std::vector<CopySpan> spans;
        for (const Seg &g : segs) {
            const size_t ib = (size_t)jobs[g.job].cols * 4;
            spans.push_back({ pin_in[k] + g.in_off, reinterpret_cast<const uint8_t *>(jobs[g.job].src) + g.r * ib, g.n * ib });
        }
        parallel_copy(spans, threads);
        bool good = hipMemcpyAsync(dev_in[k], pin_in[k], used_in, hipMemcpyHostToDevice, st) == hipSuccess;
        for (const Seg &g : segs) {
            const EhipQuantJob &j = jobs[g.job];
            const size_t nblk = (size_t)g.n * (j.cols / 32);
            const int grid = (int)std::min<size_t>(8192, (nblk + 255) / 256);
            const float *x = reinterpret_cast<const float *>(dev_in[k] + g.in_off);
            uint16_t *o = reinterpret_cast<uint16_t *>(dev_out[k] + g.out_off);
            if (j.dtype == DT_Q8) k_quant_blocks<DT_Q8><<<grid, 256, 0, st>>>(x, nblk, o);
            else k_quant_blocks<DT_Q4><<<grid, 256, 0, st>>>(x, nblk, o);
            good = good && hipGetLastError() == hipSuccess;
        }
        good = good && hipMemcpyAsync(pin_out[k], dev_out[k], used_out, hipMemcpyDeviceToHost, st) == hipSuccess &&
               hipEventRecord(ev[k], st) == hipSuccess;
        if (!good) { set_error_text("requantizer: queueing a slot's copies or kernels failed"); return false; }
        pending[k] = segs;
        segs.clear();
        return true;
    }

    bool run(const EhipQuantJob *jobs, int n_jobs) {
        std::vector<Seg> segs;
        size_t used_in = 0, used_out = 0;
        for (int i = 0; i < n_jobs; i++) {
            const EhipQuantJob &j = jobs[i];
            const size_t ib = (size_t)j.cols * 4, ob = out_row(j);
            for (int64_t r = 0; r < j.rows;) {
                const int64_t fit = (int64_t)((in_bytes - used_in) / ib);
                if (fit == 0) {
                    if (!flush(jobs, segs, used_in, used_out)) return false;
                    used_in = used_out = 0;
                    continue;
                }
                const int64_t n = std::min<int64_t>(fit, j.rows - r);
                segs.push_back({ i, r, n, used_in, used_out });
                used_in += (size_t)n * ib;
                used_out += (size_t)n * ob;
                r += n;
            }
        }
        if (!flush(jobs, segs, used_in, used_out)) return false;
        for (int t = 0; t < SLOTS; t++)
            if (!drain((next + t) % SLOTS, jobs)) return false;
        return true;
    }
};

}  // namespace

extern "C" int ehip_quantize_rows(const EhipQuantJob *jobs, int n_jobs) {
    if (n_jobs < 0 || (n_jobs > 0 && !jobs)) { set_error_text("ehip_quantize_rows: no jobs"); return -1; }
    size_t total = 0;
    for (int i = 0; i < n_jobs; i++) {
        const EhipQuantJob &j = jobs[i];
        char msg[160];
        if (j.dtype != DT_Q8 && j.dtype != DT_Q4) {
            snprintf(msg, sizeof msg, "ehip_quantize_rows: job %d: target dtype %d is not Q8_0 or Q4_0", i, j.dtype);
            set_error_text(msg);
            return -1;
        }
        if (j.cols <= 0 || j.cols % 32 || (size_t)j.cols * 4 > QuantStager::SLOT_MAX || j.rows < 0 ||
            (j.rows > 0 && (!j.src || !j.dst))) {
            snprintf(msg, sizeof msg, "ehip_quantize_rows: job %d: %lld rows of %d values cannot be quantized", i,
                     (long long)j.rows, j.cols);
            set_error_text(msg);
            return -1;
        }
        total += (size_t)j.rows * j.cols * 4;
    }
    if (total == 0) return 0;
    if (hipSetDevice(0) != hipSuccess) { set_error_text("hipSetDevice(0) failed: no usable GPU"); return -1; }
    QuantStager q(total);
    if (!q.ok) { set_error_text("requantizer: allocating the staging buffers failed"); return -1; }
    return q.run(jobs, n_jobs) ? 0 : -1;
}
