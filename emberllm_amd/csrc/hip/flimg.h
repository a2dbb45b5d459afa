// flimg.h — the K/V tile images of the matrix-core prefill attention
// (attention.hip: k_pf_kvsplit writes them, k_pf_flash16 stages them into
// LDS as they lie; the long passes' q|k|v product writes a pass's own tiles
// in its epilogue, gemm.hip).  The layout is described beside k_pf_kvsplit.
#pragma once
#include "dev_common.h"

namespace ehip {

// query rows per workgroup and keys per tile of the matrix-core attention
constexpr int FL_BR = 64, FL_BK = 64;

// the image row of key k within its tile
__device__ __forceinline__ int fl_krow(int k) {
    return (k & ~31) | ((k & 4) << 2) | ((k & 24) >> 1) | (k & 3);
}
// power-of-two exponent that brings a group maximum m into [2^14, 2^15)
__device__ __forceinline__ int fl_exp(float m) { return 15 - __builtin_amdgcn_frexp_expf(m); }
__device__ __forceinline__ uint32_t fl_pack(_Float16 a, _Float16 b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// geometry of one (kv head, tile) image, in bytes; the LDS copy is the same
// bytes at the same offsets (K and exponents in one array, V in another)
template <int HD, bool F16> struct FlImg {
    static constexpr int NP = F16 ? 1 : 2;                 // planes: hi, and lo for an fp32 cache
    static constexpr int KRB = 2 * HD;                     // K plane row bytes
    static constexpr int KRP = HD / 8;                     // 16-byte pieces per K row
    static constexpr int KBYTES = NP * FL_BK * KRB;        // K planes
    static constexpr int EBYTES = F16 ? 0 : 2 * FL_BK * 4; // int kex[64], vex[64] (fp32 cache)
    static constexpr int KE = KBYTES + EBYTES;             // first staging part
    static constexpr int VBYTES = NP * HD * FL_BK * 2;     // V^T planes, 128-byte rows
    static constexpr int HBYTES = KE + VBYTES;             // bytes per image
    static constexpr int SLAB = 1024;                      // one wave's direct-to-LDS load
    static constexpr int KE_SLABS = (KE + SLAB - 1) / SLAB, V_SLABS = VBYTES / SLAB;
    static_assert(KE % 16 == 0 && VBYTES % SLAB == 0 && (KRP & (KRP - 1)) == 0, "image geometry");
    // K row r (plane-major: plane * 64 + row), piece p
    static __device__ __forceinline__ int k_at(int r, int p) { return r * KRB + 16 * (p ^ (r & (KRP - 1))); }
    // V^T row d (plane-major: plane * HD + dim), piece p (keys 8p .. 8p + 7)
    static __device__ __forceinline__ int v_at(int d, int p) { return d * 128 + 16 * (p ^ (d & 7)); }
};

}  // namespace ehip
