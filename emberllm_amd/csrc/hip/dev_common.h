// dev_common.h — device-side layout and helpers shared by the gfx950 kernels.
//
// Weight layout in HBM (repacked at upload; the .ember file is untouched):
//   Q8_0  q: int8  [rows][cols]      row-major, rows 16-byte aligned
//         d: fp16  [rows][cols/32]   one scale per 32-weight block
//   Q4_0  q: uint8 [rows][cols/2]    16 bytes per block, byte i holds weight i
//                                    (low nibble) and weight i+16 (high nibble)
//         d: fp16  [rows][cols/32]
//   F32   q: float [rows][cols]
// The quantized payload and the scales are separate arrays so every lane
// issues aligned 16-byte loads (the file's 34/18-byte blocks are not aligned).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ehip {

enum { DT_F32 = 0, DT_Q8 = 1, DT_Q4 = 2 };
enum { ROPE_INTERLEAVED = 0, ROPE_NEOX = 1 };
constexpr int QB = 32;      // weights per quant block
constexpr int WG = 256;     // threads per workgroup (4 wave64)
// Native 4-float vector.  Arrays of HIP's float4 struct that a lambda fills
// and another reads can stay in scratch memory; arrays of this type are kept
// in registers.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
constexpr int NWAVE = WG / 64;

struct DMat {
    int dtype, rows, cols;
    const uint8_t *q;       // payload (see header comment)
    const uint16_t *d;      // fp16 scale bits, nullptr for F32
};

__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}
// float -> half, round to nearest even (hardware conversion, default mode)
__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Sum over the 64 lanes with DPP lane moves (no LDS round trips); the total
// is returned to every lane from lane 63.  The association order is fixed:
// pairs, quads, eighths, rows of 16, then rows combined.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = dpp_add<0xb1, 0xf>(v);    // quad_perm [1,0,3,2]
    v = dpp_add<0x4e, 0xf>(v);    // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xf>(v);   // row_half_mirror
    v = dpp_add<0x140, 0xf>(v);   // row_mirror: every lane of a row holds its row sum
    v = dpp_add<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
    v = dpp_add<0x143, 0xc>(v);   // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_sum(float v) { return wave_sum_dpp(v); }

// v[i] + v[i ^ 16] and v[i] + v[i ^ 32] in every lane (gfx950 lane swaps)
__device__ __forceinline__ float xor16_add(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_add(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// v[i] + v[i ^ 8] within each row of 16 (row_ror:8)
__device__ __forceinline__ float xor8_add(float v) { return dpp_add<0x128, 0xf>(v); }

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_max(float v) {
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), CTRL,
                                                               ROW_MASK, 0xf, false)));
}
__device__ __forceinline__ float wave_max(float v) {
    v = dpp_max<0xb1, 0xf>(v);
    v = dpp_max<0x4e, 0xf>(v);
    v = dpp_max<0x141, 0xf>(v);
    v = dpp_max<0x140, 0xf>(v);
    v = dpp_max<0x142, 0xa>(v);
    v = dpp_max<0x143, 0xc>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Maximum / integer sum over aligned groups of 8 lanes; every lane of the
// group receives the result.
__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xf, 0xf, false)));
    return v;
}
__device__ __forceinline__ int sum8(int v) {
    v += __builtin_amdgcn_mov_dpp(v, 0xb1, 0xf, 0xf, false);
    v += __builtin_amdgcn_mov_dpp(v, 0x4e, 0xf, 0xf, false);
    v += __builtin_amdgcn_mov_dpp(v, 0x141, 0xf, 0xf, false);
    return v;
}

// Block-wide sum over 256 threads; `red` must hold NWAVE floats.  Every
// thread receives the total.
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < NWAVE; i++) t += red[i];
    return t;
}

// Q8_0 quantization of one 32-element block held by 32 consecutive lanes
// (kernels.c:73-92): d = amax/127, inverse from the unrounded d, round half
// away from zero, clamp to +-127, scale stored as fp16.  Returns the code and
// sets *dq to the fp16-rounded scale as float (what the dot products use).
__device__ __forceinline__ int quant_q8_lane(float v, float *dq) {
    float a = fabsf(v);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off));
    float d = a / 127.0f;
    float id = d > 0.0f ? 1.0f / d : 0.0f;
    float r = roundf(v * id);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    *dq = h2f(f2h(d));
    return (int)r;
}

__device__ __forceinline__ int sdot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

}  // namespace ehip
