// libm_expf.h — expf as the reference's C library computes it, for host and
// device: glibc 2.35's single-precision exponential (sysdeps/ieee754/flt-32/
// e_expf.c with the exp2f_data.c table and cubic, the variant x86-64 selects
// on FMA hardware, where the compiler fuses the range reduction and the
// polynomial into FMAs).  x N/ln2 = k + r, |r| <= 1/2, N = 32;
// exp(x) = 2^(k/N) 2^(r/N) with 2^(k/N) from a table of 2^(i/N) (k's integer
// part added into the exponent bits) and 2^(r/N) ~ C0 r^3 + C1 r^2 + C2 r + 1,
// all in double precision, rounded once to float.  The table holds the bits
// of 2^(i/32), correctly rounded, minus i << 47.  This restatement equals the
// host library on every one of the 2^32 inputs; a correctly rounded expf
// differs from it on about one input in 1,600.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ehip {

__host__ __device__ inline float libm_expf(float x) {
    constexpr unsigned long long tab[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
    };
    constexpr double InvLn2N = 0x1.71547652b82fep+0 * 32, Shift = 0x1.8p+52;
    constexpr double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                     C2 = 0x1.62e42ff0c52d6p-1 / 32;
    const uint32_t ux = __builtin_bit_cast(uint32_t, x), abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                       // |x| >= 88, or not finite
        if (ux == 0xff800000u) return 0.0f;      // -inf
        if (abstop >= 0x7f8) return x + x;       // +inf, nan
        if (x > 0x1.62e42ep6f) return __builtin_inff();   // above log(2^128)
        if (x < -0x1.9fe368p6f) return 0.0f;     // below log(2^-150)
    }
    const double xd = (double)x;
    double kd = __builtin_fma(InvLn2N, xd, Shift);
    const unsigned long long ki = __builtin_bit_cast(unsigned long long, kd);
    kd -= Shift;
    const double r = __builtin_fma(InvLn2N, xd, -kd);
    const double sc = __builtin_bit_cast(double, tab[ki & 31] + (ki << 47));
    const double z = __builtin_fma(C0, r, C1);
    const double r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return (float)(y * sc);
}

}  // namespace ehip
