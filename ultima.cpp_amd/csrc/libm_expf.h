// Single-precision exp that returns the same bits as glibc 2.35's expf on
// x86-64 with FMA, on host and device.
//
// The reference sampler computes softmax numerators with std::exp(float)
// (src/sampler/sampler.cpp:135), i.e. glibc expf. Reproducing its bits on the
// GPU makes every downstream probability, cumulative sum and draw exactly
// reproducible instead of merely close.
//
// Method (the table-driven exp2 reduction of the ARM optimized-routines
// expf that glibc ships, sysdeps/ieee754/flt-32/e_expf.c):
//   z  = x * 32/ln2, k = round(z) (via the 1.5*2^52 shift), r = z - k
//   2^(k/32) = T[k mod 32] with the exponent bits of k/32 added
//   exp(x) ~= 2^(k/32) * (1 + C2 r + C1 r^2 + C0 r^3), all in double
// glibc's x86-64 build selects the FMA-compiled variant at run time, where the
// compiler fuses r = z - k into fma(InvLn2N, x, -k) and each polynomial step;
// the same fused operations are spelled out here. T[i] is the double nearest
// 2^(i/32) with i << 47 subtracted from its bit pattern. An exhaustive check
// over every non-NaN float (tests/test_libm_expf.py) shows bit equality with
// the host's expf.
//
// Upstream notice. The method, the table layout and the three polynomial
// coefficients follow the expf of ARM's optimized-routines
// (https://github.com/ARM-software/optimized-routines, math/expf.c and
// math/exp2f_data.c; Copyright (c) 2017-2018, Arm Limited; MIT licence), as
// shipped in the GNU C Library (sysdeps/ieee754/flt-32/e_expf.c and
// e_exp2f_data.c; Copyright (C) 2017-2022 Free Software Foundation, Inc.;
// LGPL-2.1-or-later). The table entries are the doubles nearest 2^(i/32) and
// the coefficients are those published with that method; they are restated
// here so that the device reproduces the host library's results bit for bit.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define HSAMP_HD __host__ __device__
#else
#define HSAMP_HD
#include <cmath>
#endif

namespace hsamp {

HSAMP_HD inline double bits_to_f64(uint64_t u) {
    union { uint64_t u; double d; } c{u};
    return c.d;
}
HSAMP_HD inline uint64_t f64_to_bits(double d) {
    union { double d; uint64_t u; } c{d};
    return c.u;
}
HSAMP_HD inline uint32_t f32_to_bits(float f) {
    union { float f; uint32_t u; } c{f};
    return c.u;
}

HSAMP_HD inline double fma_f64(double a, double b, double c) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_fma(a, b, c);
#else
    return std::fma(a, b, c);
#endif
}

// 2^(i/32), i = 0..31, as double bit patterns minus (i << 47).
inline constexpr uint64_t kExpT[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// expf with the table read from T (device code passes a copy in LDS).
HSAMP_HD inline float libm_expf_t(float x, const uint64_t* T) {
    constexpr double InvLn2N = 0x1.71547652b82fep+0 * 32;
    constexpr double Shift = 0x1.8p+52;
    constexpr double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    constexpr double C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    constexpr double C2 = 0x1.62e42ff0c52d6p-1 / 32;

    const uint32_t ux = f32_to_bits(x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                        // |x| >= 88 or x is NaN/inf
        if (ux == 0xff800000u) return 0.0f;       // -inf
        if (abstop >= 0x7f8) return x + x;        // NaN or +inf
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double xd = static_cast<double>(x);
    const double z = InvLn2N * xd;
    double kd = z + Shift;
    const uint64_t ki = f64_to_bits(kd);
    kd -= Shift;
    const double r = fma_f64(InvLn2N, xd, -kd);
    uint64_t t = T[ki % 32];
    t += ki << 47;
    const double s = bits_to_f64(t);
    const double zp = fma_f64(C0, r, C1);
    const double r2 = r * r;
    double y = fma_f64(C2, r, 1.0);
    y = fma_f64(zp, r2, y);
    y = y * s;
    return static_cast<float>(y);
}

HSAMP_HD inline float libm_expf(float x) { return libm_expf_t(x, kExpT); }

}  // namespace hsamp
