// expf with the results of glibc's expf (glibc >= 2.27, x86-64 FMA variant), for host and device code.
//
// The reference runtime computes every exponential of its attention with Rust's f32::exp, which calls the platform
// libm: glibc's expf, whose results are not always correctly rounded (error bound 0.502 ULP). To be bit-identical the
// GPU must therefore follow the same published algorithm (glibc sysdeps/ieee754/flt-32/e_expf.c with the table and
// coefficients of e_exp2f_data.c, from Arm's optimized-routines): x * 32 / ln2 = k + r with k the nearest integer
// (round to even via the 1.5 * 2^52 shift), 2^(k/32) from a 32-entry table, 2^(r/32) from a cubic, everything in double,
// then one rounding to float. On an x86-64 CPU with FMA glibc selects the variant built with -mfma, in which every
// a * b + c is fused: the three of the cubic, and x * 32 / ln2 in both of its uses (k + shift and the remainder r);
// that is the form below (the unfused remainder differs from the host's expf on two floats). The table and
// coefficients are the published constants; tests/test_expf.py checks the function against the host's expf on every
// float.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define VX_HD __host__ __device__
#else
#define VX_HD
#endif

namespace vx {

// tab[i] = bits(2^(i/32)) - (i << 47): 2^(i/32) rounded to double, with the exponent of k % 32 removed.
struct Exp2fTable {
    uint64_t tab[32];
};

VX_HD inline uint64_t expf_tab(uint32_t i) {
    constexpr Exp2fTable t = {{
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
    }};
    return t.tab[i];
}

VX_HD inline uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
VX_HD inline float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
VX_HD inline double bits_f64(uint64_t u) { return __builtin_bit_cast(double, u); }
VX_HD inline uint64_t f64_bits(double d) { return __builtin_bit_cast(uint64_t, d); }

// The function with the table read through tab(i) (a device caller may keep the table in LDS).
template <typename Tab>
VX_HD inline float glibc_expf_with(float x, Tab tab) {
    const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double kShift = 0x1.8p+52;
    const double kC0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double kC1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const uint32_t abstop = (f32_bits(x) >> 20) & 0x7ffu;
    if (abstop >= ((f32_bits(88.0f) >> 20) & 0x7ffu)) {
        // |x| >= 88 or x is NaN
        if (f32_bits(x) == f32_bits(-__builtin_inff())) return 0.0f;
        if (abstop >= ((f32_bits(__builtin_inff()) >> 20) & 0x7ffu)) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();  // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;             // underflow
    }
    const double xd = static_cast<double>(x);
    double kd = __builtin_fma(kInvLn2N, xd, kShift);  // k = round(x * 32 / ln2), ties to even
    const uint64_t ki = f64_bits(kd);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    uint64_t t = tab(static_cast<uint32_t>(ki % 32u));
    t += ki << (52 - 5);
    const double s = bits_f64(t);
    const double z = __builtin_fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return static_cast<float>(y);
}

VX_HD inline float glibc_expf(float x) { return glibc_expf_with(x, expf_tab); }

}  // namespace vx
