// hm_expf.h -- glibc 2.35 expf restated from its published algorithm, for
// host and device.  Compiles under hipcc (device + host) and under g++ (the
// CPU test that checks it against the host libm on every float input).
//
// Algorithm (glibc sysdeps/ieee754/flt-32/e_expf.c, from Arm's
// optimized-routines): x * N/ln2 = k + r with N = 32 and |r| <= 1/2;
// exp(x) = 2^(k/N) * 2^(r/N); 2^(k/N) = asdouble(T[k % N] + (k << 47)) where
// T[i] = bits(2^(i/32)) - (i << 47); 2^(r/N) ~ C0 r^3 + C1 r^2 + C2 r + 1;
// everything in double, one rounding to float at the end.  glibc's x86-64
// FMA variant (selected on CPUs with FMA) contracts r = InvLn2N*x - kd and
// the polynomial steps into fused multiply-adds; so does this restatement.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define HM_HD __host__ __device__ __forceinline__
#else
#define HM_HD static inline
#endif

constexpr unsigned long long kHmExp2Table[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full,
    0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,
    0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull,
    0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull,
    0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,
    0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull,
    0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull,
    0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,
    0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

// The restated expf with the table passed in: kHmExp2Table itself, or a
// copy of it in LDS (device kernels that evaluate many exponentials per
// thread keep the table there, since a per-lane index into a global table
// costs a dependent memory load per call).  The common path is computed for
// every input and the rare |x| >= 88 / inf / NaN cases are selected
// afterwards, so there are no branches; every result equals glibc's.
HM_HD float hm_expf_t(float x, const unsigned long long* table) {
    const unsigned int bits = __builtin_bit_cast(unsigned int, x);
    const unsigned int abstop = (bits >> 20) & 0x7ffu;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const unsigned long long ki = __builtin_bit_cast(unsigned long long, kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    unsigned long long t = table[ki & 31u];
    t += ki << 47;
    const double s = __builtin_bit_cast(double, t);
    const double p = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    y = y * s;
    const float common = (float)y;
    // |x| >= 88 or NaN: -inf -> 0, inf/nan -> x + x, overflow -> inf,
    // underflow -> 0, otherwise the common path.  Bit masks rather than
    // conditionals, so that the device code has no branches.
    const unsigned int m_big = 0u - (unsigned int)(abstop >= 0x42bu);
    const unsigned int m_udf = 0u - (unsigned int)(x < -0x1.9fe368p6f);
    const unsigned int m_ovf = 0u - (unsigned int)(x > 0x1.62e42ep6f);
    const unsigned int m_nan = 0u - (unsigned int)(abstop >= 0x7f8u);
    const unsigned int m_ninf = 0u - (unsigned int)(bits == 0xff800000u);
    const unsigned int cbits = __builtin_bit_cast(unsigned int, common);
    unsigned int sp = cbits & ~m_udf;
    sp = (sp & ~m_ovf) | (0x7f800000u & m_ovf);
    sp = (sp & ~m_nan) | (__builtin_bit_cast(unsigned int, x + x) & m_nan);
    sp &= ~m_ninf;
    return __builtin_bit_cast(float, (cbits & ~m_big) | (sp & m_big));
}

HM_HD float hm_expf(float x) { return hm_expf_t(x, kHmExp2Table); }

// The common path alone: equal to hm_expf_t for |x| < 88 (where none of the
// special cases applies).  Callers check the range, e.g. once for a whole
// wave, and use hm_expf_t otherwise.
HM_HD float hm_expf_small_t(float x, const unsigned long long* table) {
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const unsigned long long ki = __builtin_bit_cast(unsigned long long, kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    unsigned long long t = table[ki & 31u];
    t += ki << 47;
    const double s = __builtin_bit_cast(double, t);
    const double p = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    y = y * s;
    return (float)y;
}
