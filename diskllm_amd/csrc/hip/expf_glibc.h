/*
 * expf_glibc.h -- bit-exact restatement of the host libm expf() that the
 * reference's softmax calls (src/sampler.c:179).
 *
 * Third-party dependency: GNU C Library 2.35 (Ubuntu 2.35-0ubuntu3.11), function
 * expf, x86-64 FMA variant.  glibc's expf is the published ARM Optimized Routines
 * algorithm (Szabolcs Nagy, 2017; sysdeps/ieee754/flt-32/e_expf.c): with N = 32,
 *   z = x * N/ln2 ;  k = round(z) (via the 1.5*2^52 shift trick) ;  r = z - k
 *   2^(k/N) = asdouble(tab[k % N] + (k << (52 - 5)))
 *   exp(x) ~= 2^(k/N) * (C0 r^3 + C1 r^2 + C2 r + 1),   evaluated in double,
 * then rounded once to float.  tab[i] = bits(RN(2^(i/32))) - (i << 47) is fixed by
 * the mathematics (recomputed in high precision when this file was written);
 * C0..C2 are the published minimax coefficients scaled by N^-3, N^-2, N^-1.
 *
 * The x86-64 build of glibc compiles this routine with -mfma and contracts
 * r = z - k into one fused multiply-add; that is observable: an exhaustive test
 * over all 2^32 non-NaN inputs against the host libm gives 0 mismatches with the
 * fused form below and 2 mismatches with a separately rounded r (at
 * x = 0x1.04845ep+5 and x = -0x1.f8cbb2p+5).
 *
 * Usable on the host (g++/clang) and the device (hipcc); the 32-entry table is
 * passed in so the GPU can keep it in LDS.
 */
#ifndef DLK_EXPF_GLIBC_H
#define DLK_EXPF_GLIBC_H

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define DLK_HD __host__ __device__ __forceinline__
#else
#define DLK_HD static inline
#endif

#define DLK_EXP2_TAB_INIT                                                             \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
     0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
     0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
     0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
     0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
     0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

DLK_HD double dlk_u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }
DLK_HD uint64_t dlk_d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
DLK_HD float dlk_u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
DLK_HD uint32_t dlk_f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* The general formula of glibc 2.35 expf (x86-64 FMA variant) without its
 * special-case screen: exact for finite x in [-1000, 88.72] (below -103.97 it
 * rounds to 0 like the screened path), branch-free so loops interleave. */
DLK_HD float dlk_expf_glibc_core(float x, const uint64_t *tab) {
    const double kInvLn2N = 0x1.71547652b82fep+0 * 32;
    const double kShift = 0x1.8p+52;
    const double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double kC2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = __builtin_fma(kInvLn2N, xd, kShift);
    const uint64_t ki = dlk_d2u(kd);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    const uint64_t t = tab[ki & 31] + (ki << 47);
    const double s = dlk_u2d(t);
    const double z = __builtin_fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

/* exp(x) for float x, bit-identical to glibc 2.35 expf (x86-64 FMA variant). */
DLK_HD float dlk_expf_glibc(float x, const uint64_t *tab) {
    const uint32_t ux = dlk_f2u(x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42bu) {                         /* |x| >= 88 or NaN */
        if (ux == 0xff800000u) return 0.0f;         /* -inf */
        if (abstop >= 0x7f8u) return x + x;         /* +inf, NaN */
        if (x > 0x1.62e42ep6f) return dlk_u2f(0x7f800000u);
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    return dlk_expf_glibc_core(x, tab);
}

#endif
