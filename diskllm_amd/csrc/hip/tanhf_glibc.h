/*
 * tanhf_glibc.h -- bit-exact restatement of the host libm tanhf() that the
 * reference's logit soft-capping calls (src/core/context.c:604-606 after a
 * prefill, :873-876 after a decode step: logits[i] = cap * tanhf(logits[i] / cap)).
 *
 * Third-party dependency: GNU C Library 2.35 (Ubuntu 2.35-0ubuntu3.11), functions
 * tanhf (sysdeps/ieee754/flt-32/s_tanhf.c) and the expm1f it calls
 * (sysdeps/ieee754/flt-32/s_expm1f.c).  Both are the published fdlibm float
 * algorithms (Sun Microsystems, 1993; float conversion by Ian Lance Taylor):
 *   tanh(x) = sign(x) * (1 - 2 / (expm1(2|x|) + 2))   for 1 <= |x| < 22,
 *           = sign(x) * (-t / (t + 2)), t = expm1(-2|x|)  for 2^-55 <= |x| < 1,
 *           = x * (1 + x) below, sign(x) * 1 at and above 22;
 *   expm1(x): k = round(x / ln2), r = x - k ln2 split into hi + lo with a
 *   correction c, then expm1(r) from the rational form
 *   r - (r * e - r^2/2), R1 = 1 + r^2/2 * (Q1 + ... + Q5 (r^2/2)^4), and the
 *   result rescaled by 2^k with the per-k cases of the algorithm.
 * Every operation is one IEEE float operation in source order (x86-64 SSE, no
 * contraction), which is what the hipcc flags of this library give on the GPU
 * (-ffp-contract=off, correctly rounded float division, denormals kept).  The
 * constants are the algorithm's published float constants, written as bit
 * patterns.
 *
 * Usable on the host (gcc) and the device (hipcc).
 */
#ifndef DLK_TANHF_GLIBC_H
#define DLK_TANHF_GLIBC_H

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define DLK_TH __host__ __device__ __forceinline__
#else
#define DLK_TH static inline
#endif

DLK_TH float dlk_th_u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
DLK_TH uint32_t dlk_th_f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* expm1f for the arguments tanhf passes: finite, |x| < 44. */
DLK_TH float dlk_expm1f_glibc(float x) {
    const float kLn2Hi = dlk_th_u2f(0x3f317180u), kLn2Lo = dlk_th_u2f(0x3717f7d1u);
    const float kInvLn2 = dlk_th_u2f(0x3fb8aa3bu);
    const float kQ1 = dlk_th_u2f(0xbd088889u), kQ2 = dlk_th_u2f(0x3ad00d01u), kQ3 = dlk_th_u2f(0xb8a670cdu),
                kQ4 = dlk_th_u2f(0x36867e54u), kQ5 = dlk_th_u2f(0xb457edbbu);
    const uint32_t ux = dlk_th_f2u(x);
    const int neg = (ux >> 31) != 0;
    const uint32_t ax = ux & 0x7fffffffu;
    if (ax >= 0x4195b844u && neg) return -1.0f;       /* x <= -27 ln2 (the huge-x cases do not occur) */
    float hi, lo, c = 0.0f;
    int k;
    if (ax > 0x3eb17218u) {                            /* |x| > ln2 / 2: reduce */
        if (ax < 0x3f851592u) {                        /* |x| < 1.5 ln2 */
            if (!neg) { hi = x - kLn2Hi; lo = kLn2Lo; k = 1; }
            else { hi = x + kLn2Hi; lo = -kLn2Lo; k = -1; }
        } else {
            k = (int)(kInvLn2 * x + (neg ? -0.5f : 0.5f));
            const float t = (float)k;
            hi = x - t * kLn2Hi;                       /* exact */
            lo = t * kLn2Lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (ax < 0x33000000u) {                     /* |x| < 2^-25 */
        return x;
    } else {
        k = 0;
    }
    const float hfx = 0.5f * x;
    const float hxs = x * hfx;
    const float r1 = 1.0f + hxs * (kQ1 + hxs * (kQ2 + hxs * (kQ3 + hxs * (kQ4 + hxs * kQ5))));
    float t = 3.0f - r1 * hfx;
    float e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = (x * (e - c) - c);
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) {
        if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
        return 1.0f + 2.0f * (x - e);
    }
    float y;
    if (k <= -2 || k > 56) {
        y = 1.0f - (e - x);
        y = dlk_th_u2f(dlk_th_f2u(y) + ((uint32_t)k << 23));
        return y - 1.0f;
    }
    if (k < 23) {
        t = dlk_th_u2f(0x3f800000u - (0x1000000u >> k));   /* 1 - 2^-k */
        y = t - (e - x);
    } else {
        t = dlk_th_u2f((uint32_t)(0x7f - k) << 23);         /* 2^-k */
        y = x - (e + t);
        y += 1.0f;
    }
    return dlk_th_u2f(dlk_th_f2u(y) + ((uint32_t)k << 23));
}

/* tanhf, bit-identical to glibc 2.35 tanhf on x86-64 (NaN inputs give a NaN). */
DLK_TH float dlk_tanhf_glibc(float x) {
    const uint32_t ux = dlk_th_f2u(x);
    const uint32_t ax = ux & 0x7fffffffu;
    const int neg = (ux >> 31) != 0;
    if (ax >= 0x7f800000u) {
        if (ax > 0x7f800000u) return x + x;            /* NaN */
        return neg ? -1.0f : 1.0f;                     /* 1/x +- 1 at +-inf */
    }
    float z;
    if (ax < 0x41b00000u) {                            /* |x| < 22 */
        if (ax == 0) return x;                         /* +-0 */
        if (ax < 0x24000000u) return x * (1.0f + x);   /* |x| < 2^-55 */
        const float a = dlk_th_u2f(ax);
        if (ax >= 0x3f800000u) {                       /* |x| >= 1 */
            const float t = dlk_expm1f_glibc(2.0f * a);
            z = 1.0f - 2.0f / (t + 2.0f);
        } else {
            const float t = dlk_expm1f_glibc(-2.0f * a);
            z = -t / (t + 2.0f);
        }
    } else {
        z = 1.0f;                                      /* 1 - tiny rounds to 1 */
    }
    return neg ? -z : z;
}

/* The reference's soft-cap of one logit: cap * tanhf(x / cap). */
DLK_TH float dlk_softcap_glibc(float x, float cap) { return cap * dlk_tanhf_glibc(x / cap); }

#endif
