/*
 * aq_math.h — expf and log1pf for the f32 activations (silu, sigmoid, softplus, softmax, the DeltaNet decay),
 * restated so that they return, for every f32 argument, the same bits as the functions the reference calls.
 *
 * The reference's `f32::exp` / `f32::ln_1p` (act.rs:7-40, softmax.rs:22-49, deltanet.rs:43-86) lower to the
 * platform libm's `expf` / `log1pf`: on Linux x86-64, GNU libc. This header restates the two algorithms of GNU
 * libc 2.35 (the version of this image and of the GPU boxes), from their published sources:
 *
 *  expf   — the table method of Szabolcs Nagy's optimized-routines expf (glibc sysdeps/ieee754/flt-32/e_expf.c,
 *           e_exp2f_data.c; MIT/LGPL): x·32/ln2 = k + r, 2^(k/32) from a 32-entry table of 2^(i/32) with the
 *           exponent bits of k folded in, 2^(r/32) by a cubic, all in double, one rounding to f32 at the end.
 *           On x86-64 CPUs with FMA, glibc selects the build of that source compiled with -mfma, in which the
 *           compiler fuses x·InvLn2N into both of its additive uses and the two polynomial steps; the explicit
 *           fma() calls below are those fusions.
 *  log1pf — fdlibm's s_log1pf.c (Sun, freely distributable) in f32 arithmetic, with FreeBSD's association of the
 *           correction term, (k·ln2_lo + c), that glibc carries; no contraction.
 *
 * Both are pinned by an exhaustive sweep of all 2^32 f32 bit patterns against the platform's expf / log1pf
 * (tests/test_math.py, 0 mismatches). They use only IEEE double fma/add/mul and f32 add/sub/mul/div — each correctly
 * rounded by definition — plus integer bit operations, so the same source gives the same bits on the host (gcc,
 * fma() from libm) and on the device (hipcc, v_fma_f64; f32 division correctly rounded): compile both with
 * floating-point contraction off.
 */
#ifndef AQ_MATH_H
#define AQ_MATH_H

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define AQ_MATH_FN __host__ __device__ static inline
#define AQ_MATH_TABLE __host__ __device__ static inline
#else
#define AQ_MATH_FN static inline
#define AQ_MATH_TABLE static inline
#endif

/* 2^(i/32) rounded to double, minus i << 47 (so that adding k << 47 for k = 32q + i scales it by 2^q) */
#define AQ_EXP2_TAB_INIT                                                                                           \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,                 \
     0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,                 \
     0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,                 \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,                 \
     0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,                 \
     0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,                 \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,                 \
     0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

#if defined(__HIPCC__)
__constant__ static const uint64_t aq_exp2_tab_dev[32] = AQ_EXP2_TAB_INIT;
#endif
static const uint64_t aq_exp2_tab_host[32] = AQ_EXP2_TAB_INIT;

AQ_MATH_TABLE uint64_t aq_exp2_tab(uint32_t i) {
#if defined(__HIP_DEVICE_COMPILE__)
    return aq_exp2_tab_dev[i];
#else
    return aq_exp2_tab_host[i];
#endif
}

AQ_MATH_FN uint32_t aq_f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
AQ_MATH_FN float aq_u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

AQ_MATH_FN float aq_expf(float x) {
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32; /* 32/ln2 */
    const double shift = 0x1.8p+52;                      /* adding it rounds to an integer in the low bits */
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const uint32_t abstop = (aq_f2u(x) >> 20) & 0x7ff;
    if (abstop >= 0x42b) { /* |x| >= 88, or inf / nan */
        if (aq_f2u(x) == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();    /* x > log(2^128) */
        if (x < -0x1.9fe368p6f) return 0.0f;               /* x < log(2^-150) */
    }
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd); /* x·32/ln2 - k, |r| <= 1/2 */
    uint64_t t = aq_exp2_tab((uint32_t)(ki % 32)) + (ki << 47);
    double s;
    memcpy(&s, &t, 8);                                  /* 2^(k/32) */
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

/* log1p for an f32 argument */
AQ_MATH_FN float aq_log1pf(float x) {
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f; /* 0x3f317180, 0x3717f7d1 */
    const float lp1 = 6.6666668653e-01f, lp2 = 4.0000000596e-01f, lp3 = 2.8571429849e-01f,
                lp4 = 2.2222198546e-01f, lp5 = 1.8183572590e-01f, lp6 = 1.5313838422e-01f,
                lp7 = 1.4798198640e-01f;
    float f = 0.0f, c = 0.0f, u;
    const int32_t hx = (int32_t)aq_f2u(x);
    const int32_t ax = hx & 0x7fffffff;
    int32_t k = 1, hu = 0;
    if (hx < 0x3ed413d7) {            /* x < 0.41422 */
        if (ax >= 0x3f800000) {       /* x <= -1 */
            if (x == -1.0f) return -__builtin_inff();
            return __builtin_nanf("");
        }
        if (ax < 0x31000000) {        /* |x| < 2^-29 */
            if (ax < 0x24800000) return x;
            return x - x * x * 0.5f;
        }
        if (hx > 0 || hx <= (int32_t)0xbe95f61f) { /* -0.2929 < x < 0.41422 */
            k = 0;
            f = x;
            hu = 1;
        }
    } else if (hx >= 0x7f800000) {
        return x + x;
    }
    if (k != 0) {
        if (hx < 0x5a000000) {
            u = 1.0f + x;
            hu = (int32_t)aq_f2u(u);
            k = (hu >> 23) - 127;
            c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f); /* the rounding error of 1 + x */
            c /= u;
        } else {
            u = x;
            hu = (int32_t)aq_f2u(u);
            k = (hu >> 23) - 127;
            c = 0.0f;
        }
        hu &= 0x007fffff;
        if (hu < 0x3504f7) {
            u = aq_u2f((uint32_t)(hu | 0x3f800000)); /* u in [1, sqrt 2) */
        } else {
            k += 1;
            u = aq_u2f((uint32_t)(hu | 0x3f000000)); /* u/2 */
            hu = (0x00800000 - hu) >> 2;
        }
        f = u - 1.0f;
    }
    const float hfsq = 0.5f * f * f;
    const float kf = (float)k;
    if (hu == 0) { /* |f| < 2^-20 */
        if (f == 0.0f) {
            if (k == 0) return 0.0f;
            c += kf * ln2_lo;
            return kf * ln2_hi + c;
        }
        const float r = hfsq * (1.0f - 0.66666666666666666f * f);
        if (k == 0) return f - r;
        return kf * ln2_hi - ((r - (c + kf * ln2_lo)) - f);
    }
    const float s = f / (2.0f + f);
    const float z = s * s;
    const float r = z * (lp1 + z * (lp2 + z * (lp3 + z * (lp4 + z * (lp5 + z * (lp6 + z * lp7))))));
    if (k == 0) return f - (hfsq - s * (hfsq + r));
    return kf * ln2_hi - ((hfsq - (s * (hfsq + r) + (kf * ln2_lo + c))) - f);
}

#endif /* AQ_MATH_H */
