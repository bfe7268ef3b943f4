/*
 * aq_math.h — exp and log1p for the f32 activations (silu, sigmoid, softplus, softmax, the DeltaNet decay), built
 * only from IEEE double additions, multiplications, fused multiply-adds, divisions and rint — each correctly rounded
 * by definition — so the same source gives the same bits on the host (gcc; fma() from libm) and on the device
 * (hipcc; v_fma_f64): compile both with floating-point contraction off.
 *
 * The reference calls the platform libm's expf / log1pf (act.rs:7-40, softmax.rs:22-49, deltanet.rs:43-86), whose
 * last-ulp behaviour differs between libms; through 64 layers of Q8_K requantisation a single ulp grows into a
 * different token. Both this library and its CPU oracle therefore evaluate these functions here, in double with
 * an error of a few double ulps, then round once to f32: the correctly rounded f32 result except when the exact
 * value lies within ~1e-15 relative of a rounding boundary.
 *
 * exp:   x = k ln2 + r (Cody-Waite, ln2 split so k*LN2_HI is exact), |r| <= ln2/2, exp(r) by its Taylor series to
 *        degree 13 (truncation < 4e-18) in fused Horner steps, times 2^k built from the exponent bits.
 * log1p: small arguments by the series u - u^2/2 + u^3/3; otherwise 1 + u is exact in double for an f32 u in
 *        (2^-29, 2^29), and log(1 + u) = k ln2 + 2 atanh((m - 1)/(m + 1)) with m in [sqrt(1/2), sqrt(2)).
 */
#ifndef AQ_MATH_H
#define AQ_MATH_H

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define AQ_MATH_FN __host__ __device__ static inline
#else
#define AQ_MATH_FN static inline
#endif

#define AQ_LN2_HI 6.93147180369123816490e-01 /* ln2 with 21 trailing zero bits: k * AQ_LN2_HI is exact */
#define AQ_LN2_LO 1.90821492927058770002e-10
#define AQ_INV_LN2 1.44269504088896338700e+00

AQ_MATH_FN double aq_pow2i(int k) { /* 2^k for -1022 <= k <= 1023 */
    uint64_t bits = (uint64_t)(k + 1023) << 52;
    double d;
    memcpy(&d, &bits, 8);
    return d;
}

AQ_MATH_FN double aq_exp_d(double x) {
    if (x != x) return x;
    if (x > 709.0) return __builtin_inf();
    if (x < -740.0) return 0.0;
    const double kd = __builtin_rint(x * AQ_INV_LN2);
    const int k = (int)kd;
    const double r = __builtin_fma(-kd, AQ_LN2_LO, __builtin_fma(-kd, AQ_LN2_HI, x));
    /* Horner, highest degree first, one fused step per coefficient 1/n! */
    double p = 1.0 / 6227020800.0; /* 1/13! */
    p = __builtin_fma(p, r, 1.0 / 479001600.0);
    p = __builtin_fma(p, r, 1.0 / 39916800.0);
    p = __builtin_fma(p, r, 1.0 / 3628800.0);
    p = __builtin_fma(p, r, 1.0 / 362880.0);
    p = __builtin_fma(p, r, 1.0 / 40320.0);
    p = __builtin_fma(p, r, 1.0 / 5040.0);
    p = __builtin_fma(p, r, 1.0 / 720.0);
    p = __builtin_fma(p, r, 1.0 / 120.0);
    p = __builtin_fma(p, r, 1.0 / 24.0);
    p = __builtin_fma(p, r, 1.0 / 6.0);
    p = __builtin_fma(p, r, 0.5);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    if (k < -1000) return (p * aq_pow2i(k + 600)) * aq_pow2i(-600);
    if (k > 1000) return (p * aq_pow2i(k - 600)) * aq_pow2i(600);
    return p * aq_pow2i(k);
}

/* log(v) for a finite v > 0 */
AQ_MATH_FN double aq_log_d(double v) {
    uint64_t bits;
    memcpy(&bits, &v, 8);
    int k = (int)((bits >> 52) & 0x7FF) - 1023;
    if (k == -1023) { /* subnormal: scale up */
        v *= 18014398509481984.0; /* 2^54 */
        memcpy(&bits, &v, 8);
        k = (int)((bits >> 52) & 0x7FF) - 1023 - 54;
    }
    bits = (bits & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull; /* m in [1, 2) */
    double m;
    memcpy(&m, &bits, 8);
    if (m > 1.41421356237309504880) {
        m *= 0.5;
        k += 1;
    }
    const double s = (m - 1.0) / (m + 1.0);
    const double s2 = s * s;
    double t = 1.0 / 23.0;
    t = __builtin_fma(t, s2, 1.0 / 21.0);
    t = __builtin_fma(t, s2, 1.0 / 19.0);
    t = __builtin_fma(t, s2, 1.0 / 17.0);
    t = __builtin_fma(t, s2, 1.0 / 15.0);
    t = __builtin_fma(t, s2, 1.0 / 13.0);
    t = __builtin_fma(t, s2, 1.0 / 11.0);
    t = __builtin_fma(t, s2, 1.0 / 9.0);
    t = __builtin_fma(t, s2, 1.0 / 7.0);
    t = __builtin_fma(t, s2, 1.0 / 5.0);
    t = __builtin_fma(t, s2, 1.0 / 3.0);
    t = __builtin_fma(t, s2, 1.0);
    const double lm = 2.0 * s * t;
    const double kd = (double)k;
    return __builtin_fma(kd, AQ_LN2_LO, __builtin_fma(kd, AQ_LN2_HI, lm));
}

AQ_MATH_FN float aq_expf(float x) { return (float)aq_exp_d((double)x); }

/* log1p for an f32 argument u > -1 */
AQ_MATH_FN float aq_log1pf(float u) {
    if (u != u) return u;
    if (u == __builtin_inff()) return u;
    if (u <= -1.0f) return u == -1.0f ? -__builtin_inff() : __builtin_nanf("");
    const double d = (double)u;
    if (d < 1.0 / 536870912.0 && d > -1.0 / 536870912.0) /* |u| < 2^-29: the series is exact to 2^-87 */
        return (float)(d - (d * d) * 0.5 + (d * d * d) * (1.0 / 3.0));
    return (float)aq_log_d(1.0 + d);
}

#endif /* AQ_MATH_H */
