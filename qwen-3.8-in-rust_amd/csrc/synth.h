// synth.h — deterministic synthetic tensors, identical on the host and the device.
//
// Element i of a tensor is drawn from splitmix64(seed ^ i * odd constant); a "normal" value is the inverse normal
// CDF of that draw's top 53 bits, p = (k + 1/2) 2^-53, by Acklam's rational approximation (relative error below
// 1.2e-9; tails out to 8.3 sigma), evaluated in double with +, -, *, / only: the logarithm of the tails is an atanh
// series and the square root Newton's iteration, both written out here, so host and device compute the same bits
// (IEEE basic operations round correctly on both; contraction is off). The block quantisers below turn 256 (K-quants)
// or 32 (Q8_0/Q4_0) values into ggml blocks with plain IEEE single-precision operations (no FMA, no transcendental),
// so host and device produce the same bytes. They are this library's own min/max quantisers, not ggml's
// iterative ones: the model's bytes are the source of truth for the GPU path and the CPU reference alike.
#pragma once

#include <cstdint>

#include "../../include/aq.h"

#pragma clang fp contract(off)

#if defined(__HIPCC__)
#define AQ_HD __host__ __device__
#else
#define AQ_HD
#endif

namespace aq {

enum SynthDist : uint32_t { SYNTH_NORMAL = 0, SYNTH_UNIFORM = 1, SYNTH_CONST = 2 };

using SynthSpec = aq_synth_spec;

AQ_HD inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// ln(x) for x in (0, 1]: x = m 2^e with m in [sqrt(1/2), sqrt(2)), ln m = 2 atanh(t), t = (m - 1) / (m + 1), |t| < 0.172,
// the series to t^31 (below 1e-23 after that).
AQ_HD inline double synth_ln(double x) {
    uint64_t b;
    __builtin_memcpy(&b, &x, 8);
    int e = (int)((b >> 52) & 0x7FF) - 1023;
    b = (b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull;
    double m;
    __builtin_memcpy(&m, &b, 8);
    if (m > 1.4142135623730951) {
        m *= 0.5;
        e += 1;
    }
    const double t = (m - 1.0) / (m + 1.0), t2 = t * t;
    double s = 1.0 / 31.0;
    for (int k = 29; k >= 1; k -= 2) s = s * t2 + 1.0 / (double)k;
    return 2.0 * t * s + (double)e * 0.69314718055994531;
}

// sqrt(x) for x in [0.04, 80] (the tails' -2 ln p): Newton's iteration from an exponent-halving first guess (within
// 6 %), five steps (quadratic convergence: far below an ulp).
AQ_HD inline double synth_sqrt(double x) {
    uint64_t b;
    __builtin_memcpy(&b, &x, 8);
    b = (b >> 1) + 0x1FF8000000000000ull;
    double y;
    __builtin_memcpy(&y, &b, 8);
    for (int k = 0; k < 5; k++) y = 0.5 * (y + x / y);
    return y;
}

// The inverse of the standard normal CDF at p in (0, 1): Acklam's algorithm (central rational function for
// 0.02425 <= p <= 0.97575, tail rational functions of sqrt(-2 ln p) outside).
AQ_HD inline double synth_inv_normal(double p) {
    const double a1 = -3.969683028665376e+01, a2 = 2.209460984245205e+02, a3 = -2.759285104469687e+02,
                 a4 = 1.383577518672690e+02, a5 = -3.066479806614716e+01, a6 = 2.506628277459239e+00;
    const double b1 = -5.447609879822406e+01, b2 = 1.615858368580409e+02, b3 = -1.556989798598866e+02,
                 b4 = 6.680131188771972e+01, b5 = -1.328068155288572e+01;
    const double c1 = -7.784894002430293e-03, c2 = -3.223964580411365e-01, c3 = -2.400758277161838e+00,
                 c4 = -2.549732539343734e+00, c5 = 4.374664141464968e+00, c6 = 2.938163982698783e+00;
    const double d1 = 7.784695709041462e-03, d2 = 3.224671290700398e-01, d3 = 2.445134137142996e+00,
                 d4 = 3.754408661907416e+00;
    const double plow = 0.02425;
    if (p < plow || p > 1.0 - plow) {
        const double q = synth_sqrt(-2.0 * synth_ln(p < plow ? p : 1.0 - p));
        const double x = (((((c1 * q + c2) * q + c3) * q + c4) * q + c5) * q + c6) /
                         ((((d1 * q + d2) * q + d3) * q + d4) * q + 1.0);
        return p < plow ? x : -x;
    }
    const double q = p - 0.5, r = q * q;
    return (((((a1 * r + a2) * r + a3) * r + a4) * r + a5) * r + a6) * q /
           (((((b1 * r + b2) * r + b3) * r + b4) * r + b5) * r + 1.0);
}

// Value i: `scale` is sigma (normal) as an f32.
AQ_HD inline float synth_value(const SynthSpec &s, uint64_t i, float scale) {
    const uint64_t z = splitmix64(s.seed ^ (i * 0xD1B54A32D192ED03ull));
    if (s.dist == SYNTH_CONST) return s.a;
    if (s.dist == SYNTH_UNIFORM) {
        const float u = (float)(uint32_t)(z >> 40) * (1.0f / 16777216.0f);
        return s.a + (s.b - s.a) * u;
    }
    const double p = ((double)(z >> 11) + 0.5) * 0x1p-53;
    return s.a + (float)(synth_inv_normal(p) * (double)scale);
}

// f32 -> f16 bits, round to nearest even (the same rounding as half::f16::from_f32), in plain integer code.
AQ_HD inline uint16_t f32_to_f16_bits(float f) {
    uint32_t x;
    __builtin_memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u : 0u));
    const int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        const uint32_t shift = (uint32_t)(14 - e);
        uint32_t hm = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1u), halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t out = sign | ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (out & 1u))) out++;
    return (uint16_t)out;
}

AQ_HD inline float f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int e = -1;
            do {
                man <<= 1;
                e++;
            } while ((man & 0x400u) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    __builtin_memcpy(&f, &bits, 4);
    return f;
}

AQ_HD inline int round_i(float v) { return (int)__builtin_roundf(v); } // half away from zero, exact
AQ_HD inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// Q4_K (nmax 15) / Q5_K (nmax 31): per 32-element sub-block min/max -> 6-bit scale and min relative to the
// super-block's largest, f16 d and dmin. Packing as ggml's block_q4_K / block_q5_K (the reference's quant.rs
// unit test `scale_min_unpack_matches_ggml_packing` spells the scale packing out).
AQ_HD inline void quantize_q45k_block(const float *x, uint8_t *out, bool q5) {
    const int nmax = q5 ? 31 : 15;
    float scale[8], minv[8];
    float max_scale = 0.0f, max_min = 0.0f;
    for (int s = 0; s < 8; s++) {
        float mn = x[32 * s], mx = x[32 * s];
        for (int i = 1; i < 32; i++) {
            const float v = x[32 * s + i];
            mn = v < mn ? v : mn;
            mx = v > mx ? v : mx;
        }
        if (mn > 0.0f) mn = 0.0f;
        scale[s] = (mx - mn) / (float)nmax;
        minv[s] = -mn;
        max_scale = scale[s] > max_scale ? scale[s] : max_scale;
        max_min = minv[s] > max_min ? minv[s] : max_min;
    }
    const uint16_t d16 = f32_to_f16_bits(max_scale / 63.0f), m16 = f32_to_f16_bits(max_min / 63.0f);
    const float dq = f16_bits_to_f32(d16), dmq = f16_bits_to_f32(m16);
    int sc[8], m[8];
    for (int s = 0; s < 8; s++) {
        sc[s] = dq > 0.0f ? clampi(round_i(scale[s] / dq), 0, 63) : 0;
        m[s] = dmq > 0.0f ? clampi(round_i(minv[s] / dmq), 0, 63) : 0;
    }
    uint8_t q[256];
    for (int s = 0; s < 8; s++) {
        const float ds = dq * (float)sc[s], dm = dmq * (float)m[s];
        for (int i = 0; i < 32; i++) {
            const int v = ds > 0.0f ? round_i((x[32 * s + i] + dm) / ds) : 0;
            q[32 * s + i] = (uint8_t)clampi(v, 0, nmax);
        }
    }
    out[0] = (uint8_t)(d16 & 0xFF);
    out[1] = (uint8_t)(d16 >> 8);
    out[2] = (uint8_t)(m16 & 0xFF);
    out[3] = (uint8_t)(m16 >> 8);
    uint8_t *s12 = out + 4;
    for (int j = 0; j < 12; j++) s12[j] = 0;
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            s12[j] = (uint8_t)sc[j];
            s12[j + 4] = (uint8_t)m[j];
        } else {
            s12[j + 4] = (uint8_t)((sc[j] & 0xF) | ((m[j] & 0xF) << 4));
            s12[j - 4] |= (uint8_t)((sc[j] >> 4) << 6);
            s12[j] |= (uint8_t)((m[j] >> 4) << 6);
        }
    }
    uint8_t *qs = out + (q5 ? 48 : 16);
    for (int jp = 0; jp < 4; jp++)
        for (int i = 0; i < 32; i++)
            qs[32 * jp + i] = (uint8_t)((q[64 * jp + i] & 0xF) | ((q[64 * jp + 32 + i] & 0xF) << 4));
    if (q5) {
        uint8_t *qh = out + 16;
        for (int i = 0; i < 32; i++) {
            uint8_t h = 0;
            for (int s = 0; s < 8; s++) h |= (uint8_t)(((q[32 * s + i] >> 4) & 1) << s);
            qh[i] = h;
        }
    }
}

// Q6_K: per 16-element group scale amax/31 as int8 relative to the super-block's largest (d = max/127, f16),
// codes round(x / (d*sc)) in -32..31 stored +32. Packing as ggml's block_q6_K (ql, qh, scales, d).
AQ_HD inline void quantize_q6k_block(const float *x, uint8_t *out) {
    float scale[16], max_scale = 0.0f;
    for (int g = 0; g < 16; g++) {
        float amax = 0.0f;
        for (int i = 0; i < 16; i++) {
            const float a = __builtin_fabsf(x[16 * g + i]);
            amax = a > amax ? a : amax;
        }
        scale[g] = amax / 31.0f;
        max_scale = scale[g] > max_scale ? scale[g] : max_scale;
    }
    const uint16_t d16 = f32_to_f16_bits(max_scale / 127.0f);
    const float dq = f16_bits_to_f32(d16);
    int sc[16];
    uint8_t code[256];
    for (int g = 0; g < 16; g++) {
        sc[g] = dq > 0.0f ? clampi(round_i(scale[g] / dq), 0, 127) : 0;
        const float ds = dq * (float)sc[g];
        for (int i = 0; i < 16; i++) {
            const int v = ds > 0.0f ? round_i(x[16 * g + i] / ds) : 0;
            code[16 * g + i] = (uint8_t)(clampi(v, -32, 31) + 32);
        }
    }
    for (int h = 0; h < 2; h++)
        for (int l = 0; l < 32; l++) {
            const uint8_t q1 = code[h * 128 + l], q2 = code[h * 128 + l + 32], q3 = code[h * 128 + l + 64],
                          q4 = code[h * 128 + l + 96];
            out[h * 64 + l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
            out[h * 64 + l + 32] = (uint8_t)((q2 & 15) | ((q4 & 15) << 4));
            out[128 + h * 32 + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    for (int g = 0; g < 16; g++) out[192 + g] = (uint8_t)(int8_t)sc[g];
    out[208] = (uint8_t)(d16 & 0xFF);
    out[209] = (uint8_t)(d16 >> 8);
}

// Q8_0: d = amax/127 (f16), q = round(x/d). Q4_0: d = max/-8 with max the signed value of largest |x| (f16),
// q = floor(x/d + 8.5) clamped to 0..15 (ggml's quantize_row_q4_0_ref rule, with a divide).
AQ_HD inline void quantize_q8_0_block(const float *x, uint8_t *out) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) {
        const float a = __builtin_fabsf(x[i]);
        amax = a > amax ? a : amax;
    }
    const uint16_t d16 = f32_to_f16_bits(amax / 127.0f);
    const float dq = f16_bits_to_f32(d16);
    out[0] = (uint8_t)(d16 & 0xFF);
    out[1] = (uint8_t)(d16 >> 8);
    for (int i = 0; i < 32; i++) out[2 + i] = (uint8_t)(int8_t)(dq > 0.0f ? clampi(round_i(x[i] / dq), -127, 127) : 0);
}

AQ_HD inline void quantize_q4_0_block(const float *x, uint8_t *out) {
    float amax = 0.0f, max = 0.0f;
    for (int i = 0; i < 32; i++) {
        const float a = __builtin_fabsf(x[i]);
        if (a > amax) {
            amax = a;
            max = x[i];
        }
    }
    const uint16_t d16 = f32_to_f16_bits(max / -8.0f);
    const float dq = f16_bits_to_f32(d16);
    out[0] = (uint8_t)(d16 & 0xFF);
    out[1] = (uint8_t)(d16 >> 8);
    for (int i = 0; i < 16; i++) {
        const int a = dq != 0.0f ? clampi((int)__builtin_floorf(x[i] / dq + 8.5f), 0, 15) : 8;
        const int b = dq != 0.0f ? clampi((int)__builtin_floorf(x[i + 16] / dq + 8.5f), 0, 15) : 8;
        out[2 + i] = (uint8_t)(a | (b << 4));
    }
}

// Block `blk` (row-major over rows x blocks-per-row) of a synthetic tensor, as ggml bytes.
AQ_HD inline void synth_block(const SynthSpec &s, uint64_t blk, float scale, uint8_t *out) {
    const int be = (s.ggml_type == AQ_TYPE_Q4_0 || s.ggml_type == AQ_TYPE_Q8_0) ? 32 : 256;
    float x[256];
    const uint64_t first = blk * (uint64_t)be;
    for (int i = 0; i < be; i++) x[i] = synth_value(s, first + (uint64_t)i, scale);
    switch (s.ggml_type) {
    case AQ_TYPE_Q4_K: quantize_q45k_block(x, out, false); break;
    case AQ_TYPE_Q5_K: quantize_q45k_block(x, out, true); break;
    case AQ_TYPE_Q6_K: quantize_q6k_block(x, out); break;
    case AQ_TYPE_Q8_0: quantize_q8_0_block(x, out); break;
    case AQ_TYPE_Q4_0: quantize_q4_0_block(x, out); break;
    default: break; // F32 tensors are generated element by element (synth_value)
    }
}

inline float synth_scale(const SynthSpec &s) { return s.b; }

} // namespace aq
