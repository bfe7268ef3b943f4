/*
 * oracle_kernels.c — TEST INFRASTRUCTURE ONLY: the reference's scalar kernels restated in C (see oracle.h).
 * Compiled with -ffp-contract=off: every `a * b + c` below is a rounded multiply then a rounded add, as the
 * reference requires ("No FMA", kdot.rs:17).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "oracle_internal.h"

#include "aq_math.h"

/* ===================================================================================== f16 (half 2.7.1) */

/* quant.rs:33-36 `f16_to_f32`: exact widening, subnormals and inf/NaN included. */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do {
                man <<= 1;
                e++;
            } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* half::f16::from_f32 (q8.rs:97): round to nearest, ties to even; overflow to inf; NaN stays NaN. */
uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (man ? (0x200u | (man >> 13)) : 0));
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half_man = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_man & 1u))) half_man++;
        return (uint16_t)(sign | half_man);
    }
    uint32_t half_man = man >> 13;
    uint32_t rem = man & 0x1FFFu;
    uint32_t out = sign | ((uint32_t)e << 10) | half_man;
    if (rem > 0x1000u || (rem == 0x1000u && (half_man & 1u))) out++; /* may carry into the exponent: correct */
    return (uint16_t)out;
}

static inline float f16_at(const uint8_t *b, size_t off) {
    return or_f16_to_f32((uint16_t)(b[off] | (b[off + 1] << 8)));
}

/* ======================================================================== activation quantisers */

/* q8k.rs:76-114 `Q8KRow::quantize_scalar_into` (ggml quantize_row_q8_K_ref) + q8k.rs:190-193 pair sums. */
void or_q8k_from_f32(const float *x, size_t n, or_q8k *r) {
    size_t nb = n / 256;
    r->n = n;
    r->nb = nb;
    for (size_t b = 0; b < nb; b++) {
        const float *blk = x + b * 256;
        float amax = 0.0f, max = 0.0f;
        for (int i = 0; i < 256; i++) {
            float a = fabsf(blk[i]);
            if (a > amax) {
                amax = a;
                max = blk[i];
            }
        }
        int8_t *qs = r->qs + b * 256;
        int16_t *bs = r->bsums + b * 16;
        if (amax == 0.0f) {
            r->d[b] = 0.0f;
            memset(qs, 0, 256);
            memset(bs, 0, 32);
        } else {
            float iscale = -127.0f / max;
            for (int i = 0; i < 256; i++) {
                int q = (int)rintf(iscale * blk[i]); /* round_ties_even */
                qs[i] = (int8_t)(q < 127 ? q : 127);
            }
            for (int g = 0; g < 16; g++) {
                int s = 0;
                for (int j = 0; j < 16; j++) s += qs[16 * g + j];
                bs[g] = (int16_t)s;
            }
            r->d[b] = 1.0f / iscale;
        }
        for (int s = 0; s < 8; s++) r->q8s[b * 8 + s] = (int16_t)(bs[2 * s] + bs[2 * s + 1]);
    }
}

void or_q8k_alloc(or_q8k *r, size_t n) {
    size_t nb = n / 256;
    r->n = n;
    r->nb = nb;
    r->d = (float *)calloc(nb ? nb : 1, sizeof(float));
    r->qs = (int8_t *)calloc(n ? n : 1, 1);
    r->bsums = (int16_t *)calloc(nb * 16 + 1, sizeof(int16_t));
    r->q8s = (int16_t *)calloc(nb * 8 + 1, sizeof(int16_t));
}

void or_q8k_release(or_q8k *r) {
    free(r->d);
    free(r->qs);
    free(r->bsums);
    free(r->q8s);
    memset(r, 0, sizeof(*r));
}

/* q8k.rs:139-150 `to_ggml_bytes` */
static void q8k_to_ggml(const or_q8k *r, uint8_t *out) {
    for (size_t b = 0; b < r->nb; b++) {
        uint8_t *o = out + b * 292;
        memcpy(o, &r->d[b], 4);
        memcpy(o + 4, r->qs + b * 256, 256);
        memcpy(o + 260, r->bsums + b * 16, 32);
    }
}

/* q8k.rs:152-172 `from_ggml_bytes` */
void or_q8k_from_ggml(const uint8_t *in, size_t n, or_q8k *r) {
    r->n = n;
    r->nb = n / 256;
    for (size_t b = 0; b < r->nb; b++) {
        const uint8_t *blk = in + b * 292;
        memcpy(&r->d[b], blk, 4);
        memcpy(r->qs + b * 256, blk + 4, 256);
        memcpy(r->bsums + b * 16, blk + 260, 32);
        for (int s = 0; s < 8; s++) r->q8s[b * 8 + s] = (int16_t)(r->bsums[b * 16 + 2 * s] + r->bsums[b * 16 + 2 * s + 1]);
    }
}

void or_q8k_quantize(const float *x, size_t n, uint8_t *out) {
    or_q8k r;
    or_q8k_alloc(&r, n);
    or_q8k_from_f32(x, n, &r);
    q8k_to_ggml(&r, out);
    or_q8k_release(&r);
}

/* q8.rs:81-121 `Q8Row::quantize_scalar_into` (ggml quantize_row_q8_0_ref); d (f16 bits), d32 and the codes are
 * kept. The derived `dxs`/`off6` of q8.rs:107-120 are recomputed from the codes where the K-quant x Q8_0 dots
 * need them (q8_fine_sums below), with the same integer sums and the same single f32 product. */
void or_q8_from_f32(const float *x, size_t n, or_q8 *r) {
    size_t nb = n / 32;
    r->n = n;
    r->nb = nb;
    for (size_t b = 0; b < nb; b++) {
        const float *blk = x + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) {
            float a = fabsf(blk[i]);
            if (a > amax) amax = a;
        }
        float dd = amax / 127.0f;
        float id = dd != 0.0f ? 1.0f / dd : 0.0f;
        r->d[b] = or_f32_to_f16(dd);
        r->d32[b] = or_f16_to_f32(r->d[b]);
        for (int i = 0; i < 32; i++) {
            float q = roundf(blk[i] * id); /* round half away from zero; `as i8` saturates */
            r->qs[b * 32 + i] = (int8_t)(q > 127.0f ? 127 : (q < -128.0f ? -128 : (int)q));
        }
    }
}

void or_q8_alloc(or_q8 *r, size_t n) {
    size_t nb = n / 32;
    r->n = n;
    r->nb = nb;
    r->d = (uint16_t *)calloc(nb + 1, 2);
    r->d32 = (float *)calloc(nb + 1, 4);
    r->qs = (int8_t *)calloc(n + 1, 1);
}

void or_q8_release(or_q8 *r) {
    free(r->d);
    free(r->d32);
    free(r->qs);
    memset(r, 0, sizeof(*r));
}

void or_q8_from_ggml(const uint8_t *in, size_t n, or_q8 *r) {
    r->n = n;
    r->nb = n / 32;
    for (size_t b = 0; b < r->nb; b++) {
        r->d[b] = (uint16_t)(in[b * 34] | (in[b * 34 + 1] << 8));
        r->d32[b] = or_f16_to_f32(r->d[b]);
        memcpy(r->qs + b * 32, in + b * 34 + 2, 32);
    }
}

void or_q8_0_quantize(const float *x, size_t n, uint8_t *out) {
    or_q8 r;
    or_q8_alloc(&r, n);
    or_q8_from_f32(x, n, &r);
    for (size_t b = 0; b < r.nb; b++) {
        out[b * 34] = (uint8_t)(r.d[b] & 0xFF);
        out[b * 34 + 1] = (uint8_t)(r.d[b] >> 8);
        memcpy(out + b * 34 + 2, r.qs + b * 32, 32);
    }
    or_q8_release(&r);
}

/* ============================================================================== layouts and dequant */

size_t or_row_bytes(int type, size_t cols) {
    switch (type) {
    case AQ_TYPE_F32: return cols * 4;
    case AQ_TYPE_Q4_0: return cols / 32 * 18;
    case AQ_TYPE_Q8_0: return cols / 32 * 34;
    case AQ_TYPE_Q4_K: return cols / 256 * 144;
    case AQ_TYPE_Q5_K: return cols / 256 * 176;
    case AQ_TYPE_Q6_K: return cols / 256 * 210;
    default: return 0;
    }
}

/* quant.rs:45-51 `get_scale_min_k4` */
static inline void scale_min_k4(int j, const uint8_t *q, int *sc, int *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* quant.rs:65-219 `dequant_*` */
int or_dequant(int type, const uint8_t *src, size_t n, float *dst) {
    switch (type) {
    case AQ_TYPE_F32:
        memcpy(dst, src, n * 4);
        return 0;
    case AQ_TYPE_Q4_0:
        if (n % 32) return -1;
        for (size_t i = 0; i < n / 32; i++) {
            const uint8_t *b = src + i * 18;
            float d = f16_at(b, 0);
            for (int j = 0; j < 16; j++) {
                int x0 = (b[2 + j] & 0x0F) - 8, x1 = (b[2 + j] >> 4) - 8;
                dst[i * 32 + j] = (float)x0 * d;
                dst[i * 32 + j + 16] = (float)x1 * d;
            }
        }
        return 0;
    case AQ_TYPE_Q8_0:
        if (n % 32) return -1;
        for (size_t i = 0; i < n / 32; i++) {
            const uint8_t *b = src + i * 34;
            float d = f16_at(b, 0);
            for (int j = 0; j < 32; j++) dst[i * 32 + j] = (float)(int8_t)b[2 + j] * d;
        }
        return 0;
    case AQ_TYPE_Q4_K:
    case AQ_TYPE_Q5_K: {
        if (n % 256) return -1;
        int q5 = type == AQ_TYPE_Q5_K;
        size_t bb = q5 ? 176 : 144;
        for (size_t i = 0; i < n / 256; i++) {
            const uint8_t *b = src + i * bb;
            float d = f16_at(b, 0), min = f16_at(b, 2);
            const uint8_t *scales = b + 4;
            const uint8_t *qh = b + 16;
            const uint8_t *ql = b + (q5 ? 48 : 16);
            float *y = dst + i * 256;
            int is = 0;
            uint8_t u1 = 1, u2 = 2;
            for (int j = 0; j < 256; j += 64) {
                int sc, m;
                scale_min_k4(is, scales, &sc, &m);
                float d1 = d * (float)sc, m1 = min * (float)m;
                scale_min_k4(is + 1, scales, &sc, &m);
                float d2 = d * (float)sc, m2 = min * (float)m;
                for (int l = 0; l < 32; l++) {
                    int hi = q5 ? ((qh[l] & u1) ? 16 : 0) : 0;
                    y[j + l] = d1 * (float)((ql[l] & 0xF) + hi) - m1;
                }
                for (int l = 0; l < 32; l++) {
                    int hi = q5 ? ((qh[l] & u2) ? 16 : 0) : 0;
                    y[j + 32 + l] = d2 * (float)((ql[l] >> 4) + hi) - m2;
                }
                ql += 32;
                is += 2;
                u1 <<= 2;
                u2 <<= 2;
            }
        }
        return 0;
    }
    case AQ_TYPE_Q6_K:
        if (n % 256) return -1;
        for (size_t i = 0; i < n / 256; i++) {
            const uint8_t *b = src + i * 210;
            float d = f16_at(b, 208);
            float *y = dst + i * 256;
            for (int half = 0; half < 2; half++) {
                const uint8_t *ql = b + half * 64, *qh = b + 128 + half * 32;
                const int8_t *sc = (const int8_t *)(b + 192 + half * 8);
                float *yo = y + half * 128;
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    int q1 = ((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
                    int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    yo[l] = d * (float)sc[is] * (float)q1;
                    yo[l + 32] = d * (float)sc[is + 2] * (float)q2;
                    yo[l + 64] = d * (float)sc[is + 4] * (float)q3;
                    yo[l + 96] = d * (float)sc[is + 6] * (float)q4;
                }
            }
        }
        return 0;
    default:
        return -1;
    }
}

/* =========================================================================== K-quant x Q8_K dots */

static inline float reduce8(const float *l) { return ((l[0] + l[4]) + (l[2] + l[6])) + ((l[1] + l[5]) + (l[3] + l[7])); }
static inline float reduce4(const float *m) { return (m[0] + m[2]) + (m[1] + m[3]); }

/* Unsigned code of element j of sub-block s of one super-block (kdot.rs:78-95 closures). */
static inline int code_q45(const uint8_t *wb, int q5, int s, int j) {
    if (!q5) {
        uint8_t q = wb[16 + (s / 2) * 32 + j];
        return (s % 2 == 0) ? (q & 0xF) : (q >> 4);
    }
    uint8_t q = wb[48 + (s / 2) * 32 + j];
    int lo = (s % 2 == 0) ? (q & 0xF) : (q >> 4);
    return lo + ((wb[16 + j] & (1 << s)) ? 16 : 0);
}

/* The exact integer part of one super-block: 8 main lanes and (Q4_K/Q5_K) 4 min lanes, as kdot.rs:37-140. */
static void kq_block_isums(int type, const uint8_t *wb, const or_q8k *x, size_t sb, int32_t *sumi, int32_t *prod) {
    const int8_t *xq = x->qs + sb * 256;
    for (int i = 0; i < 8; i++) sumi[i] = 0;
    if (type == AQ_TYPE_Q6_K) {
        const uint8_t *ql_all = wb, *qh_all = wb + 128, *sc_all = wb + 192;
        const int16_t *bs = x->bsums + sb * 16;
        for (int half = 0; half < 2; half++) {
            const uint8_t *ql = ql_all + half * 64, *qh = qh_all + half * 32;
            const int8_t *sc = (const int8_t *)(sc_all + half * 8);
            for (int k = 0; k < 4; k++) {
                const int8_t *xs = xq + half * 128 + k * 32;
                for (int l = 0; l < 32; l++) {
                    int lo;
                    switch (k) {
                    case 0: lo = ql[l] & 0xF; break;
                    case 1: lo = ql[l + 32] & 0xF; break;
                    case 2: lo = ql[l] >> 4; break;
                    default: lo = ql[l + 32] >> 4; break;
                    }
                    int hi = (qh[l] >> (2 * k)) & 3;
                    int qw = lo | (hi << 4);
                    int scale = sc[2 * k + l / 16];
                    sumi[l / 4] += scale * qw * xs[l];
                }
            }
        }
        for (int i = 0; i < 8; i++) {
            int s0 = (int8_t)sc_all[2 * i], s1 = (int8_t)sc_all[2 * i + 1];
            sumi[i] -= 32 * (bs[2 * i] * s0 + bs[2 * i + 1] * s1);
        }
        if (prod)
            for (int i = 0; i < 4; i++) prod[i] = 0;
        return;
    }
    int q5 = type == AQ_TYPE_Q5_K;
    int sc[8], mn[8];
    for (int s = 0; s < 8; s++) scale_min_k4(s, wb + 4, &sc[s], &mn[s]);
    const int16_t *q8s = x->q8s + sb * 8;
    for (int i = 0; i < 4; i++) prod[i] = mn[2 * i] * q8s[2 * i] + mn[2 * i + 1] * q8s[2 * i + 1];
    for (int s = 0; s < 8; s++) {
        const int8_t *xs = xq + s * 32;
        for (int j = 0; j < 32; j++) sumi[j / 4] += sc[s] * code_q45(wb, q5, s, j) * xs[j];
    }
}

static size_t kq_block_bytes(int type) { return type == AQ_TYPE_Q4_K ? 144 : type == AQ_TYPE_Q5_K ? 176 : 210; }

/* kdot.rs:37-75 `dot_q45_k` and kdot.rs:97-140 `dot_q6_k_q8k`: the f32 part, no FMA. */
float or_dot_q8k_row(int type, const uint8_t *w, const or_q8k *x) {
    size_t bb = kq_block_bytes(type);
    float acc[8] = {0}, accm[4] = {0};
    int32_t sumi[8], prod[4];
    for (size_t sb = 0; sb < x->nb; sb++) {
        const uint8_t *wb = w + sb * bb;
        kq_block_isums(type, wb, x, sb, sumi, prod);
        float dx = x->d[sb];
        if (type == AQ_TYPE_Q6_K) {
            float d = dx * f16_at(wb, 208);
            for (int i = 0; i < 8; i++) acc[i] += d * (float)sumi[i];
        } else {
            float d = dx * f16_at(wb, 0);
            float dmin = -dx * f16_at(wb, 2);
            for (int i = 0; i < 4; i++) accm[i] += dmin * (float)prod[i];
            for (int i = 0; i < 8; i++) acc[i] += d * (float)sumi[i];
        }
    }
    if (type == AQ_TYPE_Q6_K) return reduce8(acc);
    return reduce8(acc) + reduce4(accm);
}

/* kdot.rs:176-333 the blocked form: codes and scales unpacked once per super-block, then each activation row
 * gets the arithmetic of the single-row kernel, so out[i] == or_dot_q8k_row(w, xs[i]) bit for bit. With the simd
 * switch on, the AVX2 form (oracle_simd.c, the same bits) runs instead. */
static void dot_q8k_rows_scalar(int type, const uint8_t *w, const or_q8k *const *xs, size_t t, float *out);
void or_dot_q8k_rows(int type, const uint8_t *w, const or_q8k *const *xs, size_t t, float *out) {
    if (or_simd())
        or_dot_q8k_rows_simd(type, w, xs, t, out);
    else
        dot_q8k_rows_scalar(type, w, xs, t, out);
}

static void dot_q8k_rows_scalar(int type, const uint8_t *w, const or_q8k *const *xs, size_t t, float *out) {
    size_t bb = kq_block_bytes(type);
    size_t nb = xs[0]->nb;
    float acc[16][8], accm[16][4];
    memset(acc, 0, sizeof(acc));
    memset(accm, 0, sizeof(accm));
    int codes[256];
    int sc[16], mn[8];
    for (size_t sb = 0; sb < nb; sb++) {
        const uint8_t *wb = w + sb * bb;
        if (type == AQ_TYPE_Q6_K) {
            for (int g = 0; g < 16; g++) sc[g] = (int8_t)wb[192 + g];
            for (int half = 0; half < 2; half++) {
                const uint8_t *ql = wb + half * 64, *qh = wb + 128 + half * 32;
                for (int k = 0; k < 4; k++)
                    for (int l = 0; l < 32; l++) {
                        int lo = (k == 0) ? (ql[l] & 0xF) : (k == 1) ? (ql[l + 32] & 0xF) : (k == 2) ? (ql[l] >> 4) : (ql[l + 32] >> 4);
                        int hi = (qh[l] >> (2 * k)) & 3;
                        codes[half * 128 + k * 32 + l] = lo | (hi << 4);
                    }
            }
            float dw = f16_at(wb, 208);
            for (size_t i = 0; i < t; i++) {
                const or_q8k *x = xs[i];
                float d = x->d[sb] * dw;
                const int8_t *xq = x->qs + sb * 256;
                const int16_t *bs = x->bsums + sb * 16;
                int32_t sumi[8] = {0};
                for (int e = 0; e < 256; e++) sumi[(e % 32) / 4] += sc[e / 16] * codes[e] * xq[e];
                for (int l = 0; l < 8; l++) sumi[l] -= 32 * (bs[2 * l] * sc[2 * l] + bs[2 * l + 1] * sc[2 * l + 1]);
                for (int l = 0; l < 8; l++) acc[i][l] += d * (float)sumi[l];
            }
        } else {
            int q5 = type == AQ_TYPE_Q5_K;
            float dw = f16_at(wb, 0), dminw = f16_at(wb, 2);
            for (int s = 0; s < 8; s++) {
                scale_min_k4(s, wb + 4, &sc[s], &mn[s]);
                for (int j = 0; j < 32; j++) codes[s * 32 + j] = code_q45(wb, q5, s, j);
            }
            for (size_t i = 0; i < t; i++) {
                const or_q8k *x = xs[i];
                float dx = x->d[sb];
                float d = dx * dw, dmin = -dx * dminw;
                const int8_t *xq = x->qs + sb * 256;
                const int16_t *q8s = x->q8s + sb * 8;
                for (int l = 0; l < 4; l++) {
                    int prod = mn[2 * l] * q8s[2 * l] + mn[2 * l + 1] * q8s[2 * l + 1];
                    accm[i][l] += dmin * (float)prod;
                }
                int32_t sumi[8] = {0};
                for (int s = 0; s < 8; s++)
                    for (int j = 0; j < 32; j++) sumi[j / 4] += sc[s] * codes[s * 32 + j] * xq[s * 32 + j];
                for (int l = 0; l < 8; l++) acc[i][l] += d * (float)sumi[l];
            }
        }
    }
    for (size_t i = 0; i < t; i++) out[i] = type == AQ_TYPE_Q6_K ? reduce8(acc[i]) : reduce8(acc[i]) + reduce4(accm[i]);
}

float or_dot_q8k(int type, const uint8_t *w, const uint8_t *x_q8k, size_t n) {
    or_q8k x;
    or_q8k_alloc(&x, n);
    or_q8k_from_ggml(x_q8k, n, &x);
    float v = or_dot_q8k_row(type, w, &x);
    or_q8k_release(&x);
    return v;
}

void or_dot_q8k_t(int type, const uint8_t *w, const uint8_t *const *xs, size_t t, size_t n, float *out) {
    or_q8k rows[16];
    const or_q8k *ptrs[16] = {0};
    for (size_t i = 0; i < t; i++) {
        or_q8k_alloc(&rows[i], n);
        or_q8k_from_ggml(xs[i], n, &rows[i]);
        ptrs[i] = &rows[i];
    }
    or_dot_q8k_rows(type, w, ptrs, t, out);
    for (size_t i = 0; i < t; i++) or_q8k_release(&rows[i]);
}

void or_kq_isums(int type, const uint8_t *w, const uint8_t *x_q8k, size_t n, int32_t *lanes, int32_t *mins) {
    or_q8k x;
    or_q8k_alloc(&x, n);
    or_q8k_from_ggml(x_q8k, n, &x);
    size_t bb = kq_block_bytes(type);
    int32_t prod[4];
    for (size_t sb = 0; sb < x.nb; sb++) {
        kq_block_isums(type, w + sb * bb, &x, sb, lanes + sb * 8, prod);
        for (int i = 0; i < 4; i++) mins[sb * 4 + i] = type == AQ_TYPE_Q6_K ? 0 : prod[i];
    }
    or_q8k_release(&x);
}

/* or_kq_isums over `rows` weight rows (row r at w + r * row_bytes): lanes [rows][nb][8], mins [rows][nb][4]. */
void or_kq_isums_mat(int type, const uint8_t *w, size_t rows, const uint8_t *x_q8k, size_t n, int32_t *lanes,
                     int32_t *mins) {
    const size_t nb = n / 256, rb = nb * kq_block_bytes(type);
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)rows; r++)
        or_kq_isums(type, w + (size_t)r * rb, x_q8k, n, lanes + (size_t)r * nb * 8, mins + (size_t)r * nb * 4);
}

/* ================================================================== Q8_0 / Q4_0 / F32 weight dots */

/* q8.rs:107-120 `Q8Row::derive` for one 32-block: lo = sum(q[0..16]), hi = sum(q[16..32]); dxs = d32 * f32(lo + hi)
 * (exact: an 11-bit scale times a sum of at most 12 bits); off6 = [32 lo, 0, 0, 0, 32 hi, 0, 0, 0]. */
static void q8_fine_sums(const or_q8 *x, size_t b, int32_t *lo, int32_t *hi, float *dxs) {
    int32_t l = 0, h = 0;
    for (int j = 0; j < 16; j++) l += x->qs[b * 32 + j];
    for (int j = 16; j < 32; j++) h += x->qs[b * 32 + j];
    *lo = l;
    *hi = h;
    *dxs = x->d32[b] * (float)(l + h);
}

/* dot.rs:69-99 `dot_q45_k_q8` (with the code closures of dot.rs:101-117), the `--q8-fine` form of Q4_K / Q5_K
 * (matvec.rs:129-160): per sub-block s of super-block sb, against the Q8_0 block xb = 8 sb + s, 8 exact i32 lanes
 * p32[j/4] += q*x; acc[i] += f32(p32[i]) * (d32[xb] * (d * sc)); accm[s] += (m * -dmin) * dxs[xb]; the result is
 * reduce8(acc) + reduce8(accm). No FMA. */
static float dot_q45_k_q8(int q5, const uint8_t *w, const or_q8 *x) {
    const size_t bb = q5 ? 176 : 144;
    float acc[8] = {0}, accm[8] = {0};
    for (size_t sb = 0; sb < x->nb / 8; sb++) {
        const uint8_t *wb = w + sb * bb;
        const float d = f16_at(wb, 0), dmin = f16_at(wb, 2);
        for (int s = 0; s < 8; s++) {
            int sc, m;
            scale_min_k4(s, wb + 4, &sc, &m);
            const size_t xb = sb * 8 + s;
            const int8_t *xq = x->qs + xb * 32;
            int32_t p32[8] = {0};
            for (int j = 0; j < 32; j++) p32[j / 4] += code_q45(wb, q5, s, j) * xq[j];
            const float f = x->d32[xb] * (d * (float)sc);
            for (int i = 0; i < 8; i++) acc[i] += (float)p32[i] * f;
            int32_t lo, hi;
            float dxs;
            q8_fine_sums(x, xb, &lo, &hi, &dxs);
            accm[s] += ((float)m * -dmin) * dxs;
        }
    }
    return reduce8(acc) + reduce8(accm);
}

/* dot.rs:119-160 `dot_q6_k_q8`: unsigned 6-bit codes against Q8_0 block xb = 8 sb + 4 half + k; the -32 offset is
 * taken in integer from lane 0 (32 lo) and lane 4 (32 hi); lanes 0..3 are scaled by the group scale sc[2k], lanes
 * 4..7 by sc[2k + 1]: acc[i] += f32(p32[i]) * (d32[xb] * (d * sc)); the result is reduce8(acc). */
static float dot_q6_k_q8(const uint8_t *w, const or_q8 *x) {
    float acc[8] = {0};
    for (size_t sb = 0; sb < x->nb / 8; sb++) {
        const uint8_t *wb = w + sb * 210;
        const float d = f16_at(wb, 208);
        for (int half = 0; half < 2; half++) {
            const uint8_t *ql = wb + half * 64, *qh = wb + 128 + half * 32;
            const int8_t *sc = (const int8_t *)(wb + 192 + half * 8);
            for (int k = 0; k < 4; k++) {
                const size_t xb = sb * 8 + half * 4 + k;
                const int8_t *xq = x->qs + xb * 32;
                int32_t p32[8] = {0};
                for (int l = 0; l < 32; l++) {
                    int lo;
                    switch (k) {
                    case 0: lo = ql[l] & 0xF; break;
                    case 1: lo = ql[l + 32] & 0xF; break;
                    case 2: lo = ql[l] >> 4; break;
                    default: lo = ql[l + 32] >> 4; break;
                    }
                    const int hi = (qh[l] >> (2 * k)) & 3;
                    p32[l / 4] += (lo | (hi << 4)) * xq[l];
                }
                int32_t slo, shi;
                float dxs;
                q8_fine_sums(x, xb, &slo, &shi, &dxs);
                p32[0] -= 32 * slo;
                p32[4] -= 32 * shi;
                const float f_lo = x->d32[xb] * (d * (float)sc[2 * k]);
                const float f_hi = x->d32[xb] * (d * (float)sc[2 * k + 1]);
                for (int i = 0; i < 8; i++) acc[i] += (float)p32[i] * (i < 4 ? f_lo : f_hi);
            }
        }
    }
    return reduce8(acc);
}

/* dot.rs:29-45 `dot_q8_0_q8` and dot.rs:48-66 `dot_q4_0_q8`: one f32 accumulator, blocks left to right; K-quant
 * weights take the Q8_0-grain kernels above (dot.rs:202-226 `dot_q8` routes every type). */
float or_dot_q8_row(int type, const uint8_t *w, const or_q8 *x) {
    if (or_simd() && (type == AQ_TYPE_Q8_0 || type == AQ_TYPE_Q4_0)) return or_dot_q8_row_simd(type, w, x);
    if (type == AQ_TYPE_Q4_K || type == AQ_TYPE_Q5_K) return dot_q45_k_q8(type == AQ_TYPE_Q5_K, w, x);
    if (type == AQ_TYPE_Q6_K) return dot_q6_k_q8(w, x);
    float acc = 0.0f;
    if (type == AQ_TYPE_Q8_0) {
        for (size_t b = 0; b < x->nb; b++) {
            const uint8_t *wb = w + b * 34;
            float dw = f16_at(wb, 0);
            const int8_t *xq = x->qs + b * 32;
            int32_t isum = 0;
            for (int j = 0; j < 32; j++) isum += (int8_t)wb[2 + j] * xq[j];
            acc += (dw * x->d32[b]) * (float)isum;
        }
    } else {
        for (size_t b = 0; b < x->nb; b++) {
            const uint8_t *wb = w + b * 18;
            float dw = f16_at(wb, 0);
            const int8_t *xq = x->qs + b * 32;
            int32_t isum = 0;
            for (int j = 0; j < 16; j++) {
                int lo = (wb[2 + j] & 0x0F) - 8, hi = (wb[2 + j] >> 4) - 8;
                isum += lo * xq[j] + hi * xq[j + 16];
            }
            acc += (dw * x->d32[b]) * (float)isum;
        }
    }
    return acc;
}

float or_dot_q8(int type, const uint8_t *w, const uint8_t *x_q8_0, size_t n) {
    or_q8 x;
    or_q8_alloc(&x, n);
    or_q8_from_ggml(x_q8_0, n, &x);
    float v = or_dot_q8_row(type, w, &x);
    or_q8_release(&x);
    return v;
}

/* dot.rs:180-200 `dot_f32`: 32-element partials left to right, blocks left to right, then the tail. */
float or_dot_f32(const float *w, const float *x, size_t n) {
    float acc = 0.0f;
    size_t i = 0;
    while (i + 32 <= n) {
        float part = 0.0f;
        for (int j = 0; j < 32; j++) part += w[i + j] * x[i + j];
        acc += part;
        i += 32;
    }
    float part = 0.0f;
    while (i < n) {
        part += w[i] * x[i];
        i++;
    }
    return acc + part;
}

/* ========================================================================= elementwise and row kernels */

/* rmsnorm.rs:55-69 `sum_squares_8lane` */
static float sum_squares_8lane(const float *x, size_t n) {
    size_t n8 = n / 8 * 8;
    float l[8] = {0};
    for (size_t i = 0; i < n8; i += 8)
        for (int k = 0; k < 8; k++) l[k] += x[i + k] * x[i + k];
    float ss = reduce8(l);
    for (size_t i = n8; i < n; i++) ss += x[i] * x[i];
    return ss;
}

/* rmsnorm.rs:48-53 `inv_rms` */
static float inv_rms(const float *x, size_t n, float eps) {
    float mean = sum_squares_8lane(x, n) / (float)n;
    return 1.0f / sqrtf(mean + eps);
}

/* rmsnorm.rs:25-34 `rmsnorm_scalar` */
void or_rmsnorm(const float *x, const float *w, float eps, float *y, size_t n) {
    float inv = inv_rms(x, n, eps);
    for (size_t i = 0; i < n; i++) y[i] = (x[i] * inv) * w[i];
}

/* The reference's f32 exp / log1p are the platform libm's expf / log1pf (Rust's f32::exp / f32::ln_1p lower to
 * them); the oracle calls exactly those. The device evaluates aq_math.h's restatement of the same two GNU libc
 * algorithms; or_math_sweep below compares that restatement with these calls over any range of f32 bit patterns. */
#define OR_EXPF expf
#define OR_LOG1PF log1pf

/* act.rs:7-9 `silu`, 12-14 `sigmoid`, 33-40 `softplus` */
float or_silu(float x) { return x / (1.0f + OR_EXPF(-x)); }
float or_sigmoid(float x) { return 1.0f / (1.0f + OR_EXPF(-x)); }
float or_softplus(float x) { return x > 20.0f ? x : OR_LOG1PF(OR_EXPF(x)); }
float or_expf(float x) { return OR_EXPF(x); }
float or_log1pf(float x) { return OR_LOG1PF(x); }
/* fn: 0 exp, 1 log1p, 2 silu, 3 sigmoid, 4 softplus, elementwise; restated != 0 evaluates aq_math.h's restatement
 * (the device's arithmetic) instead of the platform libm (the reference's) */
static float eval_one(int fn, float x, int restated) {
    const float e = restated ? aq_expf(-x) : OR_EXPF(-x);
    switch (fn) {
    case 0: return restated ? aq_expf(x) : OR_EXPF(x);
    case 1: return restated ? aq_log1pf(x) : OR_LOG1PF(x);
    case 2: return x / (1.0f + e);
    case 3: return 1.0f / (1.0f + e);
    default: return x > 20.0f ? x : (restated ? aq_log1pf(aq_expf(x)) : OR_LOG1PF(OR_EXPF(x)));
    }
}

void or_eval_math(int fn, const float *x, float *y, size_t n, int restated) {
    for (size_t i = 0; i < n; i++) y[i] = eval_one(fn, x[i], restated);
}

/* Compare the restatement with the platform libm on the f32 bit patterns first, first + stride, ... (count of
 * them, wrapping at 2^32), on all cores. Returns the number of arguments whose results differ in any bit (two NaNs
 * count as equal) and the first such pattern in *first_bad (0xffffffff if none). */
uint64_t or_math_sweep(int fn, uint32_t first, uint64_t count, uint32_t stride, uint32_t *first_bad) {
    uint64_t bad = 0;
    uint32_t fb = 0xffffffffu;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (int64_t i = 0; i < (int64_t)count; i++) {
        const uint32_t u = first + (uint32_t)((uint64_t)i * stride);
        float x;
        memcpy(&x, &u, 4);
        const float a = eval_one(fn, x, 0), b = eval_one(fn, x, 1);
        uint32_t ua, ub;
        memcpy(&ua, &a, 4);
        memcpy(&ub, &b, 4);
        if (ua != ub && !(a != a && b != b)) {
            bad++;
#pragma omp critical
            if (u < fb) fb = u;
        }
    }
    *first_bad = fb;
    return bad;
}

/* rmsnorm.rs:37-46 `rmsnorm_gated` */
void or_rmsnorm_gated(const float *x, const float *gate, const float *w, float eps, float *y, size_t n) {
    float inv = inv_rms(x, n, eps);
    for (size_t i = 0; i < n; i++) y[i] = (w[i] * (x[i] * inv)) * or_silu(gate[i]);
}

/* act.rs:24-30 `swiglu` */
void or_swiglu(const float *g, const float *u, float *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = or_silu(g[i]) * u[i];
}

/* softmax.rs:22-49 `softmax_scalar` */
void or_softmax(const float *x, float *y, size_t n) {
    float m = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (x[i] > m) m = x[i];
    for (size_t i = 0; i < n; i++) y[i] = OR_EXPF(x[i] - m);
    size_t n8 = n / 8 * 8;
    float l[8] = {0};
    for (size_t i = 0; i < n8; i += 8)
        for (int k = 0; k < 8; k++) l[k] += y[i + k];
    float s = reduce8(l);
    for (size_t i = n8; i < n; i++) s += y[i];
    for (size_t i = 0; i < n; i++) y[i] /= s;
}

/* rope.rs:10-12 `inv_freq` */
void or_inv_freq(size_t rope_dim, float theta, float *out) {
    for (size_t i = 0; i < rope_dim / 2; i++) out[i] = 1.0f / powf(theta, (float)(2 * i) / (float)rope_dim);
}

/* rope.rs:15-28 `cos_sin` */
void or_cos_sin(uint32_t pos, const float *inv_freq, size_t half, float *cos, float *sin) {
    float p = (float)pos;
    for (size_t i = 0; i < half; i++) {
        float angle = p * inv_freq[i];
        float s = sinf(angle), c = cosf(angle);
        cos[i] = c;
        cos[i + half] = c;
        sin[i] = s;
        sin[i + half] = s;
    }
}

/* rope.rs:31-45 `apply_rope` over `len` floats (heads x head_dim) */
void or_apply_rope(float *x, size_t len, size_t head_dim, size_t rope_dim, const float *cos, const float *sin) {
    size_t half = rope_dim / 2;
    for (size_t h = 0; h + head_dim <= len; h += head_dim) {
        float *v = x + h;
        for (size_t i = 0; i < half; i++) {
            float a = v[i], b = v[i + half];
            v[i] = a * cos[i] - b * sin[i];
            v[i + half] = b * cos[i + half] + a * sin[i + half];
        }
    }
}

/* conv.rs:11-36 `causal_conv1d_step` */
void or_conv1d_step(float *state, const float *w, size_t kernel, const float *x_new, float *out, size_t channels,
                    int act_silu) {
    for (size_t ch = 0; ch < channels; ch++) {
        float *st = state + ch * (kernel - 1);
        const float *wc = w + ch * kernel;
        float acc = 0.0f;
        for (size_t j = 0; j + 1 < kernel; j++) acc += wc[j] * st[j];
        acc += wc[kernel - 1] * x_new[ch];
        for (size_t j = 0; j + 2 < kernel; j++) st[j] = st[j + 1];
        if (kernel >= 2) st[kernel - 2] = x_new[ch];
        out[ch] = act_silu ? or_silu(acc) : acc;
    }
}

/* deltanet.rs:19-29 `l2norm` */
void or_l2norm(float *x, size_t n, float eps) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
    float inv = 1.0f / sqrtf(ss + eps);
    for (size_t i = 0; i < n; i++) x[i] *= inv;
}

/* deltanet.rs:32-35 `gate_g` */
float or_gate_g(float a, float dt_bias, float big_a) { return big_a * or_softplus(a + dt_bias); }

/* deltanet.rs:43-86 `deltanet_step` */
void or_deltanet_step(const float *q, const float *k, const float *v, float g, float beta, float *s, float *out,
                      size_t dk, size_t dv) {
    float decay = OR_EXPF(g);
    for (size_t i = 0; i < dk * dv; i++) s[i] *= decay;
    for (size_t vv = 0; vv < dv; vv++) out[vv] = 0.0f;
    for (size_t kk = 0; kk < dk; kk++) {
        const float *row = s + kk * dv;
        float kv = k[kk];
        for (size_t vv = 0; vv < dv; vv++) out[vv] += row[vv] * kv;
    }
    for (size_t vv = 0; vv < dv; vv++) out[vv] = (v[vv] - out[vv]) * beta;
    for (size_t kk = 0; kk < dk; kk++) {
        float *row = s + kk * dv;
        float kv = k[kk];
        for (size_t vv = 0; vv < dv; vv++) row[vv] += kv * out[vv];
    }
    for (size_t vv = 0; vv < dv; vv++) out[vv] = 0.0f;
    for (size_t kk = 0; kk < dk; kk++) {
        const float *row = s + kk * dv;
        float qk = q[kk];
        for (size_t vv = 0; vv < dv; vv++) out[vv] += row[vv] * qk;
    }
}
