/*
 * oracle_simd.c — TEST INFRASTRUCTURE ONLY: AVX2 forms of the oracle's weight dots, used when the process-wide
 * switch or_set_simd(1) is on (bench.py's cpu_baseline leg turns it on; tests compare it with the scalar forms).
 *
 * The reference runs its CPU path through hand-written AVX2 kernels (kernels/avx2.rs: dot_q8k / dot_q8k_t for the
 * K-quant x Q8_K dots, dot_q8 for Q8_0 / Q4_0, selected at run time in kdot.rs:147, 318 and dot.rs:206) that are
 * bit-identical to its scalar kernels (avx2.rs:1-20). These are this oracle's own vector forms of the same
 * arithmetic, bit-identical to oracle_kernels.c's scalar ones:
 *  - K-quant x Q8_K (kdot.rs:37-140): per sub-block the 32 unsigned codes against the 32 activation codes by
 *    `maddubs` (unsigned x signed byte pairs into i16; |pair| <= 63 * 128 * 2, no saturation), then `madd` against
 *    the sub-block's integer scale (i16 x i16 pairs into i32), so i32 m of the result is scale * (the dot of
 *    elements 4m .. 4m+3) — exactly the reference's lane m. Integer sums are exact in any order. The f32 part is
 *    the scalar's, lane for lane: acc[l] = acc[l] + d * f32(sumi[l]) as a rounded multiply and a rounded add
 *    (built with -ffp-contract=off), then the same reduce8 / reduce4;
 *  - Q8_0 / Q4_0 x Q8_0 (dot.rs:29-66): each block's exact i32 dot from sign-extended i16 products (`madd`), then
 *    the scalar chain acc = acc + (dw * dx) * f32(isum) block after block.
 */
#include <immintrin.h>
#include <string.h>

#include "oracle.h"
#include "oracle_internal.h"

static int g_simd = 0;
void or_set_simd(int on) { g_simd = on != 0; }
int or_simd(void) { return g_simd; }

static inline float f16_at(const uint8_t *b, size_t off) { return or_f16_to_f32((uint16_t)(b[off] | (b[off + 1] << 8))); }
static inline float reduce8(const float *l) { return ((l[0] + l[4]) + (l[2] + l[6])) + ((l[1] + l[5]) + (l[3] + l[7])); }
static inline float reduce4(const float *m) { return (m[0] + m[2]) + (m[1] + m[3]); }

/* quant.rs:45-51 get_scale_min_k4 for all 8 sub-blocks */
static inline void scales_k4(const uint8_t *q, int *sc, int *mn) {
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            sc[j] = q[j] & 63;
            mn[j] = q[j + 4] & 63;
        } else {
            sc[j] = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
            mn[j] = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
        }
    }
}

/* acc[l] = acc[l] + d * f32(sumi[l]) for the 8 lanes */
static inline __m256 lane_fma_free(__m256 acc, float d, __m256i sumi) {
    return _mm256_add_ps(acc, _mm256_mul_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi)));
}

/* kdot.rs:176-333 with the arithmetic of kdot.rs:37-140 per activation row: out[i] = W . xs[i], codes unpacked once
 * per super-block. Same contract and bits as or_dot_q8k_rows. */
void or_dot_q8k_rows_simd(int type, const uint8_t *w, const or_q8k *const *xs, size_t t, float *out) {
    const size_t nb = xs[0]->nb;
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    __m256 acc[16];
    float accm[16][4];
    for (size_t i = 0; i < t; i++) {
        acc[i] = _mm256_setzero_ps();
        accm[i][0] = accm[i][1] = accm[i][2] = accm[i][3] = 0.0f;
    }
    __m256i codes[8];
    if (type == AQ_TYPE_Q6_K) {
        for (size_t sb = 0; sb < nb; sb++) {
            const uint8_t *wb = w + sb * 210;
            const int8_t *sc = (const int8_t *)(wb + 192);
            /* codes of group (half, k): low 4 bits from ql (k = 0, 1 low nibbles of ql[0..32], ql[32..64]; k = 2, 3
             * their high nibbles), bits 4-5 = (qh[l] >> 2k) & 3 */
            for (int half = 0; half < 2; half++) {
                const __m256i qla = _mm256_loadu_si256((const __m256i *)(wb + half * 64));
                const __m256i qlb = _mm256_loadu_si256((const __m256i *)(wb + half * 64 + 32));
                const __m256i qh = _mm256_loadu_si256((const __m256i *)(wb + 128 + half * 32));
                const __m256i lo[4] = {_mm256_and_si256(qla, m4), _mm256_and_si256(qlb, m4),
                                       _mm256_and_si256(_mm256_srli_epi16(qla, 4), m4),
                                       _mm256_and_si256(_mm256_srli_epi16(qlb, 4), m4)};
                for (int k = 0; k < 4; k++) {
                    const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(qh, 2 * k), _mm256_set1_epi8(3));
                    codes[half * 4 + k] = _mm256_or_si256(lo[k], _mm256_slli_epi16(hi, 4));
                }
            }
            /* the group scales as i16 pairs: elements 0..15 of group g take sc[2g], 16..31 sc[2g + 1] */
            __m256i sv[8];
            for (int g = 0; g < 8; g++) sv[g] = _mm256_set_m128i(_mm_set1_epi16(sc[2 * g + 1]), _mm_set1_epi16(sc[2 * g]));
            const float dw = f16_at(wb, 208);
            for (size_t i = 0; i < t; i++) {
                const or_q8k *x = xs[i];
                const int8_t *xq = x->qs + sb * 256;
                __m256i sumi = _mm256_setzero_si256();
                for (int g = 0; g < 8; g++) {
                    const __m256i xv = _mm256_loadu_si256((const __m256i *)(xq + g * 32));
                    sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(_mm256_maddubs_epi16(codes[g], xv), sv[g]));
                }
                /* the -32 offset: lane l takes groups of 16 elements 2l and 2l + 1 (kdot.rs:125-129) */
                const int16_t *bs = x->bsums + sb * 16;
                int32_t off[8];
                for (int l = 0; l < 8; l++) off[l] = 32 * (bs[2 * l] * sc[2 * l] + bs[2 * l + 1] * sc[2 * l + 1]);
                sumi = _mm256_sub_epi32(sumi, _mm256_loadu_si256((const __m256i *)off));
                acc[i] = lane_fma_free(acc[i], x->d[sb] * dw, sumi);
            }
        }
    } else {
        const int q5 = type == AQ_TYPE_Q5_K;
        const size_t bb = q5 ? 176 : 144;
        for (size_t sb = 0; sb < nb; sb++) {
            const uint8_t *wb = w + sb * bb;
            int sc[8], mn[8];
            scales_k4(wb + 4, sc, mn);
            const uint8_t *qs = wb + (q5 ? 48 : 16);
            const __m256i qh = q5 ? _mm256_loadu_si256((const __m256i *)(wb + 16)) : _mm256_setzero_si256();
            for (int g = 0; g < 4; g++) { /* sub-blocks 2g (low nibbles) and 2g + 1 (high nibbles) of qs[32g ..] */
                const __m256i q = _mm256_loadu_si256((const __m256i *)(qs + g * 32));
                codes[2 * g] = _mm256_and_si256(q, m4);
                codes[2 * g + 1] = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
                if (q5)
                    for (int h = 0; h < 2; h++) { /* bit s of qh[j] is bit 4 of code j of sub-block s */
                        const int s = 2 * g + h;
                        const __m256i b = _mm256_and_si256(_mm256_srli_epi16(qh, s), _mm256_set1_epi8(1));
                        codes[s] = _mm256_or_si256(codes[s], _mm256_slli_epi16(b, 4));
                    }
            }
            __m256i sv[8];
            for (int s = 0; s < 8; s++) sv[s] = _mm256_set1_epi16((int16_t)sc[s]);
            const float dw = f16_at(wb, 0), dminw = f16_at(wb, 2);
            for (size_t i = 0; i < t; i++) {
                const or_q8k *x = xs[i];
                const float dx = x->d[sb];
                const float d = dx * dw, dmin = -dx * dminw;
                const int8_t *xq = x->qs + sb * 256;
                const int16_t *q8s = x->q8s + sb * 8;
                for (int l = 0; l < 4; l++) {
                    const int prod = mn[2 * l] * q8s[2 * l] + mn[2 * l + 1] * q8s[2 * l + 1];
                    accm[i][l] += dmin * (float)prod;
                }
                __m256i sumi = _mm256_setzero_si256();
                for (int s = 0; s < 8; s++) {
                    const __m256i xv = _mm256_loadu_si256((const __m256i *)(xq + s * 32));
                    sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(_mm256_maddubs_epi16(codes[s], xv), sv[s]));
                }
                acc[i] = lane_fma_free(acc[i], d, sumi);
            }
        }
    }
    for (size_t i = 0; i < t; i++) {
        float a[8];
        _mm256_storeu_ps(a, acc[i]);
        out[i] = type == AQ_TYPE_Q6_K ? reduce8(a) : reduce8(a) + reduce4(accm[i]);
    }
}

/* the exact sum of the 8 i32 lanes */
static inline int32_t hsum_i32(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
    return _mm_cvtsi128_si32(s);
}

/* dot.rs:29-45 `dot_q8_0_q8` and dot.rs:48-66 `dot_q4_0_q8` (Q8_0 / Q4_0 weights only). Same bits as
 * or_dot_q8_row for those types. */
float or_dot_q8_row_simd(int type, const uint8_t *w, const or_q8 *x) {
    float acc = 0.0f;
    if (type == AQ_TYPE_Q8_0) {
        for (size_t b = 0; b < x->nb; b++) {
            const uint8_t *wb = w + b * 34;
            const __m128i w0 = _mm_loadu_si128((const __m128i *)(wb + 2)), w1 = _mm_loadu_si128((const __m128i *)(wb + 18));
            const __m128i x0 = _mm_loadu_si128((const __m128i *)(x->qs + b * 32)),
                          x1 = _mm_loadu_si128((const __m128i *)(x->qs + b * 32 + 16));
            const __m256i p = _mm256_add_epi32(_mm256_madd_epi16(_mm256_cvtepi8_epi16(w0), _mm256_cvtepi8_epi16(x0)),
                                               _mm256_madd_epi16(_mm256_cvtepi8_epi16(w1), _mm256_cvtepi8_epi16(x1)));
            const int32_t isum = hsum_i32(p);
            acc += (f16_at(wb, 0) * x->d32[b]) * (float)isum;
        }
    } else {
        const __m128i m4 = _mm_set1_epi8(0x0F), e8 = _mm_set1_epi8(8);
        for (size_t b = 0; b < x->nb; b++) {
            const uint8_t *wb = w + b * 18;
            const __m128i q = _mm_loadu_si128((const __m128i *)(wb + 2));
            /* codes q - 8: elements 0..15 from the low nibbles, 16..31 from the high ones */
            const __m128i lo = _mm_sub_epi8(_mm_and_si128(q, m4), e8);
            const __m128i hi = _mm_sub_epi8(_mm_and_si128(_mm_srli_epi16(q, 4), m4), e8);
            const __m128i x0 = _mm_loadu_si128((const __m128i *)(x->qs + b * 32)),
                          x1 = _mm_loadu_si128((const __m128i *)(x->qs + b * 32 + 16));
            const __m256i p = _mm256_add_epi32(_mm256_madd_epi16(_mm256_cvtepi8_epi16(lo), _mm256_cvtepi8_epi16(x0)),
                                               _mm256_madd_epi16(_mm256_cvtepi8_epi16(hi), _mm256_cvtepi8_epi16(x1)));
            const int32_t isum = hsum_i32(p);
            acc += (f16_at(wb, 0) * x->d32[b]) * (float)isum;
        }
    }
    return acc;
}
