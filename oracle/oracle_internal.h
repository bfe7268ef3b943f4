/* oracle_internal.h — TEST INFRASTRUCTURE ONLY: types shared by the oracle's translation units. */
#ifndef AQ_ORACLE_INTERNAL_H
#define AQ_ORACLE_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

/* q8k.rs:16-23 `Q8KRow`: f32 d per block, int8 codes, 16 group sums and 8 derived sub-block sums per block. */
typedef struct or_q8k {
    size_t n, nb;
    float *d;
    int8_t *qs;
    int16_t *bsums;
    int16_t *q8s;
} or_q8k;

/* q8.rs:15-29 `Q8Row` (the fields the Q8_0 / Q4_0 kernels read). */
typedef struct or_q8 {
    size_t n, nb;
    uint16_t *d;
    float *d32;
    int8_t *qs;
} or_q8;

void or_q8k_alloc(or_q8k *r, size_t n);
void or_q8k_release(or_q8k *r);
void or_q8k_from_f32(const float *x, size_t n, or_q8k *r);
void or_q8k_from_ggml(const uint8_t *in, size_t n, or_q8k *r);
void or_q8_alloc(or_q8 *r, size_t n);
void or_q8_release(or_q8 *r);
void or_q8_from_f32(const float *x, size_t n, or_q8 *r);
void or_q8_from_ggml(const uint8_t *in, size_t n, or_q8 *r);
float or_dot_q8k_row(int type, const uint8_t *w, const or_q8k *x);
void or_dot_q8k_rows(int type, const uint8_t *w, const or_q8k *const *xs, size_t t, float *out);
float or_dot_q8_row(int type, const uint8_t *w, const or_q8 *x);
/* oracle_simd.c: AVX2 forms, bit-identical to the two above (K-quant rows; Q8_0 / Q4_0 weights) */
void or_dot_q8k_rows_simd(int type, const uint8_t *w, const or_q8k *const *xs, size_t t, float *out);
float or_dot_q8_row_simd(int type, const uint8_t *w, const or_q8 *x);

#endif
