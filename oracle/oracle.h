/*
 * oracle.h — TEST INFRASTRUCTURE ONLY. A plain-C restatement of the reference's CPU path
 * (ManeeshJupalle/Qwen-3.8-in-Rust, crates/core/src) for the speculative-decode hot path, used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker. The product (libaq) never links,
 * loads or calls it.
 *
 * Every function cites the reference function it follows. Arithmetic order, rounding and the no-FMA rule
 * follow the reference's scalar kernels exactly (the reference's AVX2 kernels are bit-identical to them,
 * kdot.rs:1-18); transcendental functions are glibc's expf/log1pf/powf/sinf/cosf, which is what Rust's f32
 * methods call on Linux.
 */
#ifndef AQ_ORACLE_H
#define AQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/aq.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- f16 (the `half` 2.7.1 crate: exact f16 -> f32, round-to-nearest-even f32 -> f16) */
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);

/* ---- activation quantisers (ggml wire layouts) */
void or_q8k_quantize(const float *x, size_t n, uint8_t *out);  /* 292 B / 256 */
void or_q8_0_quantize(const float *x, size_t n, uint8_t *out); /* 34 B / 32 */

/* ---- dequantisation of one ggml row / tensor (quant.rs:65-219). Returns 0, or -1 on a bad type/length. */
int or_dequant(int type, const uint8_t *src, size_t n, float *dst);
size_t or_row_bytes(int type, size_t cols);

/* ---- dots: one weight row (ggml bytes) against activations in ggml wire layout */
float or_dot_q8k(int type, const uint8_t *w, const uint8_t *x_q8k, size_t n);
void or_dot_q8k_t(int type, const uint8_t *w, const uint8_t *const *xs, size_t t, size_t n, float *out);
void or_kq_isums(int type, const uint8_t *w, const uint8_t *x_q8k, size_t n, int32_t *lanes, int32_t *mins);
void or_kq_isums_mat(int type, const uint8_t *w, size_t rows, const uint8_t *x_q8k, size_t n, int32_t *lanes,
                     int32_t *mins);
float or_dot_q8(int type, const uint8_t *w, const uint8_t *x_q8_0, size_t n); /* any quantised type */
float or_dot_f32(const float *w, const float *x, size_t n);

/* ---- matmul: y[c*rows + r] = W[r] . x[c] from f32 activations, quantised as the weight type requires
 * (matvec.rs:147-160 act_kind, 282-292 one_row, 511-539 matmul_impl). threads <= 0: all. With the q8-fine switch
 * on (matvec.rs:133 set_q8_fine; process-wide, read by every later matmul and model call), K-quant weights take
 * Q8_0 activations (dot.rs:69-160). */
void or_set_q8_fine(int on);
int or_q8_fine(void);
/* The AVX2 forms of the K-quant x Q8_K and Q8_0 / Q4_0 dots (oracle_simd.c; the reference's avx2.rs kernels are
 * selected the same way, kdot.rs:147, 318): process-wide, off by default; the bits are the scalar forms'. */
void or_set_simd(int on);
int or_simd(void);
void or_matmul(int type, const uint8_t *w, size_t rows, size_t cols, const float *x, size_t ncols, float *y,
               int threads);

/* ---- elementwise / row kernels */
void or_rmsnorm(const float *x, const float *w, float eps, float *y, size_t n);
void or_rmsnorm_gated(const float *x, const float *gate, const float *w, float eps, float *y, size_t n);
void or_softmax(const float *x, float *y, size_t n);
float or_expf(float x);
float or_log1pf(float x);
void or_eval_math(int fn, const float *x, float *y, size_t n, int restated);
uint64_t or_math_sweep(int fn, uint32_t first, uint64_t count, uint32_t stride, uint32_t *first_bad);
float or_silu(float x);
float or_sigmoid(float x);
float or_softplus(float x);
void or_swiglu(const float *g, const float *u, float *y, size_t n);
void or_inv_freq(size_t rope_dim, float theta, float *out);
void or_cos_sin(uint32_t pos, const float *inv_freq, size_t half, float *cos, float *sin);
void or_apply_rope(float *x, size_t len, size_t head_dim, size_t rope_dim, const float *cos, const float *sin);
void or_conv1d_step(float *state, const float *w, size_t kernel, const float *x_new, float *out, size_t channels,
                    int act_silu);
void or_l2norm(float *x, size_t n, float eps);
float or_gate_g(float a, float dt_bias, float big_a);
void or_deltanet_step(const float *q, const float *k, const float *v, float g, float beta, float *s, float *out,
                      size_t dk, size_t dv);

/* ---- model (model.rs, layers/, spec.rs). Tensors are borrowed, not copied. */
typedef struct or_model or_model;
typedef struct or_state or_state;
or_model *or_model_new(const aq_model_config *cfg, const aq_tensor *tensors, size_t n_tensors, int threads);
void or_model_free(or_model *m);
or_state *or_state_new(const or_model *m, uint32_t spec_k, uint32_t max_pos);
void or_state_free(or_state *s);
/* Model::forward_token (model.rs:486-490). logits: vocab floats (nullable). Returns argmax. */
uint32_t or_forward_token(const or_model *m, or_state *s, uint32_t id, float *logits);
/* Model::prefill + logits of the last row (model.rs:443-461, 423). Returns argmax of the last row. */
uint32_t or_prefill(const or_model *m, or_state *s, const uint32_t *ids, size_t n, float *logits_last);
/* Model::spec_prefill (spec.rs:229-272), greedy. Returns x_T. */
uint32_t or_spec_prefill(const or_model *m, or_state *s, const uint32_t *ids, size_t n);
/* Model::spec_round (spec.rs:326-433), greedy. emitted: k+1 slots. Returns m (accepted drafts). */
uint32_t or_spec_round(const or_model *m, or_state *s, uint32_t x_p, uint32_t *emitted, uint32_t *n_emitted);
/* Model::spec_set_drafts (spec.rs:436-450) and the current drafts. */
void or_spec_set_drafts(or_state *s, const uint32_t *d, size_t k);
void or_spec_get_drafts(const or_state *s, uint32_t *d);
/* The logits of row i of the last verify batch (spec.rs:316-321), vocab floats. */
void or_spec_logits_row(const or_state *s, size_t i, float *out);
/* Carried state for equality tests: position, then per DeltaNet layer rec+conv, per attention layer the KV
 * rows 0..len, then the MTP KV rows. or_state_export returns the float count when out is NULL. */
uint32_t or_state_pos(const or_state *s);
size_t or_state_export(const or_state *s, float *out);

/* ---- the sampler (sample.rs; oracle_sample.c) */
void or_rng_seed(uint64_t seed, uint64_t s[4]);
uint64_t or_rng_next(uint64_t s[4]);
float or_rng_f32(uint64_t s[4]);
typedef struct or_sampler or_sampler;
or_sampler *or_sampler_new(const aq_sampler_config *cfg, size_t vocab);
void or_sampler_free(or_sampler *sp);
void or_sampler_reseed(or_sampler *sp, uint64_t seed);
void or_sampler_rng(const or_sampler *sp, uint64_t out[4]);
int or_sampler_is_greedy(const or_sampler *sp); /* NULL counts as greedy */
size_t or_sampler_process(or_sampler *sp, const float *logits);
size_t or_sampler_kept(const or_sampler *sp, uint32_t *ids, float *probs);
uint32_t or_sampler_draw(or_sampler *sp);
uint32_t or_sampler_sample(or_sampler *sp, const float *logits);
void or_sampler_write_dense(const or_sampler *sp, float *out);
int or_sampler_accept_or_resample(or_sampler *sp, const float *target, const float *q, uint32_t d, uint32_t *tok);
/* The model calls with a sampler (NULL or temperature <= 0: greedy, as the functions above): run.rs's sampled loop
 * (prefill / forward_token then Sampler::sample) and spec.rs:229-433 with the rejection-sampling acceptance. */
uint32_t or_forward_token_s(const or_model *m, or_state *s, or_sampler *sp, uint32_t id, float *logits);
uint32_t or_prefill_s(const or_model *m, or_state *s, or_sampler *sp, const uint32_t *ids, size_t n,
                      float *logits_last);
uint32_t or_spec_prefill_s(const or_model *m, or_state *s, or_sampler *sp, const uint32_t *ids, size_t n);
uint32_t or_spec_round_s(const or_model *m, or_state *s, or_sampler *sp, uint32_t x_p, uint32_t *emitted,
                         uint32_t *n_emitted);

/* One mixer / MLP / decoder layer alone (tests/layers.rs:109-271); see oracle_model.c. */
int or_layer_run(const aq_model_config *cfg, const aq_tensor *ts, size_t n, int kind, const float *x, size_t t,
                 uint32_t start_pos, float *conv, float *rec, float *k_cache, float *v_cache, uint32_t *kv_len,
                 uint32_t kv_cap, float *y);

#ifdef __cplusplus
}
#endif
#endif
