// ops.h — launchers of the model-level kernels (ops.hip): embedding rows, RMSNorm with the fused activation
// quantiser, SwiGLU with the fused quantiser, the Gated-DeltaNet head kernel (conv + recurrence + gated norm),
// the attention prologue and decode kernels, argmax and the greedy acceptance. Every launcher returns 0 or an
// AQ_E* code and runs on `stream`.
#pragma once

#include "aq_common.h"

namespace aq {

// What a row kernel writes besides (optionally) f32: nothing, Q8_K (for K-quant weights) or Q8_0 (for Q8_0 /
// Q4_0 weights, and for K-quant weights under the q8-fine switch). F32 weights read the f32 rows
// (matvec.rs:147-160 `act_kind`).
enum QuantKind { QK_NONE = 0, QK_Q8K = 1, QK_Q80 = 2 };
inline QuantKind quant_kind_for(int weight_type) {
    if (is_kquant(weight_type)) return q8_fine() ? QK_Q80 : QK_Q8K;
    if (weight_type == AQ_TYPE_Q8_0 || weight_type == AQ_TYPE_Q4_0) return QK_Q80;
    return QK_NONE;
}

// Where a row kernel puts the quantised form: column `col0 + row` of `act`, starting at element `elem_off`
// (a multiple of 256 for Q8_K, of 32 for Q8_0). Also writes act.f32 there when `f32` is set.
struct QuantOut {
    const Act *act = nullptr;
    QuantKind kind = QK_NONE;
    size_t col0 = 0, elem_off = 0;
    bool f32 = false;
};

// out[i * out_stride + e] = dequantised row ids[i] of `w` (model.rs:364-368; Q4_K only).
int launch_embed(const Weight &w, const uint32_t *ids, size_t t, float *out, size_t out_stride, hipStream_t stream);

// y = (x * inv_rms(x)) * w per row (rmsnorm.rs:14-76), t rows of n; y_f32 optional (row stride y_stride).
int launch_rmsnorm(const float *x, size_t x_stride, const float *w, float eps, size_t n, size_t t, float *y_f32,
                   size_t y_stride, const QuantOut &q, hipStream_t stream);
// Up to two F32 matrices over the normalised rows, formed by work-groups of the norm launch itself (the DeltaNet
// ssm_alpha / ssm_beta gate rows, gated_deltanet.rs:271-274): y[i][c * rows[i] + r] = w[i] row r . normalised row
// c (dot.rs:180-200), w[i] rows[i] x n row-major.
struct NormRows {
    const float *w[2] = {nullptr, nullptr};
    float *y[2] = {nullptr, nullptr};
    int rows[2] = {0, 0};
    int t = 0; // set by the launcher: the launch's input rows
};
// Whether launch_rmsnorm_rows takes rows of n (whole 256-blocks, each chain held by 8 lanes of one wave).
bool rmsnorm_rows_fit(size_t n);
// launch_rmsnorm (no y_f32) plus the rows of `fr`, one launch.
int launch_rmsnorm_rows(const float *x, size_t x_stride, const float *w, float eps, size_t n, size_t t,
                        const QuantOut &q, const NormRows &fr, hipStream_t stream);
// Two RMSNorms of t rows of n into the same quantised rows in one launch: x with w into elements q.elem_off..,
// x2 with w2 into elements eoff2.. (the MTP's [rmsnorm(embed, enorm) | rmsnorm(h, hnorm)], mtp.rs:95-104).
int launch_rmsnorm_pair(const float *x, size_t x_stride, const float *w, const float *x2, size_t x2_stride,
                        const float *w2, size_t eoff2, float eps, size_t n, size_t t, const QuantOut &q,
                        hipStream_t stream);

// h = silu(g) * u elementwise over t rows of n (act.rs:24-30), into the quantised form (and h_f32 if set).
int launch_swiglu(const float *g, const float *u, size_t n, size_t t, float *h_f32, const QuantOut &q,
                  hipStream_t stream);

struct DnArgs {
    const float *mixed = nullptr; // t x cd conv inputs (the qkv projection)
    const float *z = nullptr;     // t x vd output gate (null: no output)
    const float *a = nullptr, *b = nullptr; // t x nv gate pre-activations (ssm_alpha / ssm_beta rows)
    const float *conv_src = nullptr;        // cd x (K-1) window
    float *conv_dst = nullptr;              // null: window not written
    const float *conv_w = nullptr;          // cd x K
    const float *ssm_a = nullptr, *dt_bias = nullptr, *ssm_norm = nullptr;
    float eps = 0.0f, qscale = 0.0f;
    float *rec = nullptr; // nv x dk x dv recurrent state
    int write_state = 0;
    float *out = nullptr; // t x vd gated-norm output (null: none)
    int out_q80 = 0;      // also the Q8_0 form of `out` into q80 (its rows = the t rows; vd and dv multiples of 32)
    Act q80;
    int t = 0, nk = 0, nv = 0, dk = 0, dv = 0, kernel = 0;
    // raw mode (the isolated recurrence): q, k (t x nk*dk), v (t x nv*dv), g, beta (t x nv) used as given
    int raw = 0;
    const float *rq = nullptr, *rk = nullptr, *rv = nullptr, *rg = nullptr, *rbeta = nullptr;
    const uint32_t *t_dev = nullptr; // multi launch: the row count, read on the device (1..8)
};
// t rows; more than 8 (a prompt chunk: projected gates, no raw mode) run as 8-row pieces inside one launch.
int launch_dn_core(const DnArgs &a, hipStream_t stream);
// n DnArgs (device array, commit form: saved gates, no output), all with the head shape of `like`: one launch.
int launch_dn_core_multi(const DnArgs *args_dev, const DnArgs &like, int n, hipStream_t stream);

struct AttnArgs {
    const float *qg = nullptr;          // t x (2*nh*hd): per head [q | gate]
    const float *kk = nullptr, *vv = nullptr; // t x nkv*hd
    const float *q_norm = nullptr, *k_norm = nullptr;
    float eps = 0.0f, scaling = 0.0f;
    const float *cos_tab = nullptr, *sin_tab = nullptr; // per position: rope_dim/2 values
    size_t start_pos = 0;        // position of row 0 (rope)
    float *q = nullptr;          // t x nh*hd scratch (post norm + rope)
    float *kcache = nullptr, *vcache = nullptr;
    size_t base = 0;             // cache rows before row 0
    size_t stride = 0;           // nkv*hd
    float *out = nullptr;        // t x nh*hd
    int out_q8k = 0; // also the Q8_K form of `out` into q8k (head_dim 256: one head row = one 256-block)
    Act q8k;
    int t = 0, nh = 0, nkv = 0, hd = 0, rd = 0;
    // Score rows in device memory for contexts whose scores do not fit the work-group's LDS: row (i, h) at
    // gsc + (i * nh + h) * gsc_stride, gsc_stride >= base + t. Null: only contexts that fit the LDS are accepted.
    float *gsc = nullptr;
    size_t gsc_stride = 0;
};
// The longest context (base + t) whose score row the attention kernel keeps in LDS for head_dim hd.
size_t attn_lds_positions(int hd);
// Norm + RoPE of q and k, K/V appended at cache rows base..base+t, then per (head, row) softmax attention over
// base + row + 1 positions with the sigmoid output gate (gqa_attention.rs:327-418).
int launch_attention(const AttnArgs &a, hipStream_t stream);

// ids[r] = argmax of row r of x (t rows of n, row stride `stride`), first maximum wins (model.rs:505-513).
// `scratch` holds at least argmax_scratch_bytes(n, t).
size_t argmax_scratch_bytes(size_t n, size_t t);
int launch_argmax(const float *x, size_t n, size_t stride, size_t t, uint32_t *ids, void *scratch, hipStream_t stream);

// The sampler (sample.hip) for the model's sampled calls; `sp` null or temperature <= 0 is greedy.
bool sampler_greedy(const aq_sampler *sp);
uint32_t sampler_vocab(const aq_sampler *sp);
int sampler_device(const aq_sampler *sp);
// Sampler::sample of one logits row into *tok_dev (sample.rs:254-257).
int sampler_sample(aq_sampler *sp, const float *logits, uint32_t *tok_dev, hipStream_t st);
// A draft (spec.rs:192-203): process + draw into *tok_dev, the kept set written densely into q_dense (vocab f32),
// whose previously written ids (q_idx, *q_n of them) are cleared first.
int sampler_draft(aq_sampler *sp, const float *logits, uint32_t *tok_dev, float *q_dense, uint32_t *q_idx,
                  uint32_t *q_n, hipStream_t st);
// The sampled acceptance of a round (spec.rs:367-380) over k + 1 logits rows: info = {m, n_emitted, keep} and
// emitted[0..n_emitted), as launch_accept.
int sampler_round(aq_sampler *sp, const float *logits, int k, const uint32_t *drafts, const float *q_dense,
                  uint32_t *emitted, uint32_t *info, hipStream_t st);

// Greedy acceptance (spec.rs:355-366): info = {m, n_emitted, keep}, emitted[0..n_emitted).
int launch_accept(const uint32_t *argmax_ids, const uint32_t *drafts, int k, uint32_t *emitted, uint32_t *info,
                  hipStream_t stream);

// y = f(x) elementwise with the device's activation functions (fn: 0 exp, 1 log1p, 2 silu, 3 sigmoid, 4 softplus).
int launch_eval_math(int fn, const float *x, float *y, size_t n, hipStream_t stream);

// batch = [x_p, drafts[0..k)]
int launch_make_batch(uint32_t x_p, const uint32_t *drafts, int k, uint32_t *batch, hipStream_t stream);

} // namespace aq
