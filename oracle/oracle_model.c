/*
 * oracle_model.c — TEST INFRASTRUCTURE ONLY: the reference's layers, model forward and greedy speculative
 * round restated in C (layers/ *.rs, model.rs, spec.rs). One batched forward serves forward_token (t = 1),
 * prefill (t = T) and the verify batch (t = k + 1): in the reference those three paths are the same per-row
 * arithmetic (layers/mod.rs:332-334, spec.rs:273-276, docs/spec.md:16-22), so one routine restates them all.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "oracle_internal.h"

typedef struct or_mat {
    int type;
    size_t rows, cols, row_bytes;
    const uint8_t *data;
} or_mat;

typedef struct or_layer {
    int attention;
    float *attn_norm, *post_norm;
    /* DeltaNet (gated_deltanet.rs:52-78) */
    or_mat qkv, gate_z, alpha, beta, ssm_out;
    float *ssm_a, *dt_bias, *conv_w, *ssm_norm;
    /* GQA (gqa_attention.rs:65-80) */
    or_mat q, k, v, o;
    float *q_norm, *k_norm;
    /* MLP (mlp.rs:27-31) */
    or_mat gate, up, down;
} or_layer;

struct or_model {
    aq_model_config cfg;
    int threads;
    or_mat embed, lm_head;
    float *output_norm;
    or_layer *layers;
    int has_mtp;
    or_layer mtp;
    or_mat eh_proj;
    float *enorm, *hnorm, *head_norm;
    float *inv_freq;
    size_t kd, vd, cd;
};

typedef struct or_kv {
    float *k, *v;
    size_t len, cap, stride;
} or_kv;

struct or_state {
    const or_model *m;
    uint32_t pos, max_pos;
    float **conv, **rec; /* per layer (NULL for attention layers) */
    or_kv *kv;           /* per layer (unused for DeltaNet layers) */
    /* speculative buffers (spec.rs:63-152) */
    uint32_t k;
    uint32_t *drafts;
    or_kv mtp_kv;
    float *logits;      /* (k+1) x vocab */
    float *normed;      /* (k+1) x hidden */
    float *mtp_hout;    /* (k+1) x hidden */
    float *hprev;       /* hidden */
    float *snapshot;
    float *saved_mixed, *saved_a, *saved_b;
    float *q_dense; /* k x vocab: the dense draft distributions of a sampled round (spec.rs:192-203) */
};

/* =============================================================================== tensors and matmul */

static const aq_tensor *find(const aq_tensor *ts, size_t n, const char *name) {
    for (size_t i = 0; i < n; i++)
        if (strcmp(ts[i].name, name) == 0) return &ts[i];
    return NULL;
}

static int get_mat(const aq_tensor *ts, size_t n, const char *name, size_t rows, size_t cols, or_mat *out) {
    const aq_tensor *t = find(ts, n, name);
    if (!t) {
        fprintf(stderr, "oracle: missing tensor %s\n", name);
        return -1;
    }
    if ((size_t)t->rows != rows || (size_t)t->cols != cols) {
        fprintf(stderr, "oracle: %s is %lldx%lld, want %zux%zu\n", name, (long long)t->rows, (long long)t->cols, rows, cols);
        return -1;
    }
    out->type = t->ggml_type;
    out->rows = rows;
    out->cols = cols;
    out->row_bytes = or_row_bytes(t->ggml_type, cols);
    out->data = (const uint8_t *)t->data;
    return 0;
}

static float *get_vec(const aq_tensor *ts, size_t n, const char *name, size_t len) {
    const aq_tensor *t = find(ts, n, name);
    if (!t || (size_t)(t->rows * t->cols) != len) {
        fprintf(stderr, "oracle: missing or mis-sized vector %s\n", name);
        return NULL;
    }
    float *v = (float *)malloc(len * sizeof(float));
    if (or_dequant(t->ggml_type, (const uint8_t *)t->data, len, v) != 0) {
        free(v);
        return NULL;
    }
    return v;
}

/* matvec.rs:127-145 `Q8_FINE` / `set_q8_fine` / `q8k_activations`: process-wide, off by default. */
static int g_q8_fine = 0;
void or_set_q8_fine(int on) { g_q8_fine = on != 0; }
int or_q8_fine(void) { return g_q8_fine; }

/* matvec.rs:147-160 `act_kind` + 282-292 `one_row` + 483-539 `matmul_impl`: y[c*rows + r] = W[r] . x[c].
 * K-quant weights take Q8_K rows through the blocked kernel (bit-identical to the single-row one), or with the
 * q8-fine switch on, Q8_0 rows one row at a time (`one_row` -> `dot_q8`); Q8_0/Q4_0 take Q8_0 rows; F32 takes f32.
 * Row-parallel; every row is computed by one thread, so thread count never changes a bit (matvec.rs:1-4). */
static void matmul(const or_mat *w, const float *x, size_t ncols, float *y, int threads) {
    size_t rows = w->rows, cols = w->cols;
    const int kq = w->type == AQ_TYPE_Q4_K || w->type == AQ_TYPE_Q5_K || w->type == AQ_TYPE_Q6_K;
    if (kq && !g_q8_fine) {
        or_q8k *acts = (or_q8k *)calloc(ncols, sizeof(or_q8k));
        const or_q8k *ptrs[16];
        for (size_t c = 0; c < ncols; c++) {
            or_q8k_alloc(&acts[c], cols);
            or_q8k_from_f32(x + c * cols, cols, &acts[c]);
        }
#pragma omp parallel for num_threads(threads) schedule(static) private(ptrs)
        for (size_t r = 0; r < rows; r++) {
            for (size_t c0 = 0; c0 < ncols; c0 += 16) {
                size_t tn = ncols - c0 < 16 ? ncols - c0 : 16;
                float out[16];
                for (size_t i = 0; i < tn; i++) ptrs[i] = &acts[c0 + i];
                or_dot_q8k_rows(w->type, w->data + r * w->row_bytes, ptrs, tn, out);
                for (size_t i = 0; i < tn; i++) y[(c0 + i) * rows + r] = out[i];
            }
        }
        for (size_t c = 0; c < ncols; c++) or_q8k_release(&acts[c]);
        free(acts);
    } else if (kq || w->type == AQ_TYPE_Q8_0 || w->type == AQ_TYPE_Q4_0) {
        or_q8 *acts = (or_q8 *)calloc(ncols, sizeof(or_q8));
        for (size_t c = 0; c < ncols; c++) {
            or_q8_alloc(&acts[c], cols);
            or_q8_from_f32(x + c * cols, cols, &acts[c]);
        }
#pragma omp parallel for num_threads(threads) schedule(static)
        for (size_t r = 0; r < rows; r++)
            for (size_t c = 0; c < ncols; c++) y[c * rows + r] = or_dot_q8_row(w->type, w->data + r * w->row_bytes, &acts[c]);
        for (size_t c = 0; c < ncols; c++) or_q8_release(&acts[c]);
        free(acts);
    } else { /* F32 x f32: matvec.rs:270-279 `dot_f32_bytes` */
#pragma omp parallel for num_threads(threads) schedule(static)
        for (size_t r = 0; r < rows; r++)
            for (size_t c = 0; c < ncols; c++)
                y[c * rows + r] = or_dot_f32((const float *)(w->data + r * w->row_bytes), x + c * cols, cols);
    }
}

void or_matmul(int type, const uint8_t *w, size_t rows, size_t cols, const float *x, size_t ncols, float *y,
               int threads) {
    or_mat m = {type, rows, cols, or_row_bytes(type, cols), w};
    matmul(&m, x, ncols, y, threads > 0 ? threads : 1);
}

/* ====================================================================================== model loading */

static int load_layer(or_model *m, const aq_tensor *ts, size_t n, uint32_t index, int attention, or_layer *L) {
    const aq_model_config *c = &m->cfg;
    char nm[160];
    size_t h = c->hidden;
#define P(s) (snprintf(nm, sizeof nm, "blk.%u." s, index), nm)
    L->attention = attention;
    if (!(L->attn_norm = get_vec(ts, n, P("attn_norm.weight"), h))) return -1;
    if (!(L->post_norm = get_vec(ts, n, P("post_attention_norm.weight"), h))) return -1;
    if (attention) {
        size_t nh = c->n_head, nkv = c->n_head_kv, hd = c->head_dim;
        if (get_mat(ts, n, P("attn_q.weight"), 2 * nh * hd, h, &L->q)) return -1;
        if (get_mat(ts, n, P("attn_k.weight"), nkv * hd, h, &L->k)) return -1;
        if (get_mat(ts, n, P("attn_v.weight"), nkv * hd, h, &L->v)) return -1;
        if (get_mat(ts, n, P("attn_output.weight"), h, nh * hd, &L->o)) return -1;
        if (!(L->q_norm = get_vec(ts, n, P("attn_q_norm.weight"), hd))) return -1;
        if (!(L->k_norm = get_vec(ts, n, P("attn_k_norm.weight"), hd))) return -1;
    } else {
        size_t nv = c->dn_n_v_heads;
        if (get_mat(ts, n, P("attn_qkv.weight"), m->cd, h, &L->qkv)) return -1;
        if (get_mat(ts, n, P("attn_gate.weight"), m->vd, h, &L->gate_z)) return -1;
        if (get_mat(ts, n, P("ssm_alpha.weight"), nv, h, &L->alpha)) return -1;
        if (get_mat(ts, n, P("ssm_beta.weight"), nv, h, &L->beta)) return -1;
        if (get_mat(ts, n, P("ssm_out.weight"), h, m->vd, &L->ssm_out)) return -1;
        if (!(L->ssm_a = get_vec(ts, n, P("ssm_a"), nv))) return -1;
        if (!(L->dt_bias = get_vec(ts, n, P("ssm_dt.bias"), nv))) return -1;
        if (!(L->conv_w = get_vec(ts, n, P("ssm_conv1d.weight"), m->cd * c->dn_conv_kernel))) return -1;
        if (!(L->ssm_norm = get_vec(ts, n, P("ssm_norm.weight"), c->dn_head_dim_v))) return -1;
    }
    if (get_mat(ts, n, P("ffn_gate.weight"), c->ffn, h, &L->gate)) return -1;
    if (get_mat(ts, n, P("ffn_up.weight"), c->ffn, h, &L->up)) return -1;
    if (get_mat(ts, n, P("ffn_down.weight"), h, c->ffn, &L->down)) return -1;
#undef P
    return 0;
}

static void free_layer(or_layer *L) {
    free(L->attn_norm);
    free(L->post_norm);
    free(L->ssm_a);
    free(L->dt_bias);
    free(L->conv_w);
    free(L->ssm_norm);
    free(L->q_norm);
    free(L->k_norm);
}

static int is_attention(const aq_model_config *c, uint32_t i) { return (i + 1) % c->full_attention_interval == 0; }

or_model *or_model_new(const aq_model_config *cfg, const aq_tensor *ts, size_t n, int threads) {
    or_model *m = (or_model *)calloc(1, sizeof(or_model));
    m->cfg = *cfg;
    m->threads = threads > 0 ? threads : 1;
    m->kd = (size_t)cfg->dn_n_k_heads * cfg->dn_head_dim_k;
    m->vd = (size_t)cfg->dn_n_v_heads * cfg->dn_head_dim_v;
    m->cd = 2 * m->kd + m->vd;
    size_t h = cfg->hidden;
    int bad = 0;
    bad |= get_mat(ts, n, "token_embd.weight", cfg->vocab, h, &m->embed);
    bad |= get_mat(ts, n, "output.weight", cfg->vocab, h, &m->lm_head);
    if (!(m->output_norm = get_vec(ts, n, "output_norm.weight", h))) bad = 1;
    m->layers = (or_layer *)calloc(cfg->n_layer, sizeof(or_layer));
    for (uint32_t i = 0; i < cfg->n_layer && !bad; i++) bad |= load_layer(m, ts, n, i, is_attention(cfg, i), &m->layers[i]);
    m->has_mtp = cfg->has_mtp != 0;
    if (m->has_mtp && !bad) {
        char nm[160];
        uint32_t mi = cfg->n_layer;
        bad |= load_layer(m, ts, n, mi, 1, &m->mtp);
        snprintf(nm, sizeof nm, "blk.%u.nextn.eh_proj.weight", mi);
        bad |= get_mat(ts, n, nm, h, 2 * h, &m->eh_proj);
        snprintf(nm, sizeof nm, "blk.%u.nextn.enorm.weight", mi);
        if (!(m->enorm = get_vec(ts, n, nm, h))) bad = 1;
        snprintf(nm, sizeof nm, "blk.%u.nextn.hnorm.weight", mi);
        if (!(m->hnorm = get_vec(ts, n, nm, h))) bad = 1;
        snprintf(nm, sizeof nm, "blk.%u.nextn.shared_head_norm.weight", mi);
        if (!(m->head_norm = get_vec(ts, n, nm, h))) bad = 1;
    }
    m->inv_freq = (float *)malloc(cfg->rope_dim / 2 * sizeof(float) + 4);
    or_inv_freq(cfg->rope_dim, cfg->rope_theta, m->inv_freq);
    if (bad) {
        or_model_free(m);
        return NULL;
    }
    return m;
}

void or_model_free(or_model *m) {
    if (!m) return;
    for (uint32_t i = 0; m->layers && i < m->cfg.n_layer; i++) free_layer(&m->layers[i]);
    free(m->layers);
    if (m->has_mtp) free_layer(&m->mtp);
    free(m->output_norm);
    free(m->enorm);
    free(m->hnorm);
    free(m->head_norm);
    free(m->inv_freq);
    free(m);
}

/* ============================================================================================ state */

static void kv_init(or_kv *kv, size_t stride, size_t cap) {
    kv->stride = stride;
    kv->cap = cap;
    kv->len = 0;
    kv->k = (float *)calloc(cap * stride + 1, sizeof(float));
    kv->v = (float *)calloc(cap * stride + 1, sizeof(float));
}

static size_t dn_state_len(const or_model *m) { return (size_t)m->cfg.dn_n_v_heads * m->cfg.dn_head_dim_k * m->cfg.dn_head_dim_v; }
static size_t dn_conv_len(const or_model *m) { return m->cd * (m->cfg.dn_conv_kernel - 1); }

or_state *or_state_new(const or_model *m, uint32_t spec_k, uint32_t max_pos) {
    const aq_model_config *c = &m->cfg;
    or_state *s = (or_state *)calloc(1, sizeof(or_state));
    s->m = m;
    s->max_pos = max_pos;
    s->conv = (float **)calloc(c->n_layer, sizeof(float *));
    s->rec = (float **)calloc(c->n_layer, sizeof(float *));
    s->kv = (or_kv *)calloc(c->n_layer, sizeof(or_kv));
    size_t n_dn = 0;
    for (uint32_t i = 0; i < c->n_layer; i++) {
        if (m->layers[i].attention) {
            kv_init(&s->kv[i], (size_t)c->n_head_kv * c->head_dim, max_pos);
        } else {
            s->conv[i] = (float *)calloc(dn_conv_len(m), sizeof(float));
            s->rec[i] = (float *)calloc(dn_state_len(m), sizeof(float));
            n_dn++;
        }
    }
    s->k = spec_k;
    if (spec_k > 0) {
        size_t t = spec_k + 1;
        s->drafts = (uint32_t *)calloc(spec_k, sizeof(uint32_t));
        kv_init(&s->mtp_kv, (size_t)c->n_head_kv * c->head_dim, max_pos + t);
        s->logits = (float *)calloc(t * c->vocab, sizeof(float));
        s->normed = (float *)calloc(t * c->hidden, sizeof(float));
        s->mtp_hout = (float *)calloc(t * c->hidden, sizeof(float));
        s->hprev = (float *)calloc(c->hidden, sizeof(float));
        s->snapshot = (float *)calloc(n_dn * (dn_state_len(m) + dn_conv_len(m)) + 1, sizeof(float));
        s->saved_mixed = (float *)calloc(n_dn * t * m->cd + 1, sizeof(float));
        s->saved_a = (float *)calloc(n_dn * t * c->dn_n_v_heads + 1, sizeof(float));
        s->saved_b = (float *)calloc(n_dn * t * c->dn_n_v_heads + 1, sizeof(float));
        s->q_dense = (float *)calloc((size_t)spec_k * c->vocab, sizeof(float));
    }
    return s;
}

void or_state_free(or_state *s) {
    if (!s) return;
    for (uint32_t i = 0; i < s->m->cfg.n_layer; i++) {
        free(s->conv[i]);
        free(s->rec[i]);
        free(s->kv[i].k);
        free(s->kv[i].v);
    }
    free(s->conv);
    free(s->rec);
    free(s->kv);
    free(s->drafts);
    free(s->mtp_kv.k);
    free(s->mtp_kv.v);
    free(s->logits);
    free(s->normed);
    free(s->mtp_hout);
    free(s->q_dense);
    free(s->hprev);
    free(s->snapshot);
    free(s->saved_mixed);
    free(s->saved_a);
    free(s->saved_b);
    free(s);
}

/* ============================================================================================ layers */

/* gated_deltanet.rs:331-375 (replay_in) and the head loop of 261-324 (forward_batch_in): per V head, for each
 * row, l2norm q/k, scale q, gates, deltanet_step, and (when out_heads) the gated RMSNorm of the output. */
static void dn_heads(const or_model *m, const or_layer *L, const float *conved, const float *z, const float *a,
                     const float *b, size_t t, float *rec, float *out_heads) {
    const aq_model_config *c = &m->cfg;
    size_t nk = c->dn_n_k_heads, nv = c->dn_n_v_heads, dk = c->dn_head_dim_k, dv = c->dn_head_dim_v;
    size_t kd = m->kd, vd = m->vd, cd = m->cd;
    float scale = 1.0f / sqrtf((float)dk);
#pragma omp parallel for num_threads(m->threads) schedule(static)
    for (size_t p = 0; p < nv; p++) {
        size_t kh = p % nk;
        float *qn = (float *)malloc(dk * sizeof(float)), *kn = (float *)malloc(dk * sizeof(float));
        float *o = (float *)malloc(dv * sizeof(float));
        for (size_t i = 0; i < t; i++) {
            const float *base = conved + i * cd;
            memcpy(qn, base + kh * dk, dk * sizeof(float));
            memcpy(kn, base + kd + kh * dk, dk * sizeof(float));
            or_l2norm(qn, dk, 1e-6f);
            or_l2norm(kn, dk, 1e-6f);
            for (size_t j = 0; j < dk; j++) qn[j] *= scale;
            float g = or_gate_g(a[i * nv + p], L->dt_bias[p], L->ssm_a[p]);
            float beta = or_sigmoid(b[i * nv + p]);
            or_deltanet_step(qn, kn, base + 2 * kd + p * dv, g, beta, rec + p * dk * dv, o, dk, dv);
            if (out_heads) or_rmsnorm_gated(o, z + i * vd + p * dv, L->ssm_norm, c->rms_eps, out_heads + i * vd + p * dv, dv);
        }
        free(qn);
        free(kn);
        free(o);
    }
}

/* gated_deltanet.rs:261-324 `forward_batch_in`; saves the conv inputs and gate pre-activations when asked
 * (spec.rs:294-301). */
static void deltanet_batch(const or_model *m, const or_layer *L, const float *x, size_t t, float *conv, float *rec,
                           float *y, float *save_mixed, float *save_a, float *save_b) {
    const aq_model_config *c = &m->cfg;
    size_t nv = c->dn_n_v_heads, vd = m->vd, cd = m->cd;
    float *mixed = (float *)malloc(t * cd * sizeof(float));
    float *z = (float *)malloc(t * vd * sizeof(float));
    float *a = (float *)malloc(t * nv * sizeof(float));
    float *b = (float *)malloc(t * nv * sizeof(float));
    float *conved = (float *)malloc(t * cd * sizeof(float));
    float *heads = (float *)malloc(t * vd * sizeof(float));
    matmul(&L->qkv, x, t, mixed, m->threads);
    matmul(&L->gate_z, x, t, z, m->threads);
    matmul(&L->alpha, x, t, a, m->threads);
    matmul(&L->beta, x, t, b, m->threads);
    for (size_t i = 0; i < t; i++) or_conv1d_step(conv, L->conv_w, c->dn_conv_kernel, mixed + i * cd, conved + i * cd, cd, 1);
    dn_heads(m, L, conved, z, a, b, t, rec, heads);
    matmul(&L->ssm_out, heads, t, y, m->threads);
    if (save_mixed) memcpy(save_mixed, mixed, t * cd * sizeof(float));
    if (save_a) memcpy(save_a, a, t * nv * sizeof(float));
    if (save_b) memcpy(save_b, b, t * nv * sizeof(float));
    free(mixed);
    free(z);
    free(a);
    free(b);
    free(conved);
    free(heads);
}

/* gated_deltanet.rs:331-375 `replay_in`: the conv and the recurrence of t saved rows, no weights. */
static void deltanet_replay(const or_model *m, const or_layer *L, const float *mixed, const float *a, const float *b,
                            size_t t, float *conv, float *rec) {
    size_t cd = m->cd;
    float *conved = (float *)malloc(t * cd * sizeof(float) + 4);
    for (size_t i = 0; i < t; i++) or_conv1d_step(conv, L->conv_w, m->cfg.dn_conv_kernel, mixed + i * cd, conved + i * cd, cd, 1);
    dn_heads(m, L, conved, NULL, a, b, t, rec, NULL);
    free(conved);
}

/* gqa_attention.rs:327-418 `forward_batch_in`: t rows at positions start.., appended to `kv`. */
static void attention_batch(const or_model *m, const or_layer *L, const float *x, size_t t, uint32_t start, or_kv *kv,
                            float *y) {
    const aq_model_config *c = &m->cfg;
    size_t nh = c->n_head, nkv = c->n_head_kv, hd = c->head_dim, rd = c->rope_dim;
    size_t group = nh / nkv;
    float *qg = (float *)malloc(t * 2 * nh * hd * sizeof(float));
    float *kk = (float *)malloc(t * nkv * hd * sizeof(float));
    float *vv = (float *)malloc(t * nkv * hd * sizeof(float));
    float *q = (float *)malloc(t * nh * hd * sizeof(float));
    float *gate = (float *)malloc(t * nh * hd * sizeof(float));
    float *attn = (float *)malloc(t * nh * hd * sizeof(float));
    float *cosv = (float *)malloc(rd * sizeof(float) + 4), *sinv = (float *)malloc(rd * sizeof(float) + 4);
    float *tmp = (float *)malloc(hd * sizeof(float));
    matmul(&L->q, x, t, qg, m->threads);
    matmul(&L->k, x, t, kk, m->threads);
    matmul(&L->v, x, t, vv, m->threads);
    size_t base = kv->len;
    for (size_t i = 0; i < t; i++) {
        or_cos_sin(start + (uint32_t)i, m->inv_freq, rd / 2, cosv, sinv);
        for (size_t h = 0; h < nh; h++) {
            const float *src = qg + i * 2 * nh * hd + h * 2 * hd;
            or_rmsnorm(src, L->q_norm, c->rms_eps, tmp, hd);
            or_apply_rope(tmp, hd, hd, rd, cosv, sinv);
            memcpy(q + i * nh * hd + h * hd, tmp, hd * sizeof(float));
            memcpy(gate + i * nh * hd + h * hd, src + hd, hd * sizeof(float));
        }
        float *krow = kk + i * nkv * hd;
        for (size_t h = 0; h < nkv; h++) {
            or_rmsnorm(krow + h * hd, L->k_norm, c->rms_eps, tmp, hd);
            or_apply_rope(tmp, hd, hd, rd, cosv, sinv);
            memcpy(krow + h * hd, tmp, hd * sizeof(float));
        }
        if (kv->len >= kv->cap) {
            fprintf(stderr, "oracle: KV cache full (%zu)\n", kv->cap);
            abort();
        }
        memcpy(kv->k + kv->len * kv->stride, krow, nkv * hd * sizeof(float));
        memcpy(kv->v + kv->len * kv->stride, vv + i * nkv * hd, nkv * hd * sizeof(float));
        kv->len++;
    }
    float scaling = powf((float)hd, -0.5f);
#pragma omp parallel for num_threads(m->threads) schedule(static)
    for (size_t h = 0; h < nh; h++) {
        size_t kvh = h / group;
        float *scores = (float *)malloc((base + t) * sizeof(float));
        float *p = (float *)malloc((base + t) * sizeof(float));
        for (size_t i = 0; i < t; i++) {
            size_t len = base + i + 1;
            const float *qh = q + i * nh * hd + h * hd;
            for (size_t tt = 0; tt < len; tt++) {
                const float *kt = kv->k + tt * kv->stride + kvh * hd;
                float acc = 0.0f;
                for (size_t d = 0; d < hd; d++) acc += qh[d] * kt[d];
                scores[tt] = acc * scaling;
            }
            or_softmax(scores, p, len);
            float *out = attn + i * nh * hd + h * hd;
            for (size_t d = 0; d < hd; d++) out[d] = 0.0f;
            for (size_t tt = 0; tt < len; tt++) {
                const float *vt = kv->v + tt * kv->stride + kvh * hd;
                for (size_t d = 0; d < hd; d++) out[d] += p[tt] * vt[d];
            }
            for (size_t d = 0; d < hd; d++) out[d] *= or_sigmoid(gate[i * nh * hd + h * hd + d]);
        }
        free(scores);
        free(p);
    }
    matmul(&L->o, attn, t, y, m->threads);
    free(qg);
    free(kk);
    free(vv);
    free(q);
    free(gate);
    free(attn);
    free(cosv);
    free(sinv);
    free(tmp);
}

/* mlp.rs:114-132 `forward_batch_in` */
static void mlp_batch(const or_model *m, const or_layer *L, const float *x, size_t t, float *y) {
    size_t ffn = m->cfg.ffn;
    float *g = (float *)malloc(t * ffn * sizeof(float)), *u = (float *)malloc(t * ffn * sizeof(float));
    float *hh = (float *)malloc(t * ffn * sizeof(float));
    matmul(&L->gate, x, t, g, m->threads);
    matmul(&L->up, x, t, u, m->threads);
    or_swiglu(g, u, hh, t * ffn);
    matmul(&L->down, hh, t, y, m->threads);
    free(g);
    free(u);
    free(hh);
}

/* layers/mod.rs:335-377 `DecoderLayer::forward_batch_in` */
static void decoder_batch(const or_model *m, const or_layer *L, const float *x, size_t t, uint32_t start, float *conv,
                          float *rec, or_kv *kv, float *y, float *sm, float *sa, float *sb) {
    size_t h = m->cfg.hidden;
    float *normed = (float *)malloc(t * h * sizeof(float)), *mixed = (float *)malloc(t * h * sizeof(float));
    float *resid = (float *)malloc(t * h * sizeof(float));
    for (size_t i = 0; i < t; i++) or_rmsnorm(x + i * h, L->attn_norm, m->cfg.rms_eps, normed + i * h, h);
    if (L->attention)
        attention_batch(m, L, normed, t, start, kv, mixed);
    else
        deltanet_batch(m, L, normed, t, conv, rec, mixed, sm, sa, sb);
    for (size_t i = 0; i < t * h; i++) resid[i] = x[i] + mixed[i];
    for (size_t i = 0; i < t; i++) or_rmsnorm(resid + i * h, L->post_norm, m->cfg.rms_eps, normed + i * h, h);
    mlp_batch(m, L, normed, t, mixed);
    for (size_t i = 0; i < t * h; i++) y[i] = resid[i] + mixed[i];
    free(normed);
    free(mixed);
    free(resid);
}

/* ============================================================================================= model */

/* model.rs:364-368 `embed_token_into` */
static void embed(const or_model *m, uint32_t id, float *out) {
    or_dequant(m->embed.type, m->embed.data + (size_t)id * m->embed.row_bytes, m->cfg.hidden, out);
}

/* model.rs:505-513 `argmax`: first max wins */
static uint32_t argmax(const float *v, size_t n) {
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return (uint32_t)best;
}

/* t tokens at the state's position through every layer (model.rs:401-413 run_layers, 443-461 prefill,
 * spec.rs:277-304 forward_batch); returns the residual rows (caller frees); advances pos. When `spec` is set the
 * DeltaNet inputs are saved per layer and row. */
static float *forward_rows(const or_model *m, or_state *s, const uint32_t *ids, size_t t, int spec) {
    size_t h = m->cfg.hidden;
    float *h0 = (float *)malloc(t * h * sizeof(float)), *h1 = (float *)malloc(t * h * sizeof(float));
    for (size_t i = 0; i < t; i++) embed(m, ids[i], h0 + i * h);
    size_t dn_i = 0, big_t = s->k + 1;
    size_t nv = m->cfg.dn_n_v_heads, cd = m->cd;
    for (uint32_t li = 0; li < m->cfg.n_layer; li++) {
        const or_layer *L = &m->layers[li];
        float *sm = NULL, *sa = NULL, *sb = NULL;
        if (spec && !L->attention) {
            size_t base = dn_i * big_t;
            sm = s->saved_mixed + base * cd;
            sa = s->saved_a + base * nv;
            sb = s->saved_b + base * nv;
        }
        decoder_batch(m, L, h0, t, s->pos, s->conv[li], s->rec[li], &s->kv[li], h1, sm, sa, sb);
        if (!L->attention) dn_i++;
        float *tmp = h0;
        h0 = h1;
        h1 = tmp;
    }
    s->pos += (uint32_t)t;
    free(h1);
    return h0;
}

/* model.rs:430-438 `logits_with` on t rows: final norm into `normed`, lm_head into `logits`. */
static void head_rows(const or_model *m, const float *hs, size_t t, float *normed, float *logits) {
    size_t h = m->cfg.hidden;
    for (size_t i = 0; i < t; i++) or_rmsnorm(hs + i * h, m->output_norm, m->cfg.rms_eps, normed + i * h, h);
    matmul(&m->lm_head, normed, t, logits, m->threads);
}

/* The next token from a logits row: argmax (greedy), or Sampler::sample (sample.rs:254-257). */
static uint32_t next_token(const float *lg, size_t vocab, or_sampler *sp) {
    return or_sampler_is_greedy(sp) ? argmax(lg, vocab) : or_sampler_sample(sp, lg);
}

uint32_t or_forward_token_s(const or_model *m, or_state *s, or_sampler *sp, uint32_t id, float *logits) {
    size_t h = m->cfg.hidden, vocab = m->cfg.vocab;
    float *hs = forward_rows(m, s, &id, 1, 0);
    float *normed = (float *)malloc(h * sizeof(float));
    float *lg = logits ? logits : (float *)malloc(vocab * sizeof(float));
    head_rows(m, hs, 1, normed, lg);
    uint32_t a = next_token(lg, vocab, sp);
    if (!logits) free(lg);
    free(normed);
    free(hs);
    return a;
}

uint32_t or_prefill_s(const or_model *m, or_state *s, or_sampler *sp, const uint32_t *ids, size_t n,
                      float *logits_last) {
    size_t h = m->cfg.hidden, vocab = m->cfg.vocab;
    float *hs = forward_rows(m, s, ids, n, 0);
    float *normed = (float *)malloc(h * sizeof(float));
    float *lg = logits_last ? logits_last : (float *)malloc(vocab * sizeof(float));
    head_rows(m, hs + (n - 1) * h, 1, normed, lg);
    uint32_t a = next_token(lg, vocab, sp);
    if (!logits_last) free(lg);
    free(normed);
    free(hs);
    return a;
}

/* ============================================================================================== MTP */

/* mtp.rs:95-104 `set_row_with`: [rmsnorm(embed(x), enorm) | rmsnorm(h, hnorm)] into cat row i. */
static void mtp_set_row(const or_model *m, float *cat, uint32_t x, const float *hvec) {
    size_t h = m->cfg.hidden;
    float *e = (float *)malloc(h * sizeof(float));
    embed(m, x, e);
    or_rmsnorm(e, m->enorm, m->cfg.rms_eps, cat, h);
    or_rmsnorm(hvec, m->hnorm, m->cfg.rms_eps, cat + h, h);
    free(e);
}

/* mtp.rs:108-127 `rows_in`: eh_proj, the block on t rows at positions kv.len.., shared_head_norm. */
static void mtp_rows(const or_model *m, or_state *s, const float *cat, size_t t, float *hout) {
    size_t h = m->cfg.hidden;
    float *u = (float *)malloc(t * h * sizeof(float)), *y = (float *)malloc(t * h * sizeof(float));
    matmul(&m->eh_proj, cat, t, u, m->threads);
    decoder_batch(m, &m->mtp, u, t, (uint32_t)s->mtp_kv.len, NULL, NULL, &s->mtp_kv, y, NULL, NULL, NULL);
    for (size_t i = 0; i < t; i++) or_rmsnorm(y + i * h, m->head_norm, m->cfg.rms_eps, hout + i * h, h);
    free(u);
    free(y);
}

/* mtp.rs:130-137 `head_in` + spec.rs:192-203 `draft_token`: argmax, or process + draw with the processed
 * distribution written densely to q_dense[i] for the acceptance rule. */
static uint32_t mtp_draft(const or_model *m, or_state *s, or_sampler *sp, const float *hrow, size_t i) {
    size_t vocab = m->cfg.vocab;
    float *lg = (float *)malloc(vocab * sizeof(float));
    matmul(&m->lm_head, hrow, 1, lg, m->threads);
    uint32_t d;
    if (or_sampler_is_greedy(sp)) {
        d = argmax(lg, vocab);
    } else {
        or_sampler_process(sp, lg);
        d = or_sampler_draw(sp);
        or_sampler_write_dense(sp, s->q_dense + i * vocab);
    }
    free(lg);
    return d;
}

/* spec.rs:205-222 `chain_drafts`: drafts from..k from the MTP hidden of row `prev` of the last rows. */
static void chain_drafts(const or_model *m, or_state *s, or_sampler *sp, size_t prev, size_t from) {
    size_t h = m->cfg.hidden;
    float *cat = (float *)malloc(2 * h * sizeof(float));
    for (size_t i = from; i < s->k; i++) {
        memcpy(s->hprev, s->mtp_hout + prev * h, h * sizeof(float));
        mtp_set_row(m, cat, s->drafts[i - 1], s->hprev);
        mtp_rows(m, s, cat, 1, s->mtp_hout);
        s->drafts[i] = mtp_draft(m, s, sp, s->mtp_hout, i);
        prev = 0;
    }
    free(cat);
}

uint32_t or_spec_prefill_s(const or_model *m, or_state *s, or_sampler *sp, const uint32_t *ids, size_t t) {
    size_t h = m->cfg.hidden, vocab = m->cfg.vocab;
    uint32_t p = s->pos;
    float *hs = forward_rows(m, s, ids, t, 0);
    float *normed = (float *)malloc(t * h * sizeof(float));
    for (size_t i = 0; i < t; i++) or_rmsnorm(hs + i * h, m->output_norm, m->cfg.rms_eps, normed + i * h, h);
    float *lg = (float *)malloc(vocab * sizeof(float));
    float *nl = (float *)malloc(h * sizeof(float));
    head_rows(m, hs + (t - 1) * h, 1, nl, lg); /* logits_of(last row) */
    uint32_t x_t = next_token(lg, vocab, sp);
    /* the MTP over the prompt: row j = (x_{j+1}, h_j), the last row's token is x_T (spec.rs:243-265) */
    if (s->mtp_kv.len > p) s->mtp_kv.len = p;
    float *cats = (float *)malloc(t * 2 * h * sizeof(float));
    for (size_t j = 0; j < t; j++) mtp_set_row(m, cats + j * 2 * h, j + 1 < t ? ids[j + 1] : x_t, normed + j * h);
    float *hout = (float *)malloc(t * h * sizeof(float));
    mtp_rows(m, s, cats, t, hout);
    memcpy(s->mtp_hout, hout + (t - 1) * h, h * sizeof(float));
    s->drafts[0] = mtp_draft(m, s, sp, s->mtp_hout, 0);
    chain_drafts(m, s, sp, 0, 1);
    free(hout);
    free(cats);
    free(nl);
    free(lg);
    free(normed);
    free(hs);
    return x_t;
}

static void snapshot(const or_model *m, or_state *s) {
    size_t off = 0, nr = dn_state_len(m), nc = dn_conv_len(m);
    for (uint32_t i = 0; i < m->cfg.n_layer; i++) {
        if (m->layers[i].attention) continue;
        memcpy(s->snapshot + off, s->rec[i], nr * sizeof(float));
        off += nr;
        memcpy(s->snapshot + off, s->conv[i], nc * sizeof(float));
        off += nc;
    }
}

static void restore(const or_model *m, or_state *s) {
    size_t off = 0, nr = dn_state_len(m), nc = dn_conv_len(m);
    for (uint32_t i = 0; i < m->cfg.n_layer; i++) {
        if (m->layers[i].attention) continue;
        memcpy(s->rec[i], s->snapshot + off, nr * sizeof(float));
        off += nr;
        memcpy(s->conv[i], s->snapshot + off, nc * sizeof(float));
        off += nc;
    }
}

uint32_t or_spec_round_s(const or_model *m, or_state *s, or_sampler *sp, uint32_t x_p, uint32_t *emitted,
                         uint32_t *n_emitted) {
    size_t h = m->cfg.hidden, vocab = m->cfg.vocab, k = s->k, t = k + 1;
    size_t nv = m->cfg.dn_n_v_heads, cd = m->cd;
    uint32_t p = s->pos;
    uint32_t *batch = (uint32_t *)malloc(t * sizeof(uint32_t));
    batch[0] = x_p;
    for (size_t i = 0; i < k; i++) batch[i + 1] = s->drafts[i];
    snapshot(m, s);
    /* verify (spec.rs:277-314) */
    float *hs = forward_rows(m, s, batch, t, 1);
    head_rows(m, hs, t, s->normed, s->logits);
    /* accept: greedy (spec.rs:355-366) or the rejection-sampling rule (spec.rs:367-380) */
    size_t mm = 0, ne = 0;
    if (or_sampler_is_greedy(sp)) {
        while (mm < k) {
            uint32_t a = argmax(s->logits + mm * vocab, vocab);
            emitted[ne++] = a;
            if (a != s->drafts[mm]) break;
            mm++;
        }
        if (mm == k) emitted[ne++] = argmax(s->logits + k * vocab, vocab);
    } else {
        while (mm < k) {
            uint32_t tok;
            const int ok = or_sampler_accept_or_resample(sp, s->logits + mm * vocab, s->q_dense + mm * vocab,
                                                         s->drafts[mm], &tok);
            emitted[ne++] = tok;
            if (!ok) break;
            mm++;
        }
        if (mm == k) emitted[ne++] = or_sampler_sample(sp, s->logits + k * vocab);
    }
    size_t keep = mm + 1;
    *n_emitted = (uint32_t)ne;
    /* roll back (spec.rs:396-415) */
    if (keep < t) {
        restore(m, s);
        size_t dn_i = 0;
        for (uint32_t li = 0; li < m->cfg.n_layer; li++) {
            const or_layer *L = &m->layers[li];
            if (L->attention) {
                s->kv[li].len = p + keep;
            } else {
                size_t base = dn_i * t;
                deltanet_replay(m, L, s->saved_mixed + base * cd, s->saved_a + base * nv, s->saved_b + base * nv, keep,
                                s->conv[li], s->rec[li]);
                dn_i++;
            }
        }
        s->pos = p + (uint32_t)keep;
    }
    /* the MTP: forget its draft rows, feed the accepted pairs, draft the next round (spec.rs:417-431) */
    s->mtp_kv.len = p;
    float *cats = (float *)malloc(keep * 2 * h * sizeof(float));
    for (size_t i = 0; i < keep; i++) mtp_set_row(m, cats + i * 2 * h, emitted[i], s->normed + i * h);
    mtp_rows(m, s, cats, keep, s->mtp_hout);
    s->drafts[0] = mtp_draft(m, s, sp, s->mtp_hout + (keep - 1) * h, 0);
    chain_drafts(m, s, sp, keep - 1, 1);
    free(cats);
    free(hs);
    free(batch);
    return (uint32_t)mm;
}

uint32_t or_forward_token(const or_model *m, or_state *s, uint32_t id, float *logits) {
    return or_forward_token_s(m, s, NULL, id, logits);
}
uint32_t or_prefill(const or_model *m, or_state *s, const uint32_t *ids, size_t n, float *logits_last) {
    return or_prefill_s(m, s, NULL, ids, n, logits_last);
}
uint32_t or_spec_prefill(const or_model *m, or_state *s, const uint32_t *ids, size_t t) {
    return or_spec_prefill_s(m, s, NULL, ids, t);
}
uint32_t or_spec_round(const or_model *m, or_state *s, uint32_t x_p, uint32_t *emitted, uint32_t *n_emitted) {
    return or_spec_round_s(m, s, NULL, x_p, emitted, n_emitted);
}

void or_spec_set_drafts(or_state *s, const uint32_t *d, size_t k) {
    for (size_t i = 0; i < k && i < s->k; i++) s->drafts[i] = d[i];
}

void or_spec_get_drafts(const or_state *s, uint32_t *d) {
    for (size_t i = 0; i < s->k; i++) d[i] = s->drafts[i];
}

void or_spec_logits_row(const or_state *s, size_t i, float *out) {
    size_t vocab = s->m->cfg.vocab;
    memcpy(out, s->logits + i * vocab, vocab * sizeof(float));
}

uint32_t or_state_pos(const or_state *s) { return s->pos; }

static size_t put(float *out, size_t off, const float *src, size_t n) {
    if (out) memcpy(out + off, src, n * sizeof(float));
    return off + n;
}

size_t or_state_export(const or_state *s, float *out) {
    const or_model *m = s->m;
    size_t off = 0;
    for (uint32_t i = 0; i < m->cfg.n_layer; i++) {
        if (m->layers[i].attention) {
            off = put(out, off, s->kv[i].k, s->kv[i].len * s->kv[i].stride);
            off = put(out, off, s->kv[i].v, s->kv[i].len * s->kv[i].stride);
        } else {
            off = put(out, off, s->rec[i], dn_state_len(m));
            off = put(out, off, s->conv[i], dn_conv_len(m));
        }
    }
    if (s->k > 0) {
        off = put(out, off, s->mtp_kv.k, s->mtp_kv.len * s->mtp_kv.stride);
        off = put(out, off, s->mtp_kv.v, s->mtp_kv.len * s->mtp_kv.stride);
    }
    return off;
}

/* ============================================================================ one layer, for the fixtures */

/* The layer tests of the reference (tests/layers.rs:109-271) run one mixer, the MLP or a whole decoder layer on
 * its own. kind: 0 DeltaNet mixer, 1 attention mixer, 2 MLP, 3 decoder with DeltaNet, 4 decoder with attention.
 * Tensors are named "blk.0.<suffix>". conv/rec (DeltaNet) and k_cache/v_cache with *kv_len (attention,
 * capacity kv_cap rows of n_head_kv*head_dim) are carried state, read and updated. */
int or_layer_run(const aq_model_config *cfg, const aq_tensor *ts, size_t n, int kind, const float *x, size_t t,
                 uint32_t start_pos, float *conv, float *rec, float *k_cache, float *v_cache, uint32_t *kv_len,
                 uint32_t kv_cap, float *y) {
    or_model m;
    memset(&m, 0, sizeof m);
    m.cfg = *cfg;
    m.threads = 3;
    m.kd = (size_t)cfg->dn_n_k_heads * cfg->dn_head_dim_k;
    m.vd = (size_t)cfg->dn_n_v_heads * cfg->dn_head_dim_v;
    m.cd = 2 * m.kd + m.vd;
    m.inv_freq = (float *)malloc(cfg->rope_dim / 2 * sizeof(float) + 4);
    or_inv_freq(cfg->rope_dim, cfg->rope_theta, m.inv_freq);
    or_layer L;
    memset(&L, 0, sizeof L);
    size_t h = cfg->hidden;
    int attention = kind == 1 || kind == 4;
    int bad = 0;
    L.attention = attention;
    if (kind >= 3) {
        bad |= !(L.attn_norm = get_vec(ts, n, "blk.0.attn_norm.weight", h));
        bad |= !(L.post_norm = get_vec(ts, n, "blk.0.post_attention_norm.weight", h));
    }
    if (kind >= 2) {
        bad |= get_mat(ts, n, "blk.0.ffn_gate.weight", cfg->ffn, h, &L.gate);
        bad |= get_mat(ts, n, "blk.0.ffn_up.weight", cfg->ffn, h, &L.up);
        bad |= get_mat(ts, n, "blk.0.ffn_down.weight", h, cfg->ffn, &L.down);
    }
    if (kind == 1 || kind == 4) {
        size_t nh = cfg->n_head, nkv = cfg->n_head_kv, hd = cfg->head_dim;
        bad |= get_mat(ts, n, "blk.0.attn_q.weight", 2 * nh * hd, h, &L.q);
        bad |= get_mat(ts, n, "blk.0.attn_k.weight", nkv * hd, h, &L.k);
        bad |= get_mat(ts, n, "blk.0.attn_v.weight", nkv * hd, h, &L.v);
        bad |= get_mat(ts, n, "blk.0.attn_output.weight", h, nh * hd, &L.o);
        bad |= !(L.q_norm = get_vec(ts, n, "blk.0.attn_q_norm.weight", hd));
        bad |= !(L.k_norm = get_vec(ts, n, "blk.0.attn_k_norm.weight", hd));
    }
    if (kind == 0 || kind == 3) {
        size_t nv = cfg->dn_n_v_heads;
        bad |= get_mat(ts, n, "blk.0.attn_qkv.weight", m.cd, h, &L.qkv);
        bad |= get_mat(ts, n, "blk.0.attn_gate.weight", m.vd, h, &L.gate_z);
        bad |= get_mat(ts, n, "blk.0.ssm_alpha.weight", nv, h, &L.alpha);
        bad |= get_mat(ts, n, "blk.0.ssm_beta.weight", nv, h, &L.beta);
        bad |= get_mat(ts, n, "blk.0.ssm_out.weight", h, m.vd, &L.ssm_out);
        bad |= !(L.ssm_a = get_vec(ts, n, "blk.0.ssm_a", nv));
        bad |= !(L.dt_bias = get_vec(ts, n, "blk.0.ssm_dt.bias", nv));
        bad |= !(L.conv_w = get_vec(ts, n, "blk.0.ssm_conv1d.weight", m.cd * cfg->dn_conv_kernel));
        bad |= !(L.ssm_norm = get_vec(ts, n, "blk.0.ssm_norm.weight", cfg->dn_head_dim_v));
    }
    or_kv kv = {k_cache, v_cache, kv_len ? *kv_len : 0, kv_cap, (size_t)cfg->n_head_kv * cfg->head_dim};
    if (!bad) {
        switch (kind) {
        case 0: deltanet_batch(&m, &L, x, t, conv, rec, y, NULL, NULL, NULL); break;
        case 1: attention_batch(&m, &L, x, t, start_pos, &kv, y); break;
        case 2: mlp_batch(&m, &L, x, t, y); break;
        default: decoder_batch(&m, &L, x, t, start_pos, conv, rec, &kv, y, NULL, NULL, NULL); break;
        }
        if (kv_len) *kv_len = (uint32_t)kv.len;
    }
    free_layer(&L);
    free(m.inv_freq);
    return bad ? -1 : 0;
}
