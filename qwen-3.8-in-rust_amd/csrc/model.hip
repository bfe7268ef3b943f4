// model.hip — the model-level C-ABI: synthetic tensor plans, the resident model, per-sequence state, the
// batched forward (token / prefill / verify), the greedy speculative round with lazy DeltaNet commit, the MTP
// draft head, and the layer / recurrence entry points the parity tests use.
//
// Host orchestration only: every number is computed by the kernels of ops.hip, matmul.hip and kq_mfma.hip, on
// the state's stream. The host learns one thing per speculative round, the number of accepted drafts (one small
// device-to-host copy), and uses it to size the commit and the MTP re-feed.
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "aq_common.h"
#include "ops.h"

namespace aq {

int weight_from_ggml(Weight &w, int type, size_t rows, size_t cols, const void *ggml, bool ggml_on_device, int device,
                     hipStream_t stream);
void free_weight(Weight &w);
int alloc_act(Act &a, size_t n, size_t ncols, int device);
void free_act(Act &a);
int synth_device(const aq_synth_spec &s, uint8_t *out, hipStream_t stream);

namespace {

constexpr int MAX_ROWS = 8;  // rows per verify / decode pass: the matrix-core matmul takes 1..8 activation columns
constexpr int PRE_ROWS = 64; // rows per prompt chunk (model.rs:443-461: one pass over the weights per chunk)

bool is_attention_layer(const aq_model_config &c, uint32_t i) {
    return c.full_attention_interval > 0 && (i + 1) % c.full_attention_interval == 0;
}

int check_config(const aq_model_config *c) {
    AQ_REQUIRE(c, "null config");
    AQ_REQUIRE(c->n_layer >= 1 && c->hidden >= 256 && c->hidden % 256 == 0, "config: hidden must be a multiple of 256");
    AQ_REQUIRE(c->ffn % 256 == 0 && c->ffn > 0, "config: ffn must be a multiple of 256");
    AQ_REQUIRE(c->vocab >= 1, "config: vocab");
    AQ_REQUIRE(c->n_head >= 1 && c->n_head_kv >= 1 && c->n_head % c->n_head_kv == 0, "config: heads");
    AQ_REQUIRE(c->head_dim % 64 == 0 && c->head_dim <= 256, "config: head_dim must be 64..256, a multiple of 64");
    AQ_REQUIRE(c->rope_dim >= 2 && c->rope_dim <= c->head_dim && c->rope_dim % 2 == 0, "config: rope_dim");
    AQ_REQUIRE(c->full_attention_interval >= 1, "config: full_attention_interval");
    AQ_REQUIRE(c->dn_n_k_heads >= 1 && c->dn_n_v_heads % c->dn_n_k_heads == 0, "config: DeltaNet heads");
    AQ_REQUIRE(c->dn_head_dim_k == 64 || c->dn_head_dim_k == 128, "config: DeltaNet head_dim_k must be 64 or 128");
    AQ_REQUIRE(c->dn_head_dim_v >= 64 && c->dn_head_dim_v <= 256 && c->dn_head_dim_v % 64 == 0, "config: head_dim_v");
    AQ_REQUIRE(c->dn_conv_kernel == 4, "config: conv kernel must be 4");
    AQ_REQUIRE(((size_t)c->dn_n_v_heads * c->dn_head_dim_v) % 256 == 0, "config: DeltaNet value width % 256");
    AQ_REQUIRE(((size_t)c->n_head * c->head_dim) % 256 == 0, "config: attention width % 256");
    return 0;
}

// ======================================================================================== synthetic plans

struct PlanEntry {
    std::string name;
    aq_synth_spec spec;
};

uint64_t tensor_seed(uint64_t seed, size_t i) {
    uint64_t z = seed + 0x9E3779B97F4A7C15ull * (uint64_t)(i + 1);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// The per-tensor types of the Q4_K_M file of the 27B hybrid (docs/data/gguf_layout.txt).
int mix_type(int mix, const std::string &kind, uint32_t layer, bool mtp) {
    if (mix == AQ_MIX_TINY) {
        if (kind == "ffn_down" || kind == "output") return AQ_TYPE_Q6_K;
        if (kind == "ssm_alpha" || kind == "ssm_beta") return AQ_TYPE_F32;
        return AQ_TYPE_Q4_K;
    }
    if (mtp) return AQ_TYPE_Q4_0; // blk.64: every matrix Q4_0 (docs/mtp.md:27-41)
    if (kind == "token_embd") return AQ_TYPE_Q4_K;
    if (kind == "output") return AQ_TYPE_Q6_K;
    if (kind == "attn_qkv") return AQ_TYPE_Q6_K;
    if (kind == "attn_gate") return AQ_TYPE_Q4_K;
    if (kind == "ssm_alpha" || kind == "ssm_beta") return AQ_TYPE_F32;
    if (kind == "ssm_out") {
        const bool q8 = layer <= 2 || (layer >= 4 && layer <= 6) || (layer >= 10 && layer <= 54 && (layer - 10) % 4 == 0) ||
                        (layer >= 56 && layer <= 58) || (layer >= 60 && layer <= 62);
        return q8 ? AQ_TYPE_Q8_0 : AQ_TYPE_Q4_K;
    }
    if (kind == "attn_q" || kind == "attn_v") {
        const bool q6 = layer == 3 || layer == 7 || layer == 19 || layer == 31 || layer == 43 || layer == 55 ||
                        layer == 59 || layer == 63;
        return q6 ? AQ_TYPE_Q6_K : AQ_TYPE_Q4_K;
    }
    if (kind == "attn_k" || kind == "attn_output") return AQ_TYPE_Q5_K;
    if (kind == "ffn_gate" || kind == "ffn_up") return AQ_TYPE_Q4_K;
    if (kind == "ffn_down") {
        const bool q6 = layer <= 7 || (layer >= 10 && layer <= 55 && (layer - 10) % 3 == 0) || layer >= 56;
        return q6 ? AQ_TYPE_Q6_K : AQ_TYPE_Q4_K;
    }
    return AQ_TYPE_F32;
}

std::vector<PlanEntry> make_plan(const aq_model_config &c, int mix, uint64_t seed) {
    std::vector<PlanEntry> plan;
    const size_t h = c.hidden, kd = (size_t)c.dn_n_k_heads * c.dn_head_dim_k,
                 vd = (size_t)c.dn_n_v_heads * c.dn_head_dim_v, cd = 2 * kd + vd;
    auto add = [&](const std::string &name, int type, size_t rows, size_t cols, uint32_t dist, float a, float b) {
        PlanEntry e;
        e.name = name;
        e.spec.ggml_type = type;
        e.spec.rows = (int64_t)rows;
        e.spec.cols = (int64_t)cols;
        e.spec.seed = tensor_seed(seed, plan.size());
        e.spec.dist = dist;
        e.spec.a = a;
        e.spec.b = b;
        plan.push_back(e);
    };
    auto mat = [&](const std::string &name, const std::string &kind, uint32_t layer, bool mtp, size_t rows, size_t cols) {
        add(name, mix_type(mix, kind, layer, mtp), rows, cols, 0, 0.0f, 0.02f);
    };
    auto ones = [&](const std::string &name, size_t n) { add(name, AQ_TYPE_F32, 1, n, 2, 1.0f, 0.0f); };
    add("token_embd.weight", mix_type(mix, "token_embd", 0, false), c.vocab, h, 0, 0.0f, 0.02f);
    auto layer = [&](uint32_t i, bool attention, bool mtp) {
        const std::string p = "blk." + std::to_string(i) + ".";
        ones(p + "attn_norm.weight", h);
        ones(p + "post_attention_norm.weight", h);
        if (attention) {
            const size_t nh = c.n_head, nkv = c.n_head_kv, hd = c.head_dim;
            mat(p + "attn_q.weight", "attn_q", i, mtp, 2 * nh * hd, h);
            mat(p + "attn_k.weight", "attn_k", i, mtp, nkv * hd, h);
            mat(p + "attn_v.weight", "attn_v", i, mtp, nkv * hd, h);
            mat(p + "attn_output.weight", "attn_output", i, mtp, h, nh * hd);
            ones(p + "attn_q_norm.weight", hd);
            ones(p + "attn_k_norm.weight", hd);
        } else {
            const size_t nv = c.dn_n_v_heads;
            mat(p + "attn_qkv.weight", "attn_qkv", i, mtp, cd, h);
            mat(p + "attn_gate.weight", "attn_gate", i, mtp, vd, h);
            mat(p + "ssm_alpha.weight", "ssm_alpha", i, mtp, nv, h);
            mat(p + "ssm_beta.weight", "ssm_beta", i, mtp, nv, h);
            mat(p + "ssm_out.weight", "ssm_out", i, mtp, h, vd);
            add(p + "ssm_a", AQ_TYPE_F32, 1, nv, 1, -16.0f, 0.0f);
            add(p + "ssm_dt.bias", AQ_TYPE_F32, 1, nv, 2, 1.0f, 0.0f);
            add(p + "ssm_conv1d.weight", AQ_TYPE_F32, cd, c.dn_conv_kernel, 0, 0.0f, 0.02f);
            ones(p + "ssm_norm.weight", c.dn_head_dim_v);
        }
        mat(p + "ffn_gate.weight", "ffn_gate", i, mtp, c.ffn, h);
        mat(p + "ffn_up.weight", "ffn_up", i, mtp, c.ffn, h);
        mat(p + "ffn_down.weight", "ffn_down", i, mtp, h, c.ffn);
    };
    for (uint32_t i = 0; i < c.n_layer; i++) layer(i, is_attention_layer(c, i), false);
    ones("output_norm.weight", h);
    add("output.weight", mix_type(mix, "output", 0, false), c.vocab, h, 0, 0.0f, 0.02f);
    if (c.has_mtp) {
        const uint32_t mi = c.n_layer;
        layer(mi, true, true);
        const std::string p = "blk." + std::to_string(mi) + ".nextn.";
        mat(p + "eh_proj.weight", "eh_proj", mi, true, h, 2 * h);
        ones(p + "enorm.weight", h);
        ones(p + "hnorm.weight", h);
        ones(p + "shared_head_norm.weight", h);
    }
    return plan;
}

size_t ggml_bytes(int type, size_t rows, size_t cols) { return rows * (cols / block_elems(type)) * block_bytes(type); }

} // namespace

// =========================================================================================== the model

struct DevLayer {
    bool attention = false;
    float *attn_norm = nullptr, *post_norm = nullptr;
    Weight qkv, gate_z, alpha, beta, ssm_out;
    float *ssm_a = nullptr, *dt_bias = nullptr, *conv_w = nullptr, *ssm_norm = nullptr;
    Weight q, k, v, o;
    float *q_norm = nullptr, *k_norm = nullptr;
    Weight gate, up, down;
};

} // namespace aq

struct aq_model {
    aq_ctx *ctx = nullptr;
    int device = 0; // the context's device, kept so that freeing never reads the context
    aq_model_config cfg{};
    size_t kd = 0, vd = 0, cd = 0;
    aq::Weight embed, lm_head;
    float *output_norm = nullptr;
    std::vector<aq::DevLayer> layers;
    bool has_mtp = false;
    aq::DevLayer mtp;
    aq::Weight eh_proj;
    float *enorm = nullptr, *hnorm = nullptr, *head_norm = nullptr;
    std::vector<float> inv_freq;
    float qscale = 0.0f, attn_scaling = 0.0f;
    std::vector<aq::Weight *> weights;
    std::vector<void *> vecs;
    aq_model_bytes bytes{};
};

namespace aq {
namespace {

void free_model(aq_model *m) {
    if (!m) return;
    for (Weight *w : m->weights) free_weight(*w);
    for (void *p : m->vecs) (void)hipFree(p);
    delete m;
}

// Where the tensors come from: a host tensor table or a synthetic plan (generated on the device).
struct Source {
    const aq_tensor *ts = nullptr;
    size_t n = 0;
    const std::vector<PlanEntry> *plan = nullptr;
    hipStream_t stream = nullptr;
    int device = 0;
    uint8_t *staging = nullptr; // device, for synthetic matrices
    size_t staging_bytes = 0;

    const aq_tensor *find(const std::string &name) const {
        for (size_t i = 0; i < n; i++)
            if (ts[i].name && name == ts[i].name) return &ts[i];
        return nullptr;
    }
    const PlanEntry *find_plan(const std::string &name) const {
        for (const PlanEntry &e : *plan)
            if (e.name == name) return &e;
        return nullptr;
    }

    int mat(aq_model *m, const std::string &name, size_t rows, size_t cols, Weight &w) {
        if (plan) {
            const PlanEntry *e = find_plan(name);
            AQ_REQUIRE(e, "model: missing tensor " + name);
            AQ_REQUIRE((size_t)e->spec.rows == rows && (size_t)e->spec.cols == cols, "model: bad shape for " + name);
            const size_t bytes = ggml_bytes(e->spec.ggml_type, rows, cols);
            if (bytes > staging_bytes) {
                if (staging) (void)hipFree(staging);
                staging = nullptr;
                staging_bytes = 0;
                if (dev_malloc(&staging, bytes) != hipSuccess) return fail(AQ_ENOMEM, "model: staging for " + name);
                staging_bytes = bytes;
            }
            int rc = synth_device(e->spec, staging, stream);
            if (!rc) rc = weight_from_ggml(w, e->spec.ggml_type, rows, cols, staging, true, device, stream);
            if (!rc) AQ_HIP(hipStreamSynchronize(stream)); // the staging buffer is reused by the next tensor
            if (rc) return rc;
        } else {
            const aq_tensor *t = find(name);
            AQ_REQUIRE(t, "model: missing tensor " + name);
            AQ_REQUIRE((size_t)t->rows == rows && (size_t)t->cols == cols,
                       "model: " + name + " is " + std::to_string(t->rows) + "x" + std::to_string(t->cols) + ", want " +
                           std::to_string(rows) + "x" + std::to_string(cols));
            AQ_REQUIRE(block_bytes(t->ggml_type) > 0, "model: unsupported type for " + name);
            AQ_REQUIRE(t->data && t->nbytes >= ggml_bytes(t->ggml_type, rows, cols), "model: short data for " + name);
            int rc = weight_from_ggml(w, t->ggml_type, rows, cols, t->data, false, device, stream);
            if (rc) return rc;
        }
        m->weights.push_back(&w);
        return 0;
    }

    int vec(aq_model *m, const std::string &name, size_t len, float *&out) {
        std::vector<float> host(len);
        if (plan) {
            const PlanEntry *e = find_plan(name);
            AQ_REQUIRE(e, "model: missing tensor " + name);
            AQ_REQUIRE((size_t)(e->spec.rows * e->spec.cols) == len && e->spec.ggml_type == AQ_TYPE_F32,
                       "model: bad vector " + name);
            int rc = aq_synth_host(&e->spec, host.data(), 1);
            if (rc) return rc;
        } else {
            const aq_tensor *t = find(name);
            AQ_REQUIRE(t, "model: missing tensor " + name);
            AQ_REQUIRE((size_t)(t->rows * t->cols) == len, "model: bad length for " + name);
            AQ_REQUIRE(t->ggml_type == AQ_TYPE_F32, "model: vector " + name + " must be F32");
            AQ_REQUIRE(t->data && t->nbytes >= len * 4, "model: short data for " + name);
            std::memcpy(host.data(), t->data, len * 4);
        }
        void *p = nullptr;
        if (dev_malloc(&p, len * 4 + 256) != hipSuccess) return fail(AQ_ENOMEM, "model: vector " + name);
        m->vecs.push_back(p);
        AQ_HIP(hipMemcpy(p, host.data(), len * 4, hipMemcpyHostToDevice));
        out = (float *)p;
        return 0;
    }
};

int load_layer(aq_model *m, Source &src, uint32_t index, bool attention, DevLayer &L) {
    const aq_model_config &c = m->cfg;
    const size_t h = c.hidden;
    const std::string p = "blk." + std::to_string(index) + ".";
    L.attention = attention;
    int rc = 0;
#define AQ_TRY(x)                                                                                             \
    do {                                                                                                      \
        rc = (x);                                                                                             \
        if (rc) return rc;                                                                                    \
    } while (0)
    AQ_TRY(src.vec(m, p + "attn_norm.weight", h, L.attn_norm));
    AQ_TRY(src.vec(m, p + "post_attention_norm.weight", h, L.post_norm));
    if (attention) {
        const size_t nh = c.n_head, nkv = c.n_head_kv, hd = c.head_dim;
        AQ_TRY(src.mat(m, p + "attn_q.weight", 2 * nh * hd, h, L.q));
        AQ_TRY(src.mat(m, p + "attn_k.weight", nkv * hd, h, L.k));
        AQ_TRY(src.mat(m, p + "attn_v.weight", nkv * hd, h, L.v));
        AQ_TRY(src.mat(m, p + "attn_output.weight", h, nh * hd, L.o));
        AQ_TRY(src.vec(m, p + "attn_q_norm.weight", hd, L.q_norm));
        AQ_TRY(src.vec(m, p + "attn_k_norm.weight", hd, L.k_norm));
    } else {
        const size_t nv = c.dn_n_v_heads;
        AQ_TRY(src.mat(m, p + "attn_qkv.weight", m->cd, h, L.qkv));
        AQ_TRY(src.mat(m, p + "attn_gate.weight", m->vd, h, L.gate_z));
        AQ_TRY(src.mat(m, p + "ssm_alpha.weight", nv, h, L.alpha));
        AQ_TRY(src.mat(m, p + "ssm_beta.weight", nv, h, L.beta));
        AQ_TRY(src.mat(m, p + "ssm_out.weight", h, m->vd, L.ssm_out));
        AQ_TRY(src.vec(m, p + "ssm_a", nv, L.ssm_a));
        AQ_TRY(src.vec(m, p + "ssm_dt.bias", nv, L.dt_bias));
        AQ_TRY(src.vec(m, p + "ssm_conv1d.weight", m->cd * c.dn_conv_kernel, L.conv_w));
        AQ_TRY(src.vec(m, p + "ssm_norm.weight", c.dn_head_dim_v, L.ssm_norm));
    }
    AQ_TRY(src.mat(m, p + "ffn_gate.weight", c.ffn, h, L.gate));
    AQ_TRY(src.mat(m, p + "ffn_up.weight", c.ffn, h, L.up));
    AQ_TRY(src.mat(m, p + "ffn_down.weight", h, c.ffn, L.down));
    return 0;
}

uint64_t wbytes(const Weight &w) { return w.base ? ggml_bytes(w.type, w.rows, w.cols) : 0; }

uint64_t layer_bytes(const aq_model *m, const DevLayer &L) {
    const uint64_t h4 = (uint64_t)m->cfg.hidden * 4;
    uint64_t b = wbytes(L.qkv) + wbytes(L.gate_z) + wbytes(L.alpha) + wbytes(L.beta) + wbytes(L.ssm_out) + wbytes(L.q) +
                 wbytes(L.k) + wbytes(L.v) + wbytes(L.o) + wbytes(L.gate) + wbytes(L.up) + wbytes(L.down) + 2 * h4;
    if (L.attention) b += 2ull * m->cfg.head_dim * 4;
    else b += (uint64_t)m->cfg.dn_n_v_heads * 8 + (uint64_t)m->cd * m->cfg.dn_conv_kernel * 4 + m->cfg.dn_head_dim_v * 4;
    return b;
}

int build_model(aq_ctx *ctx, const aq_model_config *cfg, Source &src, aq_model **out) {
    aq_model *m = new aq_model();
    m->ctx = ctx;
    m->device = ctx->device;
    m->cfg = *cfg;
    m->kd = (size_t)cfg->dn_n_k_heads * cfg->dn_head_dim_k;
    m->vd = (size_t)cfg->dn_n_v_heads * cfg->dn_head_dim_v;
    m->cd = 2 * m->kd + m->vd;
    const size_t h = cfg->hidden;
    int rc = src.mat(m, "token_embd.weight", cfg->vocab, h, m->embed);
    if (!rc && m->embed.type != AQ_TYPE_Q4_K) rc = fail(AQ_EUNSUP, "model: token_embd must be Q4_K in this build");
    if (!rc) rc = src.mat(m, "output.weight", cfg->vocab, h, m->lm_head);
    if (!rc) rc = src.vec(m, "output_norm.weight", h, m->output_norm);
    m->layers.resize(cfg->n_layer);
    for (uint32_t i = 0; i < cfg->n_layer && !rc; i++) rc = load_layer(m, src, i, is_attention_layer(*cfg, i), m->layers[i]);
    m->has_mtp = cfg->has_mtp != 0;
    if (m->has_mtp && !rc) {
        const uint32_t mi = cfg->n_layer;
        rc = load_layer(m, src, mi, true, m->mtp);
        const std::string p = "blk." + std::to_string(mi) + ".nextn.";
        if (!rc) rc = src.mat(m, p + "eh_proj.weight", h, 2 * h, m->eh_proj);
        if (!rc) rc = src.vec(m, p + "enorm.weight", h, m->enorm);
        if (!rc) rc = src.vec(m, p + "hnorm.weight", h, m->hnorm);
        if (!rc) rc = src.vec(m, p + "shared_head_norm.weight", h, m->head_norm);
    }
    if (src.staging) (void)hipFree(src.staging);
    src.staging = nullptr;
    if (rc) {
        free_model(m);
        return rc;
    }
    // rope.rs:10-12 inv_freq and the two constants, on the host as the reference computes them
    m->inv_freq.resize(cfg->rope_dim / 2);
    for (size_t i = 0; i < m->inv_freq.size(); i++)
        m->inv_freq[i] = 1.0f / powf(cfg->rope_theta, (float)(2 * i) / (float)cfg->rope_dim);
    m->qscale = 1.0f / sqrtf((float)cfg->dn_head_dim_k);
    m->attn_scaling = powf((float)cfg->head_dim, -0.5f);
    uint64_t main = wbytes(m->lm_head) + (uint64_t)h * 4;
    for (const DevLayer &L : m->layers) main += layer_bytes(m, L);
    m->bytes.main = main;
    m->bytes.lm_head = wbytes(m->lm_head);
    m->bytes.embed_row = ggml_bytes(m->embed.type, 1, h);
    m->bytes.mtp_block = m->has_mtp ? layer_bytes(m, m->mtp) + wbytes(m->eh_proj) + 3ull * h * 4 : 0;
    *out = m;
    return 0;
}

} // namespace
} // namespace aq

// ============================================================================================ the state

namespace aq {
namespace {
struct KvDev {
    float *k = nullptr, *v = nullptr;
    size_t len = 0, cap = 0, stride = 0;
};
} // namespace
} // namespace aq

struct aq_state {
    aq_model *m = nullptr;
    int device = 0; // the model's device, kept so that freeing never reads the model
    hipStream_t stream = nullptr;
    hipEvent_t ev[5] = {};
    bool ev_pending = false;
    // a prompt chunk's F32 projections run here beside the chunk's GEMMs (aux_in: their input is ready on `stream`;
    // aux_out: their outputs are, before `stream` goes on)
    hipStream_t aux = nullptr;
    hipEvent_t aux_in = nullptr, aux_out = nullptr;
    uint32_t pos = 0, max_pos = 0, k = 0;
    int par = 0; // which conv window buffer is current
    std::vector<float *> rec, conv0, conv1, sv_mixed, sv_a, sv_b;
    std::vector<aq::KvDev> kv;
    aq::KvDev mtp_kv;
    aq::Act act_h, act_ffn, act_vd, act_att, act_cat;
    float *xa = nullptr, *xb = nullptr, *y = nullptr, *mixed = nullptr, *z = nullptr, *a = nullptr, *b = nullptr;
    float *qg = nullptr, *kk = nullptr, *vv = nullptr, *qr = nullptr, *g = nullptr, *u = nullptr, *e = nullptr;
    float *logits = nullptr, *normed = nullptr, *normed_all = nullptr, *mtp_hout = nullptr;
    float *cos_tab = nullptr, *sin_tab = nullptr;
    uint32_t *ids = nullptr, *amax = nullptr, *drafts = nullptr, *emitted = nullptr, *info = nullptr, *prompt = nullptr,
             *shifted = nullptr;
    void *amax_scratch = nullptr;
    float *attn_sc = nullptr; // attention score rows [T][n_head][attn_sc_stride], when contexts outgrow the LDS
    size_t attn_sc_stride = 0;
    uint32_t *pinned = nullptr; // host, 64 words
    aq_sampler *sp = nullptr;   // the sampler of the running sampled call (null: greedy)
    float *q_dense = nullptr;   // k x vocab: each draft's dense distribution (sampled rounds)
    uint32_t *q_idx = nullptr, *q_n = nullptr; // the ids last written into each q_dense row, and their count
    aq::DnArgs *commit_args = nullptr; // device: the commit's DnArgs per DeltaNet slot, for par = 0 then par = 1
    int n_dn = 0;
    bool spec_ready = false;
    aq_spec_stats stats{};
    std::vector<void *> allocs;
};

namespace aq {
namespace {

Act col_view(const Act &a, size_t col) {
    Act v = a;
    v.ncols = a.ncols - col;
    v.f32 = a.f32 + col * a.n;
    v.qs = a.qs + col * a.n;
    v.d = a.d + col * a.nb;
    v.bs = a.bs + col * a.nb * 16;
    v.q8s = a.q8s + col * a.nb * 8;
    v.q0 = a.q0 + col * a.n;
    v.d0 = a.d0 + col * a.nb32;
    v.h0 = a.h0 + col * a.nb32;
    v.s0 = a.s0 + col * a.nb32;
    return v;
}

int dalloc(aq_state *s, size_t bytes, void **p) {
    if (dev_malloc(p, bytes + 256) != hipSuccess) return fail(AQ_ENOMEM, "state: hipMalloc of " + std::to_string(bytes));
    s->allocs.push_back(*p);
    AQ_HIP(hipMemset(*p, 0, bytes + 256));
    return 0;
}
template <typename T> int dalloc_t(aq_state *s, size_t count, T **p) {
    void *q = nullptr;
    int rc = dalloc(s, count * sizeof(T), &q);
    *p = (T *)q;
    return rc;
}

void free_state(aq_state *s) {
    if (!s) return;
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    if (s->aux) (void)hipStreamSynchronize(s->aux);
    for (void *p : s->allocs) (void)hipFree(p);
    free_act(s->act_h);
    free_act(s->act_ffn);
    free_act(s->act_vd);
    free_act(s->act_att);
    free_act(s->act_cat);
    if (s->pinned) (void)hipHostFree(s->pinned);
    for (hipEvent_t e : s->ev)
        if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : {s->aux_in, s->aux_out})
        if (e) (void)hipEventDestroy(e);
    if (s->aux) (void)hipStreamDestroy(s->aux);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    delete s;
}

// The quantised form(s) a set of consumer weights needs from one activation: the f32 rows are always written;
// Q8_K and/or Q8_0 as the weight types ask.
struct Needs {
    bool q8k = false, q80 = false;
    void add(const Weight &w) {
        if (!w.base) return;
        const QuantKind k = quant_kind_for(w.type);
        if (k == QK_Q8K) q8k = true;
        if (k == QK_Q80) q80 = true;
    }
};

// rows -> act (f32 + quantised as `nd` asks), via RMSNorm when `norm_w` is set, else a copy of f32 `src`.
int norm_into(aq_state *s, const float *x, size_t x_stride, const float *norm_w, size_t n, size_t t, Act &act,
              size_t col0, size_t elem_off, const Needs &nd, float *also_f32 = nullptr) {
    const float eps = s->m->cfg.rms_eps;
    QuantOut q;
    q.act = &act;
    q.col0 = col0;
    q.elem_off = elem_off;
    q.f32 = true;
    q.kind = nd.q8k ? QK_Q8K : (nd.q80 ? QK_Q80 : QK_NONE);
    int rc = launch_rmsnorm(x, x_stride, norm_w, eps, n, t, also_f32, n, q, s->stream);
    if (rc) return rc;
    if (nd.q8k && nd.q80) {
        Act v = col_view(act, col0);
        if (elem_off != 0 || n != act.n) return fail(AQ_EUNSUP, "norm_into: mixed quantised forms of a partial row");
        rc = launch_q8_0_quantize(v, t, v.f32, act.n, s->stream);
    }
    return rc;
}

// f32 rows already in act.f32 (columns 0..t) -> the quantised form(s).
int quantize_act(aq_state *s, Act &act, size_t t, const Needs &nd) {
    int rc = 0;
    if (nd.q8k) rc = launch_q8k_quantize(act, t, act.f32, act.n, s->stream);
    if (!rc && nd.q80) rc = launch_q8_0_quantize(act, t, act.f32, act.n, s->stream);
    return rc;
}

// y[c * rows + r] = W[r] . x[c] (+ resid) for c < t: one launch for up to MAX_ROWS columns; a prompt chunk's wider
// batches go to the many-column kernels (K-quant and Q8_0 / Q4_0 weights) or are split into MAX_ROWS-column pieces.
int mm(aq_state *s, const Weight &w, const Act &x, size_t t, float *y, const float *resid = nullptr) {
    return launch_matmul_many(w, x, t, y, resid, s->stream);
}

// Several matrices over the same activations: one grouped launch when they are K-quants of one K, optionally
// followed by (at most two) F32 matrices.
int mm_multi(aq_state *s, int n, const Weight *const *ws, float *const *ys, const Act &x, size_t t) {
    if (t > (size_t)MAX_ROWS) {
        // a prompt chunk: each matrix over all its columns; the F32 ones (few rows, latency-bound) on the auxiliary
        // stream beside the others, joined before anything after this call runs on the state's stream
        bool f32 = false;
        for (int i = 0; i < n; i++) f32 = f32 || ws[i]->type == AQ_TYPE_F32;
        if (f32) {
            AQ_HIP(hipEventRecord(s->aux_in, s->stream));
            AQ_HIP(hipStreamWaitEvent(s->aux, s->aux_in, 0));
            for (int i = 0; i < n; i++) {
                if (ws[i]->type != AQ_TYPE_F32) continue;
                const int rc = launch_matmul_many(*ws[i], x, t, ys[i], nullptr, s->aux);
                if (rc) return rc;
            }
            AQ_HIP(hipEventRecord(s->aux_out, s->aux));
        }
        for (int i = 0; i < n; i++) {
            if (ws[i]->type == AQ_TYPE_F32) continue;
            const int rc = mm(s, *ws[i], x, t, ys[i]);
            if (rc) return rc;
        }
        if (f32) AQ_HIP(hipStreamWaitEvent(s->stream, s->aux_out, 0));
        return 0;
    }
    bool grouped = is_kquant(ws[0]->type);
    int nf = 0;
    for (int i = 0; i < n; i++) {
        if (ws[i]->type == AQ_TYPE_F32) {
            nf++;
            continue;
        }
        grouped = grouped && nf == 0 && is_kquant(ws[i]->type) && ws[i]->nb == ws[0]->nb;
    }
    grouped = grouped && nf <= 2;
    if (grouped) return launch_kq_group(ws, ys, nullptr, n, x, t, s->stream);
    if (n >= 2 && n <= Q8_MAXSEG && (ws[0]->type == AQ_TYPE_Q8_0 || ws[0]->type == AQ_TYPE_Q4_0))
        return launch_q8_group(ws, ys, n, x, t, s->stream); // the MTP's Q4_0 q / k / v and gate / up
    for (int i = 0; i < n; i++) {
        const int rc = mm(s, *ws[i], x, t, ys[i]);
        if (rc) return rc;
    }
    return 0;
}

enum Mode { PLAIN = 0, VERIFY = 1 };

Needs mixer_needs(const DevLayer &L) {
    Needs nd;
    if (L.attention) {
        nd.add(L.q);
        nd.add(L.k);
        nd.add(L.v);
    } else {
        nd.add(L.qkv);
        nd.add(L.gate_z);
        nd.add(L.alpha);
        nd.add(L.beta);
    }
    return nd;
}

Needs mlp_needs(const DevLayer &L) {
    Needs nd;
    nd.add(L.gate);
    nd.add(L.up);
    return nd;
}

// The mixer on the rows in act_h (f32 + quantised): y_out = resid + mixer (resid null: y_out = mixer).
// Attention: gqa_attention.rs:327-418, K/V appended to `kv`. DeltaNet: gated_deltanet.rs:261-324; in VERIFY mode
// the recurrent state and conv window are read, not written, and the qkv / alpha / beta rows are kept in the
// layer's slot for the commit; in PLAIN mode the new conv window goes to the other buffer (the caller flips the
// parity once per pass).
// Whether a DeltaNet layer's ssm_alpha / ssm_beta rows come from its attn_norm launch (launch_rmsnorm_rows), so the
// grouped qkv / z launch carries K-quant tiles only: decode and verify batches, both gates F32 over whole 256-blocks
// and the K-quant pair grouped (not under the q8-fine switch).
bool dn_gates_in_norm(const aq_state *s, const DevLayer &L, size_t t) {
    return !L.attention && t >= 1 && t <= (size_t)MAX_ROWS && !q8_fine() && L.alpha.type == AQ_TYPE_F32 &&
           L.beta.type == AQ_TYPE_F32 && is_kquant(L.qkv.type) && is_kquant(L.gate_z.type) &&
           L.qkv.nb == L.gate_z.nb && L.alpha.cols == s->m->cfg.hidden && L.beta.cols == s->m->cfg.hidden &&
           rmsnorm_rows_fit(s->m->cfg.hidden);
}

// Where a pass's DeltaNet gate pre-activations go: in VERIFY mode the layer's slot (kept for the commit).
float *dn_alpha_out(aq_state *s, Mode mode, int dn_slot) { return mode == VERIFY ? s->sv_a[dn_slot] : s->a; }
float *dn_beta_out(aq_state *s, Mode mode, int dn_slot) { return mode == VERIFY ? s->sv_b[dn_slot] : s->b; }

// attn_norm of a DeltaNet layer into act_h (f32 + Q8_K) with its gate rows (dn_gates_in_norm), one launch.
int norm_gates_into(aq_state *s, const DevLayer &L, const float *x, size_t t, Mode mode, int dn_slot) {
    const size_t h = s->m->cfg.hidden;
    QuantOut q;
    q.act = &s->act_h;
    q.kind = QK_Q8K;
    q.f32 = true;
    NormRows fr;
    fr.w[0] = reinterpret_cast<const float *>(L.alpha.qa);
    fr.w[1] = reinterpret_cast<const float *>(L.beta.qa);
    fr.y[0] = dn_alpha_out(s, mode, dn_slot);
    fr.y[1] = dn_beta_out(s, mode, dn_slot);
    fr.rows[0] = (int)L.alpha.rows;
    fr.rows[1] = (int)L.beta.rows;
    return launch_rmsnorm_rows(x, h, L.attn_norm, s->m->cfg.rms_eps, h, t, q, fr, s->stream);
}

// gates_done: the DeltaNet gate rows are already in place (norm_gates_into).
int mixer(aq_state *s, const DevLayer &L, size_t t, size_t start_pos, KvDev *kv, int dn_slot, Mode mode, float *y_out,
          const float *resid, bool gates_done = false) {
    aq_model *m = s->m;
    const aq_model_config &c = m->cfg;
    int rc = 0;
    if (L.attention) {
        const Weight *ws[3] = {&L.q, &L.k, &L.v};
        float *ys[3] = {s->qg, s->kk, s->vv};
        if ((rc = mm_multi(s, 3, ws, ys, s->act_h, t))) return rc;
        AQ_REQUIRE(kv->len + t <= kv->cap, "attention: KV cache full");
        AttnArgs a;
        a.qg = s->qg;
        a.kk = s->kk;
        a.vv = s->vv;
        a.q_norm = L.q_norm;
        a.k_norm = L.k_norm;
        a.eps = c.rms_eps;
        a.scaling = m->attn_scaling;
        a.cos_tab = s->cos_tab;
        a.sin_tab = s->sin_tab;
        a.start_pos = start_pos;
        a.q = s->qr;
        a.kcache = kv->k;
        a.vcache = kv->v;
        a.base = kv->len;
        a.stride = kv->stride;
        a.out = s->act_att.f32;
        // the o projection reads Q8_K: each head's output row (head_dim 256) is quantised by the attention kernel
        const bool q8k = quant_kind_for(L.o.type) == QK_Q8K && c.head_dim == 256;
        a.out_q8k = q8k ? 1 : 0;
        a.q8k = s->act_att;
        a.t = (int)t;
        a.nh = (int)c.n_head;
        a.nkv = (int)c.n_head_kv;
        a.hd = (int)c.head_dim;
        a.rd = (int)c.rope_dim;
        a.gsc = s->attn_sc;
        a.gsc_stride = s->attn_sc_stride;
        // the whole chunk in one launch while its scores fit the LDS; past that, pieces of at most MAX_ROWS rows
        // (the score rows a context past the LDS keeps in device memory are that many), each piece's K/V rows
        // appended before the next piece attends to them
        const size_t qw = 2 * (size_t)c.n_head * c.head_dim, kw = kv->stride, ow = (size_t)c.n_head * c.head_dim;
        const size_t piece = kv->len + t <= attn_lds_positions((int)c.head_dim) ? t : (size_t)MAX_ROWS;
        for (size_t r0 = 0; r0 < t; r0 += piece) {
            const size_t tr = t - r0 < piece ? t - r0 : piece;
            AttnArgs ap = a;
            ap.qg = a.qg + r0 * qw;
            ap.kk = a.kk + r0 * kw;
            ap.vv = a.vv + r0 * kw;
            ap.q = a.q + r0 * ow;
            ap.out = a.out + r0 * ow;
            ap.q8k = col_view(s->act_att, r0);
            ap.start_pos = start_pos + r0;
            ap.base = kv->len;
            ap.t = (int)tr;
            if ((rc = launch_attention(ap, s->stream))) return rc;
            kv->len += tr;
        }
        if (!q8k) {
            Needs no;
            no.add(L.o);
            if ((rc = quantize_act(s, s->act_att, t, no))) return rc;
        }
        return mm(s, L.o, s->act_att, t, y_out, resid);
    }
    float *mixed = mode == VERIFY ? s->sv_mixed[dn_slot] : s->mixed;
    float *av = dn_alpha_out(s, mode, dn_slot);
    float *bv = dn_beta_out(s, mode, dn_slot);
    {
        // qkv, z and (unless the norm launch formed them) the ssm_alpha / ssm_beta gate pre-activations in one
        // launch (the gates kept for the commit)
        const Weight *ws[4] = {&L.qkv, &L.gate_z, &L.alpha, &L.beta};
        float *ys[4] = {mixed, s->z, av, bv};
        if ((rc = mm_multi(s, gates_done ? 2 : 4, ws, ys, s->act_h, t))) return rc;
    }
    DnArgs d;
    d.mixed = mixed;
    d.z = s->z;
    d.a = av;
    d.b = bv;
    d.conv_src = s->par ? s->conv1[dn_slot] : s->conv0[dn_slot];
    d.conv_dst = mode == VERIFY ? nullptr : (s->par ? s->conv0[dn_slot] : s->conv1[dn_slot]);
    d.conv_w = L.conv_w;
    d.ssm_a = L.ssm_a;
    d.dt_bias = L.dt_bias;
    d.ssm_norm = L.ssm_norm;
    d.eps = c.rms_eps;
    d.qscale = m->qscale;
    d.rec = s->rec[dn_slot];
    d.write_state = mode == VERIFY ? 0 : 1;
    d.out = s->act_vd.f32;
    // ssm_out reads Q8_0: each head's output rows are whole 32-blocks, quantised by the DeltaNet kernel itself
    const bool q80 = quant_kind_for(L.ssm_out.type) == QK_Q80 && c.dn_head_dim_v % 32 == 0;
    d.out_q80 = q80 ? 1 : 0;
    d.q80 = s->act_vd;
    d.t = (int)t;
    d.nk = (int)c.dn_n_k_heads;
    d.nv = (int)c.dn_n_v_heads;
    d.dk = (int)c.dn_head_dim_k;
    d.dv = (int)c.dn_head_dim_v;
    d.kernel = (int)c.dn_conv_kernel;
    // a prompt chunk (t > 8) runs as 8-row pieces inside the one launch, the state carried from piece to piece
    AQ_REQUIRE(t <= 8 || mode == PLAIN, "deltanet: more than 8 rows in one verify batch");
    if ((rc = launch_dn_core(d, s->stream))) return rc;
    if (!q80) {
        Needs no;
        no.add(L.ssm_out);
        if ((rc = quantize_act(s, s->act_vd, t, no))) return rc;
    }
    return mm(s, L.ssm_out, s->act_vd, t, y_out, resid);
}

// mlp.rs:114-132 on the rows in act_h: y_out = resid + down(silu(gate x) * up x).
int mlp(aq_state *s, const DevLayer &L, size_t t, float *y_out, const float *resid) {
    const size_t ffn = s->m->cfg.ffn;
    const Weight *ws[2] = {&L.gate, &L.up};
    float *ys[2] = {s->g, s->u};
    int rc = mm_multi(s, 2, ws, ys, s->act_h, t);
    if (rc) return rc;
    QuantOut q;
    q.act = &s->act_ffn;
    q.kind = quant_kind_for(L.down.type);
    if ((rc = launch_swiglu(s->g, s->u, ffn, t, q.kind == QK_NONE ? s->act_ffn.f32 : nullptr, q, s->stream))) return rc;
    return mm(s, L.down, s->act_ffn, t, y_out, resid);
}

// layers/mod.rs:335-377: h = x + mixer(rmsnorm(x)); y = h + mlp(rmsnorm(h)). x and y_out are t rows of hidden.
int decoder_layer(aq_state *s, const DevLayer &L, const float *x, size_t t, size_t start_pos, KvDev *kv, int dn_slot,
                  Mode mode, float *y_out) {
    const size_t h = s->m->cfg.hidden;
    const bool gates = dn_gates_in_norm(s, L, t);
    int rc = gates ? norm_gates_into(s, L, x, t, mode, dn_slot)
                   : norm_into(s, x, h, L.attn_norm, h, t, s->act_h, 0, 0, mixer_needs(L));
    if (!rc) rc = mixer(s, L, t, start_pos, kv, dn_slot, mode, s->y, x, gates);
    if (!rc) rc = norm_into(s, s->y, h, L.post_norm, h, t, s->act_h, 0, 0, mlp_needs(L));
    if (!rc) rc = mlp(s, L, t, y_out, s->y);
    return rc;
}

// t (<= MAX_ROWS) tokens at the state's position through every layer (model.rs:401-413, spec.rs:277-304).
// The final residual rows are left in s->xa. In VERIFY mode the DeltaNet state is read, not written, and the
// layer inputs of the recurrence are kept for the commit.
int forward_rows(aq_state *s, const uint32_t *ids_dev, size_t t, Mode mode) {
    aq_model *m = s->m;
    const size_t h = m->cfg.hidden;
    int rc = launch_embed(m->embed, ids_dev, t, s->xa, h, s->stream);
    if (rc) return rc;
    int dn = 0;
    for (uint32_t li = 0; li < m->cfg.n_layer; li++) {
        const DevLayer &L = m->layers[li];
        if ((rc = decoder_layer(s, L, s->xa, t, s->pos, &s->kv[li], L.attention ? -1 : dn, mode, s->xb))) return rc;
        if (!L.attention) dn++;
        std::swap(s->xa, s->xb);
    }
    if (mode == PLAIN) s->par ^= 1;
    s->pos += (uint32_t)t;
    return 0;
}

// model.rs:430-438: final norm of t rows (f32 into `normed`) and the lm_head into s->logits.
int head_rows(aq_state *s, const float *rows, size_t t, float *normed) {
    aq_model *m = s->m;
    const size_t h = m->cfg.hidden;
    Needs nd;
    nd.add(m->lm_head);
    int rc = norm_into(s, rows, h, m->output_norm, h, t, s->act_h, 0, 0, nd, normed);
    if (rc) return rc;
    return mm(s, m->lm_head, s->act_h, t, s->logits);
}

// ---------------------------------------------------------------------------------------------------- MTP
// mtp.rs:95-104 `set_row_with` for t rows: cat row i = [rmsnorm(embed(ids[i]), enorm) | rmsnorm(hs[i], hnorm)].
int mtp_set_rows(aq_state *s, const uint32_t *ids_dev, const float *hs, size_t t) {
    aq_model *m = s->m;
    const size_t h = m->cfg.hidden;
    Needs nd;
    nd.add(m->eh_proj);
    int rc = launch_embed(m->embed, ids_dev, t, s->e, h, s->stream);
    if (rc) return rc;
    if (nd.q8k && nd.q80) { // two quantised forms: norm_into's path (which refuses them for half rows)
        rc = norm_into(s, s->e, h, m->enorm, h, t, s->act_cat, 0, 0, nd);
        if (!rc) rc = norm_into(s, hs, h, m->hnorm, h, t, s->act_cat, 0, h, nd);
        return rc;
    }
    QuantOut q; // both halves in one launch
    q.act = &s->act_cat;
    q.col0 = 0;
    q.elem_off = 0;
    q.f32 = true;
    q.kind = nd.q8k ? QK_Q8K : (nd.q80 ? QK_Q80 : QK_NONE);
    return launch_rmsnorm_pair(s->e, h, m->enorm, hs, h, m->hnorm, h, m->cfg.rms_eps, h, t, q, s->stream);
}

// mtp.rs:108-127 `rows_in`: eh_proj, the block at positions mtp_kv.len.., shared_head_norm -> s->mtp_hout rows
// (f32) and their Q8 form in act_h for the shared lm_head.
int mtp_rows(aq_state *s, size_t t) {
    aq_model *m = s->m;
    const size_t h = m->cfg.hidden;
    int rc = mm(s, m->eh_proj, s->act_cat, t, s->xa);
    if (!rc) rc = decoder_layer(s, m->mtp, s->xa, t, s->mtp_kv.len, &s->mtp_kv, -1, PLAIN, s->xb);
    if (rc) return rc;
    Needs nd;
    nd.add(m->lm_head);
    return norm_into(s, s->xb, h, m->head_norm, h, t, s->act_h, 0, 0, nd, s->mtp_hout);
}

// mtp.rs:130-137 `head_in` + spec.rs:192-203: draft = argmax(lm_head(hout row `row`)) into drafts[i].
int mtp_draft(aq_state *s, size_t row, size_t i) {
    aq_model *m = s->m;
    const size_t vocab = m->cfg.vocab;
    Act v = col_view(s->act_h, row);
    int rc = mm(s, m->lm_head, v, 1, s->logits);
    if (rc) return rc;
    if (sampler_greedy(s->sp)) return launch_argmax(s->logits, vocab, vocab, 1, s->drafts + i, s->amax_scratch, s->stream);
    return sampler_draft(s->sp, s->logits, s->drafts + i, s->q_dense + i * vocab, s->q_idx + i * vocab, s->q_n + i,
                         s->stream);
}

// The next token from one logits row: argmax (model.rs:505-513), or Sampler::sample under a sampler.
int next_token(aq_state *s, const float *logits, uint32_t *tok_dev) {
    const size_t vocab = s->m->cfg.vocab;
    if (sampler_greedy(s->sp)) return launch_argmax(logits, vocab, vocab, 1, tok_dev, s->amax_scratch, s->stream);
    return sampler_sample(s->sp, logits, tok_dev, s->stream);
}

// spec.rs:205-222 `chain_drafts`: drafts from..k-1, each from the previous draft and the MTP hidden row `prev`.
int chain_drafts(aq_state *s, size_t prev, size_t from) {
    for (size_t i = from; i < s->k; i++) {
        int rc = mtp_set_rows(s, s->drafts + (i - 1), s->mtp_hout + prev * s->m->cfg.hidden, 1);
        if (!rc) rc = mtp_rows(s, 1);
        if (!rc) rc = mtp_draft(s, 0, i);
        if (rc) return rc;
        prev = 0;
    }
    return 0;
}

int copy_ids_in(aq_state *s, uint32_t *dev, const uint32_t *host, size_t n) {
    for (size_t i = 0; i < n; i++)
        AQ_REQUIRE(host[i] < s->m->cfg.vocab, "token id " + std::to_string(host[i]) + " out of range");
    AQ_HIP(hipMemcpyAsync(dev, host, n * 4, hipMemcpyHostToDevice, s->stream));
    return 0;
}

int sync_in(aq_state *s, void *host, const void *dev, size_t bytes) {
    AQ_HIP(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, s->stream));
    AQ_HIP(hipStreamSynchronize(s->stream));
    return 0;
}

// Prompt rows through the main model in batches; the final-norm rows of every prompt row go to normed_all,
// the last row's logits to s->logits row 0 and its argmax to s->amax[0].
int run_prompt(aq_state *s, const uint32_t *ids, size_t n) {
    aq_model *m = s->m;
    const size_t h = m->cfg.hidden;
    AQ_REQUIRE(n >= 1, "prompt: empty");
    AQ_REQUIRE(s->pos + n + MAX_ROWS <= s->max_pos, "prompt: longer than the state's max_pos");
    int rc = copy_ids_in(s, s->prompt, ids, n);
    if (rc) return rc;
    for (size_t c0 = 0; c0 < n; c0 += PRE_ROWS) {
        const size_t tc = n - c0 < (size_t)PRE_ROWS ? n - c0 : (size_t)PRE_ROWS;
        if ((rc = forward_rows(s, s->prompt + c0, tc, PLAIN))) return rc;
        Needs nd; // final norm of every row (the MTP reads them); only the last row needs the lm_head
        nd.add(m->lm_head);
        if ((rc = norm_into(s, s->xa, h, m->output_norm, h, tc, s->act_h, 0, 0, nd, s->normed_all + c0 * h))) return rc;
        if (c0 + tc == n) {
            Act v = col_view(s->act_h, tc - 1);
            if ((rc = mm(s, m->lm_head, v, 1, s->logits))) return rc;
            if ((rc = next_token(s, s->logits, s->amax))) return rc;
        }
    }
    return 0;
}

int collect_stage_times(aq_state *s) {
    if (!s->ev_pending) return 0;
    AQ_HIP(hipEventSynchronize(s->ev[4]));
    float a = 0, b = 0, c = 0;
    AQ_HIP(hipEventElapsedTime(&a, s->ev[1], s->ev[2]));
    AQ_HIP(hipEventElapsedTime(&b, s->ev[2], s->ev[3]));
    AQ_HIP(hipEventElapsedTime(&c, s->ev[3], s->ev[4]));
    s->stats.commit_ms += a;
    s->stats.refeed_ms += b;
    s->stats.chain_ms += c;
    s->ev_pending = false;
    return 0;
}

} // namespace
} // namespace aq

using namespace aq;

extern "C" {

int aq_model_plan(const aq_model_config *cfg, int mix, uint64_t seed, aq_tensor_plan *out, size_t cap, size_t *n_out) {
    int rc = check_config(cfg);
    if (rc) return rc;
    AQ_REQUIRE(mix == AQ_MIX_Q4_K_M || mix == AQ_MIX_TINY, "aq_model_plan: unknown mix");
    AQ_REQUIRE(n_out, "aq_model_plan: null n_out");
    const std::vector<PlanEntry> plan = make_plan(*cfg, mix, seed);
    *n_out = plan.size();
    if (!out) return 0;
    AQ_REQUIRE(cap >= plan.size(), "aq_model_plan: capacity too small");
    for (size_t i = 0; i < plan.size(); i++) {
        AQ_REQUIRE(plan[i].name.size() < sizeof(out[i].name), "aq_model_plan: name too long");
        std::memset(out[i].name, 0, sizeof(out[i].name));
        std::memcpy(out[i].name, plan[i].name.data(), plan[i].name.size());
        out[i].spec = plan[i].spec;
    }
    return 0;
}

int aq_model_load(aq_ctx *ctx, const aq_model_config *cfg, const aq_tensor *tensors, size_t n, aq_model **out) {
    AQ_REQUIRE(ctx && tensors && out, "aq_model_load: null argument");
    int rc = check_config(cfg);
    if (rc) return rc;
    AQ_HIP(hipSetDevice(ctx->device));
    Source src;
    src.ts = tensors;
    src.n = n;
    src.stream = ctx->stream;
    src.device = ctx->device;
    rc = build_model(ctx, cfg, src, out);
    if (!rc) AQ_HIP(hipDeviceSynchronize()); // vectors went up on the null stream, weights on the context stream
    return rc;
}

int aq_model_synth(aq_ctx *ctx, const aq_model_config *cfg, int mix, uint64_t seed, aq_model **out) {
    AQ_REQUIRE(ctx && out, "aq_model_synth: null argument");
    int rc = check_config(cfg);
    if (rc) return rc;
    AQ_REQUIRE(mix == AQ_MIX_Q4_K_M || mix == AQ_MIX_TINY, "aq_model_synth: unknown mix");
    AQ_HIP(hipSetDevice(ctx->device));
    const std::vector<PlanEntry> plan = make_plan(*cfg, mix, seed);
    Source src;
    src.plan = &plan;
    src.stream = ctx->stream;
    src.device = ctx->device;
    rc = build_model(ctx, cfg, src, out);
    if (!rc) AQ_HIP(hipDeviceSynchronize()); // vectors went up on the null stream, weights on the context stream
    return rc;
}

int aq_model_free(aq_model *m) {
    if (m) (void)hipSetDevice(m->device);
    free_model(m);
    return 0;
}

int aq_model_get_bytes(const aq_model *m, aq_model_bytes *out) {
    AQ_REQUIRE(m && out, "aq_model_get_bytes: null argument");
    *out = m->bytes;
    return 0;
}

int aq_state_new(aq_model *m, uint32_t spec_k, uint32_t max_pos, aq_state **out) {
    AQ_REQUIRE(m && out, "aq_state_new: null argument");
    AQ_REQUIRE(spec_k <= MAX_ROWS - 1, "aq_state_new: spec_k must be <= 7");
    AQ_REQUIRE(spec_k == 0 || m->has_mtp, "aq_state_new: speculative decoding needs the MTP block");
    AQ_REQUIRE(max_pos >= 1 && max_pos <= (1u << 20), "aq_state_new: max_pos");
    AQ_HIP(hipSetDevice(m->ctx->device));
    const aq_model_config &c = m->cfg;
    aq_state *s = new aq_state();
    s->m = m;
    s->device = m->device;
    s->k = spec_k;
    s->max_pos = max_pos + MAX_ROWS; // room for a verify batch past the last committed position
    const size_t T = MAX_ROWS, TP = PRE_ROWS, h = c.hidden, nv = c.dn_n_v_heads;
    const size_t cap = s->max_pos, stride = (size_t)c.n_head_kv * c.head_dim;
    const size_t rec_len = nv * c.dn_head_dim_k * c.dn_head_dim_v, conv_len = m->cd * (c.dn_conv_kernel - 1);
    int rc = 0;
#define AQ_S(x)                                                                                               \
    do {                                                                                                      \
        if (!rc) rc = (x);                                                                                    \
    } while (0)
    if (hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) != hipSuccess) rc = fail(AQ_EHIP, "state: stream");
    for (hipEvent_t &e : s->ev)
        if (!rc && hipEventCreate(&e) != hipSuccess) rc = fail(AQ_EHIP, "state: event");
    if (!rc && hipStreamCreateWithFlags(&s->aux, hipStreamNonBlocking) != hipSuccess) rc = fail(AQ_EHIP, "state: stream");
    for (hipEvent_t *e : {&s->aux_in, &s->aux_out})
        if (!rc && hipEventCreateWithFlags(e, hipEventDisableTiming) != hipSuccess) rc = fail(AQ_EHIP, "state: event");
    s->rec.assign(c.n_layer, nullptr);
    s->conv0.assign(c.n_layer, nullptr);
    s->conv1.assign(c.n_layer, nullptr);
    s->kv.assign(c.n_layer, KvDev());
    int n_dn = 0;
    for (uint32_t i = 0; i < c.n_layer && !rc; i++) {
        if (m->layers[i].attention) {
            s->kv[i].cap = cap;
            s->kv[i].stride = stride;
            AQ_S(dalloc_t(s, cap * stride, &s->kv[i].k));
            AQ_S(dalloc_t(s, cap * stride, &s->kv[i].v));
        } else {
            n_dn++;
        }
    }
    // DeltaNet state indexed by DeltaNet slot
    s->rec.assign(n_dn, nullptr);
    s->conv0.assign(n_dn, nullptr);
    s->conv1.assign(n_dn, nullptr);
    s->sv_mixed.assign(n_dn, nullptr);
    s->sv_a.assign(n_dn, nullptr);
    s->sv_b.assign(n_dn, nullptr);
    for (int i = 0; i < n_dn && !rc; i++) {
        AQ_S(dalloc_t(s, rec_len, &s->rec[i]));
        AQ_S(dalloc_t(s, conv_len, &s->conv0[i]));
        AQ_S(dalloc_t(s, conv_len, &s->conv1[i]));
        if (spec_k > 0) {
            AQ_S(dalloc_t(s, T * m->cd, &s->sv_mixed[i]));
            AQ_S(dalloc_t(s, T * nv, &s->sv_a[i]));
            AQ_S(dalloc_t(s, T * nv, &s->sv_b[i]));
        }
    }
    // score rows in device memory when a context can outgrow the attention kernel's LDS (the MTP's cache is the
    // longest: cap + T rows)
    if (cap + 2 * T > attn_lds_positions((int)c.head_dim)) {
        s->attn_sc_stride = cap + 2 * T;
        AQ_S(dalloc_t(s, T * c.n_head * s->attn_sc_stride, &s->attn_sc));
    }
    if (m->has_mtp) {
        s->mtp_kv.cap = cap + T;
        s->mtp_kv.stride = stride;
        AQ_S(dalloc_t(s, s->mtp_kv.cap * stride, &s->mtp_kv.k));
        AQ_S(dalloc_t(s, s->mtp_kv.cap * stride, &s->mtp_kv.v));
    }
    AQ_S(alloc_act(s->act_h, h, TP, m->ctx->device));
    AQ_S(alloc_act(s->act_ffn, c.ffn, TP, m->ctx->device));
    AQ_S(alloc_act(s->act_vd, m->vd, TP, m->ctx->device));
    AQ_S(alloc_act(s->act_att, (size_t)c.n_head * c.head_dim, TP, m->ctx->device));
    AQ_S(alloc_act(s->act_cat, 2 * h, T, m->ctx->device));
    AQ_S(dalloc_t(s, TP * h, &s->xa));
    AQ_S(dalloc_t(s, TP * h, &s->xb));
    AQ_S(dalloc_t(s, TP * h, &s->y));
    AQ_S(dalloc_t(s, T * h, &s->e));
    AQ_S(dalloc_t(s, TP * m->cd, &s->mixed));
    AQ_S(dalloc_t(s, TP * m->vd, &s->z));
    AQ_S(dalloc_t(s, TP * nv, &s->a));
    AQ_S(dalloc_t(s, TP * nv, &s->b));
    AQ_S(dalloc_t(s, TP * 2 * c.n_head * c.head_dim, &s->qg));
    AQ_S(dalloc_t(s, TP * stride, &s->kk));
    AQ_S(dalloc_t(s, TP * stride, &s->vv));
    AQ_S(dalloc_t(s, TP * c.n_head * c.head_dim, &s->qr));
    AQ_S(dalloc_t(s, TP * c.ffn, &s->g));
    AQ_S(dalloc_t(s, TP * c.ffn, &s->u));
    AQ_S(dalloc_t(s, T * c.vocab, &s->logits));
    AQ_S(dalloc_t(s, T * h, &s->normed));
    AQ_S(dalloc_t(s, (size_t)s->max_pos * h, &s->normed_all));
    AQ_S(dalloc_t(s, T * h, &s->mtp_hout));
    AQ_S(dalloc_t(s, T, &s->ids));
    AQ_S(dalloc_t(s, T, &s->amax));
    AQ_S(dalloc_t(s, T, &s->drafts));
    // the round's result: info[0..3) and the emitted ids at info[16..), laid out as in `pinned`, so one
    // device-to-host copy carries both
    AQ_S(dalloc_t(s, 16 + T, &s->info));
    s->emitted = s->info + 16;
    if (spec_k > 0) {
        AQ_S(dalloc_t(s, (size_t)spec_k * c.vocab, &s->q_dense));
        AQ_S(dalloc_t(s, (size_t)spec_k * c.vocab, &s->q_idx));
        AQ_S(dalloc_t(s, (size_t)spec_k, &s->q_n));
    }
    AQ_S(dalloc_t(s, s->max_pos, &s->prompt));
    AQ_S(dalloc_t(s, s->max_pos, &s->shifted));
    AQ_S(dalloc(s, argmax_scratch_bytes(c.vocab, T), &s->amax_scratch));
    // rope.rs:15-28 cos/sin per position, computed on the host as the reference does
    const size_t half = c.rope_dim / 2, npos = (size_t)s->max_pos + 2 * T;
    if (!rc) {
        std::vector<float> ct(npos * half), st(npos * half);
        for (size_t p = 0; p < npos; p++) {
            const float pf = (float)p;
            for (size_t i = 0; i < half; i++) {
                const float angle = pf * m->inv_freq[i];
                ct[p * half + i] = cosf(angle);
                st[p * half + i] = sinf(angle);
            }
        }
        AQ_S(dalloc_t(s, npos * half, &s->cos_tab));
        AQ_S(dalloc_t(s, npos * half, &s->sin_tab));
        if (!rc && hipMemcpy(s->cos_tab, ct.data(), npos * half * 4, hipMemcpyHostToDevice) != hipSuccess)
            rc = fail(AQ_EHIP, "state: rope table");
        if (!rc && hipMemcpy(s->sin_tab, st.data(), npos * half * 4, hipMemcpyHostToDevice) != hipSuccess)
            rc = fail(AQ_EHIP, "state: rope table");
    }
    if (!rc && pinned_malloc((void **)&s->pinned, 64 * 4) != hipSuccess)
        rc = fail(AQ_ENOMEM, "state: pinned");
    // the commit of a speculative round, one launch for every DeltaNet layer: the kept-row count is info[2]
    s->n_dn = n_dn;
    if (!rc && spec_k > 0 && n_dn > 0) {
        std::vector<DnArgs> ca(2 * (size_t)n_dn);
        int dn = 0;
        for (uint32_t li = 0; li < c.n_layer; li++) {
            const DevLayer &L = m->layers[li];
            if (L.attention) continue;
            for (int par = 0; par < 2; par++) {
                DnArgs &d = ca[(size_t)par * n_dn + dn];
                d.mixed = s->sv_mixed[dn];
                d.a = s->sv_a[dn];
                d.b = s->sv_b[dn];
                d.conv_src = par ? s->conv1[dn] : s->conv0[dn];
                d.conv_dst = par ? s->conv0[dn] : s->conv1[dn];
                d.conv_w = L.conv_w;
                d.ssm_a = L.ssm_a;
                d.dt_bias = L.dt_bias;
                d.ssm_norm = L.ssm_norm;
                d.eps = c.rms_eps;
                d.qscale = m->qscale;
                d.rec = s->rec[dn];
                d.write_state = 1;
                d.t = 1;
                d.t_dev = s->info + 2;
                d.nk = (int)c.dn_n_k_heads;
                d.nv = (int)c.dn_n_v_heads;
                d.dk = (int)c.dn_head_dim_k;
                d.dv = (int)c.dn_head_dim_v;
                d.kernel = (int)c.dn_conv_kernel;
            }
            dn++;
        }
        AQ_S(dalloc(s, ca.size() * sizeof(DnArgs), (void **)&s->commit_args));
        if (!rc && hipMemcpy(s->commit_args, ca.data(), ca.size() * sizeof(DnArgs), hipMemcpyHostToDevice) != hipSuccess)
            rc = fail(AQ_EHIP, "state: commit arguments");
    }
    // The clears and table uploads above ran on the null stream, which the state's non-blocking stream does not
    // wait for: finish them before the first kernel on that stream can read the buffers.
    if (!rc && hipDeviceSynchronize() != hipSuccess) rc = fail(AQ_EHIP, "state: setup sync");
#undef AQ_S
    if (rc) {
        free_state(s);
        return rc;
    }
    *out = s;
    return 0;
}

int aq_state_free(aq_state *s) {
    if (s) (void)hipSetDevice(s->device);
    free_state(s);
    return 0;
}

int aq_prefill(aq_state *s, const uint32_t *ids, size_t n, float *logits_last_host, uint32_t *argmax_out) {
    AQ_REQUIRE(s && ids, "aq_prefill: null argument");
    AQ_HIP(hipSetDevice(s->m->ctx->device));
    s->spec_ready = false; // the MTP is not fed: a round needs aq_spec_prefill again (spec.rs:337)
    int rc = run_prompt(s, ids, n);
    if (rc) return rc;
    if (logits_last_host) {
        AQ_HIP(hipMemcpyAsync(logits_last_host, s->logits, s->m->cfg.vocab * 4, hipMemcpyDeviceToHost, s->stream));
    }
    rc = sync_in(s, s->pinned, s->amax, 4);
    if (!rc && argmax_out) *argmax_out = s->pinned[0];
    return rc;
}

int aq_forward_token(aq_state *s, uint32_t id, float *logits_host, uint32_t *argmax_out) {
    AQ_REQUIRE(s, "aq_forward_token: null state");
    AQ_REQUIRE(s->pos + 1 + MAX_ROWS <= s->max_pos, "aq_forward_token: position past max_pos");
    AQ_HIP(hipSetDevice(s->m->ctx->device));
    const size_t vocab = s->m->cfg.vocab;
    s->spec_ready = false; // as in aq_prefill
    s->pinned[8] = id;
    int rc = copy_ids_in(s, s->ids, s->pinned + 8, 1);
    if (!rc) rc = forward_rows(s, s->ids, 1, PLAIN);
    if (!rc) rc = head_rows(s, s->xa, 1, s->normed);
    if (!rc) rc = next_token(s, s->logits, s->amax);
    if (rc) return rc;
    if (logits_host) AQ_HIP(hipMemcpyAsync(logits_host, s->logits, vocab * 4, hipMemcpyDeviceToHost, s->stream));
    rc = sync_in(s, s->pinned, s->amax, 4);
    if (!rc && argmax_out) *argmax_out = s->pinned[0];
    return rc;
}

int aq_spec_prefill(aq_state *s, const uint32_t *ids, size_t n, uint32_t *x_t) {
    AQ_REQUIRE(s && ids && x_t, "aq_spec_prefill: null argument");
    AQ_REQUIRE(s->k > 0, "aq_spec_prefill: state has no speculative buffers (spec_k = 0)");
    AQ_HIP(hipSetDevice(s->m->ctx->device));
    aq_model *m = s->m;
    const size_t h = m->cfg.hidden;
    const uint32_t p = s->pos;
    // spec.rs:246: the MTP holds a row for every consumed position (plus the last round's draft rows); a state
    // whose plain calls ran past them cannot be fed at the right positions
    if (s->mtp_kv.len < p)
        return fail(AQ_ESTATE, "aq_spec_prefill: the MTP has " + std::to_string(s->mtp_kv.len) + " rows for " +
                                   std::to_string(p) + " consumed positions");
    s->spec_ready = false;
    int rc = run_prompt(s, ids, n);
    if (rc) return rc;
    // the MTP over the prompt: row j = (x_{j+1}, h_j), the last row's token is x_T (spec.rs:243-265); the draft
    // rows of a used state's last round are forgotten
    s->mtp_kv.len = p;
    if (n > 1) AQ_HIP(hipMemcpyAsync(s->shifted, s->prompt + 1, (n - 1) * 4, hipMemcpyDeviceToDevice, s->stream));
    AQ_HIP(hipMemcpyAsync(s->shifted + (n - 1), s->amax, 4, hipMemcpyDeviceToDevice, s->stream));
    size_t last = 0;
    for (size_t c0 = 0; c0 < n; c0 += MAX_ROWS) {
        const size_t tc = n - c0 < (size_t)MAX_ROWS ? n - c0 : (size_t)MAX_ROWS;
        AQ_REQUIRE(s->mtp_kv.len + tc <= s->mtp_kv.cap, "aq_spec_prefill: MTP cache full");
        if ((rc = mtp_set_rows(s, s->shifted + c0, s->normed_all + c0 * h, tc))) return rc;
        if ((rc = mtp_rows(s, tc))) return rc;
        last = tc - 1;
    }
    if ((rc = mtp_draft(s, last, 0))) return rc;
    if ((rc = chain_drafts(s, last, 1))) return rc;
    rc = sync_in(s, s->pinned, s->amax, 4);
    if (rc) return rc;
    *x_t = s->pinned[0];
    s->spec_ready = true;
    return 0;
}

int aq_spec_round(aq_state *s, uint32_t x_p, uint32_t *emitted, uint32_t *n_emitted, uint32_t *m_out) {
    AQ_REQUIRE(s && emitted && n_emitted, "aq_spec_round: null argument");
    if (!s->spec_ready) return fail(AQ_ESTATE, "aq_spec_round: call aq_spec_prefill first");
    aq_model *m = s->m;
    AQ_REQUIRE(x_p < m->cfg.vocab, "aq_spec_round: x_p out of range");
    const size_t k = s->k, t = k + 1, h = m->cfg.hidden, vocab = m->cfg.vocab;
    // spec.rs:337: the MTP holds the consumed positions plus the k - 1 chained draft rows
    if (s->mtp_kv.len != s->pos + k - 1)
        return fail(AQ_ESTATE, "aq_spec_round: the MTP has " + std::to_string(s->mtp_kv.len) + " rows at position " +
                                   std::to_string(s->pos) + " (k " + std::to_string(k) + ")");
    AQ_REQUIRE(s->pos + t + MAX_ROWS <= s->max_pos, "aq_spec_round: position past max_pos");
    AQ_HIP(hipSetDevice(m->ctx->device));
    int rc = collect_stage_times(s);
    if (rc) return rc;
    const uint32_t p = s->pos;
    AQ_HIP(hipEventRecord(s->ev[0], s->stream));
    // verify (spec.rs:277-314): DeltaNet state read-only, inputs kept for the commit
    if ((rc = launch_make_batch(x_p, s->drafts, (int)k, s->ids, s->stream))) return rc;
    if ((rc = forward_rows(s, s->ids, t, VERIFY))) return rc;
    if ((rc = head_rows(s, s->xa, t, s->normed))) return rc;
    if (sampler_greedy(s->sp)) { // accept on the device (spec.rs:355-366)
        if ((rc = launch_argmax(s->logits, vocab, vocab, t, s->amax, s->amax_scratch, s->stream))) return rc;
        if ((rc = launch_accept(s->amax, s->drafts, (int)k, s->emitted, s->info, s->stream))) return rc;
    } else { // the rejection-sampling rule (spec.rs:367-380)
        if ((rc = sampler_round(s->sp, s->logits, (int)k, s->drafts, s->q_dense, s->emitted, s->info, s->stream)))
            return rc;
    }
    AQ_HIP(hipMemcpyAsync(s->pinned, s->info, (16 + t) * 4, hipMemcpyDeviceToHost, s->stream));
    AQ_HIP(hipEventRecord(s->ev[1], s->stream));
    // commit (replaces spec.rs:396-415's restore + replay): every DeltaNet layer's state advances by the kept rows
    // (info[2], read on the device) from the saved inputs, in one launch that runs while the host reads keep
    if (s->n_dn > 0) {
        DnArgs like;
        like.nk = (int)m->cfg.dn_n_k_heads;
        like.nv = (int)m->cfg.dn_n_v_heads;
        like.dk = (int)m->cfg.dn_head_dim_k;
        like.dv = (int)m->cfg.dn_head_dim_v;
        if ((rc = launch_dn_core_multi(s->commit_args + (size_t)s->par * s->n_dn, like, s->n_dn, s->stream)))
            return rc;
    }
    AQ_HIP(hipEventSynchronize(s->ev[1]));
    const uint32_t mm_ = s->pinned[0], ne = s->pinned[1], keep = s->pinned[2];
    AQ_REQUIRE(keep >= 1 && keep <= t && ne == keep, "aq_spec_round: inconsistent acceptance");
    // the KV caches forget the rejected rows
    for (uint32_t li = 0; li < m->cfg.n_layer; li++)
        if (m->layers[li].attention) s->kv[li].len = p + keep;
    s->par ^= 1;
    s->pos = p + keep;
    AQ_HIP(hipEventRecord(s->ev[2], s->stream));
    // the MTP: forget its draft rows, feed the accepted pairs, draft the next round (spec.rs:417-431)
    s->mtp_kv.len = p;
    if ((rc = mtp_set_rows(s, s->emitted, s->normed, keep))) return rc;
    if ((rc = mtp_rows(s, keep))) return rc;
    if ((rc = mtp_draft(s, keep - 1, 0))) return rc;
    AQ_HIP(hipEventRecord(s->ev[3], s->stream));
    if ((rc = chain_drafts(s, keep - 1, 1))) return rc;
    AQ_HIP(hipEventRecord(s->ev[4], s->stream));
    s->ev_pending = true;
    float vms = 0.0f;
    AQ_HIP(hipEventElapsedTime(&vms, s->ev[0], s->ev[1]));
    for (uint32_t i = 0; i < ne; i++) emitted[i] = s->pinned[16 + i];
    *n_emitted = ne;
    if (m_out) *m_out = mm_;
    s->stats.rounds++;
    s->stats.drafted += k;
    s->stats.accepted += mm_;
    s->stats.emitted += ne;
    if (mm_ <= 16) s->stats.hist[mm_]++;
    s->stats.verify_ms += vms;
    (void)h;
    return 0;
}

// ---------------------------------------------------------------------------------------- sampled calls
// The calls above with a sampler in place of argmax: the token after the prompt / after a forward is
// Sampler::sample of its logits (run.rs's sampled loop), drafts are drawn from the MTP's processed distribution, and
// a round accepts by the rejection-sampling rule (spec.rs:192-203, 241, 367-380). A greedy sampler (temperature <= 0)
// gives the greedy calls exactly, drawing nothing.
namespace {
struct SamplerScope {
    aq_state *s;
    SamplerScope(aq_state *st, aq_sampler *sp) : s(st) { s->sp = sp; }
    ~SamplerScope() { s->sp = nullptr; }
};
int check_sampler(aq_state *s, aq_sampler *sp, const char *fn) {
    AQ_REQUIRE(s && sp, std::string(fn) + ": null argument");
    AQ_REQUIRE(sampler_vocab(sp) == s->m->cfg.vocab, std::string(fn) + ": sampler vocabulary != model vocabulary");
    AQ_REQUIRE(sampler_device(sp) == s->device, std::string(fn) + ": sampler and state on different devices");
    return 0;
}
} // namespace

int aq_prefill_sampled(aq_state *s, aq_sampler *sp, const uint32_t *ids, size_t n, float *logits_last_host,
                       uint32_t *next) {
    int rc = check_sampler(s, sp, "aq_prefill_sampled");
    if (rc) return rc;
    SamplerScope g(s, sp);
    return aq_prefill(s, ids, n, logits_last_host, next);
}

int aq_forward_token_sampled(aq_state *s, aq_sampler *sp, uint32_t id, float *logits_host, uint32_t *next) {
    int rc = check_sampler(s, sp, "aq_forward_token_sampled");
    if (rc) return rc;
    SamplerScope g(s, sp);
    return aq_forward_token(s, id, logits_host, next);
}

int aq_spec_prefill_sampled(aq_state *s, aq_sampler *sp, const uint32_t *ids, size_t n, uint32_t *x_t) {
    int rc = check_sampler(s, sp, "aq_spec_prefill_sampled");
    if (rc) return rc;
    SamplerScope g(s, sp);
    return aq_spec_prefill(s, ids, n, x_t);
}

int aq_spec_round_sampled(aq_state *s, aq_sampler *sp, uint32_t x_p, uint32_t *emitted, uint32_t *n_emitted,
                          uint32_t *m_out) {
    int rc = check_sampler(s, sp, "aq_spec_round_sampled");
    if (rc) return rc;
    SamplerScope g(s, sp);
    return aq_spec_round(s, x_p, emitted, n_emitted, m_out);
}

int aq_spec_set_drafts(aq_state *s, const uint32_t *d, size_t k) {
    AQ_REQUIRE(s && d, "aq_spec_set_drafts: null argument");
    AQ_REQUIRE(k <= s->k, "aq_spec_set_drafts: more drafts than spec_k");
    if (k == 0) return 0;
    int rc = copy_ids_in(s, s->drafts, d, k);
    if (!rc) AQ_HIP(hipStreamSynchronize(s->stream));
    return rc;
}

int aq_spec_get_drafts(aq_state *s, uint32_t *d, size_t k) {
    AQ_REQUIRE(s && d, "aq_spec_get_drafts: null argument");
    AQ_REQUIRE(k <= s->k, "aq_spec_get_drafts: more drafts than spec_k");
    if (k == 0) return 0;
    int rc = sync_in(s, s->pinned, s->drafts, k * 4);
    if (!rc) std::memcpy(d, s->pinned, k * 4);
    return rc;
}

int aq_spec_logits_row(aq_state *s, size_t i, float *host_out) {
    AQ_REQUIRE(s && host_out, "aq_spec_logits_row: null argument");
    AQ_REQUIRE(i <= s->k, "aq_spec_logits_row: row out of range");
    const size_t vocab = s->m->cfg.vocab;
    AQ_HIP(hipMemcpyAsync(host_out, s->logits + i * vocab, vocab * 4, hipMemcpyDeviceToHost, s->stream));
    AQ_HIP(hipStreamSynchronize(s->stream));
    return 0;
}

int aq_spec_get_stats(aq_state *s, aq_spec_stats *out) {
    AQ_REQUIRE(s && out, "aq_spec_get_stats: null argument");
    int rc = collect_stage_times(s);
    if (rc) return rc;
    *out = s->stats;
    return 0;
}

int aq_state_pos(const aq_state *s, uint32_t *pos) {
    AQ_REQUIRE(s && pos, "aq_state_pos: null argument");
    *pos = s->pos;
    return 0;
}

int aq_state_export(aq_state *s, float *out, size_t cap, size_t *n_out) {
    AQ_REQUIRE(s && n_out, "aq_state_export: null argument");
    aq_model *m = s->m;
    const aq_model_config &c = m->cfg;
    const size_t rec_len = (size_t)c.dn_n_v_heads * c.dn_head_dim_k * c.dn_head_dim_v,
                 conv_len = m->cd * (c.dn_conv_kernel - 1);
    size_t total = 0;
    std::vector<std::pair<const float *, size_t>> parts;
    int dn = 0;
    for (uint32_t i = 0; i < c.n_layer; i++) {
        if (m->layers[i].attention) {
            parts.push_back({s->kv[i].k, s->kv[i].len * s->kv[i].stride});
            parts.push_back({s->kv[i].v, s->kv[i].len * s->kv[i].stride});
        } else {
            parts.push_back({s->rec[dn], rec_len});
            parts.push_back({s->par ? s->conv1[dn] : s->conv0[dn], conv_len});
            dn++;
        }
    }
    if (s->k > 0) {
        parts.push_back({s->mtp_kv.k, s->mtp_kv.len * s->mtp_kv.stride});
        parts.push_back({s->mtp_kv.v, s->mtp_kv.len * s->mtp_kv.stride});
    }
    for (auto &pr : parts) total += pr.second;
    *n_out = total;
    if (!out) return 0;
    AQ_REQUIRE(cap >= total, "aq_state_export: capacity too small");
    AQ_HIP(hipSetDevice(m->ctx->device));
    size_t off = 0;
    for (auto &pr : parts) {
        if (pr.second) AQ_HIP(hipMemcpyAsync(out + off, pr.first, pr.second * 4, hipMemcpyDeviceToHost, s->stream));
        off += pr.second;
    }
    AQ_HIP(hipStreamSynchronize(s->stream));
    return 0;
}

int aq_layer_run(aq_ctx *ctx, const aq_model_config *cfg, const aq_tensor *tensors, size_t n, int kind, const float *x,
                 size_t t, uint32_t start_pos, float *conv, float *rec, float *k_cache, float *v_cache,
                 uint32_t *kv_len, uint32_t kv_cap, float *y) {
    AQ_REQUIRE(ctx && cfg && tensors && x && y, "aq_layer_run: null argument");
    AQ_REQUIRE(kind >= 0 && kind <= 4, "aq_layer_run: kind must be 0..4");
    AQ_REQUIRE(t >= 1 && t <= (size_t)MAX_ROWS, "aq_layer_run: 1..8 rows");
    AQ_REQUIRE(cfg->hidden % 32 == 0 && cfg->dn_conv_kernel == 4, "aq_layer_run: config");
    const bool attention = kind == 1 || kind == 4;
    const bool dn = kind == 0 || kind == 3;
    AQ_REQUIRE(!dn || (conv && rec), "aq_layer_run: DeltaNet needs conv and rec");
    AQ_REQUIRE(!attention || (k_cache && v_cache && kv_len && *kv_len + t <= kv_cap), "aq_layer_run: KV cache");
    AQ_HIP(hipSetDevice(ctx->device));
    aq_model *m = new aq_model();
    m->ctx = ctx;
    m->device = ctx->device;
    m->cfg = *cfg;
    m->cfg.n_layer = 0;
    m->cfg.has_mtp = 0;
    m->kd = (size_t)cfg->dn_n_k_heads * cfg->dn_head_dim_k;
    m->vd = (size_t)cfg->dn_n_v_heads * cfg->dn_head_dim_v;
    m->cd = 2 * m->kd + m->vd;
    m->inv_freq.resize(cfg->rope_dim / 2);
    for (size_t i = 0; i < m->inv_freq.size(); i++)
        m->inv_freq[i] = 1.0f / powf(cfg->rope_theta, (float)(2 * i) / (float)cfg->rope_dim);
    m->qscale = 1.0f / sqrtf((float)cfg->dn_head_dim_k);
    m->attn_scaling = powf((float)cfg->head_dim, -0.5f);
    // the pieces this kind needs, named blk.0.*
    Source src;
    src.ts = tensors;
    src.n = n;
    src.stream = ctx->stream;
    src.device = ctx->device;
    DevLayer L;
    L.attention = attention;
    const size_t h = cfg->hidden;
    int rc = 0;
    if (kind >= 3) {
        rc = src.vec(m, "blk.0.attn_norm.weight", h, L.attn_norm);
        if (!rc) rc = src.vec(m, "blk.0.post_attention_norm.weight", h, L.post_norm);
    }
    if (!rc && kind >= 2) {
        rc = src.mat(m, "blk.0.ffn_gate.weight", cfg->ffn, h, L.gate);
        if (!rc) rc = src.mat(m, "blk.0.ffn_up.weight", cfg->ffn, h, L.up);
        if (!rc) rc = src.mat(m, "blk.0.ffn_down.weight", h, cfg->ffn, L.down);
    }
    if (!rc && attention) {
        const size_t nh = cfg->n_head, nkv = cfg->n_head_kv, hd = cfg->head_dim;
        rc = src.mat(m, "blk.0.attn_q.weight", 2 * nh * hd, h, L.q);
        if (!rc) rc = src.mat(m, "blk.0.attn_k.weight", nkv * hd, h, L.k);
        if (!rc) rc = src.mat(m, "blk.0.attn_v.weight", nkv * hd, h, L.v);
        if (!rc) rc = src.mat(m, "blk.0.attn_output.weight", h, nh * hd, L.o);
        if (!rc) rc = src.vec(m, "blk.0.attn_q_norm.weight", hd, L.q_norm);
        if (!rc) rc = src.vec(m, "blk.0.attn_k_norm.weight", hd, L.k_norm);
    }
    if (!rc && dn) {
        const size_t nv = cfg->dn_n_v_heads;
        rc = src.mat(m, "blk.0.attn_qkv.weight", m->cd, h, L.qkv);
        if (!rc) rc = src.mat(m, "blk.0.attn_gate.weight", m->vd, h, L.gate_z);
        if (!rc) rc = src.mat(m, "blk.0.ssm_alpha.weight", nv, h, L.alpha);
        if (!rc) rc = src.mat(m, "blk.0.ssm_beta.weight", nv, h, L.beta);
        if (!rc) rc = src.mat(m, "blk.0.ssm_out.weight", h, m->vd, L.ssm_out);
        if (!rc) rc = src.vec(m, "blk.0.ssm_a", nv, L.ssm_a);
        if (!rc) rc = src.vec(m, "blk.0.ssm_dt.bias", nv, L.dt_bias);
        if (!rc) rc = src.vec(m, "blk.0.ssm_conv1d.weight", m->cd * cfg->dn_conv_kernel, L.conv_w);
        if (!rc) rc = src.vec(m, "blk.0.ssm_norm.weight", cfg->dn_head_dim_v, L.ssm_norm);
    }
    if (rc) {
        free_model(m);
        return rc;
    }
    // a one-layer state: the model's layer list holds this layer so aq_state_new sizes the buffers
    m->cfg.n_layer = 1;
    m->cfg.full_attention_interval = attention ? 1 : 1000000;
    m->layers.push_back(L);
    aq_state *s = nullptr;
    const uint32_t cap = kv_cap > start_pos + (uint32_t)t ? kv_cap : start_pos + (uint32_t)t;
    rc = aq_state_new(m, 0, cap, &s);
    if (rc) {
        m->layers.clear();
        free_model(m);
        return rc;
    }
    const aq_model_config &c = *cfg;
    const size_t rec_len = (size_t)c.dn_n_v_heads * c.dn_head_dim_k * c.dn_head_dim_v, conv_len = m->cd * 3;
    const size_t stride = (size_t)c.n_head_kv * c.head_dim;
    auto h2d = [&](void *d, const void *hs, size_t bytes) -> int {
        AQ_HIP(hipMemcpyAsync(d, hs, bytes, hipMemcpyHostToDevice, s->stream));
        AQ_HIP(hipStreamSynchronize(s->stream));
        return 0;
    };
    auto d2h = [&](void *hs, const void *d, size_t bytes) -> int {
        AQ_HIP(hipMemcpyAsync(hs, d, bytes, hipMemcpyDeviceToHost, s->stream));
        AQ_HIP(hipStreamSynchronize(s->stream));
        return 0;
    };
    if (!rc) rc = h2d(s->xa, x, t * h * 4);
    if (!rc && dn) {
        rc = h2d(s->rec[0], rec, rec_len * 4);
        if (!rc) rc = h2d(s->conv0[0], conv, conv_len * 4);
    }
    if (!rc && attention) {
        s->kv[0].len = *kv_len;
        if (*kv_len) {
            rc = h2d(s->kv[0].k, k_cache, (size_t)*kv_len * stride * 4);
            if (!rc) rc = h2d(s->kv[0].v, v_cache, (size_t)*kv_len * stride * 4);
        }
    }
    if (!rc) {
        s->pos = start_pos;
        if (kind >= 3) {
            rc = decoder_layer(s, L, s->xa, t, start_pos, &s->kv[0], dn ? 0 : -1, PLAIN, s->xb);
        } else {
            // a mixer or the MLP alone reads x as given (no norm) and adds no residual
            AQ_HIP(hipMemcpyAsync(s->act_h.f32, s->xa, t * h * 4, hipMemcpyDeviceToDevice, s->stream));
            rc = quantize_act(s, s->act_h, t, kind == 2 ? mlp_needs(L) : mixer_needs(L));
            if (!rc) rc = kind == 2 ? mlp(s, L, t, s->xb, nullptr)
                                    : mixer(s, L, t, start_pos, &s->kv[0], dn ? 0 : -1, PLAIN, s->xb, nullptr);
        }
        if (dn) s->par = 1; // the new conv window is in the second buffer
    }
    if (!rc) rc = hipStreamSynchronize(s->stream) == hipSuccess ? 0 : fail(AQ_EHIP, "aq_layer_run: sync");
    if (!rc) rc = d2h(y, s->xb, t * h * 4);
    if (!rc && dn) {
        rc = d2h(rec, s->rec[0], rec_len * 4);
        if (!rc) rc = d2h(conv, s->par ? s->conv1[0] : s->conv0[0], conv_len * 4);
    }
    if (!rc && attention) {
        *kv_len = (uint32_t)s->kv[0].len;
        rc = d2h(k_cache, s->kv[0].k, (size_t)*kv_len * stride * 4);
        if (!rc) rc = d2h(v_cache, s->kv[0].v, (size_t)*kv_len * stride * 4);
    }
    free_state(s);
    m->layers.clear();
    free_model(m);
    return rc;
}

int aq_eval_math(aq_ctx *ctx, int fn, const float *x, float *y, size_t n) {
    AQ_REQUIRE(ctx && x && y, "aq_eval_math: null argument");
    AQ_HIP(hipSetDevice(ctx->device));
    float *d = nullptr;
    if (dev_malloc(&d, 2 * n * 4 + 256) != hipSuccess) return fail(AQ_ENOMEM, "aq_eval_math: buffer");
    int rc = hipMemcpyAsync(d, x, n * 4, hipMemcpyHostToDevice, ctx->stream) == hipSuccess ? 0 : fail(AQ_EHIP, "upload");
    if (!rc) rc = launch_eval_math(fn, d, d + n, n, ctx->stream);
    if (!rc && hipMemcpyAsync(y, d + n, n * 4, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess)
        rc = fail(AQ_EHIP, "aq_eval_math: download");
    if (hipStreamSynchronize(ctx->stream) != hipSuccess && !rc) rc = fail(AQ_EHIP, "aq_eval_math: sync");
    (void)hipFree(d);
    return rc;
}

int aq_deltanet_verify_commit_dev(aq_ctx *ctx, uint32_t nk, uint32_t nv, uint32_t dk, uint32_t dv, size_t t,
                                  size_t keep, const float *q_dev, const float *k_dev, const float *v_dev,
                                  const float *g_dev, const float *beta_dev, float *state_dev, float *out_dev) {
    AQ_REQUIRE(ctx && q_dev && k_dev && v_dev && g_dev && beta_dev && state_dev && out_dev,
               "aq_deltanet_verify_commit: null argument");
    AQ_REQUIRE(t >= 1 && t <= 8 && keep <= t, "aq_deltanet_verify_commit: 1 <= t <= 8 (one verify batch), keep <= t");
    AQ_REQUIRE(nk >= 1 && nv % nk == 0, "aq_deltanet_verify_commit: heads");
    AQ_HIP(hipSetDevice(ctx->device));
    DnArgs d;
    d.raw = 1;
    d.rq = q_dev;
    d.rk = k_dev;
    d.rv = v_dev;
    d.rg = g_dev;
    d.rbeta = beta_dev;
    d.rec = state_dev;
    d.nk = (int)nk;
    d.nv = (int)nv;
    d.dk = (int)dk;
    d.dv = (int)dv;
    // verify: every row's output from the committed state, the state untouched
    d.t = (int)t;
    d.write_state = 0;
    d.out = out_dev;
    int rc = launch_dn_core(d, ctx->stream);
    // commit: the kept rows again, state written (the outputs of the kept rows are recomputed identically)
    if (!rc && keep > 0) {
        d.t = (int)keep;
        d.write_state = 1;
        d.out = nullptr;
        rc = launch_dn_core(d, ctx->stream);
    }
    if (hipStreamSynchronize(ctx->stream) != hipSuccess && !rc) rc = fail(AQ_EHIP, "deltanet: sync");
    return rc;
}

int aq_deltanet_verify_commit(aq_ctx *ctx, uint32_t nk, uint32_t nv, uint32_t dk, uint32_t dv, size_t t, size_t keep,
                              const float *q, const float *k, const float *v, const float *g, const float *beta,
                              float *state_dev, float *out) {
    AQ_REQUIRE(ctx && q && k && v && g && beta && state_dev && out, "aq_deltanet_verify_commit: null argument");
    AQ_REQUIRE(t >= 1 && t <= 8 && keep <= t, "aq_deltanet_verify_commit: 1 <= t <= 8 (one verify batch), keep <= t");
    AQ_HIP(hipSetDevice(ctx->device));
    const size_t kd = (size_t)nk * dk, vd = (size_t)nv * dv;
    const size_t bytes[5] = {t * kd * 4, t * kd * 4, t * vd * 4, t * nv * 4, t * nv * 4};
    const float *hosts[5] = {q, k, v, g, beta};
    float *dev[6] = {};
    int rc = 0;
    for (int i = 0; i < 5 && !rc; i++) {
        if (dev_malloc(&dev[i], bytes[i] + 256) != hipSuccess) rc = fail(AQ_ENOMEM, "deltanet: inputs");
        if (!rc && hipMemcpyAsync(dev[i], hosts[i], bytes[i], hipMemcpyHostToDevice, ctx->stream) != hipSuccess)
            rc = fail(AQ_EHIP, "deltanet: upload");
    }
    if (!rc && dev_malloc(&dev[5], t * vd * 4 + 256) != hipSuccess) rc = fail(AQ_ENOMEM, "deltanet: output");
    if (!rc) rc = aq_deltanet_verify_commit_dev(ctx, nk, nv, dk, dv, t, keep, dev[0], dev[1], dev[2], dev[3], dev[4],
                                                state_dev, dev[5]);
    if (!rc && hipMemcpy(out, dev[5], t * vd * 4, hipMemcpyDeviceToHost) != hipSuccess)
        rc = fail(AQ_EHIP, "deltanet: download");
    (void)hipStreamSynchronize(ctx->stream);
    for (float *p : dev)
        if (p) (void)hipFree(p);
    return rc;
}

} // extern "C"
