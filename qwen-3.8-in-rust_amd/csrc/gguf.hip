// gguf.hip — GGUF v3 files on the host: the reader (header, metadata, tensor index; tensor data mapped, not read),
// the model contract derived from the metadata, a loader that puts a file's model in HBM, and a writer for the
// synthetic models. Host code only.
//
// Format (GGUF v3, the reference's gguf.rs:1-21 and 483-608): magic "GGUF", u32 version 3, u64 tensor count, u64
// metadata count; each metadata entry a string key, a u32 value type and the value (strings are a u64 length and
// the bytes; arrays a u32 element type, a u64 count and the elements); each tensor info a string name, u32 n_dims,
// u64 dims (ne[0] innermost), u32 ggml type and a u64 offset relative to the data section; the data section starts
// at the first multiple of general.alignment (32 when absent) past the last tensor info.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "aq_common.h"

namespace {

enum : uint32_t {
    GT_U8 = 0, GT_I8 = 1, GT_U16 = 2, GT_I16 = 3, GT_U32 = 4, GT_I32 = 5, GT_F32 = 6, GT_BOOL = 7, GT_STR = 8,
    GT_ARR = 9, GT_U64 = 10, GT_I64 = 11, GT_F64 = 12
};
constexpr uint32_t GGUF_MAGIC = 0x46554747u; // "GGUF" little-endian
constexpr uint32_t GGUF_DEFAULT_ALIGNMENT = 32;

struct Value {
    uint32_t type = 0;
    uint64_t u = 0;   // unsigned integers and bool
    int64_t i = 0;    // signed integers
    double f = 0.0;   // floats
    std::string s;
    uint32_t arr_type = 0;
    std::vector<Value> arr;
};

struct TensorInfo {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t rel_offset = 0, nbytes = 0;
};

// Bytes of `n` elements of a ggml type, 0 for a type this build does not know or a count that is not whole blocks.
uint64_t type_bytes(uint32_t type, uint64_t n) {
    const int be = aq::block_elems((int)type), bb = aq::block_bytes((int)type);
    if (be <= 0 || bb <= 0 || n % (uint64_t)be) return 0;
    uint64_t bytes;
    if (__builtin_mul_overflow(n / (uint64_t)be, (uint64_t)bb, &bytes)) return 0;
    return bytes;
}

// The fewest bytes one array element of GGUF type `t` occupies in the file (a string: its 8-byte length).
uint64_t elem_min_bytes(uint32_t t) {
    switch (t) {
    case GT_U8: case GT_I8: case GT_BOOL: return 1;
    case GT_U16: case GT_I16: return 2;
    case GT_U32: case GT_I32: case GT_F32: return 4;
    default: return 8; // GT_U64, GT_I64, GT_F64, GT_STR
    }
}

struct Reader {
    const uint8_t *p;
    uint64_t n, at = 0;
    bool ok = true;
    bool need(uint64_t k) {
        if (!ok || k > n - at) ok = false;
        return ok;
    }
    template <typename T> T get() {
        T v{};
        if (need(sizeof(T))) {
            std::memcpy(&v, p + at, sizeof(T));
            at += sizeof(T);
        }
        return v;
    }
    std::string str() {
        const uint64_t len = get<uint64_t>();
        if (!need(len)) return std::string();
        std::string s((const char *)p + at, (size_t)len);
        at += len;
        return s;
    }
    Value value(uint32_t type, int depth) {
        Value v;
        v.type = type;
        switch (type) {
        case GT_U8: v.u = get<uint8_t>(); break;
        case GT_I8: v.i = get<int8_t>(); break;
        case GT_U16: v.u = get<uint16_t>(); break;
        case GT_I16: v.i = get<int16_t>(); break;
        case GT_U32: v.u = get<uint32_t>(); break;
        case GT_I32: v.i = get<int32_t>(); break;
        case GT_F32: v.f = get<float>(); break;
        case GT_BOOL: v.u = get<uint8_t>(); break;
        case GT_STR: v.s = str(); break;
        case GT_U64: v.u = get<uint64_t>(); break;
        case GT_I64: v.i = get<int64_t>(); break;
        case GT_F64: v.f = get<double>(); break;
        case GT_ARR: {
            v.arr_type = get<uint32_t>();
            const uint64_t cnt = get<uint64_t>();
            // one level, and no more elements than the bytes left can hold (nothing is reserved for a count that
            // a crafted file inflates)
            if (!ok || depth > 0 || v.arr_type == GT_ARR || v.arr_type > GT_F64 ||
                cnt > (n - at) / elem_min_bytes(v.arr_type)) {
                ok = false;
                break;
            }
            v.arr.reserve((size_t)cnt);
            for (uint64_t k = 0; k < cnt && ok; k++) v.arr.push_back(value(v.arr_type, depth + 1));
            break;
        }
        default: ok = false;
        }
        return v;
    }
};

} // namespace

struct aq_gguf {
    std::string path;
    int fd = -1;
    uint8_t *map = nullptr;
    uint64_t file_size = 0, header_end = 0, data_offset = 0;
    uint32_t version = 0, alignment = GGUF_DEFAULT_ALIGNMENT;
    std::vector<std::pair<std::string, Value>> kv;
    std::map<std::string, size_t> kv_index;
    std::vector<TensorInfo> tensors;
    std::map<std::string, size_t> tensor_index;
};

namespace {

using aq::fail;

void close_gguf(aq_gguf *g) {
    if (!g) return;
    if (g->map) munmap(g->map, (size_t)g->file_size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

const Value *find(const aq_gguf *g, const std::string &key) {
    const auto it = g->kv_index.find(key);
    return it == g->kv_index.end() ? nullptr : &g->kv[it->second].second;
}

int get_u32(const aq_gguf *g, const std::string &key, uint32_t *out) {
    const Value *v = find(g, key);
    AQ_REQUIRE(v, "gguf: missing metadata key " + key);
    AQ_REQUIRE(v->type == GT_U32, "gguf: " + key + " is not a UINT32");
    *out = (uint32_t)v->u;
    return 0;
}

int get_f32(const aq_gguf *g, const std::string &key, float *out) {
    const Value *v = find(g, key);
    AQ_REQUIRE(v, "gguf: missing metadata key " + key);
    AQ_REQUIRE(v->type == GT_F32, "gguf: " + key + " is not a FLOAT32");
    *out = (float)v->f;
    return 0;
}

const TensorInfo *tensor(const aq_gguf *g, const std::string &name) {
    const auto it = g->tensor_index.find(name);
    return it == g->tensor_index.end() ? nullptr : &g->tensors[it->second];
}

// numpy-order rows x cols of a tensor: cols = ne[0], rows = the product of the outer dims (1 for a vector).
void rows_cols(const TensorInfo &t, int64_t *rows, int64_t *cols) {
    *cols = t.dims.empty() ? 1 : (int64_t)t.dims[0];
    int64_t r = 1;
    for (size_t d = 1; d < t.dims.size(); d++) r *= (int64_t)t.dims[d];
    *rows = r;
}

// ------------------------------------------------------------------------------------------------- writer
struct Writer {
    FILE *f = nullptr;
    uint64_t at = 0;
    bool ok = true;
    void raw(const void *p, size_t k) {
        if (ok && fwrite(p, 1, k, f) != k) ok = false;
        at += k;
    }
    template <typename T> void put(T v) { raw(&v, sizeof(T)); }
    void str(const std::string &s) {
        put<uint64_t>(s.size());
        raw(s.data(), s.size());
    }
    void key_u32(const std::string &k, uint32_t v) {
        str(k);
        put<uint32_t>(GT_U32);
        put<uint32_t>(v);
    }
    void key_f32(const std::string &k, float v) {
        str(k);
        put<uint32_t>(GT_F32);
        put<float>(v);
    }
    void key_str(const std::string &k, const std::string &v) {
        str(k);
        put<uint32_t>(GT_STR);
        str(v);
    }
    void key_bool(const std::string &k, bool v) {
        str(k);
        put<uint32_t>(GT_BOOL);
        put<uint8_t>(v ? 1 : 0);
    }
    void key_i32_array(const std::string &k, const std::vector<int32_t> &v) {
        str(k);
        put<uint32_t>(GT_ARR);
        put<uint32_t>(GT_I32);
        put<uint64_t>(v.size());
        for (int32_t x : v) put<int32_t>(x);
    }
    void key_str_array(const std::string &k, const std::vector<std::string> &v) {
        str(k);
        put<uint32_t>(GT_ARR);
        put<uint32_t>(GT_STR);
        put<uint64_t>(v.size());
        for (const auto &x : v) str(x);
    }
    void pad_to(uint64_t align) {
        static const uint8_t zeros[256] = {};
        while (at % align) raw(zeros, (size_t)std::min<uint64_t>(align - at % align, sizeof zeros));
    }
};

// Offsets relative to the data section of tensors laid out in order, each at a multiple of `alignment`.
std::vector<uint64_t> layout(const std::vector<uint64_t> &nbytes, uint32_t alignment) {
    std::vector<uint64_t> off(nbytes.size());
    uint64_t at = 0;
    for (size_t i = 0; i < nbytes.size(); i++) {
        at = (at + alignment - 1) / alignment * alignment;
        off[i] = at;
        at += nbytes[i];
    }
    return off;
}

} // namespace

extern "C" {

int aq_gguf_open(const char *path, aq_gguf **out) {
    AQ_REQUIRE(path && out, "aq_gguf_open: null argument");
    aq_gguf *g = new aq_gguf();
    g->path = path;
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) {
        close_gguf(g);
        return fail(AQ_EINVAL, std::string("aq_gguf_open: cannot open ") + path);
    }
    struct stat st;
    if (fstat(g->fd, &st) != 0 || st.st_size < 24) {
        close_gguf(g);
        return fail(AQ_EINVAL, std::string("aq_gguf_open: not a GGUF file (too short): ") + path);
    }
    g->file_size = (uint64_t)st.st_size;
    void *m = mmap(nullptr, (size_t)g->file_size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        close_gguf(g);
        return fail(AQ_ENOMEM, std::string("aq_gguf_open: mmap failed: ") + path);
    }
    g->map = (uint8_t *)m;
    Reader r{g->map, g->file_size};
    const uint32_t magic = r.get<uint32_t>();
    g->version = r.get<uint32_t>();
    const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    int rc = 0;
    if (magic != GGUF_MAGIC) rc = fail(AQ_EINVAL, "aq_gguf_open: bad magic (not a GGUF file)");
    else if (g->version != 3) rc = fail(AQ_EUNSUP, "aq_gguf_open: GGUF version " + std::to_string(g->version) + ", only 3");
    else if (n_tensors > g->file_size || n_kv > g->file_size) rc = fail(AQ_EINVAL, "aq_gguf_open: counts exceed the file");
    for (uint64_t i = 0; i < n_kv && !rc; i++) {
        std::string key = r.str();
        const uint32_t vt = r.get<uint32_t>();
        Value v = r.value(vt, 0);
        if (!r.ok) {
            rc = fail(AQ_EINVAL, "aq_gguf_open: truncated or malformed metadata at key #" + std::to_string(i));
            break;
        }
        if (!g->kv_index.emplace(key, g->kv.size()).second) {
            rc = fail(AQ_EINVAL, "aq_gguf_open: duplicate metadata key " + key);
            break;
        }
        g->kv.emplace_back(std::move(key), std::move(v));
    }
    for (uint64_t i = 0; i < n_tensors && !rc; i++) {
        TensorInfo t;
        t.name = r.str();
        const uint32_t nd = r.get<uint32_t>();
        if (!r.ok || nd == 0 || nd > 4) {
            rc = fail(AQ_EINVAL, "aq_gguf_open: tensor info #" + std::to_string(i) + ": bad dimension count");
            break;
        }
        uint64_t count = 1;
        bool wrapped = false;
        for (uint32_t d = 0; d < nd; d++) {
            t.dims.push_back(r.get<uint64_t>());
            wrapped = __builtin_mul_overflow(count, t.dims.back(), &count) || wrapped;
        }
        if (wrapped) {
            rc = fail(AQ_EINVAL, "aq_gguf_open: tensor info #" + std::to_string(i) + ": element count overflows");
            break;
        }
        t.type = r.get<uint32_t>();
        t.rel_offset = r.get<uint64_t>();
        if (!r.ok) {
            rc = fail(AQ_EINVAL, "aq_gguf_open: truncated tensor info #" + std::to_string(i));
            break;
        }
        t.nbytes = type_bytes(t.type, count);
        if (t.nbytes == 0) {
            rc = fail(AQ_EUNSUP, "aq_gguf_open: tensor " + t.name + ": ggml type " + std::to_string(t.type) +
                                     " not supported, or not whole blocks");
            break;
        }
        if (!g->tensor_index.emplace(t.name, g->tensors.size()).second) {
            rc = fail(AQ_EINVAL, "aq_gguf_open: duplicate tensor " + t.name);
            break;
        }
        g->tensors.push_back(std::move(t));
    }
    if (!rc) {
        g->header_end = r.at;
        if (const Value *a = find(g, "general.alignment")) {
            if (a->type != GT_U32 || a->u == 0 || (a->u & (a->u - 1)))
                rc = fail(AQ_EINVAL, "aq_gguf_open: general.alignment must be a power-of-two UINT32");
            else
                g->alignment = (uint32_t)a->u;
        }
    }
    if (!rc) {
        g->data_offset = (g->header_end + g->alignment - 1) / g->alignment * g->alignment;
        for (const TensorInfo &t : g->tensors) {
            // each comparison without a sum that could wrap: offset, then size, against the bytes left
            const uint64_t room = g->data_offset <= g->file_size ? g->file_size - g->data_offset : 0;
            if (t.rel_offset % g->alignment || t.rel_offset > room || t.nbytes > room - t.rel_offset) {
                rc = fail(AQ_EINVAL, "aq_gguf_open: tensor " + t.name + " misaligned or past the end of the file");
                break;
            }
        }
    }
    if (rc) {
        close_gguf(g);
        return rc;
    }
    *out = g;
    return 0;
}

int aq_gguf_close(aq_gguf *g) {
    close_gguf(g);
    return 0;
}

int aq_gguf_info(const aq_gguf *g, uint32_t *alignment, uint64_t *data_offset, uint64_t *n_tensors, uint64_t *n_kv) {
    AQ_REQUIRE(g, "aq_gguf_info: null file");
    if (alignment) *alignment = g->alignment;
    if (data_offset) *data_offset = g->data_offset;
    if (n_tensors) *n_tensors = g->tensors.size();
    if (n_kv) *n_kv = g->kv.size();
    return 0;
}

int aq_gguf_tensor(const aq_gguf *g, uint64_t i, const char **name, int32_t *ggml_type, int64_t *rows, int64_t *cols,
                   uint64_t *rel_offset, uint64_t *nbytes, const void **data) {
    AQ_REQUIRE(g && i < g->tensors.size(), "aq_gguf_tensor: no such tensor");
    const TensorInfo &t = g->tensors[i];
    if (name) *name = t.name.c_str();
    if (ggml_type) *ggml_type = (int32_t)t.type;
    int64_t r = 0, c = 0;
    rows_cols(t, &r, &c);
    if (rows) *rows = r;
    if (cols) *cols = c;
    if (rel_offset) *rel_offset = t.rel_offset;
    if (nbytes) *nbytes = t.nbytes;
    if (data) *data = g->map + g->data_offset + t.rel_offset;
    return 0;
}

int aq_gguf_get_u32(const aq_gguf *g, const char *key, uint32_t *out) {
    AQ_REQUIRE(g && key && out, "aq_gguf_get_u32: null argument");
    return get_u32(g, key, out);
}

int aq_gguf_get_f32(const aq_gguf *g, const char *key, float *out) {
    AQ_REQUIRE(g && key && out, "aq_gguf_get_f32: null argument");
    return get_f32(g, key, out);
}

int aq_gguf_get_str(const aq_gguf *g, const char *key, const char **out) {
    AQ_REQUIRE(g && key && out, "aq_gguf_get_str: null argument");
    const Value *v = find(g, key);
    AQ_REQUIRE(v, std::string("gguf: missing metadata key ") + key);
    AQ_REQUIRE(v->type == GT_STR, std::string("gguf: ") + key + " is not a STRING");
    *out = v->s.c_str();
    return 0;
}

// config.rs:146-379 `ModelConfig::from_gguf`, the part the decode path reads, with its consistency checks against
// the tensor index. The vocabulary is the length of tokenizer.ggml.tokens, or token_embd's outer dimension in a
// file without a tokenizer.
int aq_gguf_model_config(const aq_gguf *g, aq_model_config *out) {
    AQ_REQUIRE(g && out, "aq_gguf_model_config: null argument");
    const Value *arch = find(g, "general.architecture");
    AQ_REQUIRE(arch && arch->type == GT_STR, "gguf: general.architecture missing");
    const std::string a = arch->s + ".";
    uint32_t block_count = 0, nextn = 0, hidden = 0, ffn = 0, nh = 0, nkv = 0, kl = 0, vl = 0, interval = 0, rope_dim = 0;
    uint32_t conv = 0, state = 0, groups = 0, rank = 0, inner = 0;
    float eps = 0.0f, theta = 0.0f;
    int rc = 0;
#define AQ_G(fn, k, v)                                                                                        \
    if (!rc) rc = fn(g, a + k, v)
    AQ_G(get_u32, "block_count", &block_count);
    AQ_G(get_u32, "nextn_predict_layers", &nextn);
    AQ_G(get_u32, "embedding_length", &hidden);
    AQ_G(get_u32, "feed_forward_length", &ffn);
    AQ_G(get_u32, "attention.head_count", &nh);
    AQ_G(get_u32, "attention.head_count_kv", &nkv);
    AQ_G(get_u32, "attention.key_length", &kl);
    AQ_G(get_u32, "attention.value_length", &vl);
    AQ_G(get_f32, "attention.layer_norm_rms_epsilon", &eps);
    AQ_G(get_u32, "full_attention_interval", &interval);
    AQ_G(get_f32, "rope.freq_base", &theta);
    AQ_G(get_u32, "rope.dimension_count", &rope_dim);
    AQ_G(get_u32, "ssm.conv_kernel", &conv);
    AQ_G(get_u32, "ssm.state_size", &state);
    AQ_G(get_u32, "ssm.group_count", &groups);
    AQ_G(get_u32, "ssm.time_step_rank", &rank);
    AQ_G(get_u32, "ssm.inner_size", &inner);
#undef AQ_G
    if (rc) return rc;
    AQ_REQUIRE(nextn < block_count, "gguf: nextn_predict_layers >= block_count");
    AQ_REQUIRE(nextn <= 1, "gguf: this build runs one MTP layer (nextn_predict_layers " + std::to_string(nextn) + ")");
    AQ_REQUIRE(nkv > 0 && nh % nkv == 0, "gguf: head_count / head_count_kv");
    AQ_REQUIRE(rank > 0 && inner % rank == 0, "gguf: ssm.inner_size / ssm.time_step_rank");
    AQ_REQUIRE(groups > 0 && rank % groups == 0, "gguf: ssm.time_step_rank / ssm.group_count");
    AQ_REQUIRE(rope_dim <= kl, "gguf: rope.dimension_count > key_length");
    AQ_REQUIRE(vl == kl, "gguf: value_length != key_length is not supported by the attention kernels");
    AQ_REQUIRE(interval > 0, "gguf: full_attention_interval 0");
    if (const Value *sec = find(g, a + "rope.dimension_sections")) {
        AQ_REQUIRE(sec->type == GT_ARR, "gguf: rope.dimension_sections is not an array");
        int64_t sum = 0;
        for (const Value &e : sec->arr) sum += e.type == GT_I32 ? e.i : (int64_t)e.u;
        AQ_REQUIRE(sum * 2 == (int64_t)rope_dim, "gguf: rope.dimension_sections sum * 2 != rope.dimension_count");
    }
    const TensorInfo *embd = tensor(g, "token_embd.weight");
    AQ_REQUIRE(embd && embd->dims.size() == 2 && embd->dims[0] == hidden, "gguf: token_embd.weight shape");
    uint64_t vocab = embd->dims[1];
    if (const Value *tok = find(g, "tokenizer.ggml.tokens")) {
        AQ_REQUIRE(tok->type == GT_ARR && tok->arr.size() == vocab, "gguf: len(tokenizer.ggml.tokens) != token_embd rows");
    }
    const TensorInfo *outw = tensor(g, "output.weight");
    AQ_REQUIRE(outw && outw->dims == embd->dims, "gguf: output.weight missing or not the shape of token_embd");
    AQ_REQUIRE(tensor(g, "output_norm.weight"), "gguf: output_norm.weight missing");
    const uint32_t n_layer = block_count - nextn, q_dim = nh * kl, kv_dim = nkv * kl;
    const uint32_t dn_qkv = 2 * groups * state + inner;
    for (uint32_t i = 0; i < n_layer; i++) {
        const std::string b = "blk." + std::to_string(i) + ".";
        const TensorInfo *q = tensor(g, b + "attn_q.weight");
        const bool has_ssm = tensor(g, b + "ssm_a") != nullptr, by_rule = (i + 1) % interval == 0;
        AQ_REQUIRE((q != nullptr) != has_ssm, "gguf: " + b + " must hold exactly one of attn_q and ssm_a");
        AQ_REQUIRE((q != nullptr) == by_rule, "gguf: " + b + " layer type against full_attention_interval");
        if (q) {
            AQ_REQUIRE(q->dims.size() == 2 && q->dims[0] == hidden && q->dims[1] == 2ull * q_dim,
                       "gguf: " + b + "attn_q must be [hidden, 2 * q_dim] (gated attention)");
            const TensorInfo *k = tensor(g, b + "attn_k.weight");
            AQ_REQUIRE(k && k->dims.size() == 2 && k->dims[0] == hidden && k->dims[1] == kv_dim, "gguf: " + b + "attn_k shape");
        } else {
            const TensorInfo *qkv = tensor(g, b + "attn_qkv.weight"), *cw = tensor(g, b + "ssm_conv1d.weight"),
                             *sa = tensor(g, b + "ssm_a");
            AQ_REQUIRE(qkv && qkv->dims.size() == 2 && qkv->dims[0] == hidden && qkv->dims[1] == dn_qkv,
                       "gguf: " + b + "attn_qkv shape");
            AQ_REQUIRE(cw && cw->dims.size() == 2 && cw->dims[0] == conv && cw->dims[1] == dn_qkv,
                       "gguf: " + b + "ssm_conv1d shape");
            AQ_REQUIRE(sa->dims.size() == 1 && sa->dims[0] == rank, "gguf: " + b + "ssm_a shape");
        }
    }
    if (nextn) AQ_REQUIRE(tensor(g, "blk." + std::to_string(n_layer) + ".nextn.eh_proj.weight"), "gguf: nextn.eh_proj missing");
    aq_model_config c{};
    c.n_layer = n_layer;
    c.hidden = hidden;
    c.ffn = ffn;
    c.vocab = (uint32_t)vocab;
    c.n_head = nh;
    c.n_head_kv = nkv;
    c.head_dim = kl;
    c.rope_dim = rope_dim;
    c.rope_theta = theta;
    c.rms_eps = eps;
    c.full_attention_interval = interval;
    c.dn_n_k_heads = groups;
    c.dn_n_v_heads = rank;
    c.dn_head_dim_k = state;
    c.dn_head_dim_v = inner / rank;
    c.dn_conv_kernel = conv;
    c.has_mtp = nextn ? 1 : 0;
    *out = c;
    return 0;
}

int aq_model_load_gguf(aq_ctx *ctx, const char *path, aq_model **out, aq_model_config *cfg_out) {
    AQ_REQUIRE(ctx && path && out, "aq_model_load_gguf: null argument");
    aq_gguf *g = nullptr;
    int rc = aq_gguf_open(path, &g);
    if (rc) return rc;
    aq_model_config cfg{};
    rc = aq_gguf_model_config(g, &cfg);
    std::vector<aq_tensor> table(g->tensors.size());
    for (size_t i = 0; i < g->tensors.size() && !rc; i++) {
        const TensorInfo &t = g->tensors[i];
        aq_tensor &e = table[i];
        e.name = t.name.c_str();
        e.ggml_type = (int32_t)t.type;
        rows_cols(t, &e.rows, &e.cols);
        e.data = g->map + g->data_offset + t.rel_offset;
        e.nbytes = t.nbytes;
    }
    if (!rc) rc = aq_model_load(ctx, &cfg, table.data(), table.size(), out); // copies every tensor to HBM
    if (!rc && cfg_out) *cfg_out = cfg;
    close_gguf(g);
    return rc;
}

int aq_gguf_layout(const aq_tensor_plan *plan, size_t n, uint32_t alignment, uint64_t *rel_offsets) {
    AQ_REQUIRE(plan && rel_offsets, "aq_gguf_layout: null argument");
    AQ_REQUIRE(alignment && !(alignment & (alignment - 1)), "aq_gguf_layout: alignment must be a power of two");
    std::vector<uint64_t> nb(n);
    for (size_t i = 0; i < n; i++) {
        nb[i] = type_bytes((uint32_t)plan[i].spec.ggml_type, (uint64_t)plan[i].spec.rows * (uint64_t)plan[i].spec.cols);
        AQ_REQUIRE(nb[i], std::string("aq_gguf_layout: bad tensor ") + plan[i].name);
    }
    const std::vector<uint64_t> off = layout(nb, alignment);
    std::memcpy(rel_offsets, off.data(), n * sizeof(uint64_t));
    return 0;
}

// A GGUF v3 file of the synthetic model (aq_model_plan's tensors, bytes from aq_synth_host): the metadata the
// config derivation reads under architecture "qwen35", a placeholder tokenizer (vocab token strings "<id>", so the
// vocabulary is checkable), alignment 32, tensors in plan order.
int aq_gguf_write_synth(const char *path, const aq_model_config *cfg, int mix, uint64_t seed, int threads) {
    AQ_REQUIRE(path && cfg, "aq_gguf_write_synth: null argument");
    size_t n = 0;
    int rc = aq_model_plan(cfg, mix, seed, nullptr, 0, &n);
    if (rc) return rc;
    std::vector<aq_tensor_plan> plan(n);
    rc = aq_model_plan(cfg, mix, seed, plan.data(), n, &n);
    if (rc) return rc;
    std::vector<uint64_t> nb(n);
    uint64_t max_nb = 0;
    for (size_t i = 0; i < n; i++) {
        nb[i] = type_bytes((uint32_t)plan[i].spec.ggml_type, (uint64_t)plan[i].spec.rows * (uint64_t)plan[i].spec.cols);
        max_nb = std::max(max_nb, nb[i]);
    }
    const std::vector<uint64_t> off = layout(nb, GGUF_DEFAULT_ALIGNMENT);
    Writer w;
    w.f = fopen(path, "wb");
    AQ_REQUIRE(w.f, std::string("aq_gguf_write_synth: cannot create ") + path);
    const std::string a = "qwen35.";
    const uint32_t secs3 = cfg->rope_dim / 2;
    const std::vector<int32_t> sections = {(int32_t)(secs3 - secs3 / 3 - secs3 / 3), (int32_t)(secs3 / 3),
                                           (int32_t)(secs3 / 3), 0};
    std::vector<std::string> tokens(cfg->vocab);
    for (uint32_t i = 0; i < cfg->vocab; i++) tokens[i] = "<" + std::to_string(i) + ">";
    const uint64_t n_kv = 26;
    w.put<uint32_t>(GGUF_MAGIC);
    w.put<uint32_t>(3);
    w.put<uint64_t>(n);
    w.put<uint64_t>(n_kv);
    w.key_str("general.architecture", "qwen35");
    w.key_str("general.name", "aqueduct synthetic " + std::to_string(cfg->hidden));
    w.key_u32("general.alignment", GGUF_DEFAULT_ALIGNMENT);
    w.key_u32("general.file_type", mix == AQ_MIX_Q4_K_M ? 15u : 0u);
    w.key_u32("general.quantization_version", 2);
    w.key_u32(a + "block_count", cfg->n_layer + (cfg->has_mtp ? 1 : 0));
    w.key_u32(a + "nextn_predict_layers", cfg->has_mtp ? 1 : 0);
    w.key_u32(a + "context_length", 262144);
    w.key_u32(a + "embedding_length", cfg->hidden);
    w.key_u32(a + "feed_forward_length", cfg->ffn);
    w.key_u32(a + "attention.head_count", cfg->n_head);
    w.key_u32(a + "attention.head_count_kv", cfg->n_head_kv);
    w.key_u32(a + "attention.key_length", cfg->head_dim);
    w.key_u32(a + "attention.value_length", cfg->head_dim);
    w.key_f32(a + "attention.layer_norm_rms_epsilon", cfg->rms_eps);
    w.key_u32(a + "full_attention_interval", cfg->full_attention_interval);
    w.key_f32(a + "rope.freq_base", cfg->rope_theta);
    w.key_u32(a + "rope.dimension_count", cfg->rope_dim);
    w.key_i32_array(a + "rope.dimension_sections", sections);
    w.key_u32(a + "ssm.conv_kernel", cfg->dn_conv_kernel);
    w.key_u32(a + "ssm.state_size", cfg->dn_head_dim_k);
    w.key_u32(a + "ssm.group_count", cfg->dn_n_k_heads);
    w.key_u32(a + "ssm.time_step_rank", cfg->dn_n_v_heads);
    w.key_u32(a + "ssm.inner_size", cfg->dn_n_v_heads * cfg->dn_head_dim_v);
    w.key_str("tokenizer.ggml.model", "gpt2");
    w.key_str_array("tokenizer.ggml.tokens", tokens);
    for (size_t i = 0; i < n; i++) {
        const aq_synth_spec &sp = plan[i].spec;
        w.str(plan[i].name);
        const bool vec = sp.rows == 1;
        w.put<uint32_t>(vec ? 1 : 2);
        w.put<uint64_t>((uint64_t)sp.cols);
        if (!vec) w.put<uint64_t>((uint64_t)sp.rows);
        w.put<uint32_t>((uint32_t)sp.ggml_type);
        w.put<uint64_t>(off[i]);
    }
    w.pad_to(GGUF_DEFAULT_ALIGNMENT);
    const uint64_t data0 = w.at;
    std::vector<uint8_t> buf((size_t)max_nb);
    for (size_t i = 0; i < n && w.ok && !rc; i++) {
        w.pad_to(GGUF_DEFAULT_ALIGNMENT);
        if (w.at - data0 != off[i]) rc = fail(AQ_EINVAL, "aq_gguf_write_synth: layout mismatch");
        if (!rc) rc = aq_synth_host(&plan[i].spec, buf.data(), threads);
        if (!rc) w.raw(buf.data(), (size_t)nb[i]);
    }
    const bool ok = w.ok && fclose(w.f) == 0;
    if (!rc && !ok) rc = fail(AQ_EINVAL, std::string("aq_gguf_write_synth: write failed: ") + path);
    return rc;
}

} // extern "C"
