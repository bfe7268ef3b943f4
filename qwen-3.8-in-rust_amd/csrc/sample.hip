// sample.hip — the sampler on the device (the reference's sample.rs) and its C-ABI: seeded xoshiro256**, the processed
// distribution (top-k, softmax at a temperature, top-p, min-p, renormalise), draws, the dense draft distribution and
// the speculative acceptance rule accept_or_resample, plus the launchers the model's sampled calls use.
//
// Candidates. A logit and its id form one 64-bit key, (the logit's order bits, descending) << 32 | id, so ascending
// keys are the reference's order: logit descending, ties by the lower id (sample.rs:196; -0 and +0 are one key).
// top_k <= 512: every 4096-key chunk of the row is sorted in LDS (bitonic) and keeps its first top_k keys; lists are
// merged the same way until one remains. Larger top_k or none: the row's keys are radix-sorted whole (hipcub).
//
// The rest is one 256-thread work-group: elementwise steps in parallel; the reference's sequential f32 sums (the
// softmax denominator, the renormalisation, top-p's running mass, the draw's running mass, the residual's sum) by
// one lane in the reference's order. A sum over probabilities in descending order stops once the next term is below a
// quarter of the running sum's ulp: no later term can change it then (each is at most that term, up to a few ulps of
// expf's rounding), so the result is the full sequential sum's. The random state lives in device memory; lane 0 draws.
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <cmath>
#include <vector>

#include "aq_common.h"
#include "aq_math.h"
#include "ops.h"

namespace aq {
namespace {

constexpr int ST = 256;          // sampler work-group
constexpr int SZ = 4096;         // keys sorted per chunk work-group
constexpr int KMAX_FAST = 512;   // top_k up to this takes the chunked selection
constexpr int ROWS_MAX = 17;     // rows per call (k + 1 for k <= 16)
enum { OP_PROCESS = 0, OP_DRAW = 1, OP_SAMPLE = 2, OP_ACCEPT = 3, OP_DRAFT = 4, OP_ROUND = 5, OP_GREEDY_SET = 6 };

__device__ __forceinline__ uint64_t make_key(float v, uint32_t id) {
    uint32_t b = __float_as_uint(v);
    if ((b & 0x7FFFFFFFu) == 0) b = 0;                              // -0 sorts with +0
    const uint32_t asc = (b & 0x80000000u) ? ~b : (b | 0x80000000u); // ascending float order
    return ((uint64_t)(~asc) << 32) | id;
}

// Bitonic sort of SZ keys in LDS, ascending; all ST threads take part.
__device__ void bitonic_sz(uint64_t *s) {
    for (int k = 2; k <= SZ; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int t = threadIdx.x; t < SZ / 2; t += ST) {
                const int i = 2 * j * (t / j) + (t % j), l = i + j;
                const uint64_t a = s[i], b = s[l];
                const bool up = (i & k) == 0;
                if ((a > b) == up) {
                    s[i] = b;
                    s[l] = a;
                }
            }
            __syncthreads();
        }
    }
}

// Chunk c of row r: from the logits (in == nullptr: elements c*SZ ..) or from `in` (keys c*SZ .. of in_count), sorted;
// the first K keys go to out[r * out_stride + c * K ..].
__global__ void __launch_bounds__(ST) topk_chunk_kernel(const float *lg, size_t lg_stride, int vocab, const uint64_t *in,
                                                        size_t in_stride, int in_count, int K, uint64_t *out,
                                                        size_t out_stride) {
    __shared__ uint64_t s[SZ];
    const int c = blockIdx.x, r = blockIdx.y;
    for (int i = threadIdx.x; i < SZ; i += ST) {
        const int g = c * SZ + i;
        uint64_t key = ~0ull;
        if (in == nullptr) {
            if (g < vocab) key = make_key(lg[(size_t)r * lg_stride + g], (uint32_t)g);
        } else if (g < in_count) {
            key = in[(size_t)r * in_stride + g];
        }
        s[i] = key;
    }
    __syncthreads();
    bitonic_sz(s);
    for (int j = threadIdx.x; j < K; j += ST) out[(size_t)r * out_stride + (size_t)c * K + j] = s[j];
}

__global__ void __launch_bounds__(256) make_keys_kernel(const float *lg, int vocab, uint64_t *out) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < vocab) out[i] = make_key(lg[i], (uint32_t)i);
}

struct SampArgs {
    int op;
    aq_sampler_config cfg;
    int vocab, n_cand;
    const float *logits;      // row r at logits + r * vocab
    const uint64_t *keys;     // row r's sorted candidates at keys + r * key_stride
    size_t key_stride;
    uint64_t *rng;            // 4 words
    uint32_t *idx;            // the kept set: ids
    float *probs;             //               probabilities
    uint32_t *res;            // [0] n kept, [1] token, [2] accepted, [3] probs sorted descending (1) or not (0)
    uint32_t *tok_out;        // also receives the token (nullable)
    const float *q;           // OP_ACCEPT: the dense draft distribution
    uint32_t d;               //            the draft
    float *q_out;             // OP_DRAFT / OP_PROCESS dense write: the slot's dense distribution
    uint32_t *q_idx, *q_n;    //            the ids written to it last time, and their count
    const uint32_t *drafts;   // OP_ROUND: k drafts, their dense distributions at q + i * vocab
    uint32_t *emitted, *info; //           emitted tokens; info = (accepted, emitted, kept rows)
    int k;
};

__device__ __forceinline__ float quarter_ulp(float s) { return __uint_as_float(__float_as_uint(s) & 0x7F800000u) * 0x1p-25f; }

__device__ __forceinline__ uint64_t rotl64(uint64_t v, int k) { return (v << k) | (v >> (64 - k)); }

// sample.rs:34-51 xoshiro256** next / f32
__device__ uint64_t rng_next(uint64_t s[4]) {
    const uint64_t result = rotl64(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}
__device__ float rng_f32(uint64_t s[4]) { return (float)(rng_next(s) >> 40) * (1.0f / 16777216.0f); }

// Sequential f32 sum of p[0..n) (lane 0); `desc`: p is non-increasing, so the sum may stop early (file comment).
__device__ float seq_sum(const float *p, int n, bool desc) {
    float s = 0.0f;
    for (int i = 0; i < n; i++) {
        const float e = p[i];
        if (desc && e < quarter_ulp(s)) break;
        s += e;
    }
    return s;
}

// sample.rs:181-236 `process` (not greedy): the kept set into idx/probs; returns its size. Whole work-group.
__device__ int process(const SampArgs &a, const float *lg, const uint64_t *keys) {
    __shared__ float s_sum;
    __shared__ int s_n, s_first;
    const int tid = threadIdx.x, nc = a.n_cand;
    const float inv_t = 1.0f / a.cfg.temperature;
    const float m = lg[(uint32_t)keys[0]] * inv_t;
    for (int i = tid; i < nc; i += ST) {
        const uint32_t id = (uint32_t)keys[i];
        a.idx[i] = id;
        a.probs[i] = aq_expf(lg[id] * inv_t - m);
    }
    __syncthreads();
    if (tid == 0) s_sum = seq_sum(a.probs, nc, true);
    __syncthreads();
    const float sum = s_sum;
    for (int i = tid; i < nc; i += ST) a.probs[i] = a.probs[i] / sum;
    __syncthreads();
    if (tid == 0) {
        int n = nc;
        if (a.cfg.top_p < 1.0f) { // keep while the mass before the candidate is below top_p
            float cum = 0.0f;
            n = 0;
            while (n < nc && cum < a.cfg.top_p) {
                cum += a.probs[n];
                n++;
            }
            if (n < 1) n = 1;
        }
        s_n = n;
        s_first = n;
    }
    __syncthreads();
    int n = s_n;
    if (a.cfg.min_p > 0.0f) { // the first candidate after the top one below min_p * p[0] ends the set
        const float thr = a.cfg.min_p * a.probs[0];
        for (int i = 1 + tid; i < n; i += ST)
            if (!(a.probs[i] >= thr)) atomicMin(&s_first, i);
        __syncthreads();
        n = s_first;
    }
    if (tid == 0) s_sum = seq_sum(a.probs, n, true);
    __syncthreads();
    const float s = s_sum;
    for (int i = tid; i < n; i += ST) a.probs[i] = a.probs[i] / s;
    __syncthreads();
    return n;
}

// sample.rs:239-251 `draw` (lane 0). `desc`: probs non-increasing (a processed set), so the running mass may stop
// early: once it cannot grow, a u at or above it ends on the last kept id, as the reference's fall-through does.
__device__ uint32_t draw(const SampArgs &a, int n, uint64_t rs[4], bool desc) {
    const float u = rng_f32(rs);
    float cum = 0.0f;
    for (int i = 0; i < n; i++) {
        const float p = a.probs[i];
        if (desc && p < quarter_ulp(cum)) break;
        cum += p;
        if (u < cum) return a.idx[i];
    }
    return a.idx[n - 1];
}

// sample.rs:272-303 `accept_or_resample` after `process` left n kept: whole work-group; lane 0 returns the token.
__device__ uint32_t accept(const SampArgs &a, const float *lg, const uint64_t *keys, const float *q, uint32_t d, int n,
                           uint64_t rs[4], bool *ok_out) {
    __shared__ int s_pos, s_ok;
    __shared__ float s_sum;
    const int tid = threadIdx.x;
    if (tid == 0) s_pos = -1;
    __syncthreads();
    for (int i = tid; i < n; i += ST)
        if (a.idx[i] == d) s_pos = i;
    __syncthreads();
    uint32_t tok = d;
    if (tid == 0) {
        const float pd = s_pos >= 0 ? a.probs[s_pos] : 0.0f;
        const float qd = q[d];
        const float u = rng_f32(rs);
        s_ok = (qd > 0.0f && (pd >= qd || u < pd / qd)) ? 1 : 0;
    }
    __syncthreads();
    const bool ok = s_ok != 0;
    *ok_out = ok;
    if (ok) return tok;
    // the residual max(0, p - q) over the kept set, renormalised
    for (int i = tid; i < n; i += ST) a.probs[i] = fmaxf(a.probs[i] - q[a.idx[i]], 0.0f);
    __syncthreads();
    if (tid == 0) s_sum = seq_sum(a.probs, n, false);
    __syncthreads();
    const float sum = s_sum;
    if (!(sum > 0.0f)) { // p under q everywhere: the target's own distribution (sample.rs:293-297)
        const int n2 = process(a, lg, keys);
        if (tid == 0) tok = draw(a, n2, rs, true);
        return tok;
    }
    for (int i = tid; i < n; i += ST) a.probs[i] = a.probs[i] / sum;
    __syncthreads();
    if (tid == 0) tok = draw(a, n, rs, false);
    return tok;
}

__global__ void __launch_bounds__(ST) sampler_kernel(SampArgs a) {
    const int tid = threadIdx.x;
    uint64_t rs[4] = {0, 0, 0, 0};
    if (tid == 0)
        for (int i = 0; i < 4; i++) rs[i] = a.rng[i];
    __shared__ uint32_t s_tok;
    __shared__ int s_brk;
    switch (a.op) {
    case OP_GREEDY_SET: // the greedy kept set: the argmax (already in res[1]) with probability 1
        if (tid == 0) {
            a.idx[0] = a.res[1];
            a.probs[0] = 1.0f;
            a.res[0] = 1;
            a.res[3] = 1;
        }
        return;
    case OP_PROCESS:
    case OP_SAMPLE:
    case OP_DRAFT: {
        const int n = process(a, a.logits, a.keys);
        if (a.op == OP_PROCESS) {
            if (tid == 0) {
                a.res[0] = (uint32_t)n;
                a.res[3] = 1;
            }
            return;
        }
        if (tid == 0) {
            s_tok = draw(a, n, rs, true);
            a.res[0] = (uint32_t)n;
            a.res[1] = s_tok;
            a.res[3] = 1;
            if (a.tok_out) *a.tok_out = s_tok;
        }
        if (a.op == OP_DRAFT) { // spec.rs:192-203 write_dense into the slot: clear what it held, write the kept set
            const uint32_t old = *a.q_n;
            for (uint32_t j = tid; j < old; j += ST) a.q_out[a.q_idx[j]] = 0.0f;
            __syncthreads();
            for (int j = tid; j < n; j += ST) {
                a.q_out[a.idx[j]] = a.probs[j];
                a.q_idx[j] = a.idx[j];
            }
            if (tid == 0) *a.q_n = (uint32_t)n;
        }
        break;
    }
    case OP_DRAW:
        if (tid == 0) {
            s_tok = draw(a, (int)a.res[0], rs, a.res[3] != 0);
            a.res[1] = s_tok;
            if (a.tok_out) *a.tok_out = s_tok;
        }
        break;
    case OP_ACCEPT: {
        const int n = process(a, a.logits, a.keys);
        bool ok = false;
        const uint32_t tok = accept(a, a.logits, a.keys, a.q, a.d, n, rs, &ok);
        if (tid == 0) {
            a.res[0] = (uint32_t)n;
            a.res[1] = tok;
            a.res[2] = ok ? 1 : 0;
            a.res[3] = ok ? 1 : 0;
            if (a.tok_out) *a.tok_out = tok;
        }
        break;
    }
    case OP_ROUND: { // spec.rs:367-380
        const size_t v = (size_t)a.vocab;
        int m = 0;
        while (m < a.k) {
            const float *lg = a.logits + (size_t)m * v;
            const uint64_t *keys = a.keys + (size_t)m * a.key_stride;
            const int n = process(a, lg, keys);
            bool ok = false;
            const uint32_t tok = accept(a, lg, keys, a.q + (size_t)m * v, a.drafts[m], n, rs, &ok);
            if (tid == 0) {
                a.emitted[m] = tok;
                s_brk = ok ? 0 : 1;
            }
            __syncthreads();
            if (s_brk) break;
            m++;
        }
        if (m == a.k) {
            const int n = process(a, a.logits + (size_t)m * v, a.keys + (size_t)m * a.key_stride);
            if (tid == 0) a.emitted[m] = draw(a, n, rs, true);
        }
        if (tid == 0) {
            a.info[0] = (uint32_t)m;
            a.info[1] = (uint32_t)(m + 1);
            a.info[2] = (uint32_t)(m + 1);
        }
        break;
    }
    default: break;
    }
    if (tid == 0)
        for (int i = 0; i < 4; i++) a.rng[i] = rs[i];
}

} // namespace
} // namespace aq

// --------------------------------------------------------------------------------------------- the object

struct aq_sampler {
    aq_ctx *ctx = nullptr;
    int device = 0;
    aq_sampler_config cfg{};
    uint32_t vocab = 0;
    void *base = nullptr;
    uint64_t *rng = nullptr;
    uint32_t *idx = nullptr, *res = nullptr, *amax_scratch = nullptr;
    float *probs = nullptr;
    uint64_t *keys = nullptr;           // ROWS_MAX x vocab: the full sort's output rows
    uint64_t *bufa = nullptr, *bufb = nullptr; // chunk lists: ROWS_MAX x chunks x KMAX_FAST each
    uint64_t *sort_in = nullptr;        // vocab
    void *sort_tmp = nullptr;
    size_t sort_tmp_bytes = 0, chunk_stride = 0;
    uint32_t *pinned = nullptr;
    // recorded after every launch that touches the sampler's device buffers (generator state, kept set, candidate
    // lists), on whichever stream made it; every later use waits for it first, so a sampled model call still
    // queued on a state's stream and an operator call on the context stream never overlap
    hipEvent_t last = nullptr;
};

namespace aq {
namespace {

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int n_cand_of(const aq_sampler *sp) {
    const uint32_t k = sp->cfg.top_k;
    return (int)((k > 0 && k < sp->vocab) ? k : sp->vocab);
}

// The sorted candidates of `rows` logits rows (row r at logits + r * vocab): returns where row r's list starts
// (keys + r * *stride).
int candidates(aq_sampler *sp, const float *logits, int rows, hipStream_t st, const uint64_t **keys, size_t *stride) {
    AQ_REQUIRE(rows >= 1 && rows <= ROWS_MAX, "sampler: 1..17 rows");
    const int vocab = (int)sp->vocab, nc = n_cand_of(sp);
    if (nc <= KMAX_FAST) {
        int L = (vocab + SZ - 1) / SZ;
        hipLaunchKernelGGL(topk_chunk_kernel, dim3(L, rows), dim3(ST), 0, st, logits, (size_t)vocab, vocab,
                           (const uint64_t *)nullptr, (size_t)0, 0, nc, sp->bufa, sp->chunk_stride);
        uint64_t *in = sp->bufa, *out = sp->bufb;
        while (L > 1) { // every chunk of SZ keys keeps its first nc: the global first nc survive in their chunks
            const int L2 = (L * nc + SZ - 1) / SZ;
            hipLaunchKernelGGL(topk_chunk_kernel, dim3(L2, rows), dim3(ST), 0, st, (const float *)nullptr, (size_t)0,
                               vocab, (const uint64_t *)in, sp->chunk_stride, L * nc, nc, out, sp->chunk_stride);
            std::swap(in, out);
            L = L2;
        }
        *keys = in;
        *stride = sp->chunk_stride;
    } else {
        for (int r = 0; r < rows; r++) {
            hipLaunchKernelGGL(make_keys_kernel, dim3((vocab + 255) / 256), dim3(256), 0, st, logits + (size_t)r * vocab,
                               vocab, sp->sort_in);
            size_t bytes = sp->sort_tmp_bytes;
            if (hipcub::DeviceRadixSort::SortKeys(sp->sort_tmp, bytes, (const unsigned long long *)sp->sort_in,
                                                  (unsigned long long *)(sp->keys + (size_t)r * vocab), vocab, 0, 64,
                                                  st) != hipSuccess)
                return fail(AQ_EHIP, "sampler: radix sort");
        }
        *keys = sp->keys;
        *stride = sp->vocab;
    }
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "sampler: candidate launch");
}

SampArgs base_args(aq_sampler *sp, int op) {
    SampArgs a{};
    a.op = op;
    a.cfg = sp->cfg;
    a.vocab = (int)sp->vocab;
    a.n_cand = n_cand_of(sp);
    a.rng = sp->rng;
    a.idx = sp->idx;
    a.probs = sp->probs;
    a.res = sp->res;
    return a;
}

int run(const SampArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(sampler_kernel, dim3(1), dim3(ST), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "sampler launch");
}

int sync_res(aq_sampler *sp, hipStream_t st) {
    AQ_HIP(hipMemcpyAsync(sp->pinned, sp->res, 16, hipMemcpyDeviceToHost, st));
    AQ_HIP(hipStreamSynchronize(st));
    return 0;
}

// Stream st takes over the sampler: it waits for the last launch that used it (on any stream).
int join(aq_sampler *sp, hipStream_t st) {
    AQ_HIP(hipStreamWaitEvent(st, sp->last, 0));
    return 0;
}
// st's launches so far are now the sampler's last use.
int mark(aq_sampler *sp, hipStream_t st, int rc) {
    if (rc) return rc;
    AQ_HIP(hipEventRecord(sp->last, st));
    return 0;
}

} // namespace

// ------------------------------------------------------------------- launchers for the model's sampled calls
bool sampler_greedy(const aq_sampler *sp) { return sp == nullptr || sp->cfg.temperature <= 0.0f; }
uint32_t sampler_vocab(const aq_sampler *sp) { return sp->vocab; }
int sampler_device(const aq_sampler *sp) { return sp->device; }

int sampler_sample(aq_sampler *sp, const float *logits, uint32_t *tok_dev, hipStream_t st) {
    const uint64_t *keys;
    size_t stride;
    int rc = join(sp, st);
    if (!rc) rc = candidates(sp, logits, 1, st, &keys, &stride);
    if (rc) return rc;
    SampArgs a = base_args(sp, OP_SAMPLE);
    a.logits = logits;
    a.keys = keys;
    a.key_stride = stride;
    a.tok_out = tok_dev;
    return mark(sp, st, run(a, st));
}

int sampler_draft(aq_sampler *sp, const float *logits, uint32_t *tok_dev, float *q_dense, uint32_t *q_idx,
                  uint32_t *q_n, hipStream_t st) {
    const uint64_t *keys;
    size_t stride;
    int rc = join(sp, st);
    if (!rc) rc = candidates(sp, logits, 1, st, &keys, &stride);
    if (rc) return rc;
    SampArgs a = base_args(sp, OP_DRAFT);
    a.logits = logits;
    a.keys = keys;
    a.key_stride = stride;
    a.tok_out = tok_dev;
    a.q_out = q_dense;
    a.q_idx = q_idx;
    a.q_n = q_n;
    return mark(sp, st, run(a, st));
}

int sampler_round(aq_sampler *sp, const float *logits, int k, const uint32_t *drafts, const float *q_dense,
                  uint32_t *emitted, uint32_t *info, hipStream_t st) {
    const uint64_t *keys;
    size_t stride;
    int rc = join(sp, st);
    if (!rc) rc = candidates(sp, logits, k + 1, st, &keys, &stride);
    if (rc) return rc;
    SampArgs a = base_args(sp, OP_ROUND);
    a.logits = logits;
    a.keys = keys;
    a.key_stride = stride;
    a.q = q_dense;
    a.drafts = drafts;
    a.emitted = emitted;
    a.info = info;
    a.k = k;
    return mark(sp, st, run(a, st));
}

} // namespace aq

using namespace aq;

extern "C" {

int aq_sampler_new(aq_ctx *ctx, const aq_sampler_config *cfg, uint32_t vocab, aq_sampler **out) {
    AQ_REQUIRE(ctx && cfg && out, "aq_sampler_new: null argument");
    AQ_REQUIRE(vocab >= 1, "aq_sampler_new: empty vocabulary");
    AQ_REQUIRE(!(cfg->temperature > 0.0f) || std::isfinite(1.0f / cfg->temperature),
               "aq_sampler_new: temperature too small");
    AQ_HIP(hipSetDevice(ctx->device));
    aq_sampler *sp = new aq_sampler();
    sp->ctx = ctx;
    sp->device = ctx->device;
    sp->cfg = *cfg;
    sp->vocab = vocab;
    const size_t chunks = (vocab + SZ - 1) / SZ;
    sp->chunk_stride = chunks * KMAX_FAST;
    size_t tmp = 0;
    if (hipcub::DeviceRadixSort::SortKeys(nullptr, tmp, (const unsigned long long *)nullptr,
                                          (unsigned long long *)nullptr, (int)vocab, 0, 64, ctx->stream) != hipSuccess) {
        delete sp;
        return fail(AQ_EHIP, "aq_sampler_new: sort size query");
    }
    sp->sort_tmp_bytes = tmp;
    const size_t b_rng = align256(32), b_idx = align256((size_t)vocab * 4), b_probs = align256((size_t)vocab * 4),
                 b_res = align256(64), b_keys = align256((size_t)ROWS_MAX * vocab * 8),
                 b_buf = align256((size_t)ROWS_MAX * sp->chunk_stride * 8), b_in = align256((size_t)vocab * 8),
                 b_tmp = align256(tmp + 1), b_ams = align256(argmax_scratch_bytes(vocab, 1));
    const size_t total = b_rng + b_idx + b_probs + b_res + b_keys + 2 * b_buf + b_in + b_ams + b_tmp;
    if (dev_malloc(&sp->base, total) != hipSuccess) {
        delete sp;
        return fail(AQ_ENOMEM, "aq_sampler_new: hipMalloc");
    }
    uint8_t *p = (uint8_t *)sp->base;
    sp->rng = (uint64_t *)p, p += b_rng;
    sp->idx = (uint32_t *)p, p += b_idx;
    sp->probs = (float *)p, p += b_probs;
    sp->res = (uint32_t *)p, p += b_res;
    sp->keys = (uint64_t *)p, p += b_keys;
    sp->bufa = (uint64_t *)p, p += b_buf;
    sp->bufb = (uint64_t *)p, p += b_buf;
    sp->sort_in = (uint64_t *)p, p += b_in;
    sp->amax_scratch = (uint32_t *)p, p += b_ams;
    sp->sort_tmp = p;
    if (pinned_malloc((void **)&sp->pinned, 64) != hipSuccess) {
        (void)hipFree(sp->base);
        delete sp;
        return fail(AQ_ENOMEM, "aq_sampler_new: pinned buffer");
    }
    if (hipEventCreateWithFlags(&sp->last, hipEventDisableTiming) != hipSuccess) {
        sp->last = nullptr;
        aq_sampler_free(sp);
        return fail(AQ_EHIP, "aq_sampler_new: event");
    }
    int rc = aq_sampler_reseed(sp, cfg->seed);
    if (!rc && hipMemsetAsync(sp->res, 0, 64, ctx->stream) != hipSuccess) rc = fail(AQ_EHIP, "aq_sampler_new: clear");
    if (!rc && hipStreamSynchronize(ctx->stream) != hipSuccess) rc = fail(AQ_EHIP, "aq_sampler_new: sync");
    if (rc) {
        aq_sampler_free(sp);
        return rc;
    }
    *out = sp;
    return 0;
}

int aq_sampler_free(aq_sampler *sp) {
    if (!sp) return 0;
    (void)hipSetDevice(sp->device);
    if (sp->last) { // the last use may still be queued on a state's stream
        (void)hipEventSynchronize(sp->last);
        (void)hipEventDestroy(sp->last);
    }
    if (sp->base) (void)hipFree(sp->base);
    if (sp->pinned) (void)hipHostFree(sp->pinned);
    delete sp;
    return 0;
}

int aq_sampler_reseed(aq_sampler *sp, uint64_t seed) {
    AQ_REQUIRE(sp, "aq_sampler_reseed: null sampler");
    AQ_HIP(hipSetDevice(sp->device));
    uint64_t s[4], x = seed;
    for (int i = 0; i < 4; i++) { // sample.rs:21-33 splitmix64
        x += 0x9E3779B97F4A7C15ull;
        uint64_t z = x;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        s[i] = z ^ (z >> 31);
    }
    sp->cfg.seed = seed;
    if (sp->last) {
        int rc = join(sp, sp->ctx->stream);
        if (rc) return rc;
    }
    AQ_HIP(hipMemcpyAsync(sp->rng, s, 32, hipMemcpyHostToDevice, sp->ctx->stream));
    AQ_HIP(hipStreamSynchronize(sp->ctx->stream));
    return 0;
}

int aq_sampler_get_rng(aq_sampler *sp, uint64_t *out4) {
    AQ_REQUIRE(sp && out4, "aq_sampler_get_rng: null argument");
    AQ_HIP(hipSetDevice(sp->device));
    AQ_HIP(hipEventSynchronize(sp->last)); // a sampled round's draft chain may still be drawing
    AQ_HIP(hipMemcpy(out4, sp->rng, 32, hipMemcpyDeviceToHost));
    return 0;
}

int aq_sampler_process(aq_sampler *sp, const float *logits_dev, uint32_t *n_kept) {
    AQ_REQUIRE(sp && logits_dev, "aq_sampler_process: null argument");
    AQ_HIP(hipSetDevice(sp->device));
    hipStream_t st = sp->ctx->stream;
    int rc = join(sp, st);
    if (rc) return rc;
    if (sampler_greedy(sp)) {
        rc = launch_argmax(logits_dev, sp->vocab, sp->vocab, 1, sp->res + 1, sp->amax_scratch, st);
        if (!rc) rc = run(base_args(sp, OP_GREEDY_SET), st);
    } else {
        const uint64_t *keys;
        size_t stride;
        rc = candidates(sp, logits_dev, 1, st, &keys, &stride);
        if (!rc) {
            SampArgs a = base_args(sp, OP_PROCESS);
            a.logits = logits_dev;
            a.keys = keys;
            a.key_stride = stride;
            rc = run(a, st);
        }
    }
    rc = mark(sp, st, rc);
    if (!rc) rc = sync_res(sp, st);
    if (!rc && n_kept) *n_kept = sp->pinned[0];
    return rc;
}

int aq_sampler_kept(aq_sampler *sp, uint32_t *ids, float *probs, size_t cap, size_t *n) {
    AQ_REQUIRE(sp && n, "aq_sampler_kept: null argument");
    AQ_HIP(hipSetDevice(sp->device));
    int rc = join(sp, sp->ctx->stream);
    if (!rc) rc = sync_res(sp, sp->ctx->stream);
    if (rc) return rc;
    const size_t nk = sp->pinned[0];
    *n = nk;
    AQ_REQUIRE(nk <= cap || (!ids && !probs), "aq_sampler_kept: buffer smaller than the kept set");
    if (ids) AQ_HIP(hipMemcpy(ids, sp->idx, nk * 4, hipMemcpyDeviceToHost));
    if (probs) AQ_HIP(hipMemcpy(probs, sp->probs, nk * 4, hipMemcpyDeviceToHost));
    return 0;
}

int aq_sampler_draw(aq_sampler *sp, uint32_t *tok) {
    AQ_REQUIRE(sp && tok, "aq_sampler_draw: null argument");
    AQ_HIP(hipSetDevice(sp->device));
    int rc = join(sp, sp->ctx->stream);
    if (!rc) rc = sync_res(sp, sp->ctx->stream);
    if (rc) return rc;
    AQ_REQUIRE(sp->pinned[0] > 0, "aq_sampler_draw: draw before process (sample.rs:240)");
    rc = mark(sp, sp->ctx->stream, run(base_args(sp, OP_DRAW), sp->ctx->stream));
    if (!rc) rc = sync_res(sp, sp->ctx->stream);
    if (!rc) *tok = sp->pinned[1];
    return rc;
}

int aq_sampler_sample(aq_sampler *sp, const float *logits_dev, uint32_t *tok) {
    AQ_REQUIRE(sp && logits_dev && tok, "aq_sampler_sample: null argument");
    if (sampler_greedy(sp)) { // process then draw, as sample.rs:254-257: the draw consumes a number here too
        int rc = aq_sampler_process(sp, logits_dev, nullptr);
        if (!rc) rc = aq_sampler_draw(sp, tok);
        return rc;
    }
    AQ_HIP(hipSetDevice(sp->device));
    int rc = sampler_sample(sp, logits_dev, nullptr, sp->ctx->stream); // joins and marks itself
    if (!rc) rc = sync_res(sp, sp->ctx->stream);
    if (!rc) *tok = sp->pinned[1];
    return rc;
}

int aq_sampler_write_dense(aq_sampler *sp, float *dense_dev) {
    AQ_REQUIRE(sp && dense_dev, "aq_sampler_write_dense: null argument");
    AQ_HIP(hipSetDevice(sp->device));
    int rc = join(sp, sp->ctx->stream);
    if (!rc) rc = sync_res(sp, sp->ctx->stream);
    if (rc) return rc;
    // sample.rs:259-265: zeros, then the kept set (the operator-level form; the model writes it on the device)
    const size_t nk = sp->pinned[0];
    std::vector<uint32_t> ids(nk);
    std::vector<float> pr(nk), dense((size_t)sp->vocab, 0.0f);
    if (nk) {
        AQ_HIP(hipMemcpy(ids.data(), sp->idx, nk * 4, hipMemcpyDeviceToHost));
        AQ_HIP(hipMemcpy(pr.data(), sp->probs, nk * 4, hipMemcpyDeviceToHost));
    }
    for (size_t i = 0; i < nk; i++) dense[ids[i]] = pr[i];
    AQ_HIP(hipMemcpy(dense_dev, dense.data(), dense.size() * 4, hipMemcpyHostToDevice));
    return 0;
}

int aq_sampler_accept_or_resample(aq_sampler *sp, const float *target_dev, const float *q_dev, uint32_t d,
                                  int *accepted, uint32_t *tok) {
    AQ_REQUIRE(sp && target_dev && q_dev && accepted && tok, "aq_sampler_accept_or_resample: null argument");
    AQ_REQUIRE(d < sp->vocab, "aq_sampler_accept_or_resample: draft id out of range");
    AQ_HIP(hipSetDevice(sp->device));
    if (sampler_greedy(sp)) {
        int rc = aq_sampler_process(sp, target_dev, nullptr);
        if (rc) return rc;
        *tok = sp->pinned[1];
        *accepted = *tok == d;
        return 0;
    }
    hipStream_t st = sp->ctx->stream;
    const uint64_t *keys;
    size_t stride;
    int rc = join(sp, st);
    if (!rc) rc = candidates(sp, target_dev, 1, st, &keys, &stride);
    if (rc) return rc;
    SampArgs a = base_args(sp, OP_ACCEPT);
    a.logits = target_dev;
    a.keys = keys;
    a.key_stride = stride;
    a.q = q_dev;
    a.d = d;
    rc = mark(sp, st, run(a, st));
    if (!rc) rc = sync_res(sp, st);
    if (rc) return rc;
    *tok = sp->pinned[1];
    *accepted = (int)sp->pinned[2];
    return 0;
}

} // extern "C"
