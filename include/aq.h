/*
 * aq.h — C-ABI of the MI355X (gfx950) speculative-decode path for Qwen3.x hybrid (Gated-DeltaNet + gated GQA
 * + MTP) models stored in ggml K-quant blocks.
 *
 * The reference engine (ManeeshJupalle/Qwen-3.8-in-Rust, crate `aqueduct_core`) has no FFI; its drop-in points
 * are Rust functions. Each entry point below names the reference function it replaces (file:line under
 * crates/core/src/). A Rust-side FFI crate binds these symbols one to one.
 *
 * Conventions
 *  - Every function returns int: 0 = OK, < 0 = an AQ_E* code. Nothing aborts across the ABI; contract
 *    violations (the reference's assert!s, e.g. matvec.rs:338-339, kdot.rs:179-191, spec.rs:335-336) return
 *    AQ_EINVAL. aq_last_error() gives thread-local text for the last failure.
 *  - Host pointers are owned by the caller and only read/written during the call. Device memory is owned by
 *    the opaque handles, except the raw buffers of the op-level API, which the caller allocates with
 *    aq_dev_alloc.
 *  - An aq_state owns one HIP stream and is not re-entrant; an aq_model may be shared read-only by several
 *    states (the reference's `&Model` / `&mut State` split, model.rs:102-104).
 *  - Results do not depend on launch geometry; column i of a batched (verify) call equals the N = 1 call on
 *    that column, bit for bit (kdot.rs:164-173).
 */
#ifndef AQ_H
#define AQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------------------------- status codes */
#define AQ_OK 0
#define AQ_EINVAL (-1)   /* argument or shape contract violated */
#define AQ_EHIP (-2)     /* a HIP runtime call failed */
#define AQ_ENOMEM (-3)   /* device or host allocation failed */
#define AQ_EUNSUP (-4)   /* weight type / shape this build has no kernel for */
#define AQ_ESTATE (-5)   /* call out of order (e.g. spec_round before spec_prefill) */

/* ggml type ids (ggml.h enum ggml_type), the ones the Q4_K_M mix uses (gguf.rs:247-279). */
#define AQ_TYPE_F32 0
#define AQ_TYPE_Q4_0 2
#define AQ_TYPE_Q8_0 8
#define AQ_TYPE_Q4_K 12
#define AQ_TYPE_Q5_K 13
#define AQ_TYPE_Q6_K 14

/* ---------------------------------------------------------------------------------- shared plain types */

/* One tensor in ggml layout. `rows` x `cols` in numpy order (rows = ne[1], cols = ne[0]; vectors have rows 1).
 * Mirrors the reference's `WeightMat` (matvec.rs:49-119) and `TensorSource` (layers/mod.rs:31-37). */
typedef struct aq_tensor {
    const char *name; /* GGUF tensor name, e.g. "blk.3.attn_q.weight" */
    int32_t ggml_type;
    int64_t rows;
    int64_t cols;
    const void *data; /* ggml bytes */
    size_t nbytes;
} aq_tensor;

/* The model contract, the subset of `ModelConfig` (config.rs:82-137) the forward path reads. The layer
 * schedule is derived as in config.rs:238-294: layer i is full attention iff (i+1) % interval == 0. */
typedef struct aq_model_config {
    uint32_t n_layer;      /* decoder layers, without the MTP block (block_count - nextn_predict_layers) */
    uint32_t hidden;       /* embedding_length */
    uint32_t ffn;          /* feed_forward_length */
    uint32_t vocab;
    uint32_t n_head;       /* attention.head_count */
    uint32_t n_head_kv;    /* attention.head_count_kv */
    uint32_t head_dim;     /* attention.key_length */
    uint32_t rope_dim;     /* rope.dimension_count (partial rotary) */
    float rope_theta;      /* rope.freq_base */
    float rms_eps;         /* attention.layer_norm_rms_epsilon */
    uint32_t full_attention_interval;
    uint32_t dn_n_k_heads; /* ssm.group_count */
    uint32_t dn_n_v_heads; /* ssm.time_step_rank */
    uint32_t dn_head_dim_k; /* ssm.state_size */
    uint32_t dn_head_dim_v; /* ssm.inner_size / ssm.time_step_rank */
    uint32_t dn_conv_kernel;
    uint32_t has_mtp;      /* 1: blk.{n_layer} is an MTP (nextn) block */
} aq_model_config;

/* The sampler's settings (`SamplerConfig`, sample.rs:57-68): temperature <= 0 is greedy (argmax; the other fields
 * unused), top_k 0 = off, top_p >= 1 = off, min_p 0 = off; seed seeds xoshiro256** through splitmix64. */
typedef struct aq_sampler_config {
    float temperature;
    uint32_t top_k;
    float top_p;
    float min_p;
    uint64_t seed;
} aq_sampler_config;

/* Per-round counters of the speculative loop (the reference's SpecStats, spec.rs:12-59). */
typedef struct aq_spec_stats {
    uint64_t rounds, drafted, accepted, emitted;
    uint64_t hist[17];        /* hist[m]: rounds that accepted exactly m drafts (k <= 16) */
    double verify_ms, commit_ms, refeed_ms, chain_ms; /* device time per stage, summed */
} aq_spec_stats;

/* ----------------------------------------------------------------------------------------------- lifecycle */
typedef struct aq_ctx aq_ctx;
typedef struct aq_model aq_model;
typedef struct aq_state aq_state;
typedef struct aq_weight aq_weight;

const char *aq_last_error(void);
/* The hash of the sources and flags this library was built from (the build's stamp; bindings refuse a library whose
 * stamp differs from the sources beside it). No counterpart in the reference. */
const char *aq_build_hash(void);
int aq_device_count(int *out);
int aq_init(int device, aq_ctx **out);
/* Frees the context's stream and events only. Objects made from it (weights, activations, models, states) are freed
 * by their own calls, before or after this one; every other call on them needs the context alive. */
int aq_ctx_free(aq_ctx *ctx);
int aq_synchronize(aq_ctx *ctx);

/* ---------------------------------------------------------------------- raw device memory (op-level API) */
int aq_dev_alloc(aq_ctx *ctx, size_t nbytes, void **dev_out);
int aq_dev_free(aq_ctx *ctx, void *dev);
int aq_memcpy_htod(aq_ctx *ctx, void *dev, const void *host, size_t nbytes);
int aq_memcpy_dtoh(aq_ctx *ctx, void *host, const void *dev, size_t nbytes);
int aq_memcpy_dtod(aq_ctx *ctx, void *dst, const void *src, size_t nbytes);

/* --------------------------------------------------------------------------------------- operator level */

/* Device weight matrix: `rows` x `cols` ggml bytes, repacked at upload into the kernels' plane layout (the
 * integer math is unchanged; aq_weight_download returns the original ggml bytes). Replaces `WeightMat::new`
 * (matvec.rs:59-63). Types: Q4_K, Q5_K, Q6_K (K-quant x Q8_K), Q8_0, Q4_0 (x Q8_0), F32 (x f32). */
int aq_weight_upload(aq_ctx *ctx, int ggml_type, size_t rows, size_t cols, const void *ggml_bytes,
                     aq_weight **out);
int aq_weight_free(aq_weight *w);
int aq_weight_download(const aq_weight *w, void *ggml_bytes_out);

/* Activation buffer of `ncols` (1..64) rows of `n` values on the device: the f32 rows and their quantised forms (Q8_K
 * in the kernels' layout, Q8_0). Replaces `ActBuf` (matvec.rs:216-267). */
typedef struct aq_act aq_act;
int aq_act_new(aq_ctx *ctx, size_t n, size_t ncols, aq_act **out);
int aq_act_free(aq_act *a);
/* Upload `ncols` x `n` host f32 rows. */
int aq_act_set_f32(aq_act *a, const float *host, size_t ncols);
/* Quantise the f32 rows on the device for weights of `weight_type` (matvec.rs:147-160 `act_kind`): Q8_K
 * (`Q8KRow::quantize_into`, q8k.rs:54-114) for AQ_TYPE_Q4_K/Q5_K/Q6_K, Q8_0 (`Q8Row::quantize_into`, q8.rs:68-106)
 * for AQ_TYPE_Q8_0/Q4_0, and for the K-quants too while the q8-fine switch is on. */
int aq_act_quantize(aq_act *a, int weight_type, size_t ncols);
/* The quantised rows in ggml wire layout: Q8_K 292 B per 256 (q8k.rs:139-150), Q8_0 34 B per 32 (q8.rs:155-162). */
int aq_act_get_q8k(const aq_act *a, void *ggml_out, size_t ncols);
int aq_act_get_q8_0(const aq_act *a, void *ggml_out, size_t ncols);

/* y[c * rows + r] = W[r] . x[c] for c < ncols (ncols 1..64, at most the activation's columns; 1 is the matvec; past 8
 * columns the many-column matrix-core kernels, the prompt-chunk form of model.rs:443-461). Replaces `matvec`
 * (matvec.rs:336), `matmul_fn` (matvec.rs:377) and the blocked kernel `dot_q8k_t` (kdot.rs:314); under the q8-fine
 * switch, K-quant weights take `dot_q4_k_q8` / `dot_q5_k_q8` / `dot_q6_k_q8` (dot.rs:69-160). `y_dev` is a device
 * buffer of ncols * rows f32. The activation must have been quantised for w's type under the same switch. */
int aq_matmul(aq_ctx *ctx, const aq_weight *w, const aq_act *x, size_t ncols, float *y_dev);
/* aq_act_quantize and aq_matmul on the caller's HIP stream (`stream`: a hipStream_t of the context's device; NULL:
 * the context's own), returning once the work is queued, without synchronising: the forms for a caller that orders
 * its work on a stream of its own (the reference's operators, matvec.rs:336 and :377, are synchronous calls into its
 * thread pool). The caller orders the activation's f32 rows before the quantisation on that stream, and reads y_dev
 * only after the stream has reached it. Same kernels, same bits as the synchronous forms. */
int aq_act_quantize_on(aq_act *a, int weight_type, size_t ncols, void *stream);
int aq_matmul_on(aq_ctx *ctx, const aq_weight *w, const aq_act *x, size_t ncols, float *y_dev, void *stream);
/* The exact integers of the K-quant dot, from the same kernel and grid aq_matmul runs (instantiated with its
 * integer outputs on): per column c < ncols (1, 4 or 8), row and super-block the 8 i32 lane sums and (Q4_K/Q5_K) the
 * 4 i32 min products the reference keeps in `sumi` / `prod` (kdot.rs:37-140; Q6_K lanes after the -32 fold).
 * lanes_dev: ncols*rows*nb*8 ([c][row][sb][lane]); mins_dev: ncols*rows*nb*4 (zero for Q6_K). */
int aq_kq_isums(aq_ctx *ctx, const aq_weight *w, const aq_act *x, size_t ncols, int32_t *lanes_dev,
                int32_t *mins_dev);

/* The q8-fine switch: `set_q8_fine` / `q8_fine` (matvec.rs:127-145, `aqueduct run --q8-fine`, run.rs:203). Process-
 * wide, off by default. On, K-quant weights take Q8_0 activations (per-32 scales, the dots of dot.rs:69-160) instead
 * of Q8_K ones, in aq_act_quantize / aq_matmul and in every model call (forward, prefill, speculative rounds). Every
 * later call reads it: change it only while no call is running, and between a quantise and its matmul keep it
 * unchanged. aq_kq_isums is the Q8_K kernel's and returns AQ_EUNSUP while it is on. */
int aq_set_q8_fine(int on);
int aq_q8_fine(void);

/* How many device and pinned-host allocations this library has made since it was loaded (every one it makes is
 * counted). No counterpart in the reference's API: it is what its counting allocator shows in tests/decode_alloc.rs:80,
 * 185 and tests/matmul_t_alloc.rs:76-116, that a decode step, a speculative round and a blocked matmul allocate
 * nothing once their buffers exist. */
int aq_alloc_counts(uint64_t *device_allocs, uint64_t *pinned_host_allocs);

/* ids_dev[r] = argmax of row r of the t rows of n f32 at x_dev (device): `argmax` (model.rs:505-513), the first
 * maximum on ties; a NaN never becomes the maximum, and a NaN at index 0 is never replaced (the answer is 0). */
int aq_argmax(aq_ctx *ctx, const float *x_dev, size_t n, size_t t, uint32_t *ids_dev);
/* aq_argmax without any device allocation: no counterpart in the reference; for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops). Its partial results live in a fixed device array of 128 KiB
 * per GPU, held until the process ends, so t <= 16 rows of n <= 2^20 values (larger calls return AQ_EINVAL). Every
 * call on one GPU shares that array: calls that overlap on one GPU (several contexts or threads) race. Nothing in
 * it carries from one call to the next. Same results as aq_argmax. */
int aq_argmax_noalloc(aq_ctx *ctx, const float *x_dev, size_t n, size_t t, uint32_t *ids_dev);

/* ---------------------------------------------------------------------------------------------- sampler */

/* The sampler on the device: `Sampler` (sample.rs:148-303) with its xoshiro256** state in device memory. Replaces
 * `Sampler::new` (sample.rs:159), `reseed` (164). Buffers are sized for `vocab` at creation; every call below runs on
 * the context's stream and returns after it (the model's sampled calls run it on the state's stream instead: one
 * sampler is used by one call at a time). */
typedef struct aq_sampler aq_sampler;
int aq_sampler_new(aq_ctx *ctx, const aq_sampler_config *cfg, uint32_t vocab, aq_sampler **out);
int aq_sampler_free(aq_sampler *sp);
int aq_sampler_reseed(aq_sampler *sp, uint64_t seed);
/* The generator's four state words (for reproducibility checks). */
int aq_sampler_get_rng(aq_sampler *sp, uint64_t *out4);
/* `process` (sample.rs:181-236) of the vocab logits at logits_dev: the kept set (ids by probability descending,
 * probabilities summing to 1) stays on the device; n_kept (nullable) receives its size. Greedy: the argmax alone. */
int aq_sampler_process(aq_sampler *sp, const float *logits_dev, uint32_t *n_kept);
/* `kept` (sample.rs:176-179): host copies of the last kept set (cap entries at most); *n its size. */
int aq_sampler_kept(aq_sampler *sp, uint32_t *ids, float *probs, size_t cap, size_t *n);
/* `draw` (sample.rs:239-251) from the last kept set; `sample` (254-257) = process then draw. */
int aq_sampler_draw(aq_sampler *sp, uint32_t *tok);
int aq_sampler_sample(aq_sampler *sp, const float *logits_dev, uint32_t *tok);
/* `write_dense` (sample.rs:259-265): the last kept set as vocab f32 at dense_dev, zeros elsewhere. */
int aq_sampler_write_dense(aq_sampler *sp, float *dense_dev);
/* `accept_or_resample` (sample.rs:272-303): accept draft d with probability min(1, p(d)/q(d)), else a draw from
 * norm(max(0, p - q)); q_dev is the dense draft distribution (vocab f32). Greedy: accepted iff d is the argmax. */
int aq_sampler_accept_or_resample(aq_sampler *sp, const float *target_dev, const float *q_dev, uint32_t d,
                                  int *accepted, uint32_t *tok);

/* ------------------------------------------------------------------------------------ synthetic tensors */

/* A deterministic synthetic tensor: value i is drawn from splitmix64 of (seed, i) (normal: the inverse normal CDF of
 * its top 53 bits, Acklam's approximation in double with IEEE basic operations only; uniform; or constant) and quantised to ggml bytes by this library's block quantisers, with
 * plain IEEE f32 arithmetic, so the host and the device produce the same bytes. No counterpart in the reference
 * (its fixtures come from real GGUF rows and gguf-py quantisers); it builds the benchmark's random-init models. */
typedef struct aq_synth_spec {
    int32_t ggml_type;
    int64_t rows, cols;
    uint64_t seed;
    uint32_t dist; /* 0 normal(mean a, sigma b), 1 uniform [a, b), 2 constant a */
    float a, b;
} aq_synth_spec;

/* ggml bytes of the tensor on the host, `threads` workers (<= 0: all cores). */
int aq_synth_host(const aq_synth_spec *spec, void *ggml_out, int threads);
/* The same tensor generated directly on the device as an aq_weight. */
int aq_weight_synth(aq_ctx *ctx, const aq_synth_spec *spec, aq_weight **out);

/* Time `iters` launches of aq_matmul, cycling over `nw` distinct weights (so the 256 MB MALL is defeated),
 * with HIP events on the context stream. Writes the mean device time per launch in microseconds. */
int aq_matmul_time(aq_ctx *ctx, const aq_weight *const *ws, size_t nw, const aq_act *x, size_t ncols,
                   float *y_dev, int iters, double *us_per_launch);
/* The same launches with an event between each two: us_each[i] is launch i's device time (iters <= 4096), for
 * medians and spreads. No counterpart in the reference (its kernel benchmarks are Rust bench harnesses). */
int aq_matmul_time_each(aq_ctx *ctx, const aq_weight *const *ws, size_t nw, const aq_act *x, size_t ncols,
                        float *y_dev, int iters, float *us_each);
/* Measurement only, no counterpart in the reference: the mean device time of `iters` back-to-back launches of a
 * plain streaming-read kernel over `bytes` (a multiple of 16) of bufs_dev[i % nbuf] (16-byte aligned), 2048
 * partial sums into partials_dev (>= 2048 floats) — the least time any kernel needs to read that many bytes, which
 * bench.py reports beside the dominant kernel. */
int aq_read_floor_time(aq_ctx *ctx, const void *const *bufs_dev, size_t nbuf, size_t bytes, float *partials_dev,
                       int iters, double *us_per_launch);

/* ------------------------------------------------------------------------------------------- model level */

/* Type mixes of the synthetic models. AQ_MIX_Q4_K_M: the per-tensor type table of a llama.cpp Q4_K_M file of
 * the 27B hybrid (docs/data/q4km_type_breakdown.txt, docs/data/gguf_layout.txt); AQ_MIX_TINY: Q4_K for every
 * matrix except ffn_down and output (Q6_K), F32 ssm_alpha/ssm_beta. */
#define AQ_MIX_Q4_K_M 0
#define AQ_MIX_TINY 1

/* One tensor of a synthetic model: its GGUF name and how to generate it. */
typedef struct aq_tensor_plan {
    char name[64];
    aq_synth_spec spec;
} aq_tensor_plan;

/* The tensor list of a synthetic model (GGUF names, shapes as the loader checks them, types from `mix`,
 * weights ~N(0, 0.02), norm weights 1, ssm_a ~ -U(0, 16), ssm_dt.bias 1). With out == NULL only *n_out is set.
 * Replaces the reference's checkpoint builders (tools/make_tiny_checkpoint.py) for random-init models. */
int aq_model_plan(const aq_model_config *cfg, int mix, uint64_t seed, aq_tensor_plan *out, size_t cap,
                  size_t *n_out);

/* Whole model resident in device memory, from ggml tensors on the host (what a GGUF reader hands over;
 * `Model::load` model.rs:140-356 + `WeightMat::new` matvec.rs:59-63) or generated on the device from the plan
 * (same bytes as aq_synth_host of each plan entry). Matrices: Q4_K/Q5_K/Q6_K/Q8_0/Q4_0/F32; vectors F32. */
int aq_model_load(aq_ctx *ctx, const aq_model_config *cfg, const aq_tensor *tensors, size_t n, aq_model **out);
int aq_model_synth(aq_ctx *ctx, const aq_model_config *cfg, int mix, uint64_t seed, aq_model **out);
int aq_model_free(aq_model *m);

/* Bytes of the weights one pass reads: the decoder layers + output norm + lm_head (`main`), the MTP block with
 * eh_proj and its norms (`mtp_block`), the lm_head alone (`lm_head`). */
typedef struct aq_model_bytes {
    uint64_t main, mtp_block, lm_head, embed_row;
} aq_model_bytes;
int aq_model_get_bytes(const aq_model *m, aq_model_bytes *out);

/* ------------------------------------------------------------------------------------------- GGUF files */

/* A GGUF v3 file: header, metadata and tensor index parsed (`Gguf::open`, gguf.rs:483-608); the tensor data is
 * mapped read-only, not read. */
typedef struct aq_gguf aq_gguf;
int aq_gguf_open(const char *path, aq_gguf **out);
int aq_gguf_close(aq_gguf *g);
int aq_gguf_info(const aq_gguf *g, uint32_t *alignment, uint64_t *data_offset, uint64_t *n_tensors, uint64_t *n_kv);
/* Tensor i in file order (`Gguf::tensor`, gguf.rs:722): name, ggml type, rows (the outer dims; 1 for a vector) x
 * cols (ne[0]), offset relative to the data section, bytes, and a pointer to the mapped bytes. Pointers live
 * until aq_gguf_close. */
int aq_gguf_tensor(const aq_gguf *g, uint64_t i, const char **name, int32_t *ggml_type, int64_t *rows, int64_t *cols,
                   uint64_t *rel_offset, uint64_t *nbytes, const void **data);
/* Typed metadata reads (`Gguf::get_u32` / `get_f32` / `get_str`); a missing key or another type is AQ_EINVAL. */
int aq_gguf_get_u32(const aq_gguf *g, const char *key, uint32_t *out);
int aq_gguf_get_f32(const aq_gguf *g, const char *key, float *out);
int aq_gguf_get_str(const aq_gguf *g, const char *key, const char **out);
/* `ModelConfig::from_gguf` (config.rs:146-379): the model contract from the metadata, checked against the tensor
 * index (layer schedule, shapes); the vocabulary is len(tokenizer.ggml.tokens), or token_embd's rows without it. */
int aq_gguf_model_config(const aq_gguf *g, aq_model_config *out);
/* `Model::load` (model.rs:140-356) from a GGUF file: the config derived as above, every tensor copied to HBM.
 * cfg_out (nullable) receives the config. */
int aq_model_load_gguf(aq_ctx *ctx, const char *path, aq_model **out, aq_model_config *cfg_out);
/* Offsets relative to the data section of the plan's tensors written in this order at `alignment`. */
int aq_gguf_layout(const aq_tensor_plan *plan, size_t n, uint32_t alignment, uint64_t *rel_offsets);
/* A GGUF v3 file of the synthetic model: aq_model_plan's tensors (bytes as aq_synth_host, `threads` workers) under
 * the metadata keys the config derivation reads, with a placeholder tokenizer. No counterpart in the reference (its
 * tiny checkpoint comes from tools/make_tiny_checkpoint.py and llama.cpp's converter). */
int aq_gguf_write_synth(const char *path, const aq_model_config *cfg, int mix, uint64_t seed, int threads);

/* Per-sequence state: DeltaNet conv/recurrent state, KV caches, the speculative buffers (spec_k drafts,
 * 0 = plain decode only) for positions < max_pos. `Model::new_state_spec` spec.rs:184 + `State::reserve`
 * model.rs:123. spec_k <= 7. */
int aq_state_new(aq_model *m, uint32_t spec_k, uint32_t max_pos, aq_state **out);
int aq_state_free(aq_state *s);

/* `Model::prefill` (model.rs:443-461): the prompt through every layer; logits of the last row (nullable, vocab
 * floats) and their argmax. */
int aq_prefill(aq_state *s, const uint32_t *ids, size_t n, float *logits_last_host, uint32_t *argmax_out);
/* `Model::forward_token` (model.rs:486-490) + `argmax` (505-513). */
int aq_forward_token(aq_state *s, uint32_t id, float *logits_host, uint32_t *argmax_out);
/* `Model::spec_prefill` (spec.rs:229-272): the prompt, x_T = argmax of the last row, the MTP over the prompt and
 * the first k drafts. */
int aq_spec_prefill(aq_state *s, const uint32_t *ids, size_t n, uint32_t *x_t);
/* `Model::spec_round` (spec.rs:326-433), greedy: verify [x_p, d_1..d_k] in one batch, accept on the device,
 * commit the DeltaNet state of the accepted rows, truncate the KV caches, re-feed the MTP and draft the next k.
 * emitted: capacity k+1; *m = accepted drafts; *n_emitted = m+1. */
int aq_spec_round(aq_state *s, uint32_t x_p, uint32_t *emitted, uint32_t *n_emitted, uint32_t *m);
/* The same calls under a sampler (sample.rs; sampler and state on one device, sampler vocabulary = the model's): the
 * token after the prompt or a forward is `Sampler::sample` of its logits (run.rs's sampled loop; spec.rs:241);
 * drafts are drawn from the MTP's processed distribution (spec.rs:192-203); a round accepts by the rejection-sampling
 * rule `accept_or_resample`, the bonus after k acceptances is a draw (spec.rs:367-380). The sampler's random state
 * advances on the state's stream in the reference's order. A greedy sampler gives the greedy calls. */
int aq_prefill_sampled(aq_state *s, aq_sampler *sp, const uint32_t *ids, size_t n, float *logits_last_host,
                       uint32_t *next);
int aq_forward_token_sampled(aq_state *s, aq_sampler *sp, uint32_t id, float *logits_host, uint32_t *next);
int aq_spec_prefill_sampled(aq_state *s, aq_sampler *sp, const uint32_t *ids, size_t n, uint32_t *x_t);
int aq_spec_round_sampled(aq_state *s, aq_sampler *sp, uint32_t x_p, uint32_t *emitted, uint32_t *n_emitted,
                          uint32_t *m);
/* `Model::spec_set_drafts` (spec.rs:436) test hook, and the current drafts. */
int aq_spec_set_drafts(aq_state *s, const uint32_t *d, size_t k);
int aq_spec_get_drafts(aq_state *s, uint32_t *d, size_t k);
/* Row i (< k+1) of the last verify batch's logits. */
int aq_spec_logits_row(aq_state *s, size_t i, float *host_out);
int aq_spec_get_stats(aq_state *s, aq_spec_stats *out);
int aq_state_pos(const aq_state *s, uint32_t *pos);
/* The state as f32, in this order: per layer, attention: K then V rows [0, len); DeltaNet: the recurrent
 * state then the conv window; then the MTP K and V rows. With out == NULL only *n_out is set. */
int aq_state_export(aq_state *s, float *out, size_t cap, size_t *n_out);

/* One decoder piece on its own (the reference's layer tests, tests/layers.rs:109-271): kind 0 DeltaNet mixer,
 * 1 attention mixer, 2 MLP, 3 decoder layer with DeltaNet, 4 with attention; tensors "blk.0.*". x: t rows of
 * hidden (host); conv/rec (DeltaNet) and k_cache/v_cache (kv_cap rows of n_head_kv*head_dim, *kv_len used) are
 * read and updated on the host; y: t rows of hidden. */
int aq_layer_run(aq_ctx *ctx, const aq_model_config *cfg, const aq_tensor *tensors, size_t n, int kind,
                 const float *x, size_t t, uint32_t start_pos, float *conv, float *rec, float *k_cache,
                 float *v_cache, uint32_t *kv_len, uint32_t kv_cap, float *y);

/* The Gated-DeltaNet recurrence alone (deltanet.rs:43-86), with speculative rollback: from `state_dev`
 * (nv x dk x dv f32, device), t rows (1..8: one verify batch) of q, k (t x nk*dk, already normalised), v (t x nv*dv), g and beta
 * (t x nv) give out (t x nv*dv); the state is then advanced by the first `keep` rows only (keep <= t),
 * as the reference's snapshot / restore / replay leaves it (spec.rs:154-179, 396-415). Host arrays. */
int aq_deltanet_verify_commit(aq_ctx *ctx, uint32_t nk, uint32_t nv, uint32_t dk, uint32_t dv, size_t t, size_t keep,
                              const float *q, const float *k, const float *v, const float *g, const float *beta,
                              float *state_dev, float *out);
/* The same on device arrays (q_dev .. beta_dev as above, out_dev t x nv*dv): nothing allocated or copied, the two
 * launches queued on the context's stream, which is synchronised before the call returns. t is one verify batch
 * (1..8), as for the host form. */
int aq_deltanet_verify_commit_dev(aq_ctx *ctx, uint32_t nk, uint32_t nv, uint32_t dk, uint32_t dv, size_t t,
                                  size_t keep, const float *q_dev, const float *k_dev, const float *v_dev,
                                  const float *g_dev, const float *beta_dev, float *state_dev, float *out_dev);

/* The device's scalar activations, elementwise on host arrays (fn: 0 exp, 1 log1p, 2 silu, 3 sigmoid, 4 softplus;
 * act.rs:7-40). No counterpart in the reference: the parity tests use it to show the device evaluates exp and
 * log1p exactly as the CPU oracle does. */
int aq_eval_math(aq_ctx *ctx, int fn, const float *x, float *y, size_t n);

#ifdef __cplusplus
}
#endif
#endif /* AQ_H */
