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
int aq_device_count(int *out);
int aq_init(int device, aq_ctx **out);
int aq_ctx_free(aq_ctx *ctx);
int aq_synchronize(aq_ctx *ctx);

/* ---------------------------------------------------------------------- raw device memory (op-level API) */
int aq_dev_alloc(aq_ctx *ctx, size_t nbytes, void **dev_out);
int aq_dev_free(aq_ctx *ctx, void *dev);
int aq_memcpy_htod(aq_ctx *ctx, void *dev, const void *host, size_t nbytes);
int aq_memcpy_dtoh(aq_ctx *ctx, void *host, const void *dev, size_t nbytes);

/* --------------------------------------------------------------------------------------- operator level */

/* Device weight matrix: `rows` x `cols` ggml bytes, repacked at upload into the kernels' plane layout (the
 * integer math is unchanged; aq_weight_download returns the original ggml bytes). Replaces `WeightMat::new`
 * (matvec.rs:59-63). Types: Q4_K, Q5_K, Q6_K (K-quant x Q8_K), Q8_0, Q4_0 (x Q8_0), F32 (x f32). */
int aq_weight_upload(aq_ctx *ctx, int ggml_type, size_t rows, size_t cols, const void *ggml_bytes,
                     aq_weight **out);
int aq_weight_free(aq_weight *w);
int aq_weight_download(const aq_weight *w, void *ggml_bytes_out);

/* Activation buffer of `ncols` rows of `n` values on the device: the f32 rows and their quantised forms (Q8_K
 * in the kernels' layout, Q8_0). Replaces `ActBuf` (matvec.rs:216-267). */
typedef struct aq_act aq_act;
int aq_act_new(aq_ctx *ctx, size_t n, size_t ncols, aq_act **out);
int aq_act_free(aq_act *a);
/* Upload `ncols` x `n` host f32 rows. */
int aq_act_set_f32(aq_act *a, const float *host, size_t ncols);
/* Quantise the f32 rows on the device: Q8_K (`Q8KRow::quantize_into`, q8k.rs:54-114) when `kind` is
 * AQ_TYPE_Q4_K/Q5_K/Q6_K, Q8_0 (`Q8Row::quantize_into`, q8.rs:68-106) when AQ_TYPE_Q8_0/Q4_0. */
int aq_act_quantize(aq_act *a, int weight_type, size_t ncols);
/* The quantised rows in ggml wire layout: Q8_K 292 B per 256 (q8k.rs:139-150), Q8_0 34 B per 32 (q8.rs:155-162). */
int aq_act_get_q8k(const aq_act *a, void *ggml_out, size_t ncols);
int aq_act_get_q8_0(const aq_act *a, void *ggml_out, size_t ncols);

/* y[c * rows + r] = W[r] . x[c] for c < ncols (ncols 1..16; 1 is the matvec). Replaces `matvec`
 * (matvec.rs:336), `matmul_fn` (matvec.rs:377) and the blocked kernel `dot_q8k_t` (kdot.rs:314). `y_dev` is a
 * device buffer of ncols * rows f32. The activation must have been quantised for w's type. */
int aq_matmul(aq_ctx *ctx, const aq_weight *w, const aq_act *x, size_t ncols, float *y_dev);
/* Debug form of the K-quant dot for column 0: per (row, super-block) the 8 exact i32 lane sums and (Q4_K/Q5_K)
 * the 4 exact i32 min products the reference keeps in `sumi` / `prod` (kdot.rs:37-140). lanes_dev: rows*nb*8,
 * mins_dev: rows*nb*4 (zero for Q6_K). */
int aq_kq_isums(aq_ctx *ctx, const aq_weight *w, const aq_act *x, int32_t *lanes_dev, int32_t *mins_dev);

/* ------------------------------------------------------------------------------------ synthetic tensors */

/* A deterministic synthetic tensor: value i is drawn from splitmix64 of (seed, i) (normal: Irwin-Hall of four
 * 16-bit fields; uniform; or constant) and quantised to ggml bytes by this library's block quantisers, with
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

#ifdef __cplusplus
}
#endif
#endif /* AQ_H */
