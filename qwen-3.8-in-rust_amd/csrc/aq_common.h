// aq_common.h — shared definitions of the MI355X (gfx950) speculative-decode library: error handling, the
// device data layouts (weight planes, activation buffers) and small device helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/aq.h"

#pragma clang fp contract(off)

namespace aq {

// ------------------------------------------------------------------------------------------ error plumbing
void set_error(const std::string &msg);
int fail(int code, const std::string &msg);

#define AQ_HIP(call)                                                                                          \
    do {                                                                                                      \
        hipError_t e_ = (call);                                                                               \
        if (e_ != hipSuccess)                                                                                 \
            return ::aq::fail(AQ_EHIP, std::string(#call) + ": " + hipGetErrorString(e_) + " at " + __FILE__ +  \
                                           ":" + std::to_string(__LINE__));                                   \
    } while (0)

#define AQ_REQUIRE(cond, msg)                                                                                 \
    do {                                                                                                      \
        if (!(cond)) return ::aq::fail(AQ_EINVAL, msg);                                                       \
    } while (0)

// ------------------------------------------------------------------------------------------- block layouts
// ggml block sizes (ggml-common.h; the reference's quant.rs:15-20).
constexpr int QK_K = 256;
constexpr int QK32 = 32;
inline int block_elems(int t) { return (t == AQ_TYPE_Q4_0 || t == AQ_TYPE_Q8_0) ? 32 : (t == AQ_TYPE_F32 ? 1 : 256); }
inline int block_bytes(int t) {
    switch (t) {
    case AQ_TYPE_F32: return 4;
    case AQ_TYPE_Q4_0: return 18;
    case AQ_TYPE_Q8_0: return 34;
    case AQ_TYPE_Q4_K: return 144;
    case AQ_TYPE_Q5_K: return 176;
    case AQ_TYPE_Q6_K: return 210;
    default: return 0;
    }
}
inline bool is_kquant(int t) { return t == AQ_TYPE_Q4_K || t == AQ_TYPE_Q5_K || t == AQ_TYPE_Q6_K; }

// The q8-fine switch (matvec.rs:127-145 `Q8_FINE`, `set_q8_fine`): process-wide, off by default. On, K-quant weights
// take Q8_0 activations (per-32 scales) through launch_kq_q8f instead of Q8_K ones; every later quantiser choice and
// K-quant launch reads it, so it is changed only while no call is running.
bool q8_fine();
void set_q8_fine(bool on);

// Device weight planes. A ggml row of `nb` blocks is split into planes so that every kernel load is an aligned
// vector load; the integer math is unchanged (the GGUF bytes are the source of truth and aq_weight_download
// restores them exactly).
//
// K-quants are stored by tile: tile (row >> 2, sb) = 4 consecutive rows x 1 super-block, tiles in row-group-major
// order (tile index (row >> 2) * nb + sb, rows padded to a multiple of 4), so the 16 (lane pair, row) threads of
// a matrix-core block read one contiguous 256-byte run per load. Within a tile, r = row & 3 and lane l = p + 4h
// (p = l & 3, h = l >> 2):
//   Q4_K: qa 512 B  codes: qa[h*256 + (p*4 + r)*16 + q*4 + b] = qs[32q + 4l + b] (q = sub-block pair 0..3)
//         sc  64 B  per row r at r*16: f16 d, f16 dmin, then the 12 packed 6-bit scale/min bytes (as stored)
//   Q5_K: as Q4_K plus qb 128 B: qb[(p*4 + r)*8 + h*4 + b] = qh[4l + b]
//   Q6_K: qa 512 B  ql: qa[h*256 + (p*4 + r)*16 + (g*2 + k)*4 + b] = ql[g*64 + k*32 + 4l + b] (g = half, k = 0/1)
//         qb 256 B  qh: qb[(p*4 + r)*16 + h*8 + g*4 + b] = qh[g*32 + 4l + b]
//         sc  64 B  int8 group scales of row r at r*16       dm 8 B  f16 d of row r at r*2
// Lane l (0..7) of a super-block owns elements 32s + 4l + b (s = sub-block 0..7, b = 0..3): the lane of the
// reference's 8 exact i32 partial sums (kdot.rs:1-18).
// Per 32-block (Q8_0 / Q4_0): qa 32 B / 16 B codes (as stored), dm 2 B f16 d, row-major. F32: qa = the rows.
__host__ __device__ inline size_t kq_tile(size_t row, size_t sb, size_t nb) { return (row >> 2) * nb + sb; }
__host__ __device__ inline size_t kq_qa_off(size_t row, size_t sb, size_t nb, int l) {
    return kq_tile(row, sb, nb) * 512 + (size_t)(l >> 2) * 256 + (size_t)((l & 3) * 4 + (int)(row & 3)) * 16;
}
__host__ __device__ inline size_t kq_sc_off(size_t row, size_t sb, size_t nb) {
    return kq_tile(row, sb, nb) * 64 + (row & 3) * 16;
}
// Q5_K qh bytes of lane l (4 B); Q6_K qh bytes of lane l (8 B: halves g = 0, 1)
__host__ __device__ inline size_t kq_qb5_off(size_t row, size_t sb, size_t nb, int l) {
    return kq_tile(row, sb, nb) * 128 + (size_t)((l & 3) * 4 + (int)(row & 3)) * 8 + (size_t)(l >> 2) * 4;
}
__host__ __device__ inline size_t kq_qb6_off(size_t row, size_t sb, size_t nb, int l) {
    return kq_tile(row, sb, nb) * 256 + (size_t)((l & 3) * 4 + (int)(row & 3)) * 16 + (size_t)(l >> 2) * 8;
}
__host__ __device__ inline size_t kq_dm_off(size_t row, size_t sb, size_t nb) {
    return kq_tile(row, sb, nb) * 8 + (row & 3) * 2;
}
// Activation Q8_K codes are stored by lane slot slot(l) = 2*(l&3) + (l>>2) (0,4,1,5,2,6,3,7), so lanes j and
// j+4, the pair one kernel thread owns, are adjacent.
__host__ __device__ inline int lane_slot(int l) { return 2 * (l & 3) + (l >> 2); }

// Weight loads marked non-temporal (the `nt` bit): each weight byte is read once per round, so its lines are the
// first the caches give up, and what the round reads again (activations, the DeltaNet state, the gate rows, the KV
// cache) stays resident instead of being pushed out by ~17 GB of weights per round (K-quant and Q8_0 / Q4_0 weight
// loads: the greedy --spec 3 round 8.05 -> 7.76 ms).
typedef unsigned int kq_nt_u4 __attribute__((ext_vector_type(4)));
typedef unsigned int kq_nt_u2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ld_nt4(const uint8_t *p) {
    const kq_nt_u4 v = __builtin_nontemporal_load(reinterpret_cast<const kq_nt_u4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld_nt2(const uint8_t *p) {
    const kq_nt_u2 v = __builtin_nontemporal_load(reinterpret_cast<const kq_nt_u2 *>(p));
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ld_nt1(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p));
}
__device__ __forceinline__ uint16_t ld_nth(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(p));
}

struct Weight {
    int type = 0;
    size_t rows = 0, cols = 0, nb = 0; // nb: blocks per row
    uint8_t *base = nullptr;            // one allocation holding every plane
    uint8_t *qa = nullptr, *qb = nullptr, *sc = nullptr, *dm = nullptr;
    size_t qa_bytes = 0, qb_bytes = 0, sc_bytes = 0, dm_bytes = 0; // per block
    size_t total = 0;
    int device = 0;
};

// Device activation buffer: `ncols` rows of `n` values.
//   f32   : ncols x n
//   Q8_K  : qs  ncols x n int8, by lane per 256-block: qs[blk*256 + slot(l)*32 + s*4 + b] = q[blk*256 + 32s + 4l + b]
//           d   ncols x nb f32; bs ncols x nb x 16 i16 (group sums); q8s ncols x nb x 8 i16 (sub-block sums)
//   Q8_0  : q0  ncols x n int8 (natural order); d0 ncols x n/32 f32 (the f16 scale widened); h0 the f16 bits;
//           s0  ncols x n/32 i32 (sum of the block's codes, for the Q4_0 -8 offset)
struct Act {
    size_t n = 0, ncols = 0, nb = 0, nb32 = 0;
    float *f32 = nullptr;
    int8_t *qs = nullptr;
    float *d = nullptr;
    int16_t *bs = nullptr, *q8s = nullptr;
    int8_t *q0 = nullptr;
    float *d0 = nullptr;
    uint16_t *h0 = nullptr;
    int32_t *s0 = nullptr;
    void *base = nullptr;
    int device = 0;
};

// Every device and pinned-host allocation of the library goes through these two, which count it
// (aq_alloc_counts: what shows that a decode step or a speculative round allocates nothing).
hipError_t dev_malloc_raw(void **p, size_t bytes);
hipError_t pinned_malloc(void **p, size_t bytes);
template <typename T> hipError_t dev_malloc(T **p, size_t bytes) { return dev_malloc_raw((void **)p, bytes); }

// ----------------------------------------------------------------------------------------- kernel launchers
// All launches go to `stream`; they return 0 or an AQ_E* code.
int launch_q8k_quantize(const Act &a, size_t ncols, const float *src, size_t src_stride, hipStream_t stream);
int launch_q8_0_quantize(const Act &a, size_t ncols, const float *src, size_t src_stride, hipStream_t stream);
int launch_matmul(const Weight &w, const Act &x, size_t ncols, float *y, const float *resid, hipStream_t stream);
// The K-quant kernel with its exact integers written out: per column c, row r, super-block sb, lanes[((c * rows + r)
// * nb + sb) * 8 + l] (Q6_K after the -32 fold) and mins[... * 4 + i] (zero for Q6_K); y as launch_matmul.
int kq_isums_run(const Weight &w, const Act &x, size_t ncols, float *y, int32_t *lanes, int32_t *mins,
                 hipStream_t stream);
// The matrix-core K-quant kernel (kq_mfma.hip); launch_matmul routes K-quant weights here.
int launch_kq_mfma(const Weight &w, const Act &x, size_t ncols, float *y, const float *resid, hipStream_t stream);
// n matrices that read the same activations (y_i = W_i x [+ resid_i]): K-quants of one K, as few launches as
// their types allow (up to three matrices and two types per launch), then at most two F32 matrices that join the
// last launch. resids may be null.
int launch_kq_group(const Weight *const *ws, float *const *ys, const float *const *resids, int n, const Act &x,
                    size_t ncols, hipStream_t stream);
// K-quant weights x Q8_0 activations (kq_q8f.hip, dot.rs:69-160); launch_matmul routes K-quant weights here when
// the q8-fine switch is on. y as launch_matmul; ncols 1..16.
int launch_kq_q8f(const Weight &w, const Act &x, size_t ncols, float *y, const float *resid, hipStream_t stream);
// Many columns (a prompt chunk): K-quant x Q8_K and Q8_0 / Q4_0 x Q8_0 on the 16x16x32 matrix cores (kq_gemm.hip).
int launch_gemm(const Weight &w, const Act &x, size_t ncols, float *y, const float *resid, hipStream_t stream);
// Any column count: launch_matmul up to 8 columns, launch_gemm past that where it applies, else 8-column pieces.
int launch_matmul_many(const Weight &w, const Act &x, size_t ncols, float *y, const float *resid, hipStream_t stream);
int launch_repack(Weight &w, const uint8_t *ggml_dev, bool to_planes, hipStream_t stream);
// n matrices that read the same activations, all Q8_0 or all Q4_0 of one K (y_i = W_i x, no residual): one launch
// of the wave kernel for up to Q8_MAXSEG of them when its activation staging fits and ncols <= 4, else one launch
// each. ncols 1..8.
constexpr int Q8_MAXSEG = 3;
int launch_q8_group(const Weight *const *ws, float *const *ys, int n, const Act &x, size_t ncols, hipStream_t stream);

} // namespace aq

struct aq_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
};

struct aq_weight {
    aq_ctx *ctx = nullptr;
    aq::Weight w;
};

struct aq_act {
    aq_ctx *ctx = nullptr;
    aq::Act a;
};
