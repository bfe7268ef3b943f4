// ops.hip — the model-level kernels around the matmuls: embedding rows, RMSNorm + activation quantiser, SwiGLU +
// quantiser, the Gated-DeltaNet head kernel, attention, argmax and greedy acceptance.
//
// Every kernel reproduces the reference's scalar arithmetic in the reference's order (products and sums rounded
// one by one, no FMA; sequential sums stay sequential, in one thread), so its outputs equal the CPU path's bit
// for bit wherever the reference is exact IEEE arithmetic; exp and log1p are evaluated in double and rounded
// once (quant_dev.h).
#include <cmath>

#include "ops.h"
#include "quant_dev.h"

namespace aq {
namespace {

// ------------------------------------------------------------------------------------------------ embedding
// model.rs:364-368 `embed_token_into` -> quant.rs:102-133 `dequant_q4_k`: y = (d*sc)*q - (dmin*m) per element,
// read from the Q4_K planes (sub-block s, position p = 4l + b: nibble of qa[slot(l)*16 + (s/2)*4 + b]).
__global__ void __launch_bounds__(256) embed_q4k_kernel(Weight w, const uint32_t *ids, float *out, size_t out_stride) {
    const size_t i = blockIdx.y, sb = blockIdx.x;
    size_t row = ids[i];
    if (row >= w.rows) row = w.rows - 1; // ids are validated by the host; keep every access in bounds regardless
    const int e = threadIdx.x, s = e >> 5, p = e & 31, l = p >> 2, b = p & 3;
    const uint8_t byte = w.qa[kq_qa_off(row, sb, w.nb, l) + (s >> 1) * 4 + b];
    const int q = (s & 1) ? (byte >> 4) : (byte & 0xF);
    const uint8_t *rec = w.sc + kq_sc_off(row, sb, w.nb);
    const float d = f16_to_f32((uint16_t)(rec[0] | (rec[1] << 8)));
    const float dmin = f16_to_f32((uint16_t)(rec[2] | (rec[3] << 8)));
    const uint8_t *sc12 = rec + 4;
    int sc, m;
    if (s < 4) { // quant.rs:45-51 get_scale_min_k4
        sc = sc12[s] & 63;
        m = sc12[s + 4] & 63;
    } else {
        sc = (sc12[s + 4] & 0xF) | ((sc12[s - 4] >> 6) << 4);
        m = (sc12[s + 4] >> 4) | ((sc12[s] >> 6) << 4);
    }
    const float d1 = d * (float)sc, m1 = dmin * (float)m;
    out[i * out_stride + sb * 256 + e] = d1 * (float)q - m1;
}

// -------------------------------------------------------------------------------------------------- rmsnorm
// rmsnorm.rs:25-76: ss = reduce8 of 8 interleaved sequential lanes (+ sequential tail), mean = ss/n,
// inv = 1/sqrt(mean + eps), y = (x*inv)*w. One work-group per row; the row sits in LDS; 8 threads run the
// 8 lane chains. Then the quantised form is written from LDS.
__global__ void __launch_bounds__(256) rmsnorm_kernel(const float *x, size_t x_stride, const float *w, float eps, int n,
                                                      float *y, size_t y_stride, Act qa, int kind, size_t col0,
                                                      size_t eoff, int act_f32) {
    extern __shared__ float xs[]; // 2n + 16: the row, 16 partials, the weights
    float *red = xs + n;
    const int row = blockIdx.x, tid = threadIdx.x;
    float *wsh = red + 16; // the norm weights, staged like the row
    copy_rows_in(xs, x + (size_t)row * x_stride, n, tid, 256);
    copy_rows_in(wsh, w, n, tid, 256);
    __syncthreads();
    const int n8 = n / 8 * 8;
    if (tid < 8) red[tid] = seq_sum<true>(xs, tid, n8, 8, 0.0f);
    __syncthreads();
    if (tid == 0) {
        float ss = reduce8_f(red);
        for (int i = n8; i < n; i++) ss += xs[i] * xs[i];
        const float mean = ss / (float)n;
        red[8] = 1.0f / sqrtf(mean + eps);
    }
    __syncthreads();
    const float inv = red[8];
    for (int i = tid; i < n; i += 256) {
        const float v = (xs[i] * inv) * wsh[i];
        xs[i] = v;
        if (y) y[(size_t)row * y_stride + i] = v;
        if (act_f32) qa.f32[(col0 + row) * qa.n + eoff + i] = v;
    }
    __syncthreads();
    if (kind == QK_Q8K) {
        const int wave = tid >> 6, lane = tid & 63;
        for (int blk = wave; blk < n / 256; blk += 4) {
            const float v4[4] = {xs[blk * 256 + lane * 4], xs[blk * 256 + lane * 4 + 1], xs[blk * 256 + lane * 4 + 2],
                                 xs[blk * 256 + lane * 4 + 3]};
            q8k_block_store(qa, col0 + row, eoff / 256 + blk, v4, lane);
        }
    } else if (kind == QK_Q80) {
        for (int blk = tid; blk < n / 32; blk += 256) q8_0_block_store(qa, col0 + row, eoff / 32 + blk, xs + blk * 32);
    }
}

// The same, for rows of float4s (the model's shapes), 512 threads: each thread keeps its float4s of x and w in
// registers from the first load to the output; the squares go to LDS transposed (chain l's terms contiguous); the 8
// chain lanes add 24 terms from registers while the next 24 are read, so only the adds (about 4.5 cycles each) are
// on the critical path, not the LDS latency. Work-group (row, slice) computes the whole chain of its row and then
// writes only its slice of the normalised row (whole 256-blocks), so the quantiser work spreads over the slices'
// work-groups; with Q8_K output, wave w holds whole 256-blocks (its float4s are block w + 8r, lane order), so the
// quantiser runs on registers.
constexpr int RN_THREADS = 512, RN_ROUNDS = 8; // n <= 4 * 512 * 8
// float4 rounds per thread an instance needs: with 8 lanes per chain (PL < 0) a chain holds at most 8 * -PL terms,
// so n / 4 <= 16 * -PL + 1 (the vector path takes n % 4 == 0, the chains n8 = n / 8 * 8 elements)
__host__ __device__ constexpr int rn_rounds(int pl) {
    return pl < 0 ? (16 * -pl + 1 + RN_THREADS - 1) / RN_THREADS : RN_ROUNDS;
}

__host__ __device__ inline int rn_chain_stride(int n) { // floats per chain row in LDS: 4 (mod 32), 16-byte rows
    const int clen = n / 8;
    return (clen + 31) / 32 * 32 + 4;
}

// FR (with PL < 0 and n a multiple of 256): a one-dimensional grid, the t x nslice norm work-groups first, then
// t x 8 ceil(nrows / 8) work-groups each forming row g of the F32 matrices in `fr` over normalised row c instead of
// writing a slice. Work-group i runs on XCD i mod 8 (the dispatcher's round robin), so the F32-rows index puts the
// t work-groups of one row g on one XCD: 8 rows x t columns per group of 8 t, column-major within the group.
template <int PL, bool FR = false>
__global__ void __launch_bounds__(RN_THREADS) rmsnorm_vec_kernel(const float *x, size_t x_stride, const float *w,
                                                                 float eps, int n, float *y, size_t y_stride, Act qa,
                                                                 int kind, size_t col0, size_t eoff, int act_f32,
                                                                 const float *x2, size_t x2_stride, const float *w2,
                                                                 size_t eoff2, int nslice, NormRows fr) {
    if (blockIdx.z == 1) { // a pair launch: the second input, its norm weights and its place in the output row
        x = x2;
        x_stride = x2_stride;
        w = w2;
        eoff = eoff2;
    }
    extern __shared__ float sm[]; // 8 chains of squares, 16 floats, then (Q8_0 output only) the normalised row
    const int tid = threadIdx.x, lane = tid & 63;
    int row = blockIdx.x, ys = blockIdx.y; // the input row, and the slice (>= nslice: F32 row ys - nslice)
    if constexpr (FR) {
        const int id = (int)blockIdx.x, nn = nslice * fr.t;
        if (id < nn) {
            row = id % fr.t;
            ys = id / fr.t;
        } else {
            const int k = id - nn, grp = k / (8 * fr.t), rem = k % (8 * fr.t);
            row = rem / 8;
            ys = nslice + grp * 8 + rem % 8;
        }
    }
    const int n4 = n >> 2, n8 = n / 8 * 8, clen = n8 / 8, cs = rn_chain_stride(n);
    const bool frw = FR && ys >= nslice; // uniform: an F32-rows work-group
    const int g = ys - nslice;
    if (frw && g >= fr.rows[0] && g >= fr.rows[1]) return; // past both matrices' rows (uniform)
    // this work-group's slice of the output: float4s [o0, o1), whole 256-blocks (an F32-rows one: the whole row)
    const int nblk = n4 / 64;
    const int o0 = !frw && nslice > 1 ? ys * nblk / nslice * 64 : 0;
    const int o1 = !frw && nslice > 1 ? (ys + 1) * nblk / nslice * 64 : n4;
    float *sq = sm, *red = sm + 8 * cs, *xs = red + 16;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)row * x_stride);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    constexpr int R = rn_rounds(PL);
    float4 xv[R], wv[R], fv[FR ? 2 : 1][R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int i4 = tid + r * RN_THREADS;
        if (i4 < n4) xv[r] = x4[i4];
        if (i4 >= o0 && i4 < o1) wv[r] = w4[i4]; // the norm weights of this work-group's slice only
        if constexpr (FR) {
#pragma unroll
            for (int i = 0; i < 2; i++)
                if (frw && g < fr.rows[i] && i4 < n4) {
                    // weights read once per pass (94 MB over the 27B shape's 48 layers): non-temporal, like the
                    // matmuls' weights, so the DeltaNet state and the KV rows stay in the memory-side cache
                    const uint4 u = ld_nt4(reinterpret_cast<const uint8_t *>(fr.w[i] + (size_t)g * n) + (size_t)i4 * 16);
                    fv[i][r] = make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z),
                                           __uint_as_float(u.w));
                }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int i4 = tid + r * RN_THREADS;
        if (i4 < n4) {
            const float c[4] = {xv[r].x, xv[r].y, xv[r].z, xv[r].w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int e = 4 * i4 + k;
                if (e < n8) sq[(e & 7) * cs + (e >> 3)] = c[k] * c[k];
            }
        }
    }
    __syncthreads();
    if constexpr (PL < 0) {
        // all 8 chains in wave 0, each on its own SIMD pass: chain c in lanes 8c..8c+7, lane 8c+j holds the chain's
        // terms T*j .. T*j + T - 1 in registers (zeros past the chain's end); after each lane's terms the running
        // sum moves one lane up (DPP row shift), so lane 8c+7 ends with chain c summed in order. One wave on its
        // SIMD issues an add every pass; chains in 8 waves would share each SIMD between two of them.
        constexpr int T = -PL;
        static_assert(T % 4 == 0, "whole float4s of terms per lane");
        if (tid < 64) {
            const int c = lane >> 3, j = lane & 7;
            const float4 *src = reinterpret_cast<const float4 *>(sq + c * cs + T * j);
            float r[T];
#pragma unroll
            for (int k = 0; k < T / 4; k++) {
                // clen is a multiple of 4 on this path, so a float4 lies wholly inside or outside the chain
                const float4 f = T * j + 4 * k < clen ? src[k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                r[4 * k] = f.x;
                r[4 * k + 1] = f.y;
                r[4 * k + 2] = f.z;
                r[4 * k + 3] = f.w;
            }
            float acc = 0.0f;
#pragma unroll
            for (int m = 0; m < 8; m++) {
                if (m > 0) acc = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc),
                                                                                      0x111, 0xF, 0xF, false));
#pragma unroll
                for (int k = 0; k < T; k++) acc += r[k];
            }
            if (j == 7) red[c] = acc;
        }
    } else if constexpr (PL > 0) {
        // chain w runs in wave w: lane m holds the chain's terms PL*m .. PL*m + PL - 1 in registers; the running sum
        // moves one lane up after each lane's terms (DPP wave shift), so lane 63 ends with the whole chain, summed in
        // order with every term an add of a register (no LDS read on the chain's path)
        const int wave = tid >> 6;
        float acc = 0.0f;
        if (wave < 8) {
            const float *c = sq + wave * cs + PL * lane;
            float r[PL];
#pragma unroll
            for (int k = 0; k < PL; k++) r[k] = PL * lane + k < clen ? c[k] : 0.0f;
#pragma unroll 4
            for (int m = 0; m < 64; m++) {
                if (m > 0) acc = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc),
                                                                                      0x138, 0xF, 0xF, false));
#pragma unroll
                for (int k = 0; k < PL; k++) acc += r[k];
            }
        }
        if (lane == 63 && wave < 8) red[wave] = acc;
    } else if (tid < 8) { // chain tid, 6 float4s per batch from LDS, two batches in flight
        const float *c = sq + tid * cs;
        const float4 *c4 = reinterpret_cast<const float4 *>(c);
        const int nq = clen / 4;
        float acc = 0.0f;
        constexpr int B = 6; // at most 15 LDS reads may be waited for one by one (the counter's width)
        // whole double batches without guards (a guard per term costs a branch), then the remaining float4s
        const int nfull = nq / (2 * B) * (2 * B);
        auto rd = [&](float4 *buf, int v0) {
#pragma unroll
            for (int k = 0; k < B; k++) buf[k] = c4[v0 + k];
        };
        auto add = [&](const float4 *buf) {
#pragma unroll
            for (int k = 0; k < B; k++) {
                acc += buf[k].x;
                acc += buf[k].y;
                acc += buf[k].z;
                acc += buf[k].w;
            }
        };
        if (nfull > 0) {
            float4 ba[B], bb[B];
            rd(ba, 0);
            for (int v0 = 0; v0 < nfull; v0 += 2 * B) {
                rd(bb, v0 + B);
                add(ba);
                if (v0 + 2 * B < nfull) rd(ba, v0 + 2 * B);
                add(bb);
            }
        }
        for (int v = nfull; v < nq; v++) {
            const float4 f = c4[v];
            acc += f.x;
            acc += f.y;
            acc += f.z;
            acc += f.w;
        }
        for (int u = nq * 4; u < clen; u++) acc += c[u];
        red[tid] = acc;
    }
    __syncthreads();
    if (tid == 0) {
        float ss = reduce8_f(red);
        const float *xr = x + (size_t)row * x_stride;
        for (int i = n8; i < n; i++) ss += xr[i] * xr[i];
        const float mean = ss / (float)n;
        red[8] = 1.0f / sqrtf(mean + eps);
    }
    __syncthreads();
    const float inv = red[8];
    if constexpr (FR) {
        if (frw) {
            // dot.rs:180-200 over the normalised row (the values the slices write): the 32-element block b is the
            // float4s 8b..8b+7, held by lanes 8k..8k+7 of one wave in element order; its partial is summed left to
            // right from 0 by passing the running sum one lane up (DPP row shift) after each lane's four products,
            // so lane 8k+7 ends with it. Then the partials are added block by block in one chain per matrix (below),
            // and the empty tail's `acc + part` (+0.0f).
            const int nb32 = n / 32;
            float *part = sq; // the chains are summed (the barrier above)
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int i4 = tid + r * RN_THREADS;
                if (i4 < n4) { // n4 is a multiple of 64 here: wave-uniform, every lane of the wave on the DPP path
                    const float v[4] = {(xv[r].x * inv) * wv[r].x, (xv[r].y * inv) * wv[r].y,
                                        (xv[r].z * inv) * wv[r].z, (xv[r].w * inv) * wv[r].w};
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        if (g >= fr.rows[i]) continue; // uniform
                        const float p[4] = {fv[i][r].x * v[0], fv[i][r].y * v[1], fv[i][r].z * v[2],
                                            fv[i][r].w * v[3]};
                        float acc = 0.0f;
#pragma unroll
                        for (int m = 0; m < 8; m++) {
                            if (m > 0)
                                acc = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                                    0, __builtin_bit_cast(int, acc), 0x111, 0xF, 0xF,
                                                                    false));
#pragma unroll
                            for (int k = 0; k < 4; k++) acc += p[k];
                        }
                        if ((lane & 7) == 7) part[i * nb32 + (i4 >> 3)] = acc;
                    }
                }
            }
            __syncthreads();
            // matrix i's chain in lanes 8i..8i+7 of wave 0: lane 8i + j holds partials jS..jS+S-1 in registers
            // (+0.0f past the row's n / 32 <= -PL / 4 * 8 blocks: the sum from +0.0f is never -0.0f, so they change
            // nothing), the running sum passed one lane up after each lane's terms, so lane 8i + 7 ends with it
            if (tid < 16) {
                constexpr int S = PL < 0 ? -PL / 4 : 1;
                const int i = tid >> 3, j = tid & 7;
                const float *pc = part + i * nb32 + j * S;
                float rv[S];
#pragma unroll
                for (int k = 0; k < S; k++) rv[k] = j * S + k < nb32 ? pc[k] : 0.0f;
                float acc = 0.0f;
#pragma unroll
                for (int m = 0; m < 8; m++) {
                    if (m > 0)
                        acc = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, acc),
                                                                                   0x111, 0xF, 0xF, false));
#pragma unroll
                    for (int k = 0; k < S; k++) acc += rv[k];
                }
                const int rows_i = i ? fr.rows[1] : fr.rows[0];
                if (j == 7 && g < rows_i) (i ? fr.y[1] : fr.y[0])[(size_t)row * rows_i + g] = acc + 0.0f;
            }
            return;
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int i4 = tid + r * RN_THREADS;
        // n4 is a multiple of 64 when the output is Q8_K: the conditions are wave-uniform there
        if (i4 < n4 && i4 >= o0 && i4 < o1) {
            const float v[4] = {(xv[r].x * inv) * wv[r].x, (xv[r].y * inv) * wv[r].y, (xv[r].z * inv) * wv[r].z,
                                (xv[r].w * inv) * wv[r].w};
            const float4 v4 = make_float4(v[0], v[1], v[2], v[3]);
            if (y) *reinterpret_cast<float4 *>(y + (size_t)row * y_stride + 4 * i4) = v4;
            if (act_f32) *reinterpret_cast<float4 *>(qa.f32 + (col0 + row) * qa.n + eoff + 4 * i4) = v4;
            if (kind == QK_Q8K) q8k_block_store(qa, col0 + row, eoff / 256 + (i4 >> 6), v, lane);
            if (kind == QK_Q80) reinterpret_cast<float4 *>(xs)[i4] = v4;
        }
    }
    if (kind == QK_Q80) {
        // one lane per element, a half wave per 32-block: the slice is whole 256-blocks, so each pass of the loop
        // is whole half waves (the last pass may leave whole waves idle)
        __syncthreads();
        for (int e = 4 * o0 + tid; e < 4 * o1; e += RN_THREADS)
            q8_0_block_half(qa, col0 + row, (size_t)(eoff + e) / 32, xs[e], lane);
    }
}

// --------------------------------------------------------------------------------------------------- swiglu
// act.rs:24-30: h = silu(g) * u. Q8_K: one wave per 256-block; Q8_0 / none: one lane per element, a half wave per
// 32-block.
__global__ void __launch_bounds__(256) swiglu_q8k_kernel(const float *g, const float *u, size_t n, size_t total,
                                                         float *h, Act qa, size_t col0) {
    const int lane = threadIdx.x & 63;
    const size_t blk = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= total) return;
    const size_t nb = n / 256, row = blk / nb, b = blk % nb;
    const size_t e = row * n + b * 256 + lane * 4;
    const float4 gv = *reinterpret_cast<const float4 *>(g + e), uv = *reinterpret_cast<const float4 *>(u + e);
    const float v[4] = {silu_f(gv.x) * uv.x, silu_f(gv.y) * uv.y, silu_f(gv.z) * uv.z, silu_f(gv.w) * uv.w};
    if (h) *reinterpret_cast<float4 *>(h + e) = make_float4(v[0], v[1], v[2], v[3]);
    q8k_block_store(qa, col0 + row, b, v, lane);
}

__global__ void __launch_bounds__(256) swiglu_q80_kernel(const float *g, const float *u, size_t n, size_t total,
                                                         float *h, Act qa, size_t col0, int quant) {
    // one lane per element, one Q8_0 block per 32-lane half wave (n % 32 == 0, so a half never spans two blocks and
    // is past the end as a whole or not at all); the block's d, codes and code sum by the half's reductions
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x, blk = e / 32;
    const bool live = blk < total;
    const int lane = (int)(threadIdx.x & 63);
    float v = 0.0f;
    if (live) {
        v = silu_f(g[e]) * u[e];
        if (h) h[e] = v;
    }
    const size_t nb = n / 32, row = blk / nb, b = blk % nb;
    if (quant && live) q8_0_block_half(qa, col0 + row, b, v, lane); // `live` is uniform over each half wave
}

// ------------------------------------------------------------------------------------------ Gated DeltaNet
// One work-group of 512 threads per V head p (K head p % nk, gated_deltanet.rs:172). Per row
// (gated_deltanet.rs:261-375, deltanet.rs:19-86, conv.rs:11-36):
//   conv step + SiLU of the head's q/k/v channels; l2norm(q), l2norm(k) (eps 1e-6, sequential sums);
//   q *= 1/sqrt(dk); g = ssm_a * softplus(a + dt_bias); beta = sigmoid(b);
//   S *= exp(g); kv = sum_k S[k][v] k[k]; delta = (v - kv) beta; S[k][v] += k[k] delta; o = sum_k S[k][v] q[k];
//   y = (w * (o * inv_rms(o))) * silu(z)  (rmsnorm.rs:37-46).
// Only the recurrence is sequential over rows, so everything else runs for all rows at once, each sum still in
// the reference's order:
//   A  every thread: conv + SiLU of whole channels over all rows, silu(z), and the 32-element alpha/beta partials
//      (dot.rs:180-200);
//   B  waves 4 and 6: the 2t l2norm sums, 8 lanes per sum; waves 5 and 7: the alpha / beta block chains, then the
//      decays / betas per row; waves 0-3: the state column of thread j (S[.][j], registers) is loaded meanwhile;
//   C  thread j < dv: the recurrence of column j, row after row, with no barrier between rows;
//   D  wave 0: the output RMS of each row (8 lanes of the reduce8 pattern per row); thread j < dv: the gated
//      output, and its Q8_0 form per half wave.
// The state is written back only when asked (write_state); the conv windows go to conv_dst (a second buffer, so
// work-groups sharing a K head never read a window another one has already advanced): v channels by every head,
// q/k channels by head p == kh.
constexpr int DN_TMAX = 8;      // rows per DeltaNet launch
constexpr int DN_THREADS = 512; // waves 0-3 hold state columns (dv <= 256); 4-6 run the per-row sums

// Parts per state column in the recurrence: as many as the work-group holds (H * DV <= DN_THREADS), at most four,
// with whole float4s of keys per part.
template <int DK, int DV>
constexpr int dn_parts() {
    return (4 * DV <= DN_THREADS && DK % 16 == 0) ? 4 : (2 * DV <= DN_THREADS && DK % 8 == 0) ? 2 : 1;
}

template <int DK, int DV>
constexpr int dn_kh() { return DK / dn_parts<DK, DV>(); }

// Rows r0 .. r0 + t - 1 (t <= DN_TMAX) of the launch's rows. `s` is the thread's part of the state column: loaded
// from a.rec when `first`, written back when `last` (and a.write_state), carried in registers between the pieces of
// one launch otherwise. The conv window of a piece after the first is the three input rows before it. TT > 0: the
// row count is TT (the input loops run over exactly those rows), else t_in.
template <int DK, int DV, bool CHUNK = false, int TT = 0>
__device__ __forceinline__ void dn_core_body(const DnArgs &a, const int p, const int t_in, float (&s)[dn_kh<DK, DV>()],
                                             const int r0, const bool first, const bool last) {
    static_assert(TT >= 0 && TT <= DN_TMAX, "rows per launch");
    constexpr int TM = TT ? TT : DN_TMAX; // the input loops' bound
    const int t = TT ? TT : t_in;
    // CHUNK: the host admits no raw rows, so that path compiles away
    const bool raw_ = !CHUNK && a.raw;
    static_assert(DK <= 256 && DV <= 256 && DN_THREADS >= 448 && DN_TMAX * 2 <= 16, "DeltaNet work-group shape");
    __shared__ float sq[DN_TMAX][DK], sk[DN_TMAX][DK], sv[DN_TMAX][DV], sz[DN_TMAX][DV], so[DN_TMAX][DV];
    __shared__ float rdec[DN_TMAX], rbeta[DN_TMAX], rq[DN_TMAX], rk[DN_TMAX], ro[DN_TMAX];
    const int j = threadIdx.x, lane = j & 63, wave = j >> 6;
    const int kh = p % a.nk;
    const int kd = a.nk * DK, vd = a.nv * DV, cd = 2 * kd + vd;
    const bool gated = a.out && !raw_;
    // the gate inputs, loaded before phase A so their latency hides behind it: wave 5 computes the decays and
    // wave 7 the betas (lane i = row i), each in its own wave so neither waits for the other's branch
    const bool gate_lane = (wave == 5 || wave == 7) && lane < t;
    const int gr = wave == 5 ? 0 : 1;
    float gv = 0.0f, gsa = 0.0f, gdt = 0.0f;
    if (gate_lane) {
        gv = raw_ ? (gr == 0 ? a.rg : a.rbeta)[(size_t)(r0 + lane) * a.nv + p]
                  : (gr == 0 ? a.a : a.b)[(size_t)(r0 + lane) * a.nv + p];
        if (gr == 0 && !raw_) {
            gsa = a.ssm_a[p];
            gdt = a.dt_bias[p];
        }
    }
    const float nrm_w = gated && j < t * DV ? a.ssm_norm[j % DV] : 0.0f; // phase D's norm weight (thread's column)
    // the state column, split by key: thread j holds keys [h KH, h KH + KH) of column c = j % DV, part h = j / DV;
    // its loads are issued first, so their latency passes under phase A's loads (both are latency-bound phases)
    constexpr int H = dn_parts<DK, DV>(), KH = DK / H;
    const int c = j % DV, h = j / DV;
    const bool has_col = h < H;
    float *srec = a.rec + (size_t)p * DK * DV;
    if (has_col && first) {
#pragma unroll
        for (int k = 0; k < KH; k++) s[k] = srec[(size_t)(h * KH + k) * DV + c];
    }

    // ---- A: channels over all rows
    if (raw_) {
        for (int e = j; e < t * DK; e += DN_THREADS) {
            const int i = e / DK, c = e % DK;
            sq[i][c] = a.rq[(size_t)(r0 + i) * kd + kh * DK + c];
            sk[i][c] = a.rk[(size_t)(r0 + i) * kd + kh * DK + c];
        }
        for (int e = j; e < t * DV; e += DN_THREADS) {
            const int i = e / DV, c = e % DV;
            sv[i][c] = a.rv[(size_t)(r0 + i) * vd + p * DV + c];
        }
    } else {
        // task c: q channel c (c < DK), k channel c - DK, v channel c - 2 DK (conv, conv.rs:11-36), then the
        // z channels (silu only)
        const int n_conv = 2 * DK + DV, n_task = n_conv + (gated ? DV : 0);
        for (int c = j; c < n_task; c += DN_THREADS) {
            if (c < n_conv) {
                const int kind = c < DK ? 0 : c < 2 * DK ? 1 : 2;
                const int cc = kind == 2 ? c - 2 * DK : c - kind * DK;
                const int ch = kind == 0 ? kh * DK + cc : kind == 1 ? kd + kh * DK + cc : 2 * kd + p * DV + cc;
                float seq[TM + 3];
#pragma unroll
                for (int e = 0; e < 3; e++)
                    seq[e] = first ? a.conv_src[(size_t)ch * 3 + e] : a.mixed[(size_t)(r0 - 3 + e) * cd + ch];
                float cw[4];
#pragma unroll
                for (int e = 0; e < 4; e++) cw[e] = a.conv_w[(size_t)ch * 4 + e];
#pragma unroll
                for (int i = 0; i < TM; i++) seq[3 + i] = a.mixed[(size_t)(r0 + (i < t ? i : t - 1)) * cd + ch];
                float *dst = kind == 0 ? &sq[0][cc] : kind == 1 ? &sk[0][cc] : &sv[0][cc];
                const int dstride = kind == 2 ? DV : DK;
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    if (i < t) {
                        float acc = 0.0f;
                        acc += cw[0] * seq[i];
                        acc += cw[1] * seq[i + 1];
                        acc += cw[2] * seq[i + 2];
                        acc += cw[3] * seq[i + 3];
                        dst[i * dstride] = silu_f(acc);
                    }
                }
                if (a.conv_dst && last && (kind == 2 || p == kh)) {
#pragma unroll
                    for (int i = 0; i <= TM; i++) // the window after row t - 1: seq[t .. t + 2]
                        if (i == t)
                            for (int e = 0; e < 3; e++) a.conv_dst[(size_t)ch * 3 + e] = seq[i + e];
                }
            } else {
                const int cc = c - n_conv;
                float zr[TM];
#pragma unroll
                for (int i = 0; i < TM; i++) zr[i] = a.z[(size_t)(r0 + (i < t ? i : t - 1)) * vd + p * DV + cc];
#pragma unroll
                for (int i = 0; i < TM; i++)
                    if (i < t) sz[i][cc] = silu_f(zr[i]);
            }
        }
    }
    __syncthreads();

    // ---- B: norms (waves 4 and 6) and gates (waves 5 and 7)
    if constexpr (DK % 32 == 0) {
        // chain c = the sum of squares of q (c even) or k (c odd) of row c / 2, in 8 lanes of wave 4 (chains 0-7) or
        // 6 (8-15): lane m of the chain holds its terms m*T .. m*T + T - 1 as registers and the running sum moves
        // one lane up after each lane's terms (DPP row shift), so lane 7 of the group ends with the whole sum,
        // added in order
        if ((wave == 4 || wave == 6) && !raw_) {
            constexpr int T = DK / 8;
            const int c = (wave == 4 ? 0 : 8) + (lane >> 3), m = lane & 7, cc = c < 2 * t ? c : 0;
            const float4 *x4 = reinterpret_cast<const float4 *>((cc & 1) ? sk[cc >> 1] : sq[cc >> 1]) + m * (T / 4);
            float r[T];
#pragma unroll
            for (int u = 0; u < T / 4; u++) {
                const float4 f = x4[u];
                r[4 * u] = f.x * f.x;
                r[4 * u + 1] = f.y * f.y;
                r[4 * u + 2] = f.z * f.z;
                r[4 * u + 3] = f.w * f.w;
            }
            float ss = 0.0f;
#pragma unroll
            for (int st = 0; st < 8; st++) {
                if (st > 0) ss = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, ss),
                                                                                      0x111, 0xF, 0xF, false));
#pragma unroll
                for (int u = 0; u < T; u++) ss += r[u];
            }
            if (m == 7 && c < 2 * t) {
                const float inv = 1.0f / sqrtf(ss + 1e-6f); // deltanet.rs:19-29 l2norm
                if (c & 1)
                    rk[c >> 1] = inv;
                else
                    rq[c >> 1] = inv;
            }
        }
    } else if (wave == 4 && !raw_ && lane < 2 * t) { // one sum per lane
        const int i = lane >> 1;
        const float ss = seq_sum<true>((lane & 1) ? sk[i] : sq[i], 0, DK, 1, 0.0f);
        const float inv = 1.0f / sqrtf(ss + 1e-6f); // deltanet.rs:19-29 l2norm
        if (lane & 1)
            rk[i] = inv;
        else
            rq[i] = inv;
    }
    if (gate_lane) {
        const int i = lane;
        const float v = gv;
        if (gr == 0) {
            const float g = raw_ ? v : gsa * softplus_f(v + gdt); // deltanet.rs:32-35 gate_g
            rdec[i] = exp_f(g);
        } else {
            rbeta[i] = raw_ ? v : sigmoid_f(v);
        }
    }
    __syncthreads();
    if (!raw_) {
        for (int e = j; e < t * DK; e += DN_THREADS) {
            const int i = e / DK, cc = e % DK;
            sq[i][cc] = (sq[i][cc] * rq[i]) * a.qscale;
            sk[i][cc] = sk[i][cc] * rk[i];
        }
        __syncthreads();
    }

    // ---- C: the recurrence of column c (deltanet.rs:43-86), row after row. Each part updates its keys' state and
    // forms their products in parallel (S *= decay, S k; then S += k delta, S q); the two sums over k stay one
    // left-to-right chain from 0, handed from part to part in key order through LDS, so kv and o are the
    // reference's sequential sums. Every thread meets the barriers. The two sums hand over through separate
    // slots, so the next row's kv hand-off never overwrites an o hand-off still being read.
    __shared__ float xfer[DV], xfer2[DV], xdelta[DV];
    for (int i = 0; i < t; i++) {
        float pk[KH];
        float kv = 0.0f;
        const float4 *k4 = reinterpret_cast<const float4 *>(sk[i] + h * KH);
        const float4 *q4 = reinterpret_cast<const float4 *>(sq[i] + h * KH);
        if (has_col) {
            const float decay = rdec[i];
#pragma unroll
            for (int u = 0; u < KH / 4; u++) {
                const float4 kb = k4[u];
                const float kk[4] = {kb.x, kb.y, kb.z, kb.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    s[4 * u + e] *= decay;
                    pk[4 * u + e] = s[4 * u + e] * kk[e];
                }
            }
        }
#pragma unroll
        for (int hh = 0; hh < H; hh++) {
            if (has_col && h == hh) {
                if (hh > 0) kv = xfer[c];
#pragma unroll
                for (int k = 0; k < KH; k++) kv += pk[k];
                if (hh + 1 < H) xfer[c] = kv;
                else xdelta[c] = (sv[i][c] - kv) * rbeta[i];
            }
            __syncthreads();
        }
        float ov = 0.0f;
        if (has_col) {
            const float delta = xdelta[c];
#pragma unroll
            for (int u = 0; u < KH / 4; u++) {
                const float4 kb = k4[u], qb = q4[u];
                const float kk[4] = {kb.x, kb.y, kb.z, kb.w}, qq[4] = {qb.x, qb.y, qb.z, qb.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    s[4 * u + e] += kk[e] * delta;
                    pk[4 * u + e] = s[4 * u + e] * qq[e];
                }
            }
        }
#pragma unroll
        for (int hh = 0; hh < H; hh++) {
            if (has_col && h == hh) {
                if (hh > 0) ov = xfer2[c];
#pragma unroll
                for (int k = 0; k < KH; k++) ov += pk[k];
                if (hh + 1 < H) {
                    xfer2[c] = ov;
                } else if (raw_) {
                    if (a.out) a.out[(size_t)(r0 + i) * vd + p * DV + c] = ov;
                } else {
                    so[i][c] = ov;
                }
            }
            if (hh + 1 < H) __syncthreads();
        }
    }
    if (has_col && a.write_state && last) {
#pragma unroll
        for (int k = 0; k < KH; k++) srec[(size_t)(h * KH + k) * DV + c] = s[k];
    }

    // ---- D: gated RMSNorm of each output row
    if (gated) {
        __syncthreads();
        if (wave == 0) {
            constexpr int n8 = DV / 8 * 8;
            const int i = lane >> 3, m = lane & 7;
            const float part8 = i < t ? seq_sum<true>(so[i < t ? i : 0], m, n8, 8, 0.0f) : 0.0f;
            // reduce8 on the DPP network: lane m + (l_m + l_m+4), then lanes 0, 1 + the pair two up, then lane 0
            // + lane 1: ((l0 + l4) + (l2 + l6)) + ((l1 + l5) + (l3 + l7))
            float r8 = part8;
            r8 = r8 + __int_as_float(dpp_mov<0x104>(__float_as_int(r8))); // row_shl:4
            r8 = r8 + __int_as_float(dpp_mov<0x102>(__float_as_int(r8))); // row_shl:2
            r8 = r8 + __int_as_float(dpp_mov<0x101>(__float_as_int(r8))); // row_shl:1
            if (m == 0 && i < t) {
                float ss = r8;
                for (int e = n8; e < DV; e++) ss += so[i][e] * so[i][e];
                ro[i] = 1.0f / sqrtf(ss / (float)DV + a.eps);
            }
        }
        __syncthreads();
        // the gated output, and with out_q80 its Q8_0 form (quant.rs quantize_q8_0): thread j takes row j / DV,
        // column j % DV (rows past DN_THREADS / DV in further passes); the head's rows are whole 32-blocks, one per
        // half wave (uniform over each half wave: DV % 32 == 0)
        for (int e = j; e < t * DV; e += DN_THREADS) {
            const int i = e / DV, jc = e % DV;
            const float w = e == j ? nrm_w : a.ssm_norm[jc];
            const float v = (w * (so[i][jc] * ro[i])) * sz[i][jc];
            a.out[(size_t)(r0 + i) * vd + p * DV + jc] = v;
            if (a.out_q80) q8_0_block_half(a.q80, r0 + i, (size_t)p * (DV / 32) + (jc >> 5), v, lane);
        }
    }
}

// TT > 0: a.t == TT rows (the verify's k + 1 and decode's 1 take such an instance), else any row count up to 8
template <int DK, int DV, int TT>
__global__ void __launch_bounds__(DN_THREADS) dn_core_kernel(DnArgs a) {
    float s[dn_kh<DK, DV>()];
    dn_core_body<DK, DV, false, TT>(a, (int)blockIdx.x, a.t, s, 0, true, true);
}

// A prompt chunk of more than DN_TMAX rows in one launch (gated_deltanet.rs:197-199 steps the recurrence token by
// token): pieces of DN_TMAX rows in order, the state column kept in registers from piece to piece and each piece's
// conv window taken from the three input rows before it.
template <int DK, int DV>
__global__ void __launch_bounds__(DN_THREADS) dn_core_chunk_kernel(DnArgs a) {
    float s[dn_kh<DK, DV>()];
    for (int r0 = 0; r0 < a.t; r0 += DN_TMAX) {
        if (r0 > 0) __syncthreads(); // the previous piece's LDS rows are read to the end before they are rewritten
        const int tp = a.t - r0 < DN_TMAX ? a.t - r0 : DN_TMAX;
        dn_core_body<DK, DV, true>(a, (int)blockIdx.x, tp, s, r0, r0 == 0, r0 + DN_TMAX >= a.t);
    }
}

// Several layers' heads in one launch (the commit of every DeltaNet layer after a speculative round): work-group
// (p, y) runs head p of args[y]; the row count is read on the device when t_dev is set.
template <int DK, int DV>
__global__ void __launch_bounds__(DN_THREADS) dn_core_multi_kernel(const DnArgs *args) {
    const DnArgs &a = args[blockIdx.y];
    const int t = a.t_dev ? (int)*a.t_dev : a.t;
    if (t < 1 || t > DN_TMAX) return; // uniform: a row count the host validates before it is used
    float s[dn_kh<DK, DV>()];
    dn_core_body<DK, DV>(a, (int)blockIdx.x, t, s, 0, true, true);
}

// ---------------------------------------------------------------------------------------------- attention
// gqa_attention.rs:327-418 per row: q/k per-head RMSNorm (rmsnorm.rs) then RoPE on the first rope_dim dims
// (rope.rs:31-45: pairs (i, i + rd/2)); K and V appended to the cache. One work-group per (head, row).
__global__ void __launch_bounds__(256) attn_prep_kernel(AttnArgs a) {
    __shared__ float xs[256], red[16];
    const int hh = blockIdx.x, i = blockIdx.y, d = threadIdx.x, hd = a.hd;
    const bool isq = hh < a.nh;
    const float *src = isq ? a.qg + (size_t)i * 2 * a.nh * hd + (size_t)hh * 2 * hd
                           : a.kk + (size_t)i * a.nkv * hd + (size_t)(hh - a.nh) * hd;
    const float *w = isq ? a.q_norm : a.k_norm;
    xs[d] = src[d];
    __syncthreads();
    const int n8 = hd / 8 * 8;
    if (d < 8) red[d] = seq_sum<true>(xs, d, n8, 8, 0.0f);
    __syncthreads();
    if (d == 0) {
        float ss = reduce8_f(red);
        for (int e = n8; e < hd; e++) ss += xs[e] * xs[e];
        red[8] = 1.0f / sqrtf(ss / (float)hd + a.eps);
    }
    __syncthreads();
    const float y = (xs[d] * red[8]) * w[d];
    __syncthreads();
    xs[d] = y;
    __syncthreads();
    const int half = a.rd / 2;
    const size_t pos = a.start_pos + i;
    const float *cs = a.cos_tab + pos * half, *sn = a.sin_tab + pos * half;
    float r = y;
    if (d < half) {
        r = xs[d] * cs[d] - xs[d + half] * sn[d];
    } else if (d < a.rd) {
        const int e = d - half;
        r = xs[d] * cs[e] + xs[e] * sn[e];
    }
    if (isq) {
        a.q[(size_t)i * a.nh * hd + (size_t)hh * hd + d] = r;
    } else {
        const int kvh = hh - a.nh;
        const size_t crow = a.base + i;
        a.kcache[crow * a.stride + (size_t)kvh * hd + d] = r;
        a.vcache[crow * a.stride + (size_t)kvh * hd + d] = a.vv[(size_t)i * a.nkv * hd + (size_t)kvh * hd + d];
    }
}

// Scores (sequential dot over head_dim, times scaling), softmax (softmax.rs:22-49: max, exp, 8-lane sum, divide),
// weighted V sum (sequential over positions), times sigmoid(gate).
// GSC: the score row lives in device memory (a.gsc) instead of LDS, for contexts past attn_lds_positions; the
// arithmetic and its order are the same.
template <bool GSC>
__global__ void __launch_bounds__(256) attn_core_kernel(AttnArgs a) {
    extern __shared__ float sm[]; // hd + (base + t, unless GSC) + 32
    const int h = blockIdx.x, i = blockIdx.y, tid = threadIdx.x, hd = a.hd;
    const int kvh = h / (a.nh / a.nkv);
    const size_t len = a.base + i + 1;
    float *qs = sm;
    float *sc = GSC ? a.gsc + ((size_t)i * a.nh + h) * a.gsc_stride : sm + hd;
    float *red = GSC ? sm + hd : sc + a.base + a.t;
    for (int d = tid; d < hd; d += 256) qs[d] = a.q[(size_t)i * a.nh * hd + (size_t)h * hd + d];
    __syncthreads();
    float mx = -INFINITY;
    for (size_t tt = tid; tt < len; tt += 256) {
        const float *kr = a.kcache + tt * a.stride + (size_t)kvh * hd;
        float acc = 0.0f;
        int d = 0;
        // 16 float4s in flight while the previous 16 are summed (double buffer); the sum stays sequential in d
        const float4 *k4 = reinterpret_cast<const float4 *>(kr);
        const int ng = hd / 64;
        float4 ka[16], kb[16];
        if (ng > 0) {
#pragma unroll
            for (int u = 0; u < 16; u++) ka[u] = k4[u];
        }
        for (int g = 0; g < ng; g++) {
            if (g + 1 < ng) {
#pragma unroll
                for (int u = 0; u < 16; u++) kb[u] = k4[(g + 1) * 16 + u];
            }
            const float *qg = qs + g * 64;
#pragma unroll
            for (int u = 0; u < 16; u++) {
                acc += qg[4 * u] * ka[u].x;
                acc += qg[4 * u + 1] * ka[u].y;
                acc += qg[4 * u + 2] * ka[u].z;
                acc += qg[4 * u + 3] * ka[u].w;
            }
#pragma unroll
            for (int u = 0; u < 16; u++) ka[u] = kb[u];
        }
        d = ng * 64;
        for (; d < hd; d += 8) { // hd % 8 == 0
            const float4 k0 = *reinterpret_cast<const float4 *>(kr + d);
            const float4 k1 = *reinterpret_cast<const float4 *>(kr + d + 4);
            acc += qs[d] * k0.x;
            acc += qs[d + 1] * k0.y;
            acc += qs[d + 2] * k0.z;
            acc += qs[d + 3] * k0.w;
            acc += qs[d + 4] * k1.x;
            acc += qs[d + 5] * k1.y;
            acc += qs[d + 6] * k1.z;
            acc += qs[d + 7] * k1.w;
        }
        const float v = acc * a.scaling;
        sc[tt] = v;
        mx = v > mx ? v : mx;
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(mx, off);
        mx = o > mx ? o : mx;
    }
    if ((tid & 63) == 0) red[16 + (tid >> 6)] = mx;
    __syncthreads();
    mx = red[16];
    for (int wv = 1; wv < 4; wv++) mx = red[16 + wv] > mx ? red[16 + wv] : mx;
    for (size_t tt = tid; tt < len; tt += 256) sc[tt] = exp_f(sc[tt] - mx);
    __syncthreads();
    const size_t n8 = len / 8 * 8;
    if (tid < 8) red[tid] = seq_sum<false>(sc, tid, (int)n8, 8, 0.0f);
    __syncthreads();
    if (tid == 0) {
        float s = reduce8_f(red);
        for (size_t e = n8; e < len; e++) s += sc[e];
        red[8] = s;
    }
    __syncthreads();
    const float ssum = red[8];
    for (size_t tt = tid; tt < len; tt += 256) sc[tt] = sc[tt] / ssum;
    __syncthreads();
    for (int d = tid; d < hd; d += 256) {
        const float *vc = a.vcache + (size_t)kvh * hd + d;
        float acc = 0.0f;
        // 16 positions' loads in flight while the previous 16 are summed (double buffer); the sum stays
        // sequential in tt. The last batch may be partial: its loads are clamped to the last position (all issued
        // together, like a full batch's) and only the positions before len are added.
        constexpr int VB = 16;
        const size_t ng = (len + VB - 1) / VB;
        float va[VB], vb[VB];
        auto vload = [&](float *buf, size_t g) {
#pragma unroll
            for (int u = 0; u < VB; u++) {
                const size_t tt = g * VB + u;
                buf[u] = vc[(tt < len ? tt : len - 1) * a.stride];
            }
        };
        vload(va, 0);
        for (size_t g = 0; g < ng; g++) {
            if (g + 1 < ng) vload(vb, g + 1);
            if ((g + 1) * VB <= len) {
#pragma unroll
                for (int u = 0; u < VB; u++) acc += sc[g * VB + u] * va[u];
            } else {
#pragma unroll
                for (int u = 0; u < VB; u++)
                    if (g * VB + u < len) acc += sc[g * VB + u] * va[u];
            }
#pragma unroll
            for (int u = 0; u < VB; u++) va[u] = vb[u];
        }
        const float gate = a.qg[(size_t)i * 2 * a.nh * hd + (size_t)h * 2 * hd + hd + d];
        const float o = acc * sigmoid_f(gate);
        a.out[(size_t)i * a.nh * hd + (size_t)h * hd + d] = o;
        if (a.out_q8k) qs[d] = o; // q is no longer read
    }
    if (a.out_q8k) { // uniform: this head's output row is block h of row i's Q8_K form (hd == 256)
        __syncthreads();
        if (tid < 64) {
            const float v[4] = {qs[4 * tid], qs[4 * tid + 1], qs[4 * tid + 2], qs[4 * tid + 3]};
            q8k_block_store(a.q8k, i, h, v, tid);
        }
    }
}

// ------------------------------------------------------------------------------------------------- argmax
constexpr size_t ARGMAX_CHUNK = 2048;

__device__ __forceinline__ void amax_merge(float &bv, uint32_t &bi, float ov, uint32_t oi) {
    if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
    }
}

__device__ __forceinline__ void amax_block(float &bv, uint32_t &bi, float *sv, uint32_t *si) {
    for (int off = 32; off >= 1; off >>= 1) amax_merge(bv, bi, __shfl_xor(bv, off), __shfl_xor(bi, off));
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) amax_merge(bv, bi, sv[w], si[w]);
    }
}

__global__ void __launch_bounds__(256) argmax_partial_kernel(const float *x, size_t n, size_t stride, float *pv,
                                                             uint32_t *pi, int nchunk) {
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    const int c = blockIdx.x, r = blockIdx.y;
    const float *xr = x + (size_t)r * stride;
    const size_t lo = (size_t)c * ARGMAX_CHUNK, hi = lo + ARGMAX_CHUNK < n ? lo + ARGMAX_CHUNK : n;
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (size_t e = lo + threadIdx.x; e < hi; e += 8 * 256) { // 8 loads in flight per thread
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = e + u * 256 < hi ? xr[e + u * 256] : -INFINITY;
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (e + u * 256 < hi) amax_merge(bv, bi, v[u], (uint32_t)(e + u * 256));
    }
    amax_block(bv, bi, sv, si);
    if (threadIdx.x == 0) {
        pv[(size_t)r * nchunk + c] = bv;
        pi[(size_t)r * nchunk + c] = bi;
    }
}

// model.rs:505-513: best = 0, replaced by i only when v[i] > v[best]. So a NaN never replaces the best, a NaN at
// index 0 is never replaced (the answer is 0), and among equal maxima the first wins. The partial kernels skip NaN
// (a comparison with NaN is false); here the row's first value decides the NaN case.
__global__ void __launch_bounds__(64) argmax_final_kernel(const float *x, size_t stride, const float *pv,
                                                          const uint32_t *pi, int nchunk, uint32_t *ids) {
    __shared__ float sv[1];
    __shared__ uint32_t si[1];
    const int r = blockIdx.x;
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (int c = threadIdx.x; c < nchunk; c += 64) amax_merge(bv, bi, pv[(size_t)r * nchunk + c], pi[(size_t)r * nchunk + c]);
    amax_block(bv, bi, sv, si);
    if (threadIdx.x == 0) {
        const float v0 = x[(size_t)r * stride];
        ids[r] = (v0 != v0 || bi == 0xFFFFFFFFu) ? 0u : bi;
    }
}

// -------------------------------------------------------------------------------------------- acceptance
// spec.rs:355-366: walk the drafts while the verify argmax agrees; emit the verify argmax at each step, plus the
// bonus token when every draft was accepted.
__global__ void accept_kernel(const uint32_t *ids, const uint32_t *drafts, int k, uint32_t *emitted, uint32_t *info) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    int m = 0, ne = 0;
    while (m < k) {
        const uint32_t a = ids[m];
        emitted[ne++] = a;
        if (a != drafts[m]) break;
        m++;
    }
    if (m == k) emitted[ne++] = ids[k];
    info[0] = (uint32_t)m;
    info[1] = (uint32_t)ne;
    info[2] = (uint32_t)(m + 1);
}

__global__ void make_batch_kernel(uint32_t x_p, const uint32_t *drafts, int k, uint32_t *batch) {
    const int i = threadIdx.x;
    if (i == 0) batch[0] = x_p;
    else if (i <= k) batch[i] = drafts[i - 1];
}

// fn: 0 exp, 1 log1p, 2 silu, 3 sigmoid, 4 softplus (the device forms every kernel above uses)
__global__ void eval_math_kernel(int fn, const float *x, float *y, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    float r;
    switch (fn) {
    case 0: r = exp_f(v); break;
    case 1: r = aq_log1pf(v); break;
    case 2: r = silu_f(v); break;
    case 3: r = sigmoid_f(v); break;
    default: r = softplus_f(v); break;
    }
    y[i] = r;
}

int launched(const char *what) {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail(AQ_EHIP, std::string(what) + " launch: " + hipGetErrorString(e));
}

} // namespace

int launch_embed(const Weight &w, const uint32_t *ids, size_t t, float *out, size_t out_stride, hipStream_t stream) {
    AQ_REQUIRE(w.type == AQ_TYPE_Q4_K, "embed: token_embd must be Q4_K in this build");
    if (t == 0) return 0;
    hipLaunchKernelGGL(embed_q4k_kernel, dim3((unsigned)w.nb, (unsigned)t), dim3(256), 0, stream, w, ids, out, out_stride);
    return launched("embed");
}

// Chain terms per lane of the vector kernel for rows of n: 8 lanes per chain in one wave when a chain is whole
// float4s and fits (negative counts), else one wave per chain (the smallest built count that holds a chain), else 0
// (the chains read from LDS).
static int rn_pick_pl(size_t n) {
    const int clen = (int)(n / 8), need8 = (clen + 7) / 8, need = (clen + 63) / 64;
    const int t8s[] = {4, 8, 16, 24, 32, 48, 64, 80, 96};
    const int pls[] = {1, 2, 4, 6, 8, 10, 12, 16};
    int pl = 0;
    if (clen % 4 == 0)
        for (int c : t8s)
            if (!pl && c >= need8) pl = -c;
    for (int c : pls)
        if (!pl && c >= need) pl = c;
    return pl;
}

bool rmsnorm_rows_fit(size_t n) {
    return n > 0 && n % 256 == 0 && n <= (size_t)4 * RN_THREADS * RN_ROUNDS && rn_pick_pl(n) < 0 &&
           ((size_t)8 * rn_chain_stride((int)n) + 16) * sizeof(float) <= 65536;
}

// x2 set: a pair launch (grid z = 2), the second input normalised with w2 into elements eoff2.. of the same output
// rows; it needs the vector kernel, and falls back to two launches where that does not apply. fr set: the F32 rows
// of fr by work-groups past the slices (grid y), in the same launch.
static int rmsnorm_launch(const float *x, size_t x_stride, const float *w, float eps, size_t n, size_t t, float *y_f32,
                          size_t y_stride, const QuantOut &q, hipStream_t stream, const float *x2, size_t x2_stride,
                          const float *w2, size_t eoff2, const NormRows *fr = nullptr) {
    AQ_REQUIRE(n > 0 && n <= 16384, "rmsnorm: row length must be 1..16384");
    if (t == 0) return 0;
    if (x2) {
        AQ_REQUIRE(q.act && !y_f32, "rmsnorm pair: the output is the quantised rows only");
        // the second input's place in the output rows, checked as the first's is below
        AQ_REQUIRE(eoff2 + n <= q.act->n, "rmsnorm pair: quantised output out of range");
        AQ_REQUIRE(q.kind != QK_Q8K || eoff2 % 256 == 0, "rmsnorm pair: Q8_K needs 256-blocks");
        AQ_REQUIRE(q.kind != QK_Q80 || eoff2 % 32 == 0, "rmsnorm pair: Q8_0 needs 32-blocks");
    }
    Act act{};
    if (q.act) {
        act = *q.act;
        AQ_REQUIRE(q.col0 + t <= act.ncols && q.elem_off + n <= act.n, "rmsnorm: quantised output out of range");
        AQ_REQUIRE(q.kind != QK_Q8K || (n % 256 == 0 && q.elem_off % 256 == 0), "rmsnorm: Q8_K needs 256-blocks");
        AQ_REQUIRE(q.kind != QK_Q80 || (n % 32 == 0 && q.elem_off % 32 == 0), "rmsnorm: Q8_0 needs 32-blocks");
    } else {
        AQ_REQUIRE(q.kind == QK_NONE && !q.f32, "rmsnorm: quantised output without a buffer");
    }
    const auto al16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    const bool vec = n % 4 == 0 && n <= 4 * RN_THREADS * RN_ROUNDS && x_stride % 4 == 0 && al16(x) && al16(w) &&
                     (!y_f32 || (y_stride % 4 == 0 && al16(y_f32))) &&
                     (!q.f32 || (act.n % 4 == 0 && q.elem_off % 4 == 0 && al16(act.f32))) &&
                     (!x2 || (x2_stride % 4 == 0 && al16(x2) && al16(w2) && (!q.f32 || eoff2 % 4 == 0)));
    const size_t vshmem = ((size_t)8 * rn_chain_stride((int)n) + 16 + (q.kind == QK_Q80 ? n : 0)) * sizeof(float);
    if (x2 && !(vec && vshmem <= 65536)) { // the pair as two launches
        QuantOut q2 = q;
        q2.elem_off = eoff2;
        const int rc = rmsnorm_launch(x, x_stride, w, eps, n, t, nullptr, 0, q, stream, nullptr, 0, nullptr, 0);
        return rc ? rc : rmsnorm_launch(x2, x2_stride, w2, eps, n, t, nullptr, 0, q2, stream, nullptr, 0, nullptr, 0);
    }
    int nfr = 0;
    if (fr) {
        AQ_REQUIRE(!x2 && !y_f32 && vec && rmsnorm_rows_fit(n), "rmsnorm rows: unsupported shape");
        for (int i = 0; i < 2; i++) {
            AQ_REQUIRE(fr->rows[i] >= 0 && fr->rows[i] <= 4096, "rmsnorm rows: row count");
            AQ_REQUIRE(!fr->rows[i] || (fr->w[i] && fr->y[i] && al16(fr->w[i])), "rmsnorm rows: buffers");
            nfr = fr->rows[i] > nfr ? fr->rows[i] : nfr;
        }
    }
    if (vec && vshmem <= 65536) {
        const size_t shmem = vshmem;
        // slices of whole 256-blocks (about five blocks each) when the row is made of them
        const int nblk = n % 256 == 0 ? (int)(n / 256) : 0;
        const unsigned slices = nblk >= 8 ? (unsigned)((nblk + 4) / 5) : 1;
        const int pl = rn_pick_pl(n);
        AQ_REQUIRE(n / 4 <= (size_t)rn_rounds(pl) * RN_THREADS, "rmsnorm: row longer than the kernel's rounds");
        const dim3 grid = fr ? dim3((unsigned)(t * (slices + 8 * ((nfr + 7) / 8)))) // the F32-rows index, in the kernel
                             : dim3((unsigned)t, slices, x2 ? 2u : 1u);
        if (!x2) { // the kernel's second-input arguments, unread with one input
            x2 = x;
            x2_stride = x_stride;
            w2 = w;
            eoff2 = q.elem_off;
        }
        NormRows frv = fr ? *fr : NormRows{};
        frv.t = (int)t;
        if (fr) {
            switch (pl) {
#define AQ_RNF(P)                                                                                             \
    case P:                                                                                                   \
        hipLaunchKernelGGL((rmsnorm_vec_kernel<P, true>), grid, dim3(RN_THREADS), shmem, stream, x, x_stride, w, eps, \
                           (int)n, y_f32, y_stride, act, (int)q.kind, q.col0, q.elem_off, q.f32 ? 1 : 0, x2,        \
                           x2_stride, w2, eoff2, (int)slices, frv);                                           \
        break;
                AQ_RNF(-4) AQ_RNF(-8) AQ_RNF(-16) AQ_RNF(-24) AQ_RNF(-32) AQ_RNF(-48) AQ_RNF(-64) AQ_RNF(-80) AQ_RNF(-96)
#undef AQ_RNF
            default: return fail(AQ_EUNSUP, "rmsnorm rows: chain form");
            }
            return launched("rmsnorm rows");
        }
        switch (pl) {
#define AQ_RN(P)                                                                                              \
    case P:                                                                                                   \
        hipLaunchKernelGGL((rmsnorm_vec_kernel<P>), grid, dim3(RN_THREADS), shmem, stream, x, x_stride, w, eps, (int)n, \
                           y_f32, y_stride, act, (int)q.kind, q.col0, q.elem_off, q.f32 ? 1 : 0, x2, x2_stride, w2,  \
                           eoff2, (int)slices, frv);                                                          \
        break;
            AQ_RN(0) AQ_RN(1) AQ_RN(2) AQ_RN(4) AQ_RN(6) AQ_RN(8) AQ_RN(10) AQ_RN(12) AQ_RN(16)
            AQ_RN(-4) AQ_RN(-8) AQ_RN(-16) AQ_RN(-24) AQ_RN(-32) AQ_RN(-48) AQ_RN(-64) AQ_RN(-80) AQ_RN(-96)
#undef AQ_RN
        }
        return launched("rmsnorm");
    }
    const size_t shmem = (2 * n + 16) * sizeof(float);
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)t), dim3(256), shmem, stream, x, x_stride, w, eps, (int)n, y_f32,
                       y_stride, act, (int)q.kind, q.col0, q.elem_off, q.f32 ? 1 : 0);
    return launched("rmsnorm");
}

int launch_rmsnorm(const float *x, size_t x_stride, const float *w, float eps, size_t n, size_t t, float *y_f32,
                   size_t y_stride, const QuantOut &q, hipStream_t stream) {
    return rmsnorm_launch(x, x_stride, w, eps, n, t, y_f32, y_stride, q, stream, nullptr, 0, nullptr, 0);
}

int launch_rmsnorm_rows(const float *x, size_t x_stride, const float *w, float eps, size_t n, size_t t,
                        const QuantOut &q, const NormRows &fr, hipStream_t stream) {
    return rmsnorm_launch(x, x_stride, w, eps, n, t, nullptr, 0, q, stream, nullptr, 0, nullptr, 0, &fr);
}

int launch_rmsnorm_pair(const float *x, size_t x_stride, const float *w, const float *x2, size_t x2_stride,
                        const float *w2, size_t eoff2, float eps, size_t n, size_t t, const QuantOut &q,
                        hipStream_t stream) {
    AQ_REQUIRE(x2 && w2, "rmsnorm pair: no second input");
    return rmsnorm_launch(x, x_stride, w, eps, n, t, nullptr, 0, q, stream, x2, x2_stride, w2, eoff2);
}

int launch_swiglu(const float *g, const float *u, size_t n, size_t t, float *h_f32, const QuantOut &q,
                  hipStream_t stream) {
    if (t == 0) return 0;
    Act act{};
    if (q.act) {
        act = *q.act;
        AQ_REQUIRE(q.col0 + t <= act.ncols && q.elem_off == 0 && n == act.n, "swiglu: quantised output shape");
    }
    if (q.kind == QK_Q8K) {
        AQ_REQUIRE(n % 256 == 0, "swiglu: Q8_K needs n % 256 == 0");
        const size_t total = t * (n / 256);
        hipLaunchKernelGGL(swiglu_q8k_kernel, dim3((unsigned)((total + 3) / 4)), dim3(256), 0, stream, g, u, n, total,
                           h_f32, act, q.col0);
    } else {
        AQ_REQUIRE(n % 32 == 0, "swiglu: n % 32 != 0");
        AQ_REQUIRE(q.kind == QK_Q80 || h_f32, "swiglu: no output");
        const size_t total = t * (n / 32);
        hipLaunchKernelGGL(swiglu_q80_kernel, dim3((unsigned)((total * 32 + 255) / 256)), dim3(256), 0, stream, g, u,
                           n, total, h_f32, act, q.col0, q.kind == QK_Q80 ? 1 : 0);
    }
    return launched("swiglu");
}

int launch_dn_core(const DnArgs &a, hipStream_t stream) {
    AQ_REQUIRE(a.t >= 1 && a.nk >= 1 && a.nv >= 1 && a.nv % a.nk == 0, "deltanet: head counts");
    AQ_REQUIRE(a.dv >= 1 && a.dv <= 256, "deltanet: head_dim_v must be 1..256");
    AQ_REQUIRE(a.rec, "deltanet: no state");
    if (!a.raw) {
        AQ_REQUIRE(a.kernel == 4, "deltanet: conv kernel must be 4 in this build");
        AQ_REQUIRE(a.mixed && a.a && a.b && a.conv_src && a.conv_w && a.ssm_a && a.dt_bias, "deltanet: inputs");
        AQ_REQUIRE(!a.out || (a.z && a.ssm_norm), "deltanet: output needs z and ssm_norm");
        AQ_REQUIRE(!a.out_q80 || (a.out && a.dv % 32 == 0 && a.q80.q0 && a.q80.n == (size_t)a.nv * a.dv &&
                                  a.q80.ncols >= (size_t)a.t),
                   "deltanet: Q8_0 output needs whole 32-blocks and a buffer of t rows of nv * dv");
    } else {
        AQ_REQUIRE(a.rq && a.rk && a.rv && a.rg && a.rbeta, "deltanet: raw inputs");
    }
    AQ_REQUIRE(a.t <= DN_TMAX || (!a.raw && a.t <= 4096),
               "deltanet: more than 8 rows in one launch need the projected gates (no raw mode) and t <= 4096");
    AQ_REQUIRE(a.raw || (a.a && a.b), "deltanet: gate inputs");
    const int threads = DN_THREADS;
    const int key = a.dk * 1000 + a.dv;
    switch (key) {
#define AQ_DN(K, V)                                                                                           \
    case K * 1000 + V:                                                                                        \
        if (a.t == 4)                                                                                         \
            hipLaunchKernelGGL((dn_core_kernel<K, V, 4>), dim3((unsigned)a.nv), dim3(threads), 0, stream, a);  \
        else if (a.t == 1)                                                                                    \
            hipLaunchKernelGGL((dn_core_kernel<K, V, 1>), dim3((unsigned)a.nv), dim3(threads), 0, stream, a);  \
        else if (a.t <= DN_TMAX)                                                                              \
            hipLaunchKernelGGL((dn_core_kernel<K, V, 0>), dim3((unsigned)a.nv), dim3(threads), 0, stream, a);  \
        else                                                                                                  \
            hipLaunchKernelGGL((dn_core_chunk_kernel<K, V>), dim3((unsigned)a.nv), dim3(threads), 0, stream, a); \
        break;
        AQ_DN(8, 8) AQ_DN(16, 16) AQ_DN(32, 32) AQ_DN(64, 64) AQ_DN(128, 128) AQ_DN(128, 256) AQ_DN(64, 128)
#undef AQ_DN
    default: return fail(AQ_EUNSUP, "deltanet: head dims (k, v) not built: " + std::to_string(a.dk) + ", " +
                                        std::to_string(a.dv));
    }
    return launched("deltanet");
}

int launch_dn_core_multi(const DnArgs *args_dev, const DnArgs &like, int n, hipStream_t stream) {
    AQ_REQUIRE(n >= 1 && args_dev, "deltanet: no layers");
    AQ_REQUIRE(!like.raw && !like.out, "deltanet multi: commit form only (saved gates, no output)");
    const int key = like.dk * 1000 + like.dv;
    switch (key) {
#define AQ_DN(K, V)                                                                                           \
    case K * 1000 + V:                                                                                        \
        hipLaunchKernelGGL((dn_core_multi_kernel<K, V>), dim3((unsigned)like.nv, (unsigned)n), dim3(DN_THREADS), 0, \
                           stream, args_dev);                                                                 \
        break;
        AQ_DN(8, 8) AQ_DN(16, 16) AQ_DN(32, 32) AQ_DN(64, 64) AQ_DN(128, 128) AQ_DN(128, 256) AQ_DN(64, 128)
#undef AQ_DN
    default: return fail(AQ_EUNSUP, "deltanet: head dims (k, v) not built: " + std::to_string(like.dk) + ", " +
                                        std::to_string(like.dv));
    }
    return launched("deltanet multi");
}

int launch_attention(const AttnArgs &a, hipStream_t stream) {
    AQ_REQUIRE(a.t >= 1 && a.nh >= 1 && a.nkv >= 1 && a.nh % a.nkv == 0, "attention: head counts");
    AQ_REQUIRE(a.hd >= 8 && a.hd <= 256 && a.hd % 8 == 0, "attention: head_dim must be a multiple of 8, <= 256");
    AQ_REQUIRE(a.rd >= 2 && a.rd <= a.hd && a.rd % 2 == 0, "attention: rope_dim");
    hipLaunchKernelGGL(attn_prep_kernel, dim3((unsigned)(a.nh + a.nkv), (unsigned)a.t), dim3(a.hd), 0, stream, a);
    int rc = launched("attention prologue");
    if (rc) return rc;
    AQ_REQUIRE(!a.out_q8k || (a.hd == 256 && a.q8k.qs && a.q8k.n == (size_t)a.nh * 256 && a.q8k.ncols >= (size_t)a.t),
               "attention: Q8_K output needs head_dim 256 and a buffer of t rows of nh * 256");
    if (a.base + a.t <= attn_lds_positions(a.hd)) {
        const size_t shmem = (a.hd + a.base + a.t + 32) * sizeof(float);
        hipLaunchKernelGGL(attn_core_kernel<false>, dim3((unsigned)a.nh, (unsigned)a.t), dim3(256), shmem, stream, a);
    } else {
        AQ_REQUIRE(a.gsc && a.base + a.t <= a.gsc_stride, "attention: context longer than the state's score rows");
        const size_t shmem = (a.hd + 32) * sizeof(float);
        hipLaunchKernelGGL(attn_core_kernel<true>, dim3((unsigned)a.nh, (unsigned)a.t), dim3(256), shmem, stream, a);
    }
    return launched("attention");
}

size_t attn_lds_positions(int hd) { return 65536 / sizeof(float) - (size_t)hd - 32; }

size_t argmax_scratch_bytes(size_t n, size_t t) {
    const size_t nchunk = (n + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK;
    return t * nchunk * 8 + 256;
}

int launch_argmax(const float *x, size_t n, size_t stride, size_t t, uint32_t *ids, void *scratch, hipStream_t stream) {
    AQ_REQUIRE(n >= 1 && t >= 1, "argmax: empty");
    const int nchunk = (int)((n + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK);
    float *pv = (float *)scratch;
    uint32_t *pi = (uint32_t *)((uint8_t *)scratch + ((t * nchunk * 4 + 255) & ~(size_t)255));
    hipLaunchKernelGGL(argmax_partial_kernel, dim3((unsigned)nchunk, (unsigned)t), dim3(256), 0, stream, x, n, stride,
                       pv, pi, nchunk);
    int rc = launched("argmax");
    if (rc) return rc;
    hipLaunchKernelGGL(argmax_final_kernel, dim3((unsigned)t), dim3(64), 0, stream, x, stride, pv, pi, nchunk, ids);
    return launched("argmax final");
}

int launch_accept(const uint32_t *argmax_ids, const uint32_t *drafts, int k, uint32_t *emitted, uint32_t *info,
                  hipStream_t stream) {
    hipLaunchKernelGGL(accept_kernel, dim3(1), dim3(64), 0, stream, argmax_ids, drafts, k, emitted, info);
    return launched("accept");
}

int launch_eval_math(int fn, const float *x, float *y, size_t n, hipStream_t stream) {
    AQ_REQUIRE(fn >= 0 && fn <= 4, "eval_math: fn must be 0..4");
    if (n == 0) return 0;
    hipLaunchKernelGGL(eval_math_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, fn, x, y, n);
    return launched("eval_math");
}

int launch_make_batch(uint32_t x_p, const uint32_t *drafts, int k, uint32_t *batch, hipStream_t stream) {
    AQ_REQUIRE(k >= 0 && k < 64, "make_batch: k");
    hipLaunchKernelGGL(make_batch_kernel, dim3(1), dim3(64), 0, stream, x_p, drafts, k, batch);
    return launched("make_batch");
}

} // namespace aq
