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
    const size_t wsb = row * w.nb + sb;
    const int e = threadIdx.x, s = e >> 5, p = e & 31, l = p >> 2, b = p & 3;
    const uint8_t byte = w.qa[wsb * 128 + lane_slot(l) * 16 + (s >> 1) * 4 + b];
    const int q = (s & 1) ? (byte >> 4) : (byte & 0xF);
    const uint8_t *rec = w.sc + wsb * 16;
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

// --------------------------------------------------------------------------------------------------- swiglu
// act.rs:24-30: h = silu(g) * u. Q8_K: one wave per 256-block; Q8_0 / none: one lane per 32-block.
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
    const size_t blk = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= total) return;
    const size_t nb = n / 32, row = blk / nb, b = blk % nb;
    const size_t e = row * n + b * 32;
    float v[32], gv[32], uv[32];
#pragma unroll
    for (int i = 0; i < 32; i++) {
        gv[i] = g[e + i];
        uv[i] = u[e + i];
    }
    for (int i = 0; i < 32; i++) v[i] = silu_f(gv[i]) * uv[i];
    if (h)
        for (int i = 0; i < 32; i++) h[e + i] = v[i];
    if (quant) q8_0_block_store(qa, col0 + row, b, v);
}

// ------------------------------------------------------------------------------------------ Gated DeltaNet
// One work-group per V head p (K head p % nk, gated_deltanet.rs:172); thread j owns column j of the head's
// state S[k][v] (row-major, dk x dv) in registers, and the conv windows of channels q_j, k_j, v_j.
// Per row (gated_deltanet.rs:261-375, deltanet.rs:19-86, conv.rs:11-36):
//   conv step + SiLU of the head's q/k/v channels; l2norm(q), l2norm(k) (eps 1e-6, sequential sums);
//   q *= 1/sqrt(dk); g = ssm_a * softplus(a + dt_bias); beta = sigmoid(b);
//   S *= exp(g); kv = sum_k S[k][v] k[k]; delta = (v - kv) beta; S[k][v] += k[k] delta; o = sum_k S[k][v] q[k];
//   y = (w * (o * inv_rms(o))) * silu(z)  (rmsnorm.rs:37-46).
// Each column's sums run in its own thread in the reference's order. The state is written back only when asked
// (write_state); the conv windows go to conv_dst (a second buffer, so work-groups sharing a K head never read a
// window another one has already advanced): v channels by every head, q/k channels by head p == kh.
__device__ __forceinline__ float conv_step(float win[3], const float c[4], float x) {
    float acc = 0.0f;
    acc += c[0] * win[0];
    acc += c[1] * win[1];
    acc += c[2] * win[2];
    acc += c[3] * x;
    win[0] = win[1];
    win[1] = win[2];
    win[2] = x;
    return silu_f(acc);
}

constexpr int DN_TMAX = 8;      // rows per DeltaNet launch
constexpr int DN_BLK_MAX = 256; // 32-blocks of the alpha/beta rows (hidden <= 8192)

template <int DK, int DV>
__global__ void __launch_bounds__(256) dn_core_kernel(DnArgs a) {
    constexpr int NT = ((DK > DV ? DK : DV) + 63) / 64 * 64;
    __shared__ float qn[DK], kn[DK], ob[DV], red[16];
    __shared__ float in_q[DN_TMAX][DK], in_k[DN_TMAX][DK], in_v[DN_TMAX][DV], in_z[DN_TMAX][DV];
    __shared__ float gab[2][DN_TMAX]; // per row: a (or g), b (or beta)
    const int p = blockIdx.x, j = threadIdx.x;
    const int kh = p % a.nk, t = a.t;
    const int kd = a.nk * DK, vd = a.nv * DV, cd = 2 * kd + vd;
    const bool has_qk = j < DK, has_v = j < DV;
    const int jq = has_qk ? j : 0, jv = has_v ? j : 0; // in-range indices for the lanes past a head's width
    const int chq = kh * DK + jq, chk = kd + kh * DK + jq, chv = 2 * kd + p * DV + jv;

    // ---- every row's inputs to LDS up front (one round trip instead of one per row)
    for (int i = 0; i < t; i++) {
        if (a.raw) {
            if (has_qk) {
                in_q[i][j] = a.rq[(size_t)i * kd + kh * DK + j];
                in_k[i][j] = a.rk[(size_t)i * kd + kh * DK + j];
            }
            if (has_v) in_v[i][j] = a.rv[(size_t)i * vd + p * DV + j];
        } else {
            const float *mrow = a.mixed + (size_t)i * cd;
            if (has_qk) {
                in_q[i][j] = mrow[chq];
                in_k[i][j] = mrow[chk];
            }
            if (has_v) {
                in_v[i][j] = mrow[chv];
                if (a.z) in_z[i][j] = a.z[(size_t)i * vd + p * DV + j];
            }
        }
    }
    if (a.raw) {
        if (j < t) {
            gab[0][j] = a.rg[(size_t)j * a.nv + p];
            gab[1][j] = a.rbeta[(size_t)j * a.nv + p];
        }
    } else if (!a.x) {
        if (j < t) {
            gab[0][j] = a.a[(size_t)j * a.nv + p];
            gab[1][j] = a.b[(size_t)j * a.nv + p];
        }
    } else {
        // gated_deltanet.rs:271-274 ssm_alpha / ssm_beta rows of this head on the t input rows, dot.rs:180-200:
        // 32-element partials left to right (one thread per block and row), then the block chain (one thread per
        // (row, input)), `acc + part` with the short tail (0.0f when there is none).
        __shared__ float part[2][DN_TMAX][DN_BLK_MAX];
        const int n = a.hidden, nblk = (n + 31) / 32;
        for (int task = j; task < 2 * nblk; task += NT) {
            const int r = task / nblk, b = task % nblk;
            const float *w = (r == 0 ? a.w_alpha : a.w_beta) + (size_t)p * n;
            const int e0 = b * 32, ne = n - e0 < 32 ? n - e0 : 32;
            float wv[32];
            if (ne == 32 && (n & 3) == 0) {
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const float4 f = *reinterpret_cast<const float4 *>(w + e0 + 4 * u);
                    wv[4 * u] = f.x;
                    wv[4 * u + 1] = f.y;
                    wv[4 * u + 2] = f.z;
                    wv[4 * u + 3] = f.w;
                }
                for (int i = 0; i < t; i++) {
                    const float *xr = a.x + (size_t)i * a.x_stride + e0;
                    float xv[32];
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        const float4 f = *reinterpret_cast<const float4 *>(xr + 4 * u);
                        xv[4 * u] = f.x;
                        xv[4 * u + 1] = f.y;
                        xv[4 * u + 2] = f.z;
                        xv[4 * u + 3] = f.w;
                    }
                    float pt = 0.0f;
#pragma unroll
                    for (int e = 0; e < 32; e++) pt += wv[e] * xv[e];
                    part[r][i][b] = pt;
                }
            } else {
                for (int i = 0; i < t; i++) {
                    const float *xr = a.x + (size_t)i * a.x_stride + e0;
                    float pt = 0.0f;
                    for (int e = 0; e < ne; e++) pt += w[e0 + e] * xr[e];
                    part[r][i][b] = pt;
                }
            }
        }
        __syncthreads();
        if (j < 2 * t) {
            const int r = j / t, i = j % t;
            float v = seq_sum<false>(&part[r][i][0], 0, nblk, 1, 0.0f);
            if (n % 32 == 0) v = v + 0.0f;
            gab[r][i] = v;
            (r == 0 ? a.a : a.b)[(size_t)i * a.nv + p] = v; // kept for the commit
        }
    }

    // ---- state and conv windows
    float wq[3] = {0, 0, 0}, wk[3] = {0, 0, 0}, wv[3] = {0, 0, 0};
    float cq[4] = {0, 0, 0, 0}, ck[4] = {0, 0, 0, 0}, cv[4] = {0, 0, 0, 0};
    if (!a.raw) {
        for (int e = 0; e < 3; e++) {
            wq[e] = a.conv_src[(size_t)chq * 3 + e];
            wk[e] = a.conv_src[(size_t)chk * 3 + e];
            wv[e] = a.conv_src[(size_t)chv * 3 + e];
        }
        for (int e = 0; e < 4; e++) {
            cq[e] = a.conv_w[(size_t)chq * 4 + e];
            ck[e] = a.conv_w[(size_t)chk * 4 + e];
            cv[e] = a.conv_w[(size_t)chv * 4 + e];
        }
    }
    float s[DK];
    float *srec = a.rec + (size_t)p * DK * DV;
#pragma unroll
    for (int k = 0; k < DK; k++) s[k] = srec[(size_t)k * DV + jv];
    const float big_a = a.raw ? 0.0f : a.ssm_a[p], dtb = a.raw ? 0.0f : a.dt_bias[p];
    const int tk = NT > 64 ? 64 : 1; // the k-norm chain runs in another wave when there is one
    __syncthreads();

    for (int i = 0; i < t; i++) {
        float vval = 0.0f;
        if (a.raw) {
            if (has_qk) {
                qn[j] = in_q[i][j];
                kn[j] = in_k[i][j];
            }
            if (has_v) vval = in_v[i][j];
        } else {
            if (has_qk) {
                qn[j] = conv_step(wq, cq, in_q[i][j]);
                kn[j] = conv_step(wk, ck, in_k[i][j]);
            }
            if (has_v) vval = conv_step(wv, cv, in_v[i][j]);
        }
        __syncthreads();
        float g, beta;
        if (a.raw) {
            g = gab[0][i];
            beta = gab[1][i];
        } else {
            if (j == 0 || j == tk) { // deltanet.rs:19-29 l2norm, eps 1e-6
                const float ss = seq_sum<true>(j == 0 ? qn : kn, 0, DK, 1, 0.0f);
                red[j == 0 ? 0 : 1] = 1.0f / sqrtf(ss + 1e-6f);
            }
            __syncthreads();
            if (has_qk) {
                const float qv = qn[j] * red[0];
                qn[j] = qv * a.qscale;
                kn[j] = kn[j] * red[1];
            }
            __syncthreads();
            g = big_a * softplus_f(gab[0][i] + dtb); // deltanet.rs:32-35 gate_g
            beta = sigmoid_f(gab[1][i]);
        }
        float ov = 0.0f;
        { // deltanet.rs:43-86, column j of the head's state
            const float decay = exp_f(g);
#pragma unroll
            for (int k = 0; k < DK; k++) s[k] *= decay;
            float kv = 0.0f;
#pragma unroll
            for (int k = 0; k < DK; k++) kv += s[k] * kn[k];
            const float delta = (vval - kv) * beta;
#pragma unroll
            for (int k = 0; k < DK; k++) s[k] += kn[k] * delta;
#pragma unroll
            for (int k = 0; k < DK; k++) ov += s[k] * qn[k];
        }
        if (a.out) {
            if (a.raw) {
                if (has_v) a.out[(size_t)i * vd + p * DV + j] = ov;
            } else {
                if (has_v) ob[j] = ov;
                __syncthreads();
                constexpr int n8 = DV / 8 * 8;
                if (j < 8) red[4 + j] = seq_sum<true>(ob, j, n8, 8, 0.0f);
                __syncthreads();
                if (j == 0) {
                    float ss = reduce8_f(red + 4);
                    for (int e = n8; e < DV; e++) ss += ob[e] * ob[e];
                    red[2] = 1.0f / sqrtf(ss / (float)DV + a.eps);
                }
                __syncthreads();
                if (has_v) {
                    const size_t o = (size_t)i * vd + p * DV + j;
                    a.out[o] = (a.ssm_norm[j] * (ov * red[2])) * silu_f(in_z[i][j]);
                }
            }
        }
        __syncthreads(); // qn, kn, ob, red are rewritten by the next row
    }
    if (a.write_state && has_v) {
#pragma unroll
        for (int k = 0; k < DK; k++) srec[(size_t)k * DV + j] = s[k];
    }
    if (a.conv_dst && !a.raw) {
        if (has_v)
            for (int e = 0; e < 3; e++) a.conv_dst[(size_t)chv * 3 + e] = wv[e];
        if (has_qk && p == kh)
            for (int e = 0; e < 3; e++) {
                a.conv_dst[(size_t)chq * 3 + e] = wq[e];
                a.conv_dst[(size_t)chk * 3 + e] = wk[e];
            }
    }
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
__global__ void __launch_bounds__(256) attn_core_kernel(AttnArgs a) {
    extern __shared__ float sm[]; // hd + (base + t) + 32
    const int h = blockIdx.x, i = blockIdx.y, tid = threadIdx.x, hd = a.hd;
    const int kvh = h / (a.nh / a.nkv);
    const size_t len = a.base + i + 1;
    float *qs = sm, *sc = sm + hd, *red = sc + a.base + a.t;
    for (int d = tid; d < hd; d += 256) qs[d] = a.q[(size_t)i * a.nh * hd + (size_t)h * hd + d];
    __syncthreads();
    float mx = -INFINITY;
    for (size_t tt = tid; tt < len; tt += 256) {
        const float *kr = a.kcache + tt * a.stride + (size_t)kvh * hd;
        float acc = 0.0f;
        int d = 0;
        for (; d + 32 <= hd; d += 32) { // 8 loads in flight; the sum stays sequential in d
            float4 kv4[8];
#pragma unroll
            for (int u = 0; u < 8; u++) kv4[u] = *reinterpret_cast<const float4 *>(kr + d + 4 * u);
#pragma unroll
            for (int u = 0; u < 8; u++) {
                acc += qs[d + 4 * u] * kv4[u].x;
                acc += qs[d + 4 * u + 1] * kv4[u].y;
                acc += qs[d + 4 * u + 2] * kv4[u].z;
                acc += qs[d + 4 * u + 3] * kv4[u].w;
            }
        }
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
        size_t tt = 0;
        for (; tt + 8 <= len; tt += 8) { // 8 loads in flight; the sum stays sequential in tt
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = vc[(tt + u) * a.stride];
#pragma unroll
            for (int u = 0; u < 8; u++) acc += sc[tt + u] * v[u];
        }
        for (; tt < len; tt++) acc += sc[tt] * vc[tt * a.stride];
        const float gate = a.qg[(size_t)i * 2 * a.nh * hd + (size_t)h * 2 * hd + hd + d];
        a.out[(size_t)i * a.nh * hd + (size_t)h * hd + d] = acc * sigmoid_f(gate);
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

__global__ void __launch_bounds__(64) argmax_final_kernel(const float *pv, const uint32_t *pi, int nchunk,
                                                          uint32_t *ids) {
    __shared__ float sv[1];
    __shared__ uint32_t si[1];
    const int r = blockIdx.x;
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (int c = threadIdx.x; c < nchunk; c += 64) amax_merge(bv, bi, pv[(size_t)r * nchunk + c], pi[(size_t)r * nchunk + c]);
    amax_block(bv, bi, sv, si);
    if (threadIdx.x == 0) ids[r] = bi == 0xFFFFFFFFu ? 0u : bi;
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

int launch_rmsnorm(const float *x, size_t x_stride, const float *w, float eps, size_t n, size_t t, float *y_f32,
                   size_t y_stride, const QuantOut &q, hipStream_t stream) {
    AQ_REQUIRE(n > 0 && n <= 16384, "rmsnorm: row length must be 1..16384");
    if (t == 0) return 0;
    Act act{};
    if (q.act) {
        act = *q.act;
        AQ_REQUIRE(q.col0 + t <= act.ncols && q.elem_off + n <= act.n, "rmsnorm: quantised output out of range");
        AQ_REQUIRE(q.kind != QK_Q8K || (n % 256 == 0 && q.elem_off % 256 == 0), "rmsnorm: Q8_K needs 256-blocks");
        AQ_REQUIRE(q.kind != QK_Q80 || (n % 32 == 0 && q.elem_off % 32 == 0), "rmsnorm: Q8_0 needs 32-blocks");
    } else {
        AQ_REQUIRE(q.kind == QK_NONE && !q.f32, "rmsnorm: quantised output without a buffer");
    }
    const size_t shmem = (2 * n + 16) * sizeof(float);
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)t), dim3(256), shmem, stream, x, x_stride, w, eps, (int)n, y_f32,
                       y_stride, act, (int)q.kind, q.col0, q.elem_off, q.f32 ? 1 : 0);
    return launched("rmsnorm");
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
        hipLaunchKernelGGL(swiglu_q80_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, g, u, n,
                           total, h_f32, act, q.col0, q.kind == QK_Q80 ? 1 : 0);
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
    } else {
        AQ_REQUIRE(a.rq && a.rk && a.rv && a.rg && a.rbeta, "deltanet: raw inputs");
    }
    AQ_REQUIRE(a.t <= DN_TMAX, "deltanet: at most 8 rows per launch");
    AQ_REQUIRE(a.raw || a.x || (a.a && a.b), "deltanet: gate inputs");
    AQ_REQUIRE(!a.x || (a.w_alpha && a.w_beta && a.a && a.b && a.hidden > 0 && a.hidden <= 32 * DN_BLK_MAX),
               "deltanet: alpha/beta projection");
    const int threads = ((a.dk > a.dv ? a.dk : a.dv) + 63) / 64 * 64;
    const int key = a.dk * 1000 + a.dv;
    switch (key) {
#define AQ_DN(K, V)                                                                                           \
    case K * 1000 + V: hipLaunchKernelGGL((dn_core_kernel<K, V>), dim3((unsigned)a.nv), dim3(threads), 0, stream, a); break;
        AQ_DN(8, 8) AQ_DN(16, 16) AQ_DN(32, 32) AQ_DN(64, 64) AQ_DN(128, 128) AQ_DN(128, 256) AQ_DN(64, 128)
#undef AQ_DN
    default: return fail(AQ_EUNSUP, "deltanet: head dims (k, v) not built: " + std::to_string(a.dk) + ", " +
                                        std::to_string(a.dv));
    }
    return launched("deltanet");
}

int launch_attention(const AttnArgs &a, hipStream_t stream) {
    AQ_REQUIRE(a.t >= 1 && a.nh >= 1 && a.nkv >= 1 && a.nh % a.nkv == 0, "attention: head counts");
    AQ_REQUIRE(a.hd >= 8 && a.hd <= 256 && a.hd % 8 == 0, "attention: head_dim must be a multiple of 8, <= 256");
    AQ_REQUIRE(a.rd >= 2 && a.rd <= a.hd && a.rd % 2 == 0, "attention: rope_dim");
    hipLaunchKernelGGL(attn_prep_kernel, dim3((unsigned)(a.nh + a.nkv), (unsigned)a.t), dim3(a.hd), 0, stream, a);
    int rc = launched("attention prologue");
    if (rc) return rc;
    const size_t shmem = (a.hd + a.base + a.t + 32) * sizeof(float);
    AQ_REQUIRE(shmem <= 160 * 1024, "attention: context too long for one work-group's LDS");
    hipLaunchKernelGGL(attn_core_kernel, dim3((unsigned)a.nh, (unsigned)a.t), dim3(256), shmem, stream, a);
    return launched("attention");
}

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
    hipLaunchKernelGGL(argmax_final_kernel, dim3((unsigned)t), dim3(64), 0, stream, pv, pi, nchunk, ids);
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
