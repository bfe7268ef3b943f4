// kq_q8f.hip — K-quant weights x Q8_0 activations: the reference's opt-in `--q8-fine` form (matvec.rs:127-160
// `set_q8_fine` / `act_kind`, dot.rs:69-160 `dot_q4_k_q8` / `dot_q5_k_q8` / `dot_q6_k_q8`).
//
// Arithmetic (per weight row and activation column, no FMA): for every 32-element sub-block s of super-block sb,
// against the activation's Q8_0 block xb = 8 sb + s, eight exact i32 lanes p32[i] = sum over elements 4i..4i+3 of
// code * x; Q6_K takes its -32 offset in integer from lane 0 (32 * sum x[0..16]) and lane 4 (32 * sum x[16..32]).
// Then acc[i] += f32(p32[i]) * (d32[xb] * (d * sc)) with sc the sub-block scale (Q6_K: the group scale of lanes 0..3
// or 4..7), in sub-block order; Q4_K / Q5_K also accm[s] += (m[s] * -dmin) * (d32[xb] * f32(sum x[xb])) in
// super-block order. The result is reduce8(acc) [+ reduce8(accm)], reduce8(v) = ((v0+v4)+(v2+v6)) + ((v1+v5)+(v3+v7)).
//
// Mapping. Thread (row, lane l) runs the chains acc[l] and accm[l] of its row for NC activation columns, super-blocks
// in order. Its weight bytes are one 16-byte load of the tile plane per super-block (the lane's 4 codes of all 8
// sub-blocks) plus the row's scales; its activation codes are the 4 bytes 4l..4l+3 of each Q8_0 block, read from
// the natural-order code plane (the same buffer the Q8_0 / Q4_0 kernels read). A 64-lane wave holds 8 rows x 8 lanes;
// the 8 lanes of a row are adjacent, so the Q6_K half-block sums (4 lanes) are two DPP adds and the final reduce8 is
// three exchanges within the row's 8 lanes, in the reference's pairing. Work-group: 256 threads = 32 rows.
#include "aq_common.h"
#include "quant_dev.h"

namespace aq {
namespace {

constexpr int Q8F_ROWS = 32; // rows per 256-thread work-group

struct Q8fArgs {
    const uint8_t *qa, *qb, *sc, *dm;
    int rows, nb; // weight rows; super-blocks per row
    const int8_t *xq;  // ncols x n codes, natural order
    const float *xd;   // ncols x nb32 block scales (the f16 widened)
    const int32_t *xs; // ncols x nb32 code sums
    size_t n, nb32;
    int ncols;
    float *y;
    const float *resid;
};

__device__ __forceinline__ float f16lo(uint32_t w) {
    _Float16 f;
    const uint16_t h = (uint16_t)(w & 0xFFFF);
    __builtin_memcpy(&f, &h, 2);
    return (float)f;
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b) { return __builtin_amdgcn_sdot4((int)a, (int)b, 0, false); }

// quant.rs:45-51 get_scale_min_k4 over the 12 packed bytes (words w1..w3 of the row's 16-byte scale record).
__device__ __forceinline__ void scales_k4(uint32_t w1, uint32_t w2, uint32_t w3, int sc[8], int mn[8]) {
    const uint8_t q[12] = {(uint8_t)w1, (uint8_t)(w1 >> 8), (uint8_t)(w1 >> 16), (uint8_t)(w1 >> 24),
                           (uint8_t)w2, (uint8_t)(w2 >> 8), (uint8_t)(w2 >> 16), (uint8_t)(w2 >> 24),
                           (uint8_t)w3, (uint8_t)(w3 >> 8), (uint8_t)(w3 >> 16), (uint8_t)(w3 >> 24)};
#pragma unroll
    for (int s = 0; s < 4; s++) {
        sc[s] = q[s] & 63;
        mn[s] = q[s + 4] & 63;
        sc[s + 4] = (q[s + 8] & 0xF) | ((q[s] >> 6) << 4);
        mn[s + 4] = (q[s + 8] >> 4) | ((q[s + 4] >> 6) << 4);
    }
}

// Exchange within the 8 adjacent lanes of a row: the value of lane (l ^ m).
__device__ __forceinline__ float xor_row(float v, int m) { return __shfl_xor(v, m, 64); }

// reduce8 of the values the 8 lanes of a row hold (lane l: v_l); every lane of the row gets the result.
__device__ __forceinline__ float row_reduce8(float v) {
    const float a = v + xor_row(v, 4); // lanes 0..3: v0+v4, v1+v5, v2+v6, v3+v7
    const float b = a + xor_row(a, 2); // lane 0: (v0+v4)+(v2+v6); lane 1: (v1+v5)+(v3+v7)
    return b + xor_row(b, 1);
}

template <int T, int NC>
__global__ void __launch_bounds__(256) kq_q8f_kernel(Q8fArgs a) {
    const int tid = threadIdx.x, l = tid & 7;
    const int row = blockIdx.x * Q8F_ROWS + (tid >> 3);
    const int c0 = blockIdx.y * NC;
    const size_t r = (size_t)min(row, a.rows - 1); // the rows past the end read the last row and write nothing
    const size_t nb = (size_t)a.nb;
    float acc[NC], accm[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) acc[c] = accm[c] = 0.0f;
    for (size_t sb = 0; sb < nb; sb++) {
        const uint4 q = *reinterpret_cast<const uint4 *>(a.qa + kq_qa_off(r, sb, nb, l));
        const uint4 s4 = *reinterpret_cast<const uint4 *>(a.sc + kq_sc_off(r, sb, nb));
        uint32_t code[8];   // the lane's 4 codes of sub-block s, one byte each
        float dsc[8];       // d * sc of the scale that multiplies this lane in sub-block s
        float mind = 0.0f;  // Q4_K / Q5_K: m[l] * -dmin, the min of sub-block l
        if constexpr (T == AQ_TYPE_Q6_K) {
            const uint2 h = *reinterpret_cast<const uint2 *>(a.qb + kq_qb6_off(r, sb, nb, l));
            const float d = f16lo(*reinterpret_cast<const uint16_t *>(a.dm + kq_dm_off(r, sb, nb)));
            const uint32_t qw[4] = {q.x, q.y, q.z, q.w}, hw[2] = {h.x, h.y}, sw[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const int g = s >> 2, k = s & 3; // half, sub-block within the half (dot.rs:128-141)
                const uint32_t lo = (qw[g * 2 + (k & 1)] >> (4 * (k >> 1))) & 0x0F0F0F0Fu;
                const uint32_t hi = ((hw[g] >> (2 * k)) & 0x03030303u) << 4;
                code[s] = lo | hi;
                const int gi = 2 * s + (l >> 2); // group scale sc[g*8 + 2k] (lanes 0..3) or sc[g*8 + 2k + 1]
                const int scv = (int8_t)(sw[gi >> 2] >> (8 * (gi & 3)));
                dsc[s] = d * (float)scv;
            }
        } else {
            const float d = f16lo(s4.x), dmin = f16lo(s4.x >> 16);
            int sc[8], mn[8];
            scales_k4(s4.y, s4.z, s4.w, sc, mn);
            const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
            uint32_t h5 = 0;
            if constexpr (T == AQ_TYPE_Q5_K) h5 = *reinterpret_cast<const uint32_t *>(a.qb + kq_qb5_off(r, sb, nb, l));
#pragma unroll
            for (int s = 0; s < 8; s++) {
                uint32_t c = (qw[s >> 1] >> (4 * (s & 1))) & 0x0F0F0F0Fu;
                if constexpr (T == AQ_TYPE_Q5_K) c |= ((h5 >> s) & 0x01010101u) << 4;
                code[s] = c;
                dsc[s] = d * (float)sc[s];
            }
            int ml = mn[0];
#pragma unroll
            for (int s = 1; s < 8; s++) ml = l == s ? mn[s] : ml;
            mind = (float)ml * -dmin;
        }
#pragma unroll
        for (int c = 0; c < NC; c++) {
            if (c0 + c >= a.ncols) break;
            const size_t col = (size_t)(c0 + c);
            const uint32_t *xw = reinterpret_cast<const uint32_t *>(a.xq + col * a.n + sb * 256) + l;
            const float *xd = a.xd + col * a.nb32 + sb * 8;
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const uint32_t xv = xw[s * 8];
                int p = sdot4(code[s], xv);
                if constexpr (T == AQ_TYPE_Q6_K) {
                    // 32 * (sum of the x codes of this lane's half-block), taken from lanes 0 and 4 only
                    int hs = sdot4(xv, 0x01010101u);
                    hs += dpp_mov<0xB1>(hs); // quad_perm [1,0,3,2]
                    hs += dpp_mov<0x4E>(hs); // quad_perm [2,3,0,1]
                    if ((l & 3) == 0) p -= 32 * hs;
                }
                const float f = xd[s] * dsc[s];
                acc[c] += (float)p * f;
            }
            if constexpr (T != AQ_TYPE_Q6_K) {
                const float dxs = xd[l] * (float)a.xs[col * a.nb32 + sb * 8 + l];
                accm[c] += mind * dxs;
            }
        }
    }
#pragma unroll
    for (int c = 0; c < NC; c++) {
        float v = row_reduce8(acc[c]);
        if constexpr (T != AQ_TYPE_Q6_K) v = v + row_reduce8(accm[c]);
        if (c0 + c < a.ncols && l == 0 && row < a.rows) {
            const size_t o = (size_t)(c0 + c) * a.rows + row;
            a.y[o] = a.resid ? a.resid[o] + v : v;
        }
    }
}

template <int T>
int launch_t(const Q8fArgs &a, hipStream_t stream) {
    const unsigned gx = (unsigned)((a.rows + Q8F_ROWS - 1) / Q8F_ROWS);
    // columns per thread: all of them up to 4, else groups of 4 (the chains are per column, so the split is free)
    if (a.ncols <= 1) {
        hipLaunchKernelGGL((kq_q8f_kernel<T, 1>), dim3(gx, 1), dim3(256), 0, stream, a);
    } else if (a.ncols == 2) {
        hipLaunchKernelGGL((kq_q8f_kernel<T, 2>), dim3(gx, 1), dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL((kq_q8f_kernel<T, 4>), dim3(gx, (unsigned)((a.ncols + 3) / 4)), dim3(256), 0, stream, a);
    }
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "kq_q8f launch");
}

} // namespace

int launch_kq_q8f(const Weight &w, const Act &x, size_t ncols, float *y, const float *resid, hipStream_t stream) {
    AQ_REQUIRE(is_kquant(w.type), "kq_q8f: K-quant weights only");
    AQ_REQUIRE(w.cols == x.n && w.cols % 256 == 0, "kq_q8f: activation length must equal the weight's columns "
                                                    "(a multiple of 256, matvec.rs:73-77)");
    AQ_REQUIRE(ncols >= 1 && ncols <= x.ncols && ncols <= 16, "kq_q8f: ncols out of range");
    AQ_REQUIRE(w.rows >= 1 && w.rows <= (size_t)INT32_MAX, "kq_q8f: rows out of range");
    Q8fArgs a{};
    a.qa = w.qa;
    a.qb = w.qb;
    a.sc = w.sc;
    a.dm = w.dm;
    a.rows = (int)w.rows;
    a.nb = (int)w.nb;
    a.xq = x.q0;
    a.xd = x.d0;
    a.xs = x.s0;
    a.n = x.n;
    a.nb32 = x.nb32;
    a.ncols = (int)ncols;
    a.y = y;
    a.resid = resid;
    switch (w.type) {
    case AQ_TYPE_Q4_K: return launch_t<AQ_TYPE_Q4_K>(a, stream);
    case AQ_TYPE_Q5_K: return launch_t<AQ_TYPE_Q5_K>(a, stream);
    default: return launch_t<AQ_TYPE_Q6_K>(a, stream);
    }
}

} // namespace aq
