// kq_gemm.hip — weight x activation products over many columns (a prompt chunk's rows: model.rs:443-461 prefill,
// where every projection is a matmul over the chunk's tokens, matvec.rs:369-393). Each output equals the single-
// column dot bit for bit: the integer lane sums are exact and each output's f32 chains advance super-block by
// super-block (block by block for Q8_0 / Q4_0) in the reference's order.
//
// K-quants x Q8_K (kdot.rs:37-140, 176-333) on v_mfma_i32_16x16x32_i8. The reference's lane l of a super-block is
// the 32 elements 32s + 4l + b (s = sub-block, b = 0..3), and its sum is sum_s sc[s] * sum_b q * x. One matrix-core
// product over K = 32 covers exactly lane l: k-group g of the operands (lanes 16g .. 16g + 15) takes sub-blocks 2g and
// 2g + 1, four elements each; the scale goes into the weight operand as digits small enough that digit * code fits
// an int8 (Q4_K: 6-bit scales in two base-8 digits, codes <= 15; Q5_K: three base-4 digits, codes <= 31; Q6_K:
// signed 8-bit group scales in four balanced base-5 digits in -2..2, unsigned codes <= 63, and the reference's -32
// offset taken from the activation's 16-element group sums into lane l exactly as kdot.rs:125-129 does). The digit
// products chain through the accumulator (c = digit_hi product; c = c * base + next digit's product ...), so the
// result is the exact lane sum for a 16-row x 16-column tile. The f32 part then runs per output in the lanes that
// hold it (4 rows x 1 column per lane): acc[l] += (dx * d) * f32(sumi[l]), accm[i] += (-dx * dmin) * f32(prod[i]),
// no FMA, and reduce8(acc) [+ reduce4(accm)] at the end.
//
// Q8_0 / Q4_0 x Q8_0 (dot.rs:29-66): one product over K = 32 is one block's exact i32 sum for the tile (Q4_0: the
// unsigned codes, less 8 * the activation block's code sum), then acc += (dw * dx) * f32(isum) per output.
//
// Work: a wave owns 16 rows x 16 columns for all of K (its super-block's loads issued one step ahead); a 256-thread
// work-group the same 16 rows x 64 columns. Rows and columns past the ends are read clamped and not written.
#include "aq_common.h"

namespace aq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mma(uint64_t a, uint64_t b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8((long)a, (long)b, c, 0, 0, 0);
}
__device__ __forceinline__ uint64_t pack2(uint32_t lo, uint32_t hi) { return (uint64_t)lo | ((uint64_t)hi << 32); }
__device__ __forceinline__ float h2f(uint32_t bits16) {
    _Float16 f;
    const uint16_t h = (uint16_t)(bits16 & 0xFFFF);
    __builtin_memcpy(&f, &h, 2);
    return (float)f;
}
// Each byte of x (values <= 126) negated, as int8: (0x80 - v) without borrows, then the top bit flipped.
__device__ __forceinline__ uint32_t neg_bytes(uint32_t x) { return (0x80808080u - x) ^ 0x80808080u; }

// The 6-bit scale and min of sub-block s from a Q4_K / Q5_K record's 12 packed bytes (quant.rs:45-51).
__device__ __forceinline__ void scale_min(const uint32_t w[3], int s, int &sc, int &m) {
    const uint8_t *q = reinterpret_cast<const uint8_t *>(w);
    if (s < 4) {
        sc = q[s] & 63;
        m = q[s + 4] & 63;
    } else {
        sc = (q[s + 4] & 0xF) | ((q[s - 4] >> 6) << 4);
        m = (q[s + 4] >> 4) | ((q[s] >> 6) << 4);
    }
}

// Balanced base-5 digits (each in -2..2, low digit first) of a signed 8-bit scale, as four signed bytes.
__device__ __forceinline__ uint32_t digits5(int v) {
    uint32_t out = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int d = v % 5; // in -4..4 (C truncation)
        if (d > 2) d -= 5;
        if (d < -2) d += 5;
        v = (v - d) / 5;
        out |= (uint32_t)(uint8_t)(int8_t)d << (8 * i);
    }
    return out;
}
// The operand bytes x (codes <= 63) times a digit in -2..2.
__device__ __forceinline__ uint32_t times_digit(uint32_t x, int d) {
    const uint32_t p = x * (uint32_t)(d < 0 ? -d : d);
    return d < 0 ? neg_bytes(p) : p;
}

struct GemmArgs {
    const uint8_t *qa, *qb, *sc, *dm;
    int rows, nb, ncols;
    // Q8_K activations (lane-slot order) or Q8_0 (natural order)
    const int8_t *xq;
    const float *xd;
    const int16_t *xbs, *xq8s;
    const int32_t *xs0;
    size_t n;
    float *y;
    const float *resid;
};

__device__ __forceinline__ int sdot2(uint32_t a, uint32_t b) {
    typedef short s16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(s16x2, a), __builtin_bit_cast(s16x2, b), 0, false);
}
// Two signed bytes of w (byte k and k + 1) as an i16 pair.
__device__ __forceinline__ uint32_t i8pair(uint32_t w, int k) {
    const int lo = (int)(int8_t)(w >> (8 * k)), hi = (int)(int8_t)(w >> (8 * k + 8));
    return ((uint32_t)lo & 0xFFFFu) | ((uint32_t)hi << 16);
}

// What one super-block step of a wave reads: the weight operand's codes (row li, lanes 0..7, sub-blocks 2g and
// 2g + 1) and its scale record, the scale records of the lane's four output rows, and the column's activation
// operand, scale and group / sub-block sums. Loaded one super-block ahead of its use.
template <int T>
struct GemmLd {
    uint32_t w[8], w2[8], h[8];
    uint4 sa, se[4];
    uint32_t d6[4];
    uint64_t bx[8];
    float dx;
    uint4 s8a, s8b;
};

template <int T>
__device__ __forceinline__ void gemm_load(const GemmArgs &a, GemmLd<T> &L, size_t sb, size_t ra, const int rj[4],
                                          size_t col, int g) {
    const size_t nb = (size_t)a.nb;
#pragma unroll
    for (int l = 0; l < 8; l++) {
        if constexpr (T == AQ_TYPE_Q6_K) {
            const uint2 w = *reinterpret_cast<const uint2 *>(a.qa + kq_qa_off(ra, sb, nb, l) + 8 * (g >> 1));
            L.w[l] = w.x;
            L.w2[l] = w.y;
            L.h[l] = *reinterpret_cast<const uint32_t *>(a.qb + kq_qb6_off(ra, sb, nb, l) + 4 * (g >> 1));
        } else {
            L.w[l] = *reinterpret_cast<const uint32_t *>(a.qa + kq_qa_off(ra, sb, nb, l) + 4 * g);
            if constexpr (T == AQ_TYPE_Q5_K) L.h[l] = *reinterpret_cast<const uint32_t *>(a.qb + kq_qb5_off(ra, sb, nb, l));
        }
        L.bx[l] = *reinterpret_cast<const uint64_t *>(a.xq + col * a.n + sb * 256 + (size_t)lane_slot(l) * 32 + 8 * g);
    }
    L.sa = *reinterpret_cast<const uint4 *>(a.sc + kq_sc_off(ra, sb, nb));
#pragma unroll
    for (int j = 0; j < 4; j++) {
        L.se[j] = *reinterpret_cast<const uint4 *>(a.sc + kq_sc_off((size_t)rj[j], sb, nb));
        if constexpr (T == AQ_TYPE_Q6_K) L.d6[j] = *reinterpret_cast<const uint16_t *>(a.dm + kq_dm_off((size_t)rj[j], sb, nb));
    }
    L.dx = a.xd[col * nb + sb];
    if constexpr (T == AQ_TYPE_Q6_K) {
        L.s8a = reinterpret_cast<const uint4 *>(a.xbs + (col * nb + sb) * 16)[0];
        L.s8b = reinterpret_cast<const uint4 *>(a.xbs + (col * nb + sb) * 16)[1];
    } else {
        L.s8a = *reinterpret_cast<const uint4 *>(a.xq8s + (col * nb + sb) * 8);
    }
}

// K-quant x Q8_K, one 16-row x 16-column tile per wave: the work-group's four waves take four column tiles of the
// same rows (their weight reads share the caches).
template <int T>
__global__ void __launch_bounds__(256) kq_gemm_kernel(GemmArgs a) {
    constexpr int ND = T == AQ_TYPE_Q4_K ? 2 : (T == AQ_TYPE_Q5_K ? 3 : 4); // digits
    constexpr int BASE = T == AQ_TYPE_Q4_K ? 8 : (T == AQ_TYPE_Q5_K ? 4 : 5);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, li = lane & 15;
    const int r0 = (int)blockIdx.x * 16;
    const int c0 = ((int)blockIdx.y * 4 + wave) * 16;
    if (c0 >= a.ncols) return; // whole waves past the end (no barriers in this kernel)
    const size_t nb = (size_t)a.nb;
    const size_t ra = (size_t)min(r0 + li, a.rows - 1); // this lane's weight-operand row
    int rj[4];                                           // the rows of this lane's outputs: 4g + j
#pragma unroll
    for (int j = 0; j < 4; j++) rj[j] = min(r0 + 4 * g + j, a.rows - 1);
    const size_t col = (size_t)min(c0 + li, a.ncols - 1);

    float acc[4][8], accm[4][4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
        for (int l = 0; l < 8; l++) acc[j][l] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) accm[j][i] = 0.0f;
    }
    GemmLd<T> cur, nxt;
    gemm_load<T>(a, cur, 0, ra, rj, col, g);
    for (size_t sb = 0; sb < nb; sb++) {
        gemm_load<T>(a, nxt, sb + 1 < nb ? sb + 1 : sb, ra, rj, col, g); // in flight during this step

        // the weight operand's digits: the scales of sub-blocks 2g and 2g + 1 (Q6_K: per lane half, l < 4 / l >= 4)
        int dga[ND], dgb[ND], dgc[ND], dgd[ND];
        if constexpr (T == AQ_TYPE_Q6_K) {
            const uint32_t sw = g == 0 ? cur.sa.x : g == 1 ? cur.sa.y : g == 2 ? cur.sa.z : cur.sa.w;
            const uint32_t da = digits5((int8_t)sw), dc = digits5((int8_t)(sw >> 8));
            const uint32_t db = digits5((int8_t)(sw >> 16)), dd = digits5((int8_t)(sw >> 24));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                dga[i] = (int8_t)(da >> (8 * i));
                dgb[i] = (int8_t)(db >> (8 * i));
                dgc[i] = (int8_t)(dc >> (8 * i));
                dgd[i] = (int8_t)(dd >> (8 * i));
            }
        } else {
            const uint32_t w3[3] = {cur.sa.y, cur.sa.z, cur.sa.w};
            int sca, scb, mdum;
            scale_min(w3, 2 * g, sca, mdum);
            scale_min(w3, 2 * g + 1, scb, mdum);
            constexpr int BB = T == AQ_TYPE_Q4_K ? 3 : 2;
#pragma unroll
            for (int i = 0; i < ND; i++) {
                dga[i] = dgc[i] = (sca >> (BB * i)) & ((1 << BB) - 1);
                dgb[i] = dgd[i] = (scb >> (BB * i)) & ((1 << BB) - 1);
            }
        }

        // the exact lane sums of the tile: sumi[l][j] for output rows 4g + j of this lane's column
        int sumi[8][4];
#pragma unroll
        for (int l = 0; l < 8; l++) {
            uint32_t lo, hi;
            if constexpr (T == AQ_TYPE_Q6_K) {
                const int sh = 4 * (g & 1);
                lo = ((cur.w[l] >> sh) & 0x0F0F0F0Fu) | (((cur.h[l] >> sh) & 0x03030303u) << 4);
                hi = ((cur.w2[l] >> sh) & 0x0F0F0F0Fu) | (((cur.h[l] >> (sh + 2)) & 0x03030303u) << 4);
            } else {
                lo = cur.w[l] & 0x0F0F0F0Fu;
                hi = (cur.w[l] >> 4) & 0x0F0F0F0Fu;
                if constexpr (T == AQ_TYPE_Q5_K) {
                    lo |= ((cur.h[l] >> (2 * g)) & 0x01010101u) << 4;
                    hi |= ((cur.h[l] >> (2 * g + 1)) & 0x01010101u) << 4;
                }
            }
            const int *da = l < 4 ? dga : dgc, *db = l < 4 ? dgb : dgd;
            v4i c = {0, 0, 0, 0};
#pragma unroll
            for (int i = ND - 1; i >= 0; i--) {
                if (i < ND - 1) {
#pragma unroll
                    for (int e = 0; e < 4; e++) c[e] *= BASE;
                }
                uint32_t alo, ahi;
                if constexpr (T == AQ_TYPE_Q6_K) {
                    alo = times_digit(lo, da[i]);
                    ahi = times_digit(hi, db[i]);
                } else {
                    alo = lo * (uint32_t)da[i];
                    ahi = hi * (uint32_t)db[i];
                }
                c = mma(pack2(alo, ahi), cur.bx[l], c);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) sumi[l][j] = c[j];
        }

        // the f32 chains of the lane's four outputs (kdot.rs:37-140), in super-block order
        const float dx = cur.dx;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if constexpr (T == AQ_TYPE_Q6_K) {
                const float d = dx * h2f(cur.d6[j]);
                const uint32_t sw[4] = {cur.se[j].x, cur.se[j].y, cur.se[j].z, cur.se[j].w};
                const uint32_t bsw[8] = {cur.s8a.x, cur.s8a.y, cur.s8a.z, cur.s8a.w,
                                         cur.s8b.x, cur.s8b.y, cur.s8b.z, cur.s8b.w};
#pragma unroll
                for (int l = 0; l < 8; l++) {
                    // kdot.rs:125-129: lane l less 32 * (bs[2l] sc[2l] + bs[2l + 1] sc[2l + 1])
                    const int off = sdot2(bsw[l], i8pair(sw[l >> 1], 2 * (l & 1)));
                    acc[j][l] += d * (float)(sumi[l][j] - 32 * off);
                }
            } else {
                const float d = dx * h2f(cur.se[j].x), dmin = -dx * h2f(cur.se[j].x >> 16);
                // the 8 mins as bytes (quant.rs:45-51): sub-blocks 0..3 from bytes 4..7, 4..7 from bytes 8..11 + 0..3
                const uint32_t mlo = cur.se[j].z & 0x3F3F3F3Fu;
                const uint32_t mhi = ((cur.se[j].w >> 4) & 0x0F0F0F0Fu) | ((cur.se[j].z >> 2) & 0x30303030u);
                const uint32_t q8w[4] = {cur.s8a.x, cur.s8a.y, cur.s8a.z, cur.s8a.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t m2 = __builtin_amdgcn_perm(0u, i < 2 ? mlo : mhi, (i & 1) ? 0x0C030C02u : 0x0C010C00u);
                    accm[j][i] += dmin * (float)sdot2(m2, q8w[i]); // m[2i] q8s[2i] + m[2i+1] q8s[2i+1]
                }
#pragma unroll
                for (int l = 0; l < 8; l++) acc[j][l] += d * (float)sumi[l][j];
            }
        }
        cur = nxt;
    }

    const int ocol = c0 + li;
    if (ocol < a.ncols) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int row = r0 + 4 * g + j;
            if (row >= a.rows) continue;
            const float *l8 = acc[j];
            float v = ((l8[0] + l8[4]) + (l8[2] + l8[6])) + ((l8[1] + l8[5]) + (l8[3] + l8[7])); // reduce8
            if constexpr (T != AQ_TYPE_Q6_K) {
                const float *m4 = accm[j];
                v = v + ((m4[0] + m4[2]) + (m4[1] + m4[3])); // reduce4
            }
            const size_t o = (size_t)ocol * a.rows + row;
            a.y[o] = a.resid ? a.resid[o] + v : v;
        }
    }
}

// Q8_0 / Q4_0 weights x Q8_0 activations: one block per product, on the same tiles (eight waves per SIMD hide the
// loads' latency).
template <int T>
__global__ void __launch_bounds__(256) q8_gemm_kernel(GemmArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, li = lane & 15;
    const int r0 = (int)blockIdx.x * 16;
    const int c0 = ((int)blockIdx.y * 4 + wave) * 16;
    if (c0 >= a.ncols) return;
    const size_t nb = (size_t)a.nb; // 32-blocks per row
    const size_t ra = (size_t)min(r0 + li, a.rows - 1);
    int rj[4];
#pragma unroll
    for (int j = 0; j < 4; j++) rj[j] = min(r0 + 4 * g + j, a.rows - 1);
    const size_t col = (size_t)min(c0 + li, a.ncols - 1);
    constexpr int BB = T == AQ_TYPE_Q8_0 ? 32 : 16; // code bytes per block
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto load_w = [&](size_t b) -> uint64_t {
        if constexpr (T == AQ_TYPE_Q8_0) return *reinterpret_cast<const uint64_t *>(a.qa + (ra * nb + b) * BB + 8 * g);
        // elements 8g .. 8g + 7: bytes 8 (g & 1) .., low nibbles for g < 2, high for g >= 2
        const uint64_t w = *reinterpret_cast<const uint64_t *>(a.qa + (ra * nb + b) * BB + 8 * (g & 1));
        return (w >> (4 * (g >> 1))) & 0x0F0F0F0F0F0F0F0Full;
    };
    for (size_t b = 0; b < nb; b++) {
        const uint64_t wa = load_w(b);
        const uint64_t bx = *reinterpret_cast<const uint64_t *>(a.xq + col * a.n + b * 32 + 8 * g);
        float dw[4];
#pragma unroll
        for (int j = 0; j < 4; j++) dw[j] = h2f(*reinterpret_cast<const uint16_t *>(a.dm + ((size_t)rj[j] * nb + b) * 2));
        const float dx = a.xd[col * nb + b];
        int off = 0;
        if constexpr (T == AQ_TYPE_Q4_0) off = 8 * a.xs0[col * nb + b]; // dot.rs:48-66: codes less 8
        v4i c = {0, 0, 0, 0};
        c = mma(wa, bx, c);
#pragma unroll
        for (int j = 0; j < 4; j++) acc[j] += (dw[j] * dx) * (float)(c[j] - off);
    }
    const int ocol = c0 + li;
    if (ocol < a.ncols) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int row = r0 + 4 * g + j;
            if (row >= a.rows) continue;
            const size_t o = (size_t)ocol * a.rows + row;
            a.y[o] = a.resid ? a.resid[o] + acc[j] : acc[j];
        }
    }
}

template <int T>
int launch_kq_t(const GemmArgs &ga, hipStream_t stream) {
    const dim3 grid((unsigned)((ga.rows + 15) / 16), (unsigned)((ga.ncols + 63) / 64));
    hipLaunchKernelGGL((kq_gemm_kernel<T>), grid, dim3(256), 0, stream, ga);
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "kq_gemm launch");
}
template <int T>
int launch_q8_t(const GemmArgs &ga, hipStream_t stream) {
    const dim3 grid((unsigned)((ga.rows + 15) / 16), (unsigned)((ga.ncols + 63) / 64));
    hipLaunchKernelGGL((q8_gemm_kernel<T>), grid, dim3(256), 0, stream, ga);
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "q8_gemm launch");
}

} // namespace

int launch_gemm(const Weight &w, const Act &x, size_t ncols, float *y, const float *resid, hipStream_t stream) {
    AQ_REQUIRE(ncols >= 1 && ncols <= x.ncols, "gemm: ncols out of range");
    AQ_REQUIRE(w.cols == x.n, "gemm: activation length != weight columns");
    AQ_REQUIRE(w.rows >= 1 && w.rows <= (size_t)INT32_MAX && ncols <= (size_t)INT32_MAX, "gemm: shape");
    GemmArgs ga{};
    ga.qa = w.qa;
    ga.qb = w.qb;
    ga.sc = w.sc;
    ga.dm = w.dm;
    ga.rows = (int)w.rows;
    ga.nb = (int)w.nb;
    ga.ncols = (int)ncols;
    ga.n = x.n;
    ga.y = y;
    ga.resid = resid;
    if (is_kquant(w.type)) {
        AQ_REQUIRE(w.cols % 256 == 0, "gemm: K-quant columns must be a multiple of 256");
        ga.xq = x.qs;
        ga.xd = x.d;
        ga.xbs = x.bs;
        ga.xq8s = x.q8s;
        switch (w.type) {
        case AQ_TYPE_Q4_K: return launch_kq_t<AQ_TYPE_Q4_K>(ga, stream);
        case AQ_TYPE_Q5_K: return launch_kq_t<AQ_TYPE_Q5_K>(ga, stream);
        default: return launch_kq_t<AQ_TYPE_Q6_K>(ga, stream);
        }
    }
    AQ_REQUIRE(w.type == AQ_TYPE_Q8_0 || w.type == AQ_TYPE_Q4_0, "gemm: weight type");
    AQ_REQUIRE(w.cols % 32 == 0, "gemm: Q8_0 / Q4_0 columns must be a multiple of 32");
    ga.xq = x.q0;
    ga.xd = x.d0;
    ga.xs0 = x.s0;
    if (w.type == AQ_TYPE_Q8_0) return launch_q8_t<AQ_TYPE_Q8_0>(ga, stream);
    return launch_q8_t<AQ_TYPE_Q4_0>(ga, stream);
}

} // namespace aq
