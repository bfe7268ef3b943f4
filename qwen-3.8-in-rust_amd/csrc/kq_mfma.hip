// kq_mfma.hip — the K-quant x Q8_K matmul (N = 1 matvec and the N = k+1 verify batch) on gfx950 matrix cores.
//
// Same integers and floats as the reference (kdot.rs:37-140 and the blocked kdot.rs:176-333): per super-block the
// 8 exact i32 lane sums (lane l = elements 4l..4l+3 of each 32-element sub-block, the scale multiplied in as an
// integer), the 4 Q4_K/Q5_K min lanes, the Q6_K -32 fold; then acc[l] += (dx*dw) * float(sum) super-block by
// super-block without FMA, and the ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)) [+ (m0+m2)+(m1+m3)] reduction. Only how
// the exact integers are produced is new:
//
//  * v_mfma_i32_4x4x4_16b_i8 computes 16 independent 4x4x4 int8 products. Block b of one instruction is
//    (row group g, lane j): its K = 4 elements are lane j's 4 positions of one sub-block, so it yields the lane-j
//    partial of that sub-block for 4 weight rows x 4 activation columns, exactly (int32). A = activations (A row i
//    = column c), B = weight codes (B column = weight row). Register layout, measured on the device: A and B of
//    block b at lanes 4b+i / 4b+j, D[i][j] at lane 4b+j, VGPR i.
//  * Thread t = 16g + 4j + r of a wave owns weight row 4g + r (16 rows per wave) and the two reference lanes j and
//    j+4: one instruction set with blocks (g, j) computes lane j, a second one lane j+4. Per-row work (scale
//    decode, the min lanes) is shared by the row's 4 threads instead of 8, and every min lane j (0..3) is a thread.
//  * Q4_K / Q5_K: the 6-bit sub-block scale is split into 3-bit (2-bit) digits folded into the int8 weight operand
//    (sb_products_split), so the MFMA accumulator sums the scaled sub-block dots; Q6_K (int8 scales) multiplies
//    each MFMA partial by its scale with a full-rate 24-bit integer mad.
//  * Results go to VGPRs (built with -amdgpu-mfma-vgpr-form): no accumulator-register copies.
//  * Activations are staged in LDS per chunk of super-blocks, double-buffered (chunk k+1 is fetched into registers
//    while chunk k is computed); weights stream from HBM as 16-byte loads, prefetched PF super-blocks ahead.
//  * Matrices with few rows split K across KS waves of the work-group: wave w takes super-blocks w, w+KS, ...;
//    after every round the waves exchange their f32 products through LDS and each adds them to its copy of the
//    chain in super-block order, which keeps the chain the reference's sequential sum bit for bit.
#include "aq_common.h"

namespace aq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

struct MfArgs {
    const uint8_t *qa, *qb, *sc, *dm;
    int rows, nb;
    const int8_t *xqs;   // ncols x n, by lane slot
    const float *xd;     // ncols x nb
    const int16_t *xbs;  // ncols x nb x 16
    const int16_t *xq8s; // ncols x nb x 8
    size_t xcol;
    float *y;
    const float *resid;
};

__device__ __forceinline__ float h2f(uint32_t bits16) {
    _Float16 f;
    const uint16_t h = (uint16_t)bits16;
    __builtin_memcpy(&f, &h, 2);
    return (float)f;
}

__device__ __forceinline__ v4i mfma(uint32_t a, uint32_t b) {
    return __builtin_amdgcn_mfma_i32_4x4x4i8((int)a, (int)b, (v4i){0, 0, 0, 0}, 0, 0, 0);
}
__device__ __forceinline__ v4i mfma_acc(uint32_t a, uint32_t b, v4i c) {
    return __builtin_amdgcn_mfma_i32_4x4x4i8((int)a, (int)b, c, 0, 0, 0);
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u16x2 as_u16x2(uint32_t w) { return __builtin_bit_cast(u16x2, w); }
__device__ __forceinline__ uint32_t as_u32(u16x2 v) { return __builtin_bit_cast(uint32_t, v); }

__device__ __forceinline__ int sbyte(uint32_t w, int i) { return (int)(int8_t)(w >> (8 * i)); }
__device__ __forceinline__ int ubyte(uint32_t w, int i) { return (int)((w >> (8 * i)) & 0xFF); }

// The weight bytes of one super-block one thread needs (lanes j and j+4 of its row).
template <int TYPE>
struct WRegs {
    uint4 qa0, qa1; // codes of lane j, lane j+4
    uint4 sc;       // Q4_K/Q5_K: d, dmin, 12 scale bytes; Q6_K: 16 int8 scales
    uint4 qb;       // Q5_K: .x, .y = qh of lanes j, j+4; Q6_K: .x,.y lane j (h 0,1), .z,.w lane j+4
    uint32_t d6;    // Q6_K: f16 d
};

template <int TYPE>
__device__ __forceinline__ void load_w(WRegs<TYPE> &w, const MfArgs &a, size_t wsb, int j) {
    const uint4 *q = reinterpret_cast<const uint4 *>(a.qa + wsb * 128 + j * 32);
    w.qa0 = q[0];
    w.qa1 = q[1];
    w.sc = *reinterpret_cast<const uint4 *>(a.sc + wsb * 16);
    if constexpr (TYPE == AQ_TYPE_Q5_K) {
        const uint2 h = *reinterpret_cast<const uint2 *>(a.qb + wsb * 32 + j * 8);
        w.qb = make_uint4(h.x, h.y, 0, 0);
    } else if constexpr (TYPE == AQ_TYPE_Q6_K) {
        w.qb = *reinterpret_cast<const uint4 *>(a.qb + wsb * 64 + j * 16);
        w.d6 = *reinterpret_cast<const uint16_t *>(a.dm + wsb * 2);
    }
}

// The products of one super-block for one thread: pr0/pr1 = (dx*dw)*float(lane sum) of lanes j and j+4, pm the
// Q4_K/Q5_K min product of min lane j, for every column. xq: the super-block's codes, 256 bytes per column (lane-slot
// order, XS bytes per column); xd: its f32 scales per column; xm: its activation-sum pairs [pair][ncp].
// kdot.rs:37-140 per lane.
template <int TYPE, int NC, int XS = 256>
__device__ __forceinline__ void sb_products(const WRegs<TYPE> &wv, const int8_t *xq, const float *xd,
                                            const uint32_t *xm, int ncp, int j, int r, float *pr0, float *pr1,
                                            float *pm) {
    constexpr int NCG = (NC + 3) / 4;
    constexpr bool Q6 = TYPE == AQ_TYPE_Q6_K;
    uint32_t code0[8], code1[8]; // 4 unsigned codes per sub-block, lanes j and j+4
    int scl0[8], scl1[8];        // integer scale per sub-block, lanes j and j+4
    int mn0 = 0, mn1 = 0;        // Q4_K/Q5_K mins of sub-blocks 2j, 2j+1 (min lane j)
    int os00 = 0, os01 = 0, os10 = 0, os11 = 0; // Q6_K -32 fold scales: groups 2l, 2l+1 of l = j, j+4
    float dw, dminw = 0.0f;
    if constexpr (Q6) {
        const uint32_t ql0[4] = {wv.qa0.x, wv.qa0.y, wv.qa0.z, wv.qa0.w};
        const uint32_t ql1[4] = {wv.qa1.x, wv.qa1.y, wv.qa1.z, wv.qa1.w};
        const uint32_t qh0[2] = {wv.qb.x, wv.qb.y}, qh1[2] = {wv.qb.z, wv.qb.w};
        const uint32_t sw[4] = {wv.sc.x, wv.sc.y, wv.sc.z, wv.sc.w};
#pragma unroll
        for (int hh = 0; hh < 2; hh++)
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int s = hh * 4 + kk;
                const int li = kk < 2 ? hh * 2 + kk : hh * 2 + kk - 2, sh = kk < 2 ? 0 : 4;
                code0[s] = ((ql0[li] >> sh) & 0x0F0F0F0Fu) | (((qh0[hh] >> (2 * kk)) & 0x03030303u) << 4);
                code1[s] = ((ql1[li] >> sh) & 0x0F0F0F0Fu) | (((qh1[hh] >> (2 * kk)) & 0x03030303u) << 4);
                const int gi = hh * 8 + 2 * kk; // lane j (< 4) uses group gi, lane j+4 group gi+1
                scl0[s] = sbyte(sw[gi >> 2], gi & 3);
                scl1[s] = sbyte(sw[(gi + 1) >> 2], (gi + 1) & 3);
            }
        // groups 2l, 2l+1: l = j -> bytes 2j, 2j+1 of word j/2; l = j+4 -> word 2 + j/2
        os00 = sbyte(sw[j >> 1], 2 * (j & 1));
        os01 = sbyte(sw[j >> 1], 2 * (j & 1) + 1);
        os10 = sbyte(sw[2 + (j >> 1)], 2 * (j & 1));
        os11 = sbyte(sw[2 + (j >> 1)], 2 * (j & 1) + 1);
        dw = h2f(wv.d6);
    } else {
        const uint32_t q0 = wv.sc.y, q1 = wv.sc.z, q2 = wv.sc.w;
        const uint32_t sc_lo = q0 & 0x3F3F3F3Fu, mn_lo = q1 & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (q2 & 0x0F0F0F0Fu) | ((q0 >> 2) & 0x30303030u);
        const uint32_t mn_hi = ((q2 >> 4) & 0x0F0F0F0Fu) | ((q1 >> 2) & 0x30303030u);
        const uint32_t mnw = j < 2 ? mn_lo : mn_hi;
        mn0 = ubyte(mnw, 2 * (j & 1));
        mn1 = ubyte(mnw, 2 * (j & 1) + 1);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            scl0[s] = scl1[s] = ubyte(sc_lo, s);
            scl0[s + 4] = scl1[s + 4] = ubyte(sc_hi, s);
        }
        const uint32_t w0[4] = {wv.qa0.x, wv.qa0.y, wv.qa0.z, wv.qa0.w};
        const uint32_t w1[4] = {wv.qa1.x, wv.qa1.y, wv.qa1.z, wv.qa1.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            code0[2 * q] = w0[q] & 0x0F0F0F0Fu;
            code0[2 * q + 1] = (w0[q] >> 4) & 0x0F0F0F0Fu;
            code1[2 * q] = w1[q] & 0x0F0F0F0Fu;
            code1[2 * q + 1] = (w1[q] >> 4) & 0x0F0F0F0Fu;
        }
        if constexpr (TYPE == AQ_TYPE_Q5_K) {
#pragma unroll
            for (int s = 0; s < 8; s++) {
                code0[s] |= ((wv.qb.x >> s) & 0x01010101u) << 4;
                code1[s] |= ((wv.qb.y >> s) & 0x01010101u) << 4;
            }
        }
        dw = h2f(wv.sc.x & 0xFFFF);
        dminw = h2f(wv.sc.x >> 16);
    }
#pragma unroll
    for (int cg = 0; cg < NCG; cg++) {
        const int cA = cg * 4 + r < NC ? cg * 4 + r : 0; // this thread's A-operand column
        const uint4 *xp = reinterpret_cast<const uint4 *>(xq + cA * XS + j * 64);
        const uint4 va = xp[0], vb = xp[1], vc = xp[2], vd = xp[3];
        const uint32_t x0[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w}; // lane j
        const uint32_t x1[8] = {vc.x, vc.y, vc.z, vc.w, vd.x, vd.y, vd.z, vd.w}; // lane j+4
        int s0[4] = {0, 0, 0, 0}, s1[4] = {0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const v4i d0 = mfma(x0[s], code0[s]);
            const v4i d1 = mfma(x1[s], code1[s]);
#pragma unroll
            for (int c = 0; c < 4; c++) {
                if (cg * 4 + c < NC) { // the block's columns past NC are padding
                    s0[c] += __mul24(scl0[s], d0[c]); // |d| <= 4*63*127 fits 24 bits
                    s1[c] += __mul24(scl1[s], d1[c]);
                }
            }
        }
        const float4 dx4 = *reinterpret_cast<const float4 *>(xd + cg * 4);
        const float dxs[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
        const uint4 m0 = *reinterpret_cast<const uint4 *>(xm + j * ncp + cg * 4);
        const uint32_t mw0[4] = {m0.x, m0.y, m0.z, m0.w};
        uint32_t mw1[4] = {0, 0, 0, 0};
        if constexpr (Q6) {
            const uint4 m1 = *reinterpret_cast<const uint4 *>(xm + (j + 4) * ncp + cg * 4);
            mw1[0] = m1.x;
            mw1[1] = m1.y;
            mw1[2] = m1.z;
            mw1[3] = m1.w;
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int col = cg * 4 + c;
            if (col < NC) {
                const float dd = dxs[c] * dw;
                const int lo0 = (int)(int16_t)(mw0[c] & 0xFFFF), hi0 = (int)(int16_t)(mw0[c] >> 16);
                if constexpr (Q6) {
                    const int lo1 = (int)(int16_t)(mw1[c] & 0xFFFF), hi1 = (int)(int16_t)(mw1[c] >> 16);
                    pr0[col] = dd * (float)(s0[c] - 32 * (lo0 * os00 + hi0 * os01));
                    pr1[col] = dd * (float)(s1[c] - 32 * (lo1 * os10 + hi1 * os11));
                } else {
                    pr0[col] = dd * (float)s0[c];
                    pr1[col] = dd * (float)s1[c];
                    pm[col] = (-dxs[c] * dminw) * (float)(mn0 * lo0 + mn1 * hi0);
                }
            }
        }
    }
}

// Q4_K / Q5_K products with the sub-block scale inside the matrix-core operand. A 6-bit scale sc is split into
// digits of DB bits (sc = sum_i digit_i << (DB*i); DB = 3 for Q4_K codes <= 15, DB = 2 for Q5_K codes <= 31), so
// code * digit <= 105 (resp. 93) is an int8: one 32-bit multiply scales the 4 packed code bytes of a sub-block
// without carries, and the MFMA accumulator sums sc_i-weighted dots over the 8 sub-blocks. The lane sum is then
// sum_i D_i << (DB*i) = sum_s sc[s] * dot_s exactly — the same integer as kdot.rs:37-95 — with no per-output
// scale multiply.
template <int TYPE, int NC, int XS = 256>
__device__ __forceinline__ void sb_products_split(const WRegs<TYPE> &wv, const int8_t *xq, const float *xd,
                                                  const uint32_t *xm, int ncp, int j, int r, float *pr0,
                                                  float *pr1, float *pm) {
    constexpr int NCG = (NC + 3) / 4;
    constexpr int DB = TYPE == AQ_TYPE_Q4_K ? 3 : 2;   // digit bits
    constexpr int ND = TYPE == AQ_TYPE_Q4_K ? 2 : 3;   // digits of a 6-bit scale
    constexpr uint32_t DM = (1u << DB) - 1u;
    const uint32_t q0 = wv.sc.y, q1 = wv.sc.z, q2 = wv.sc.w;
    const uint32_t sc_lo = q0 & 0x3F3F3F3Fu, mn_lo = q1 & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (q2 & 0x0F0F0F0Fu) | ((q0 >> 2) & 0x30303030u);
    const uint32_t mn_hi = ((q2 >> 4) & 0x0F0F0F0Fu) | ((q1 >> 2) & 0x30303030u);
    const uint32_t mnw = j < 2 ? mn_lo : mn_hi;
    const int mn0 = ubyte(mnw, 2 * (j & 1)), mn1 = ubyte(mnw, 2 * (j & 1) + 1);
    // digit words: byte s of dig[i][0] (s < 4) / dig[i][1] (s >= 4) = digit i of sc[s]
    uint32_t dig[ND][2];
#pragma unroll
    for (int i = 0; i < ND; i++) {
        dig[i][0] = (sc_lo >> (DB * i)) & (DM * 0x01010101u);
        dig[i][1] = (sc_hi >> (DB * i)) & (DM * 0x01010101u);
    }
    uint32_t code0[8], code1[8];
    const uint32_t w0[4] = {wv.qa0.x, wv.qa0.y, wv.qa0.z, wv.qa0.w};
    const uint32_t w1[4] = {wv.qa1.x, wv.qa1.y, wv.qa1.z, wv.qa1.w};
#pragma unroll
    for (int q = 0; q < 4; q++) {
        code0[2 * q] = w0[q] & 0x0F0F0F0Fu;
        code0[2 * q + 1] = (w0[q] >> 4) & 0x0F0F0F0Fu;
        code1[2 * q] = w1[q] & 0x0F0F0F0Fu;
        code1[2 * q + 1] = (w1[q] >> 4) & 0x0F0F0F0Fu;
    }
    if constexpr (TYPE == AQ_TYPE_Q5_K) {
#pragma unroll
        for (int s = 0; s < 8; s++) {
            code0[s] |= ((wv.qb.x >> s) & 0x01010101u) << 4;
            code1[s] |= ((wv.qb.y >> s) & 0x01010101u) << 4;
        }
    }
    const float dw = h2f(wv.sc.x & 0xFFFF), dminw = h2f(wv.sc.x >> 16);
#pragma unroll
    for (int cg = 0; cg < NCG; cg++) {
        const int cA = cg * 4 + r < NC ? cg * 4 + r : 0;
        const uint4 *xp = reinterpret_cast<const uint4 *>(xq + cA * XS + j * 64);
        const uint4 va = xp[0], vb = xp[1], vc = xp[2], vd = xp[3];
        const uint32_t x0[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w}; // lane j
        const uint32_t x1[8] = {vc.x, vc.y, vc.z, vc.w, vd.x, vd.y, vd.z, vd.w}; // lane j+4
        v4i a0[ND], a1[ND];
#pragma unroll
        for (int i = 0; i < ND; i++) a0[i] = a1[i] = (v4i){0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < 8; s++) {
#pragma unroll
            for (int i = 0; i < ND; i++) {
                // digit i of sc[s] in both 16-bit halves, then one packed 16-bit multiply per code word (the four
                // byte products stay below 256, so no carry crosses a byte)
                const uint32_t sel = (uint32_t)(s & 3) | 0x0C00u | ((uint32_t)(s & 3) << 16) | 0x0C000000u;
                const u16x2 d2 = as_u16x2(__builtin_amdgcn_perm(0u, dig[i][s >> 2], sel));
                a0[i] = mfma_acc(x0[s], as_u32(as_u16x2(code0[s]) * d2), a0[i]);
                a1[i] = mfma_acc(x1[s], as_u32(as_u16x2(code1[s]) * d2), a1[i]);
            }
        }
        const float4 dx4 = *reinterpret_cast<const float4 *>(xd + cg * 4);
        const float dxs[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
        const uint4 m0 = *reinterpret_cast<const uint4 *>(xm + j * ncp + cg * 4);
        const uint32_t mw0[4] = {m0.x, m0.y, m0.z, m0.w};
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int col = cg * 4 + c;
            if (col < NC) {
                int s0 = a0[ND - 1][c], s1 = a1[ND - 1][c];
#pragma unroll
                for (int i = ND - 2; i >= 0; i--) {
                    s0 = (s0 << DB) + a0[i][c];
                    s1 = (s1 << DB) + a1[i][c];
                }
                const float dd = dxs[c] * dw;
                const int lo0 = (int)(int16_t)(mw0[c] & 0xFFFF), hi0 = (int)(int16_t)(mw0[c] >> 16);
                pr0[col] = dd * (float)s0;
                pr1[col] = dd * (float)s1;
                pm[col] = (-dxs[c] * dminw) * (float)(mn0 * lo0 + mn1 * hi0);
            }
        }
    }
}

// LDS chunk (per super-block of the chunk): codes xq[CH][NC][256] (by lane slot), f32 scales xd[CH][NCP] and
// activation-sum pairs xm[CH][8][NCP] (pair i = sums 2i, 2i+1: Q4_K/Q5_K sub-block sums (i < 4), Q6_K group sums),
// NCP = NC rounded up to 4 so a thread reads its 4 columns with one 16-byte load.
template <int NC, int CH>
struct Lds {
    static constexpr int NCP = (NC + 3) / 4 * 4;
    int8_t xq[CH][NC][256];
    float xd[CH][NCP];
    uint32_t xm[CH][8][NCP];
};

template <int TYPE, int NC, int KS, int PF, int CH>
__global__ void __launch_bounds__(256) kq_mfma_kernel(MfArgs a) {
    static_assert(CH % (KS * PF) == 0, "a chunk must hold whole prefetch rounds");
    constexpr int RG = 4 / KS;                      // row groups (16 rows each) per work-group
    constexpr int NCG = (NC + 3) / 4;               // column groups of 4
    constexpr int NCP = Lds<NC, CH>::NCP;
    constexpr int NV = (CH * NC * 16 + 255) / 256;  // 16-byte code vectors per thread per chunk
    constexpr int NM = CH * NC;                     // (super-block, column) meta entries per chunk
    static_assert(NV <= 4 && NM <= 256, "staging shape");
    constexpr bool Q6 = TYPE == AQ_TYPE_Q6_K;
    __shared__ Lds<NC, CH> lds_buf[2];
    __shared__ float xch[KS > 1 ? RG : 1][KS > 1 ? 2 : 1][KS][3 * NC][64];

    const int t = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int rg = wid / KS, w = wid % KS;
    const int g = t >> 4, j = (t >> 2) & 3, r = t & 3;
    int row = ((int)blockIdx.x * RG + rg) * 16 + 4 * g + r;
    const bool valid = row < a.rows;
    if (!valid) row = a.rows - 1;
    const int nb = a.nb;
    const int nchunks = (nb + CH - 1) / CH;
    const size_t rowsb = (size_t)row * nb;

    float acc0[NC], acc1[NC], accm[NC]; // lane j, lane j+4, min lane j
#pragma unroll
    for (int i = 0; i < NC; i++) acc0[i] = acc1[i] = accm[i] = 0.0f;

    WRegs<TYPE> wr[PF];
#pragma unroll
    for (int p = 0; p < PF; p++) load_w<TYPE>(wr[p], a, rowsb + min(w + p * KS, nb - 1), j);
    int parity = 0;

    // ---- activation chunk staging (named registers, never an array: arrays here get demoted to scratch)
    uint4 sv0 = make_uint4(0, 0, 0, 0), sv1 = sv0, sv2 = sv0, sv3 = sv0, sm0 = sv0, sm1 = sv0;
    float sd = 0.0f;
#define AQ_STAGE_VEC(I, SV, BODY)                                                                             \
    if constexpr (I < NV) {                                                                                   \
        const int v = (int)threadIdx.x + I * 256;                                                             \
        const int c = v / (CH * 16), rem = v % (CH * 16), sbi = rem / 16, o = (rem % 16) * 16;                \
        BODY(SV)                                                                                              \
    }
    auto stage_load = [&](int k) {
        const int c0 = k * CH, ch = nb - c0 < CH ? nb - c0 : CH;
#define AQ_LOAD_BODY(SV)                                                                                      \
    if (c < NC && sbi < ch)                                                                                   \
        SV = *reinterpret_cast<const uint4 *>(a.xqs + (size_t)c * a.xcol + (size_t)(c0 + sbi) * 256 + o);
        AQ_STAGE_VEC(0, sv0, AQ_LOAD_BODY)
        AQ_STAGE_VEC(1, sv1, AQ_LOAD_BODY)
        AQ_STAGE_VEC(2, sv2, AQ_LOAD_BODY)
        AQ_STAGE_VEC(3, sv3, AQ_LOAD_BODY)
#undef AQ_LOAD_BODY
        const int e = (int)threadIdx.x;
        if (e < NM) {
            const int c = e / CH, sbi = e % CH;
            if (sbi < ch) {
                const size_t xm = (size_t)c * nb + c0 + sbi;
                sd = a.xd[xm];
                if constexpr (Q6) {
                    sm0 = reinterpret_cast<const uint4 *>(a.xbs + xm * 16)[0];
                    sm1 = reinterpret_cast<const uint4 *>(a.xbs + xm * 16)[1];
                } else {
                    sm0 = *reinterpret_cast<const uint4 *>(a.xq8s + xm * 8);
                }
            }
        }
    };
    auto stage_store = [&](int buf) {
        Lds<NC, CH> &L = lds_buf[buf];
#define AQ_STORE_BODY(SV)                                                                                     \
    if (c < NC) *reinterpret_cast<uint4 *>(&L.xq[sbi][c][o]) = SV;
        AQ_STAGE_VEC(0, sv0, AQ_STORE_BODY)
        AQ_STAGE_VEC(1, sv1, AQ_STORE_BODY)
        AQ_STAGE_VEC(2, sv2, AQ_STORE_BODY)
        AQ_STAGE_VEC(3, sv3, AQ_STORE_BODY)
#undef AQ_STORE_BODY
        const int e = (int)threadIdx.x;
        if (e < NM) {
            const int c = e / CH, sbi = e % CH;
            L.xd[sbi][c] = sd;
            L.xm[sbi][0][c] = sm0.x;
            L.xm[sbi][1][c] = sm0.y;
            L.xm[sbi][2][c] = sm0.z;
            L.xm[sbi][3][c] = sm0.w;
            if constexpr (Q6) {
                L.xm[sbi][4][c] = sm1.x;
                L.xm[sbi][5][c] = sm1.y;
                L.xm[sbi][6][c] = sm1.z;
                L.xm[sbi][7][c] = sm1.w;
            }
        }
    };
#undef AQ_STAGE_VEC
    stage_load(0);
    stage_store(0);
    if (nchunks > 1) stage_load(1);
    __syncthreads();

    for (int k = 0; k < nchunks; k++) {
        const int c0 = k * CH;
        const int ch = nb - c0 < CH ? nb - c0 : CH;
        const Lds<NC, CH> &L = lds_buf[k & 1];

        auto process = [&](const WRegs<TYPE> &wv, const int sbi, float *pr0, float *pr1, float *pm) {
            if constexpr (TYPE == AQ_TYPE_Q6_K)
                sb_products<TYPE, NC>(wv, &L.xq[sbi][0][0], &L.xd[sbi][0], &L.xm[sbi][0][0], NCP, j, r, pr0, pr1, pm);
            else
                sb_products_split<TYPE, NC>(wv, &L.xq[sbi][0][0], &L.xd[sbi][0], &L.xm[sbi][0][0], NCP, j, r, pr0, pr1,
                                            pm);
        };

        for (int rb = 0; rb < ch; rb += KS * PF) {
#pragma unroll
            for (int p = 0; p < PF; p++) {
                const int round0 = rb + p * KS; // first super-block (chunk-relative) of this round
                if (round0 < ch) {              // uniform across the work-group
                    const int sbi = round0 + w;
                    float pr0[NC], pr1[NC], pm[NC];
#pragma unroll
                    for (int c = 0; c < NC; c++) pr0[c] = pr1[c] = pm[c] = 0.0f;
                    if (sbi < ch) {
                        process(wr[p], sbi, pr0, pr1, pm);
                        load_w<TYPE>(wr[p], a, rowsb + min(c0 + sbi + PF * KS, nb - 1), j);
                    }
                    if constexpr (KS == 1) {
#pragma unroll
                        for (int c = 0; c < NC; c++) {
                            acc0[c] += pr0[c];
                            acc1[c] += pr1[c];
                            if constexpr (!Q6) accm[c] += pm[c];
                        }
                    } else {
                        float(*x)[3 * NC][64] = xch[rg][parity];
#pragma unroll
                        for (int c = 0; c < NC; c++) {
                            x[w][c][t] = pr0[c];
                            x[w][NC + c][t] = pr1[c];
                            x[w][2 * NC + c][t] = pm[c];
                        }
                        __syncthreads();
                        const int live = ch - round0 < KS ? ch - round0 : KS; // super-blocks in this round
#pragma unroll
                        for (int w2 = 0; w2 < KS; w2++) {
                            if (w2 < live) {
#pragma unroll
                                for (int c = 0; c < NC; c++) {
                                    acc0[c] += x[w2][c][t];
                                    acc1[c] += x[w2][NC + c][t];
                                    if constexpr (!Q6) accm[c] += x[w2][2 * NC + c][t];
                                }
                            }
                        }
                        parity ^= 1;
                    }
                }
            }
        }
        if (k + 1 < nchunks) {
            stage_store((k + 1) & 1);
            if (k + 2 < nchunks) stage_load(k + 2);
        }
        __syncthreads();
    }
    // ---------------------------------------------------------------- reduce the 8 lanes of each row
    // lanes j and j+4 are in one thread; j sits at t = 16g + 4j + r: xor 8 pairs j with j^2, xor 4 with j^1.
    if (w != 0) return; // every wave of a row group holds the same chain; wave 0 writes
#pragma unroll
    for (int col = 0; col < NC; col++) {
        float v = acc0[col] + acc1[col]; // l_j + l_{j+4}
        v = v + __shfl_xor(v, 8);
        v = v + __shfl_xor(v, 4);
        if constexpr (!Q6) {
            float m = accm[col];
            m = m + __shfl_xor(m, 8); // m0+m2, m1+m3
            m = m + __shfl_xor(m, 4);
            v = v + m;
        }
        if (j == 0 && valid) {
            const size_t o = (size_t)col * a.rows + row;
            a.y[o] = a.resid ? a.resid[o] + v : v;
        }
    }
}

// Whole-K variant: the activations of all nb super-blocks are copied to LDS once, behind one barrier, so the
// weight prefetch ring is never drained by a staging wait; the main loop has no data-dependent branch around a
// load (a round past the end of K is computed on clamped indices and its products are not added). Column stride
// KQ_XS = 256 + 16 bytes puts the 4 columns a wave reads at once in different LDS banks.
//
// One launch can cover up to three matrices that read the same activations (gate and up; q, k and v; the
// DeltaNet qkv and z projections): the work-groups are laid out segment after segment, each segment with its own
// weights, output and K-quant type (one of the kernel's two types), so the staging and the launch are shared.
constexpr int KQ_XS = 272;
constexpr int KQ_MAXSEG = 3;

struct KqSeg {
    const uint8_t *qa, *qb, *sc, *dm;
    float *y;
    const float *resid;
    int rows, type, wg_end; // wg_end: one past this segment's last work-group
};
struct KqGroup {
    KqSeg seg[KQ_MAXSEG];
    int nseg, nb;
    const int8_t *xqs;
    const float *xd;
    const int16_t *xbs, *xq8s;
    size_t xcol;
};

inline size_t kq_full_lds_bytes(int nb, int nc, bool has45, bool has6) {
    const int ncp = (nc + 3) / 4 * 4, np = (has45 ? 4 : 0) + (has6 ? 8 : 0);
    return (size_t)nb * nc * KQ_XS + (size_t)nb * ncp * 4 + (size_t)nb * np * ncp * 4;
}

// Activations of every super-block to LDS: codes [sb][column][KQ_XS], scales [sb][NCP], activation-sum pairs
// [sb][NP][NCP]: the 4 sub-block-sum pairs (Q4_K/Q5_K segments, HAS45) and then the 8 group-sum pairs (Q6_K
// segments, HAS6).
template <int NC, bool HAS45, bool HAS6>
__device__ __forceinline__ void kq_stage(const KqGroup &G, int8_t *sxq, float *sxd, uint32_t *sxm) {
    constexpr int NCP = (NC + 3) / 4 * 4;
    constexpr int NP = (HAS45 ? 4 : 0) + (HAS6 ? 8 : 0), P6 = HAS45 ? 4 : 0;
    const int nb = G.nb;
    // 16 threads per (column, super-block) record of 256 codes, two records per thread group in flight
    const int o = threadIdx.x & 15, nrec = nb * NC;
    for (int r0 = (int)threadIdx.x >> 4; r0 < nrec; r0 += 32) {
        const int ra = r0, rb = r0 + 16 < nrec ? r0 + 16 : r0; // the second record, or the first again
        const int ca = ra / nb, sa = ra - ca * nb, cb = rb / nb, sbb = rb - cb * nb;
        const uint4 va = *reinterpret_cast<const uint4 *>(G.xqs + (size_t)ca * G.xcol + (size_t)sa * 256 + o * 16);
        const uint4 vb = *reinterpret_cast<const uint4 *>(G.xqs + (size_t)cb * G.xcol + (size_t)sbb * 256 + o * 16);
        *reinterpret_cast<uint4 *>(sxq + ((size_t)sa * NC + ca) * KQ_XS + o * 16) = va;
        *reinterpret_cast<uint4 *>(sxq + ((size_t)sbb * NC + cb) * KQ_XS + o * 16) = vb;
    }
    for (int e = (int)threadIdx.x; e < nb * NC; e += 256) {
        const int c = e / nb, sb = e % nb;
        const size_t m = (size_t)c * nb + sb;
        sxd[sb * NCP + c] = G.xd[m];
        if constexpr (HAS45) {
            const uint4 p0 = *reinterpret_cast<const uint4 *>(G.xq8s + m * 8);
            sxm[(sb * NP + 0) * NCP + c] = p0.x;
            sxm[(sb * NP + 1) * NCP + c] = p0.y;
            sxm[(sb * NP + 2) * NCP + c] = p0.z;
            sxm[(sb * NP + 3) * NCP + c] = p0.w;
        }
        if constexpr (HAS6) {
            const uint4 g0 = reinterpret_cast<const uint4 *>(G.xbs + m * 16)[0];
            const uint4 g1 = reinterpret_cast<const uint4 *>(G.xbs + m * 16)[1];
            const uint32_t pv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
            for (int q = 0; q < 8; q++) sxm[(sb * NP + P6 + q) * NCP + c] = pv[q];
        }
    }
}

// One segment's work-group: rows wg*RG*16 .. +RG*16 of the segment's matrix, K split KS ways across waves.
// xch: [RG][2][KS][3 NC][64] exchange floats. HAS45 / HAS6: the staging's pair sets (this segment's type reads
// its own).
template <int TYPE, int NC, int KS, int PF, bool HAS45, bool HAS6>
__device__ __forceinline__ void kq_full_run(const KqGroup &G, const KqSeg &sg, int wg, int8_t *sxq, float *sxd,
                                            uint32_t *sxm, float *xch) {
    constexpr int RG = 4 / KS;
    constexpr int NCP = (NC + 3) / 4 * 4;
    constexpr bool Q6 = TYPE == AQ_TYPE_Q6_K;
    constexpr int NP = (HAS45 ? 4 : 0) + (HAS6 ? 8 : 0), POFF = Q6 && HAS45 ? 4 : 0;
    MfArgs a{};
    a.qa = sg.qa;
    a.qb = sg.qb;
    a.sc = sg.sc;
    a.dm = sg.dm;
    a.rows = sg.rows;
    a.nb = G.nb;
    const int nb = G.nb;
    const int t = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int rg = wid / KS, w = wid % KS;
    const int g = t >> 4, j = (t >> 2) & 3, r = t & 3;
    int row = (wg * RG + rg) * 16 + 4 * g + r;
    const bool valid = row < a.rows;
    if (!valid) row = a.rows - 1;
    const size_t rowsb = (size_t)row * nb;

    // the first PF rounds of weights fly while the activations are staged
    WRegs<TYPE> wr[PF];
#pragma unroll
    for (int p = 0; p < PF; p++) load_w<TYPE>(wr[p], a, rowsb + min(w + p * KS, nb - 1), j);
    kq_stage<NC, HAS45, HAS6>(G, sxq, sxd, sxm);
    __syncthreads();

    float acc0[NC], acc1[NC], accm[NC]; // lane j, lane j+4, min lane j
#pragma unroll
    for (int i = 0; i < NC; i++) acc0[i] = acc1[i] = accm[i] = 0.0f;
    int parity = 0;
    const int nr = (nb + KS - 1) / KS; // rounds of KS super-blocks (wave w takes super-block round*KS + w)

    auto round_body = [&](WRegs<TYPE> &wv, const int round, const bool prefetch) {
        const int sb = round * KS + w;
        const int sbc = sb < nb ? sb : nb - 1;
        float pr0[NC], pr1[NC], pm[NC];
#pragma unroll
        for (int c = 0; c < NC; c++) pm[c] = 0.0f;
        const int8_t *xq = sxq + (size_t)sbc * NC * KQ_XS;
        const float *xd = sxd + sbc * NCP;
        const uint32_t *xm = sxm + (sbc * NP + POFF) * NCP;
        if constexpr (Q6)
            sb_products<TYPE, NC, KQ_XS>(wv, xq, xd, xm, NCP, j, r, pr0, pr1, pm);
        else
            sb_products_split<TYPE, NC, KQ_XS>(wv, xq, xd, xm, NCP, j, r, pr0, pr1, pm);
        if (prefetch) {
            load_w<TYPE>(wv, a, rowsb + min(sb + PF * KS, nb - 1), j);
            __builtin_amdgcn_sched_barrier(0); // issue the refill here, not after the later rounds' compute
        }
        const int live = nb - round * KS < KS ? nb - round * KS : KS; // super-blocks in this round
        if constexpr (KS == 1) {
#pragma unroll
            for (int c = 0; c < NC; c++) {
                acc0[c] += pr0[c];
                acc1[c] += pr1[c];
                if constexpr (!Q6) accm[c] += pm[c];
            }
        } else {
            float *x = xch + (size_t)(rg * 2 + parity) * KS * 3 * NC * 64; // [KS][3 NC][64]
#pragma unroll
            for (int c = 0; c < NC; c++) {
                x[(w * 3 * NC + c) * 64 + t] = pr0[c];
                x[(w * 3 * NC + NC + c) * 64 + t] = pr1[c];
                x[(w * 3 * NC + 2 * NC + c) * 64 + t] = pm[c];
            }
            __syncthreads();
#pragma unroll
            for (int w2 = 0; w2 < KS; w2++) {
                if (w2 < live) {
#pragma unroll
                    for (int c = 0; c < NC; c++) {
                        acc0[c] += x[(w2 * 3 * NC + c) * 64 + t];
                        acc1[c] += x[(w2 * 3 * NC + NC + c) * 64 + t];
                        if constexpr (!Q6) accm[c] += x[(w2 * 3 * NC + 2 * NC + c) * 64 + t];
                    }
                }
            }
            parity ^= 1;
        }
    };
    const int nfull = nr / PF * PF;
    for (int rd = 0; rd < nfull; rd += PF) {
#pragma unroll
        for (int p = 0; p < PF; p++) round_body(wr[p], rd + p, true);
    }
#pragma unroll
    for (int p = 0; p < PF; p++)
        if (nfull + p < nr) round_body(wr[p], nfull + p, false);

    if (w != 0) return; // every wave of a row group holds the same chain; wave 0 writes
#pragma unroll
    for (int col = 0; col < NC; col++) {
        float v = acc0[col] + acc1[col]; // l_j + l_{j+4}
        v = v + __shfl_xor(v, 8);
        v = v + __shfl_xor(v, 4);
        if constexpr (!Q6) {
            float m = accm[col];
            m = m + __shfl_xor(m, 8); // m0+m2, m1+m3
            m = m + __shfl_xor(m, 4);
            v = v + m;
        }
        if (j == 0 && valid) {
            const size_t o = (size_t)col * a.rows + row;
            sg.y[o] = sg.resid ? sg.resid[o] + v : v;
        }
    }
}

template <int T0, int T1, int NC, int KS, int PF>
__global__ void __launch_bounds__(256) kq_group_kernel(KqGroup G) {
    constexpr int RG = 4 / KS;
    constexpr bool HAS6 = T0 == AQ_TYPE_Q6_K || T1 == AQ_TYPE_Q6_K;
    constexpr bool HAS45 = T0 != AQ_TYPE_Q6_K || T1 != AQ_TYPE_Q6_K;
    constexpr int NCP = (NC + 3) / 4 * 4;
    extern __shared__ __align__(16) uint8_t kq_lds[];
    __shared__ float xch[(KS > 1 ? RG : 1) * (KS > 1 ? 2 : 1) * KS * 3 * NC * 64];
    int si = 0; // this work-group's segment (uniform)
    while (si + 1 < G.nseg && (int)blockIdx.x >= G.seg[si].wg_end) si++;
    const KqSeg &sg = G.seg[si];
    const int wg = (int)blockIdx.x - (si ? G.seg[si - 1].wg_end : 0);
    int8_t *sxq = reinterpret_cast<int8_t *>(kq_lds);
    float *sxd = reinterpret_cast<float *>(kq_lds + (size_t)G.nb * NC * KQ_XS);
    uint32_t *sxm = reinterpret_cast<uint32_t *>(sxd + (size_t)G.nb * NCP);
    if (T0 == T1 || sg.type == T0)
        kq_full_run<T0, NC, KS, PF, HAS45, HAS6>(G, sg, wg, sxq, sxd, sxm, xch);
    else
        kq_full_run<T1, NC, KS, PF, HAS45, HAS6>(G, sg, wg, sxq, sxd, sxm, xch);
}

template <int TYPE, int NC, int KS>
int launch_ks(const MfArgs &args, hipStream_t stream) {
    // prefetch depth and chunk (CH a multiple of KS * PF; two chunk buffers in LDS), from a sweep on MI355X of the
    // 27B shapes at N = 1, 4: fewer registers and smaller chunks beat deeper prefetch at this occupancy
    constexpr int PF = KS == 1 ? 4 : 2;
    constexpr int CH = KS * PF;
    constexpr int ROWS = 64 / KS;
    const dim3 grid((unsigned)((args.rows + ROWS - 1) / ROWS)), block(256);
    hipLaunchKernelGGL((kq_mfma_kernel<TYPE, NC, KS, PF, CH>), grid, block, 0, stream, args);
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "kq_mfma launch");
}

// The chunked kernel (activations staged a chunk at a time): the fallback when the whole-K staging does not fit
// the CU's LDS. K is split across waves when the rows alone give too few waves to keep HBM busy.
template <int TYPE, int NC>
int launch_chunked_nc(const MfArgs &args, hipStream_t stream) {
    const int waves = (args.rows + 15) / 16;
    if (waves >= 2048 || args.nb < 8) return launch_ks<TYPE, NC, 1>(args, stream);
    if (waves >= 1024) return launch_ks<TYPE, NC, 2>(args, stream);
    return launch_ks<TYPE, NC, 4>(args, stream);
}

template <int TYPE>
int launch_chunked(const MfArgs &args, size_t ncols, hipStream_t stream) {
    switch (ncols) {
    case 1: return launch_chunked_nc<TYPE, 1>(args, stream);
    case 2: return launch_chunked_nc<TYPE, 2>(args, stream);
    case 3: return launch_chunked_nc<TYPE, 3>(args, stream);
    case 4: return launch_chunked_nc<TYPE, 4>(args, stream);
    case 5: return launch_chunked_nc<TYPE, 5>(args, stream);
    case 6: return launch_chunked_nc<TYPE, 6>(args, stream);
    case 7: return launch_chunked_nc<TYPE, 7>(args, stream);
    case 8: return launch_chunked_nc<TYPE, 8>(args, stream);
    default: return fail(AQ_EINVAL, "kq_mfma: ncols must be 1..8");
    }
}

constexpr int KQ_LDS_MAX = 160 * 1024 - 512; // a CU's LDS, less a margin

template <int NC>
constexpr size_t kq_xch_bytes() { return (size_t)2 * 2 * 2 * 3 * NC * 64 * 4; } // the same for KS = 2 and KS = 4

template <int T0, int T1, int NC, int KS>
int launch_group_ks(KqGroup G, size_t lds, hipStream_t stream) {
    constexpr int PF = 2;
    constexpr int ROWS = 64 / KS;
    int wgs = 0;
    for (int i = 0; i < G.nseg; i++) {
        wgs += (G.seg[i].rows + ROWS - 1) / ROWS;
        G.seg[i].wg_end = wgs;
    }
    if (lds > 64 * 1024) {
        static bool raised = false; // once per instantiation: allow dynamic LDS up to the CU's size
        if (!raised) {
            const void *fn = reinterpret_cast<const void *>(&kq_group_kernel<T0, T1, NC, KS, PF>);
            AQ_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)(KQ_LDS_MAX - kq_xch_bytes<NC>())));
            raised = true;
        }
    }
    hipLaunchKernelGGL((kq_group_kernel<T0, T1, NC, KS, PF>), dim3((unsigned)wgs), dim3(256), lds, stream, G);
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "kq_mfma launch");
}

// Returns 1 (nothing launched) when the whole-K staging does not fit. The split from a sweep on MI355X of the 27B
// shapes: long rows (K >= 12288) and tall groups at N > 1 split K in two, the rest in four.
template <int T0, int T1, int NC>
int launch_group_nc(const KqGroup &G, int rows, hipStream_t stream) {
    constexpr bool HAS6 = T0 == AQ_TYPE_Q6_K || T1 == AQ_TYPE_Q6_K;
    constexpr bool HAS45 = T0 != AQ_TYPE_Q6_K || T1 != AQ_TYPE_Q6_K;
    const size_t lds = kq_full_lds_bytes(G.nb, NC, HAS45, HAS6);
    if (lds + kq_xch_bytes<NC>() > (size_t)KQ_LDS_MAX) return 1;
    if (G.nb >= 48 || (NC > 1 && rows >= 12288)) return launch_group_ks<T0, T1, NC, 2>(G, lds, stream);
    return launch_group_ks<T0, T1, NC, 4>(G, lds, stream);
}

template <int T0, int T1>
int launch_group_t(const KqGroup &G, int rows, size_t ncols, hipStream_t stream) {
    switch (ncols) {
    case 1: return launch_group_nc<T0, T1, 1>(G, rows, stream);
    case 2: return launch_group_nc<T0, T1, 2>(G, rows, stream);
    case 3: return launch_group_nc<T0, T1, 3>(G, rows, stream);
    case 4: return launch_group_nc<T0, T1, 4>(G, rows, stream);
    case 5: return launch_group_nc<T0, T1, 5>(G, rows, stream);
    case 6: return launch_group_nc<T0, T1, 6>(G, rows, stream);
    case 7: return launch_group_nc<T0, T1, 7>(G, rows, stream);
    case 8: return launch_group_nc<T0, T1, 8>(G, rows, stream);
    default: return fail(AQ_EINVAL, "kq_mfma: ncols must be 1..8");
    }
}

MfArgs single_args(const Weight &w, const Act &x, float *y, const float *resid) {
    MfArgs args{};
    args.qa = w.qa;
    args.qb = w.qb;
    args.sc = w.sc;
    args.dm = w.dm;
    args.rows = (int)w.rows;
    args.nb = (int)w.nb;
    args.xqs = x.qs;
    args.xd = x.d;
    args.xbs = x.bs;
    args.xq8s = x.q8s;
    args.xcol = x.n;
    args.y = y;
    args.resid = resid;
    return args;
}

// One launch over segments [i0, i1) of at most two K-quant types; the chunked kernel per segment if the staging
// does not fit.
int launch_run(const Weight *const *ws, float *const *ys, const float *const *resids, int i0, int i1, const Act &x,
               size_t ncols, hipStream_t stream) {
    KqGroup G{};
    G.nseg = i1 - i0;
    G.nb = (int)ws[i0]->nb;
    G.xqs = x.qs;
    G.xd = x.d;
    G.xbs = x.bs;
    G.xq8s = x.q8s;
    G.xcol = x.n;
    int t0 = 99, t1 = 0, rows = 0;
    for (int i = i0; i < i1; i++) {
        const Weight &w = *ws[i];
        KqSeg &sg = G.seg[i - i0];
        sg.qa = w.qa;
        sg.qb = w.qb;
        sg.sc = w.sc;
        sg.dm = w.dm;
        sg.y = ys[i];
        sg.resid = resids ? resids[i] : nullptr;
        sg.rows = (int)w.rows;
        sg.type = w.type;
        rows += (int)w.rows;
        t0 = w.type < t0 ? w.type : t0;
        t1 = w.type > t1 ? w.type : t1;
    }
    int rc = 1;
    constexpr int Q4 = AQ_TYPE_Q4_K, Q5 = AQ_TYPE_Q5_K, Q6 = AQ_TYPE_Q6_K;
    if (t0 == Q4 && t1 == Q4) rc = launch_group_t<Q4, Q4>(G, rows, ncols, stream);
    else if (t0 == Q5 && t1 == Q5) rc = launch_group_t<Q5, Q5>(G, rows, ncols, stream);
    else if (t0 == Q6 && t1 == Q6) rc = launch_group_t<Q6, Q6>(G, rows, ncols, stream);
    else if (t0 == Q4 && t1 == Q5) rc = launch_group_t<Q4, Q5>(G, rows, ncols, stream);
    else if (t0 == Q4 && t1 == Q6) rc = launch_group_t<Q4, Q6>(G, rows, ncols, stream);
    else if (t0 == Q5 && t1 == Q6) rc = launch_group_t<Q5, Q6>(G, rows, ncols, stream);
    if (rc != 1) return rc;
    for (int i = i0; i < i1; i++) {
        const MfArgs args = single_args(*ws[i], x, ys[i], resids ? resids[i] : nullptr);
        switch (ws[i]->type) {
        case Q4: rc = launch_chunked<Q4>(args, ncols, stream); break;
        case Q5: rc = launch_chunked<Q5>(args, ncols, stream); break;
        default: rc = launch_chunked<Q6>(args, ncols, stream); break;
        }
        if (rc) return rc;
    }
    return 0;
}

} // namespace

int launch_kq_group(const Weight *const *ws, float *const *ys, const float *const *resids, int n, const Act &x,
                    size_t ncols, hipStream_t stream) {
    AQ_REQUIRE(n >= 1 && ws && ys, "kq_mfma: no matrices");
    AQ_REQUIRE(ncols >= 1 && ncols <= 8, "kq_mfma: ncols must be 1..8");
    for (int i = 0; i < n; i++) {
        AQ_REQUIRE(is_kquant(ws[i]->type), "kq_mfma: not a K-quant type");
        AQ_REQUIRE(ws[i]->nb == ws[0]->nb, "kq_mfma: grouped matrices must share K");
        AQ_REQUIRE(ws[i]->cols == x.n, "kq_mfma: activation length != weight columns");
    }
    // consecutive runs of at most KQ_MAXSEG matrices and two types per launch
    int i0 = 0;
    while (i0 < n) {
        int i1 = i0 + 1, ta = ws[i0]->type, tb = ta;
        while (i1 < n && i1 - i0 < KQ_MAXSEG) {
            const int t = ws[i1]->type;
            if (t != ta && t != tb) {
                if (ta != tb) break;
                tb = t;
            }
            i1++;
        }
        const int rc = launch_run(ws, ys, resids, i0, i1, x, ncols, stream);
        if (rc) return rc;
        i0 = i1;
    }
    return 0;
}

int launch_kq_mfma(const Weight &w, const Act &x, size_t ncols, float *y, const float *resid, hipStream_t stream) {
    const Weight *ws[1] = {&w};
    float *ys[1] = {y};
    const float *rs[1] = {resid};
    return launch_kq_group(ws, ys, rs, 1, x, ncols, stream);
}

} // namespace aq
