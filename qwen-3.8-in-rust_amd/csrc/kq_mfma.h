// kq_mfma.h — the K-quant x Q8_K matmul (N = 1 matvec and the N = k+1 verify batch) on gfx950 matrix cores.
//
// Same integers and floats as the reference (kdot.rs:37-140 and the blocked kdot.rs:176-333): per super-block the
// 8 exact i32 lane sums (lane l = elements 4l..4l+3 of each 32-element sub-block, the scale multiplied in as an
// integer), the 4 Q4_K/Q5_K min lanes, the Q6_K -32 fold; then acc[l] += (dx*dw) * float(sum) super-block by
// super-block without FMA, and the ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)) [+ (m0+m2)+(m1+m3)] reduction. Only how
// the exact integers are produced is new:
//
//  * v_mfma_i32_4x4x4_16b_i8 computes 16 independent 4x4x4 int8 products. Block b of one instruction is
//    (q, j): its K = 4 elements are lane j's 4 positions of one sub-block, so it yields the lane-j partial of that
//    sub-block for 4 weight rows x 4 activation columns, exactly (int32). A = activations (A row i = column c),
//    B = weight codes (B column = weight row). Register layout, measured on the device: A and B of block b at lanes
//    4b+i / 4b+j, D[i][j] at lane 4b+j, VGPR i.
//  * Thread 4b + r (b = 4q + j) owns weight row r of its block's row group and the two reference lanes j and j+4:
//    one instruction set computes lane j, a second one lane j+4. q names a (row group, K slice) pair: a wave covers
//    16 / KSW rows and KSW consecutive super-blocks per round (kq_wave_run).
//  * Q4_K / Q5_K: the 6-bit sub-block scale is split into 3-bit (2-bit) digits folded into the int8 weight operand
//    (sb_products_split), so the MFMA accumulator sums the scaled sub-block dots; Q6_K (int8 scales) multiplies
//    each MFMA partial by its scale with a full-rate 24-bit integer mad.
//  * Results go to VGPRs (built with -amdgpu-mfma-vgpr-form): no accumulator-register copies.
//  * Weights are read from tiled planes (4 rows x 1 super-block per tile, aq_common.h) into a register ring PF
//    rounds deep; activations are staged in LDS (all of K, or chunks of it) once per work-group.
#pragma once
#include "aq_common.h"

#include <algorithm>
#include <map>
#include <mutex>

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

// a.lo * b.lo + a.hi * b.hi of two signed 16-bit pairs (v_dot2_i32_i16), exact in i32
typedef short s16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ int sdot2(uint32_t a, uint32_t b) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(s16x2, a), __builtin_bit_cast(s16x2, b), 0, false);
}
// the same with the zero addend as the instruction's inline constant (the builtin's two-operand form takes an extra
// register move to clear its accumulator)
__device__ __forceinline__ int sdot2z(uint32_t a, uint32_t b) {
    int r;
    __asm__("v_dot2_i32_i16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// A 4 x 4 transpose of 16-lane rows across four registers: on entry row q (lanes 16q..16q+15) of p_k holds chain k's
// value for K slice q; on exit row q of p_m holds chain q's value for K slice m. Two v_permlane16_swap (odd rows of
// the first register with even rows of the second), then two v_permlane32_swap (upper half of the first with lower
// half of the second), all within the wave's registers.
__device__ __forceinline__ void xpose4(float &p0, float &p1, float &p2, float &p3) {
    const auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, p0), __builtin_bit_cast(unsigned, p1),
                                                    false, false);
    const auto b = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, p2), __builtin_bit_cast(unsigned, p3),
                                                    false, false);
    const auto c = __builtin_amdgcn_permlane32_swap(a[0], b[0], false, false);
    const auto d = __builtin_amdgcn_permlane32_swap(a[1], b[1], false, false);
    p0 = __builtin_bit_cast(float, (unsigned)c[0]);
    p2 = __builtin_bit_cast(float, (unsigned)c[1]);
    p1 = __builtin_bit_cast(float, (unsigned)d[0]);
    p3 = __builtin_bit_cast(float, (unsigned)d[1]);
}

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

// Tile `tile` (= (row >> 2) * nb + sb), row r = row & 3 within it, lane pair j (tiled planes, aq_common.h): the
// 16 (j, r) threads of a matrix-core block read contiguous 256-byte runs. Offsets are 32-bit (every plane is below
// 4 GiB), so the loads take the uniform plane base plus one 32-bit lane offset.
template <int TYPE>
__device__ __forceinline__ void load_w(WRegs<TYPE> &w, const MfArgs &a, uint32_t tile, int r, int j) {
    const uint32_t jr = (uint32_t)(j * 4 + r);
    const uint8_t *qa = a.qa + (tile * 512u + jr * 16u);
    w.qa0 = ld_nt4(qa);       // lane j
    w.qa1 = ld_nt4(qa + 256); // lane j + 4
    w.sc = ld_nt4(a.sc + (tile * 64u + (uint32_t)r * 16u));
    if constexpr (TYPE == AQ_TYPE_Q5_K) {
        const uint2 h = ld_nt2(a.qb + (tile * 128u + jr * 8u));
        w.qb = make_uint4(h.x, h.y, 0, 0);
    } else if constexpr (TYPE == AQ_TYPE_Q6_K) {
        w.qb = ld_nt4(a.qb + (tile * 256u + jr * 16u));
        w.d6 = ld_nth(a.dm + (tile * 8u + (uint32_t)r * 2u));
    }
}

// The products of one super-block for one thread: pr0/pr1 = (dx*dw)*float(lane sum) of lanes j and j+4, pm the
// Q4_K/Q5_K min product of min lane j, for every column. xq: the super-block's codes, 256 bytes per column (lane-slot
// order, XS bytes per column); xd: its f32 scales per column; xm: its activation-sum pairs [pair][ncp].
// kdot.rs:37-140 per lane.
// With IS, the exact integers behind the products are also returned: is0/is1 the lane sums of lanes j and j+4
// (Q6_K: after the -32 fold), ism the min product of min lane j (Q4_K/Q5_K), per column.
template <int TYPE, int NC, int XS = 256, bool IS = false>
__device__ __forceinline__ void sb_products(const WRegs<TYPE> &wv, const int8_t *xq, const float *xd,
                                            const uint32_t *xm, int ncp, int j, int r, float *pr0, float *pr1,
                                            float *pm, int *is0 = nullptr, int *is1 = nullptr,
                                            int *ism = nullptr) {
    constexpr int NCG = (NC + 3) / 4;
    constexpr bool Q6 = TYPE == AQ_TYPE_Q6_K;
    uint32_t code0[8], code1[8]; // 4 unsigned codes per sub-block, lanes j and j+4
    int scl0[8], scl1[8];        // integer scale per sub-block, lanes j and j+4
    int mn0 = 0, mn1 = 0;        // Q4_K/Q5_K mins of sub-blocks 2j, 2j+1 (min lane j)
    int os00 = 0, os01 = 0, os10 = 0, os11 = 0; // Q6_K -32 fold scales: groups 2l, 2l+1 of l = j, j+4
    uint32_t osp0 = 0, osp1 = 0;                 // the same as signed 16-bit pairs
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
        osp0 = ((uint32_t)os00 & 0xFFFFu) | ((uint32_t)os01 << 16);
        osp1 = ((uint32_t)os10 & 0xFFFFu) | ((uint32_t)os11 << 16);
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
                    // the -32 fold: lo * os_a + hi * os_b as one dot2 of the 16-bit pairs, exact
                    const int i0 = s0[c] - 32 * sdot2(osp0, mw0[c]), i1 = s1[c] - 32 * sdot2(osp1, mw1[c]);
                    pr0[col] = dd * (float)i0;
                    pr1[col] = dd * (float)i1;
                    if constexpr (IS) {
                        is0[col] = i0;
                        is1[col] = i1;
                        ism[col] = 0;
                    }
                } else {
                    const int im = mn0 * lo0 + mn1 * hi0;
                    pr0[col] = dd * (float)s0[c];
                    pr1[col] = dd * (float)s1[c];
                    pm[col] = (-dxs[c] * dminw) * (float)im;
                    if constexpr (IS) {
                        is0[col] = s0[c];
                        is1[col] = s1[c];
                        ism[col] = im;
                    }
                }
            }
        }
    }
}

// The DB-bit digits of the 8 six-bit sub-block scales (the bytes of sc_lo, sc_hi) as 16-bit pairs: the halves of
// dig[i][p] are digit i of scales 2p and 2p + 1. The digits are split byte-parallel (one shift and mask per digit
// and word), then one byte permute per pair; the words are opaque to the compiler, so a half reaches both halves of
// the code multiply through its operand select rather than a re-derived shift.
template <int DB, int ND>
__device__ __forceinline__ void kq_digits(uint32_t sc_lo, uint32_t sc_hi, uint32_t (&dig)[ND][4]) {
    constexpr uint32_t BM = ((1u << DB) - 1u) * 0x01010101u;
#pragma unroll
    for (int i = 0; i < ND; i++) {
        const uint32_t dlo = (sc_lo >> (DB * i)) & BM, dhi = (sc_hi >> (DB * i)) & BM;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint32_t b0 = (uint32_t)(2 * (p & 1));
            dig[i][p] = __builtin_amdgcn_perm(0u, p < 2 ? dlo : dhi, b0 | 0x0C00u | ((b0 + 1u) << 16) | 0x0C000000u);
            __asm__("" : "+v"(dig[i][p]));
        }
    }
}

// Q4_K / Q5_K products with the sub-block scale inside the matrix-core operand. A 6-bit scale sc is split into
// digits of DB bits (sc = sum_i digit_i << (DB*i); DB = 3 for Q4_K codes <= 15, DB = 2 for Q5_K codes <= 31), so
// code * digit <= 105 (resp. 93) is an int8: one 32-bit multiply scales the 4 packed code bytes of a sub-block
// without carries, and the MFMA accumulator sums sc_i-weighted dots over the 8 sub-blocks. The lane sum is then
// sum_i D_i << (DB*i) = sum_s sc[s] * dot_s exactly — the same integer as kdot.rs:37-95 — with no per-output
// scale multiply.
template <int TYPE, int NC, int XS = 256, bool IS = false>
__device__ __forceinline__ void sb_products_split(const WRegs<TYPE> &wv, const int8_t *xq, const float *xd,
                                                  const uint32_t *xm, int ncp, int j, int r, float *pr0,
                                                  float *pr1, float *pm, int *is0 = nullptr, int *is1 = nullptr,
                                                  int *ism = nullptr) {
    constexpr int NCG = (NC + 3) / 4;
    constexpr int DB = TYPE == AQ_TYPE_Q4_K ? 3 : 2;   // digit bits
    constexpr int ND = TYPE == AQ_TYPE_Q4_K ? 2 : 3;   // digits of a 6-bit scale
    // up to four columns: the activation reads go out first, so their LDS latency passes under the unpacking (the
    // same in the Q6_K path costs 25 registers: three waves per SIMD instead of four)
    uint4 xh[4];
    float4 dxh;
    uint4 mh;
    if constexpr (NCG == 1) {
        const uint4 *xp = reinterpret_cast<const uint4 *>(xq + (r < NC ? r : 0) * XS + j * 64);
#pragma unroll
        for (int u = 0; u < 4; u++) xh[u] = xp[u];
        dxh = *reinterpret_cast<const float4 *>(xd);
        mh = *reinterpret_cast<const uint4 *>(xm + j * ncp);
        __builtin_amdgcn_sched_barrier(0);
    }
    const uint32_t q0 = wv.sc.y, q1 = wv.sc.z, q2 = wv.sc.w;
    const uint32_t sc_lo = q0 & 0x3F3F3F3Fu, mn_lo = q1 & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (q2 & 0x0F0F0F0Fu) | ((q0 >> 2) & 0x30303030u);
    const uint32_t mn_hi = ((q2 >> 4) & 0x0F0F0F0Fu) | ((q1 >> 2) & 0x30303030u);
    const uint32_t mnw = j < 2 ? mn_lo : mn_hi;
    // the min lane's two mins as a 16-bit pair, for one dot2 per column against the activation-sum pair
    const uint32_t mnp = __builtin_amdgcn_perm(0u, mnw, (uint32_t)(2 * (j & 1)) | 0x0C00u |
                                                          ((uint32_t)(2 * (j & 1) + 1) << 16) | 0x0C000000u);
    // digit pair words: the 16-bit halves of dig[i][p] are digit i of sc[2p] and sc[2p + 1]; a packed multiply
    // broadcasts one half to both halves of the code word (op_sel), so no per-sub-block byte shuffle is needed
    uint32_t dig[ND][4];
    kq_digits<DB, ND>(sc_lo, sc_hi, dig);
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
        const uint4 va = NCG == 1 ? xh[0] : xp[0], vb = NCG == 1 ? xh[1] : xp[1], vc = NCG == 1 ? xh[2] : xp[2],
                    vd = NCG == 1 ? xh[3] : xp[3];
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
                const u16x2 dp = as_u16x2(dig[i][s >> 1]);
                const u16x2 d2 = (s & 1) ? (u16x2){dp.y, dp.y} : (u16x2){dp.x, dp.x};
                a0[i] = mfma_acc(x0[s], as_u32(as_u16x2(code0[s]) * d2), a0[i]);
                a1[i] = mfma_acc(x1[s], as_u32(as_u16x2(code1[s]) * d2), a1[i]);
            }
        }
        const float4 dx4 = NCG == 1 ? dxh : *reinterpret_cast<const float4 *>(xd + cg * 4);
        const float dxs[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
        const uint4 m0 = NCG == 1 ? mh : *reinterpret_cast<const uint4 *>(xm + j * ncp + cg * 4);
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
                const int im = sdot2z(mnp, mw0[c]); // mn0 * lo0 + mn1 * hi0, exact
                pr0[col] = dd * (float)s0;
                pr1[col] = dd * (float)s1;
                pm[col] = (-dxs[c] * dminw) * (float)im;
                if constexpr (IS) {
                    is0[col] = s0;
                    is1[col] = s1;
                    ism[col] = im;
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------ the wave-split kernel
// The activations of all nb super-blocks are copied to LDS once per work-group, behind its only barrier (column
// stride KQ_XS = 256 + 16 bytes puts the 4 columns a wave reads at once in different LDS banks); weights stream
// from HBM into a register ring PF rounds deep.
//
// The 16 matrix-core blocks of a wave are (q, j): j = the lane pair (j, j+4), q = (row group rg, K slice ks) with
// KSW K slices per wave (2 or 4) and 4 / KSW row groups of 4 rows: a wave owns 16 / KSW rows and in round rd its
// K slice ks computes super-block rd * KSW + ks. Matrices split K four ways inside the wave, so a wave covers 4 rows
// and the grid holds enough waves even for the 5120-row ones; K below 4 super-blocks and the lm_head at N > 1 take
// two slices (kq_pick_ksw). The f32 chains stay the reference's sequential sums: each round the K slices hand their
// products to the chain owners — by register transposes with four slices, through the wave's own LDS slot with two
// (no work-group barrier; one wave's LDS accesses execute in order) — and the owner of a chain adds the KSW products
// in super-block order.
//
// One launch can cover up to three matrices that read the same activations (gate and up; q, k and v; the
// DeltaNet qkv and z projections): the work-groups are laid out segment after segment, each segment with its own
// weights, output and K-quant type (one of the kernel's two types), so the staging and the launch are shared.
constexpr int KQ_XS = 272;
constexpr int KQ_MAXSEG = 5; // up to three K-quant segments plus two F32 ones

struct KqSeg {
    const uint8_t *qa, *qb, *sc, *dm;
    float *y;
    const float *resid;
    int rows, type, wg_end; // wg_end: one past this segment's last work-group
    int nwg;                // this segment's work-groups
};
struct KqGroup {
    KqSeg seg[KQ_MAXSEG];
    int nseg, nb;
    const float *xf; // the f32 activation rows (F32 segments)
    int chk; // super-blocks per activation staging chunk: nb, or a multiple of KSW * PF
    const int8_t *xqs;
    const float *xd;
    const int16_t *xbs, *xq8s;
    size_t xcol;
    int32_t *isl, *ism; // integer check (IS instances only): lane sums [col][row][sb][8], min products [..][4]
};

// Activations of every super-block to LDS: codes [sb][column][KQ_XS], scales [sb][NCP], activation-sum pairs
// [sb][NP][NCP]: the 4 sub-block-sum pairs (Q4_K/Q5_K segments, HAS45) and then the 8 group-sum pairs (Q6_K
// segments, HAS6).
// Activations of super-blocks s0 .. s0 + ns - 1 to LDS slots 0 .. ns - 1: codes [slot][column][KQ_XS], scales
// [slot][NCP], activation-sum pairs [slot][NP][NCP] (the 4 sub-block-sum pairs for Q4_K/Q5_K segments, HAS45, then
// the 8 group-sum pairs for Q6_K segments, HAS6). 16 threads per (column, super-block) record of 256 codes, two
// records per thread group in flight (few registers: the weight ring stays resident).
template <int NC, bool HAS45, bool HAS6, int B = 2>
__device__ __forceinline__ void kq_stage(const KqGroup &G, int8_t *sxq, float *sxd, uint32_t *sxm, int s0, int ns) {
    constexpr int NCP = (NC + 3) / 4 * 4;
    constexpr int NP = (HAS45 ? 4 : 0) + (HAS6 ? 8 : 0), P6 = HAS45 ? 4 : 0;
    const int nb = G.nb;
    const uint32_t o = threadIdx.x & 15u, g = threadIdx.x >> 4, nrec = (uint32_t)(ns * NC);
    // B records per thread in flight: all B loads are issued before the first LDS write (past the end a thread
    // reloads and rewrites the last record, so every load is issued and the wait counts stay exact)
    for (uint32_t r0 = 0; r0 < nrec; r0 += 16u * B) { // uniform
        uint4 v[B];
#pragma unroll
        for (int i = 0; i < B; i++) {
            // record r = (super-block r / NC, column r % NC): NC is a constant, so no division by a runtime value
            const uint32_t rc = min(r0 + g + 16u * i, nrec - 1u), sb = rc / NC, c = rc - sb * NC;
            v[i] = *reinterpret_cast<const uint4 *>(G.xqs + (c * (uint32_t)G.xcol + (s0 + sb) * 256u + o * 16u));
        }
#pragma unroll
        for (int i = 0; i < B; i++) {
            const uint32_t rc = min(r0 + g + 16u * i, nrec - 1u), sb = rc / NC, c = rc - sb * NC;
            *reinterpret_cast<uint4 *>(sxq + ((sb * NC + c) * KQ_XS + o * 16u)) = v[i];
        }
    }
    for (int e = (int)threadIdx.x; e < nrec; e += 256) {
        const int sb = e / NC, c = e - sb * NC;
        const size_t m = (size_t)c * nb + s0 + sb;
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

// kq_stage split in two for the first chunk: the loads into registers (every load issued, clamped into the
// activations, so the compiler's wait counts stay exact), then, after the first weight loads are issued, the LDS
// writes. Waiting for a record then waits only for what was issued before it. Five records per 16-thread group
// (80 records: 4 columns of K = 5120), held in named registers.
template <bool HAS45, bool HAS6>
struct KqStageRegs {
    uint4 r0, r1, r2, r3, r4;
    float d;
    uint4 q8, b0, b1;
};
constexpr int KQ_STAGE_REGS = 5 * 16; // records the register staging holds

template <int NC>
__device__ __forceinline__ uint4 kq_rec_load(const KqGroup &G, int i, int nrec) {
    // unsigned 32-bit index math (the activations are far below 4 GiB): a constant divisor and one offset register
    const uint32_t rc = min((threadIdx.x >> 4) + 16u * (uint32_t)i, (uint32_t)nrec - 1u);
    const uint32_t sb = rc / NC, c = rc - sb * NC;
    return *reinterpret_cast<const uint4 *>(G.xqs + (c * (uint32_t)G.xcol + sb * 256u + (threadIdx.x & 15u) * 16u));
}
template <int NC>
__device__ __forceinline__ void kq_rec_store(int8_t *sxq, const uint4 v, int i, int nrec) {
    // past the end a thread rewrites the last record with the bytes it loaded from there: no branches
    const uint32_t rc = min((threadIdx.x >> 4) + 16u * (uint32_t)i, (uint32_t)nrec - 1u);
    const uint32_t sb = rc / NC, c = rc - sb * NC;
    *reinterpret_cast<uint4 *>(sxq + ((sb * NC + c) * KQ_XS + (threadIdx.x & 15u) * 16u)) = v;
}
template <int NC, bool HAS45, bool HAS6>
__device__ __forceinline__ void kq_stage_load(const KqGroup &G, KqStageRegs<HAS45, HAS6> &R, int ns) {
    const int nb = G.nb, nrec = ns * NC;
    R.r0 = kq_rec_load<NC>(G, 0, nrec);
    R.r1 = kq_rec_load<NC>(G, 1, nrec);
    R.r2 = kq_rec_load<NC>(G, 2, nrec);
    R.r3 = kq_rec_load<NC>(G, 3, nrec);
    R.r4 = kq_rec_load<NC>(G, 4, nrec);
    const uint32_t e = min(threadIdx.x, (uint32_t)nrec - 1u), sb = e / NC, c = e - sb * NC;
    const uint32_t m = c * (uint32_t)nb + sb;
    R.d = G.xd[m];
    if constexpr (HAS45) R.q8 = *reinterpret_cast<const uint4 *>(G.xq8s + m * 8);
    if constexpr (HAS6) {
        R.b0 = reinterpret_cast<const uint4 *>(G.xbs + m * 16)[0];
        R.b1 = reinterpret_cast<const uint4 *>(G.xbs + m * 16)[1];
    }
}
template <int NC, bool HAS45, bool HAS6>
__device__ __forceinline__ void kq_stage_store(const KqStageRegs<HAS45, HAS6> &R, int8_t *sxq, float *sxd,
                                               uint32_t *sxm, int ns) {
    constexpr int NCP = (NC + 3) / 4 * 4;
    constexpr int NP = (HAS45 ? 4 : 0) + (HAS6 ? 8 : 0), P6 = HAS45 ? 4 : 0;
    const int nrec = ns * NC;
    kq_rec_store<NC>(sxq, R.r0, 0, nrec);
    kq_rec_store<NC>(sxq, R.r1, 1, nrec);
    kq_rec_store<NC>(sxq, R.r2, 2, nrec);
    kq_rec_store<NC>(sxq, R.r3, 3, nrec);
    kq_rec_store<NC>(sxq, R.r4, 4, nrec);
    const uint32_t e = min(threadIdx.x, (uint32_t)nrec - 1u), sb = e / NC, c = e - sb * NC;
    sxd[sb * NCP + c] = R.d;
    if constexpr (HAS45) {
        const uint32_t pv[4] = {R.q8.x, R.q8.y, R.q8.z, R.q8.w};
#pragma unroll
        for (int q = 0; q < 4; q++) sxm[(sb * NP + q) * NCP + c] = pv[q];
    }
    if constexpr (HAS6) {
        const uint32_t pv[8] = {R.b0.x, R.b0.y, R.b0.z, R.b0.w, R.b1.x, R.b1.y, R.b1.z, R.b1.w};
#pragma unroll
        for (int q = 0; q < 8; q++) sxm[(sb * NP + P6 + q) * NCP + c] = pv[q];
    }
}

// The exchange slot of one wave: KSW blocks (one per K slice) of NCH chains x NI chain owners, the block stride
// padded to NI modulo 64 floats so both the writes (by slice) and the owners' reads hit distinct banks.
// With XP (chains handed over by register transposes, xpose4) the slot holds only the final chains [chain][owner].
template <int NCH, int KSW, bool XP = false>
struct KqXch {
    static constexpr int NI = 64 / KSW;
    static constexpr int S = NCH * NI + (((NI - NCH * NI) % 64) + 64) % 64;
    static constexpr int FLOATS = XP ? NCH * NI : (KSW > 1 ? KSW * S : 1);
};
// the chains of a kernel instance go through register transposes: four K slices (the chains in groups of four, the
// last group padded with zeros)
template <int NC, int KSW>
constexpr bool kq_xp() { return KSW == 4; }

template <int NC>
constexpr int kq_nch_max() { return 3 * NC; }

// One wave's share of one segment: tiles of RW = 16 / KSW rows, the wave's tiles being gw, gw + nw, ... (gw the
// wave's index within the segment, nw the segment's waves). The rounds of all its tiles form one stream, so the
// weight ring runs on across tile boundaries. Per round: the products of the K slice, handed to the chain owners
// through the wave's LDS slot; per tile: the lane reduction ((l0+l4)+(l2+l6))+((l1+l5)+(l3+l7)) [+ (m0+m2)+(m1+m3)]
// (kdot.rs:1-18) and the store. With chunked staging (G.chk < nb) every wave runs exactly one tile (idle ones on
// clamped rows), because all waves of the work-group meet at the chunk barriers.
template <int TYPE, int NC, int KSW, int PF, bool HAS45, bool HAS6, bool IS, bool FULL>
__device__ __forceinline__ void kq_wave_run(const KqGroup &G, const KqSeg &sg, int wg, int8_t *sxq, float *sxd,
                                            uint32_t *sxm, float *xw) {
    static_assert(KSW == 2 || KSW == 4, "K slices per wave");
    constexpr int RW = 16 / KSW;                        // rows per tile
    constexpr int NCP = (NC + 3) / 4 * 4;
    constexpr bool Q6 = TYPE == AQ_TYPE_Q6_K;
    constexpr int NP = (HAS45 ? 4 : 0) + (HAS6 ? 8 : 0), POFF = Q6 && HAS45 ? 4 : 0;
    constexpr int NCH = (Q6 ? 2 : 3) * NC;              // f32 chains of one (row, lane pair): j, j+4, min j
    constexpr int NO = (NCH + KSW - 1) / KSW;           // chains this thread keeps
    using X = KqXch<3 * NC, KSW, kq_xp<NC, KSW>()>;     // slot sized for the largest NCH of the kernel
    constexpr int NI = X::NI;
    MfArgs a{};
    a.qa = sg.qa;
    a.qb = sg.qb;
    a.sc = sg.sc;
    a.dm = sg.dm;
    a.rows = sg.rows;
    a.nb = G.nb;
    const int nb = G.nb;
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); // uniform: the tile bookkeeping is scalar
    const int b = lane >> 2, r = lane & 3, j = b & 3, q = b >> 2;
    const int rg = q / KSW, ks = q % KSW;
    const int idx = (rg * 4 + j) * 4 + r; // chain owner index within the wave (0..NI-1)
    const int chk = G.chk;
    const int ntile = (a.rows + RW - 1) / RW;
    const int gw = wg * 4 + wid, nw = sg.nwg * 4;
    int mt = gw < ntile ? (ntile - 1 - gw) / nw + 1 : 0; // tiles of this wave
    if (chk < nb) mt = 1;                                 // chunked: one tile per wave (idle waves included)
    const int nr = (nb + KSW - 1) / KSW;                  // rounds per tile
    const int nit = mt * nr;
    // this thread's weight row in tile k of the wave (clamped into the matrix), and its row group's first tile
    auto tile_row = [&](int k) {
        const int rw0 = (gw + k * nw) * RW;
        const int rr_ = rw0 + rg * 4 + r;
        return rr_ < a.rows ? rr_ : a.rows - 1;
    };
    // the prefetch cursor: tile pk (clamped to the wave's last tile), round prd; ptile = this thread's row group's
    // first tile plus its K slice, so a round's tile is ptile + prd * KSW (clamped to the row's last super-block)
    int pk = 0, prd = 0;
    uint32_t ptile = (uint32_t)(tile_row(0) >> 2) * (uint32_t)nb + (uint32_t)ks, plast = ptile - ks + nb - 1;
    int prr = tile_row(0) & 3;
    auto issue = [&](WRegs<TYPE> &wv) {
        const uint32_t tl = ptile + (uint32_t)(prd * KSW);
        load_w<TYPE>(wv, a, tl < plast ? tl : plast, prr, j);
        if (++prd == nr) {
            prd = 0;
            if (pk + 1 < mt) {
                pk++;
                const int row = tile_row(pk);
                ptile = (uint32_t)(row >> 2) * (uint32_t)nb + (uint32_t)ks;
                plast = ptile - ks + nb - 1;
                prr = row & 3;
            }
        }
    };
    WRegs<TYPE> wr[PF];

    // the first chunk's activations: loaded into registers ahead of the first PF rounds of weights when they fit
    // (then writing them to LDS waits only for them), else staged after those weights are issued
    const int ns0 = chk < nb ? chk : nb;
    if (ns0 * NC <= KQ_STAGE_REGS) { // uniform
        KqStageRegs<HAS45, HAS6> R;
        kq_stage_load<NC>(G, R, ns0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < PF; p++) issue(wr[p]);
        __builtin_amdgcn_sched_barrier(0);
        kq_stage_store<NC>(R, sxq, sxd, sxm, ns0);
    } else {
#pragma unroll
        for (int p = 0; p < PF; p++) issue(wr[p]);
        kq_stage<NC, HAS45, HAS6>(G, sxq, sxd, sxm, 0, ns0);
    }
    __syncthreads();
    if (nit == 0) return; // no barrier follows (with chunks every wave has a tile)
    int s0 = 0; // first super-block of the staged chunk

    float acc[NO];
#pragma unroll
    for (int i = 0; i < NO; i++) acc[i] = 0.0f;
    int ck = 0, crd = 0; // the compute cursor: tile, round

    // a finished tile: every owner's final chains to the slot [chain][owner], then one lane per (row, column)
    auto finish_tile = [&]() {
#pragma unroll
        for (int m = 0; m < NO; m++) {
            const int k = ks + KSW * m;
            if (k < NCH) xw[k * NI + idx] = acc[m];
            acc[m] = 0.0f;
        }
        __asm__ volatile("" ::: "memory");
        if (lane < RW * NC) {
            const int col = lane / RW, rw = lane % RW;
            const int orow = (gw + ck * nw) * RW + rw;
            const int base = (rw >> 2) * 16 + (rw & 3); // idx of lane pair 0 of this row
            float a0[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) a0[jj] = xw[col * NI + base + 4 * jj] + xw[(NC + col) * NI + base + 4 * jj];
            float v = (a0[0] + a0[2]) + (a0[1] + a0[3]);
            if constexpr (!Q6) {
                const float *m = xw + (2 * NC + col) * NI + base;
                v = v + ((m[0] + m[8]) + (m[4] + m[12]));
            }
            if (orow < a.rows) {
                const size_t o = (size_t)col * a.rows + orow;
                sg.y[o] = sg.resid ? sg.resid[o] + v : v;
            }
        }
        __asm__ volatile("" ::: "memory");
    };

    // FULL: nb is a multiple of KSW, so every round's K slices are all live (a kernel of its own: the partial
    // rounds' guards, a select per chain and slice, stay out of its loop)
    auto round_body = [&](WRegs<TYPE> &wv, const bool prefetch) {
        const int sb = crd * KSW + ks;
        const int sbc = FULL || sb < nb ? sb : nb - 1;
        float pr[3][NC];
#pragma unroll
        for (int c = 0; c < NC; c++) pr[2][c] = 0.0f;
        const int ls = sbc - s0; // LDS slot
        const int8_t *xq = sxq + (size_t)ls * NC * KQ_XS;
        const float *xd = sxd + ls * NCP;
        const uint32_t *xm = sxm + (ls * NP + POFF) * NCP;
        int ip[3][IS ? NC : 1];
        if constexpr (Q6)
            sb_products<TYPE, NC, KQ_XS, IS>(wv, xq, xd, xm, NCP, j, r, pr[0], pr[1], pr[2], ip[0], ip[1], ip[2]);
        else
            sb_products_split<TYPE, NC, KQ_XS, IS>(wv, xq, xd, xm, NCP, j, r, pr[0], pr[1], pr[2], ip[0], ip[1],
                                                   ip[2]);
        if constexpr (IS) { // the exact integers of this (row, super-block), lanes j and j+4, min lane j
            const int orow = (gw + ck * nw) * RW + rg * 4 + r;
            if (sb < nb && orow < a.rows) {
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    const size_t o = ((size_t)c * a.rows + orow) * nb + sb;
                    G.isl[o * 8 + j] = ip[0][c];
                    G.isl[o * 8 + j + 4] = ip[1][c];
                    G.ism[o * 4 + j] = ip[2][c];
                }
            }
        }
        // every product is final here (the empty asm pins its computation above the refill), so no use of the
        // consumed weight registers sinks below it
#pragma unroll
        for (int k = 0; k < NCH; k++) __asm__ volatile("" : "+v"(pr[k / NC][k % NC]));
        if (prefetch) {
            // the refill goes into the registers just consumed, so the ring keeps its registers across the loop's
            // back edge (no copies, no drain of the loads in flight)
            __builtin_amdgcn_sched_barrier(0);
            issue(wv);
            __builtin_amdgcn_sched_barrier(0);
        }
        // super-blocks in this round (uniform)
        const int live = FULL ? KSW : nb - crd * KSW < KSW ? nb - crd * KSW : KSW;
        if constexpr (KSW == 4) {
            // chains in groups of four by register transposes (the last group padded with zeros): the owner of
            // chain 4m + ks (K slice ks) then holds its four products in super-block order
#pragma unroll
            for (int m = 0; m < (NCH + 3) / 4; m++) {
                float q[4];
#pragma unroll
                for (int u = 0; u < 4; u++) q[u] = 4 * m + u < NCH ? pr[(4 * m + u) / NC][(4 * m + u) % NC] : 0.0f;
                xpose4(q[0], q[1], q[2], q[3]);
                acc[m] += q[0];
                if (live > 1) acc[m] += q[1];
                if (live > 2) acc[m] += q[2];
                if (live > 3) acc[m] += q[3];
            }
        } else {
#pragma unroll
        for (int k = 0; k < NCH; k++) xw[ks * X::S + k * NI + idx] = pr[k / NC][k % NC];
        __asm__ volatile("" ::: "memory");
        if (live == KSW) { // all K slices live: the owners' reads issue together
#pragma unroll
            for (int m = 0; m < NO; m++) {
                const int k = ks + KSW * m;
                if (k < NCH) {
#pragma unroll
                    for (int k2 = 0; k2 < KSW; k2++) acc[m] += xw[k2 * X::S + k * NI + idx];
                }
            }
        } else {
#pragma unroll
            for (int m = 0; m < NO; m++) {
                const int k = ks + KSW * m;
                if (k < NCH) {
#pragma unroll
                    for (int k2 = 0; k2 < KSW; k2++)
                        if (k2 < live) acc[m] += xw[k2 * X::S + k * NI + idx];
                }
            }
        }
        __asm__ volatile("" ::: "memory");
        }
        if (++crd == nr) { // uniform across the wave
            finish_tile();
            crd = 0;
            ck++;
        }
    };
    // the next staging chunk when round crd starts past the staged one (chunks hold whole groups of PF rounds;
    // chunked launches run one tile per wave, so the round counter is the item counter)
    auto next_chunk = [&]() {
        if (crd * KSW >= s0 + chk) { // uniform across the work-group
            __syncthreads();
            s0 += chk;
            kq_stage<NC, HAS45, HAS6>(G, sxq, sxd, sxm, s0, nb - s0 < chk ? nb - s0 : chk);
            __syncthreads();
        }
    };
    const int nfull = nit / PF * PF;
    for (int i = 0; i < nfull; i += PF) {
        next_chunk();
#pragma unroll
        for (int p = 0; p < PF; p++) round_body(wr[p], true);
    }
    if (nfull < nit) next_chunk();
#pragma unroll
    for (int p = 0; p < PF; p++)
        if (nfull + p < nit) round_body(wr[p], false);
}

// An F32 segment (the DeltaNet ssm_alpha / ssm_beta rows, dot.rs:180-200 via matvec.rs:270-279): one row per
// work-group, so it is done long before the K-quant work-groups beside it. Thread t takes 32-element blocks t,
// t + 256, ...: each block's partial is a left-to-right sum from 0 (product, then add), two columns at a time,
// written to LDS; after the work-group's barrier lane c chains column c's partials block by block, and the
// reference's `acc + part` with the absent tail adds 0.0f when n is a multiple of 32. `part` holds NC x ceil(n / 32)
// floats.
template <int NC>
__device__ __forceinline__ void kq_f32_run(const KqGroup &G, const KqSeg &sg, int wg, float *part) {
    const int row = wg;
    if (row >= sg.rows) return; // uniform: no barrier is met
    const int n = (int)G.xcol, nblk = (n + 31) / 32;
    const float *w = reinterpret_cast<const float *>(sg.qa) + (size_t)row * n;
    for (int b = (int)threadIdx.x; b < nblk; b += (int)blockDim.x) {
        const int e0 = b * 32, ne = n - e0 < 32 ? n - e0 : 32;
        if (ne == 32) {
            float wv[32];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const float4 f = *reinterpret_cast<const float4 *>(w + e0 + 4 * u);
                wv[4 * u] = f.x, wv[4 * u + 1] = f.y, wv[4 * u + 2] = f.z, wv[4 * u + 3] = f.w;
            }
            // two columns' sums interleaved (independent chains, each still left to right); one pair at a time
            // keeps the registers below the K-quant path's
#pragma unroll 1
            for (int c0 = 0; c0 < NC; c0 += 2) {
                constexpr int G2 = NC < 2 ? NC : 2;
                float xv[G2][32];
#pragma unroll
                for (int g = 0; g < G2; g++) {
                    const float *xr = G.xf + (size_t)(c0 + g < NC ? c0 + g : NC - 1) * n + e0;
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        const float4 f = *reinterpret_cast<const float4 *>(xr + 4 * u);
                        xv[g][4 * u] = f.x, xv[g][4 * u + 1] = f.y, xv[g][4 * u + 2] = f.z, xv[g][4 * u + 3] = f.w;
                    }
                }
                float pt[G2];
#pragma unroll
                for (int g = 0; g < G2; g++) pt[g] = 0.0f;
#pragma unroll
                for (int e = 0; e < 32; e++)
#pragma unroll
                    for (int g = 0; g < G2; g++) pt[g] += wv[e] * xv[g][e];
#pragma unroll
                for (int g = 0; g < G2; g++)
                    if (c0 + g < NC) part[(c0 + g) * nblk + b] = pt[g];
            }
        } else {
            for (int c = 0; c < NC; c++) {
                const float *xr = G.xf + (size_t)c * n + e0;
                float pt = 0.0f;
                for (int e = 0; e < ne; e++) pt += w[e0 + e] * xr[e];
                part[c * nblk + b] = pt;
            }
        }
    }
    __syncthreads();
    if (threadIdx.x < NC) {
        const float *pc = part + threadIdx.x * nblk;
        float acc = 0.0f;
        int b = 0;
        for (; b + 16 <= nblk; b += 16) { // 16 reads in flight, the sum still in block order
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = pc[b + u];
#pragma unroll
            for (int u = 0; u < 16; u++) acc += v[u];
        }
        for (; b < nblk; b++) acc += pc[b];
        if (n % 32 == 0) acc = acc + 0.0f;
        const size_t o = (size_t)threadIdx.x * sg.rows + row;
        sg.y[o] = sg.resid ? sg.resid[o] + acc : acc;
    }
}

// Up to four columns (four K slices, no Q5_K) the kernel fits 128 VGPRs without spilling, i.e. four waves per SIMD
// (16 per CU, every wave slot of a CU with four work-groups); the bound keeps the compiler there (Q4_K at N = 4: 134
// VGPRs otherwise, three waves per SIMD, and a quarter of a 4352-wave launch waiting for slots).
template <int T0, int T1, int NC, int KSW, int PF>
constexpr int kq_waves_per_eu() {
    return NC <= 4 && KSW == 4 && T0 != AQ_TYPE_Q5_K && T1 != AQ_TYPE_Q5_K ? 4 : 1;
}
template <int T0, int T1, int NC, int KSW, int PF, bool IS, bool FULL>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kq_waves_per_eu<T0, T1, NC, KSW, PF>())))
kq_wave_kernel(KqGroup G) {
    constexpr bool HAS6 = T0 == AQ_TYPE_Q6_K || T1 == AQ_TYPE_Q6_K;
    constexpr bool HAS45 = T0 != AQ_TYPE_Q6_K || T1 != AQ_TYPE_Q6_K;
    constexpr int NCP = (NC + 3) / 4 * 4;
    using X = KqXch<3 * NC, KSW, kq_xp<NC, KSW>()>;
    extern __shared__ __align__(16) uint8_t kq_lds[];
    __shared__ float xch[4 * X::FLOATS];
    int si = 0; // this work-group's segment (uniform)
    while (si + 1 < G.nseg && (int)blockIdx.x >= G.seg[si].wg_end) si++;
    const KqSeg &sg = G.seg[si];
    const int wg = (int)blockIdx.x - (si ? G.seg[si - 1].wg_end : 0);
    if (sg.type == AQ_TYPE_F32) { // uniform: F32 work-groups stage nothing and meet only their own barrier
        kq_f32_run<NC>(G, sg, wg, reinterpret_cast<float *>(kq_lds));
        return;
    }
    const int ns = G.chk < G.nb ? G.chk : G.nb; // super-blocks staged at a time
    int8_t *sxq = reinterpret_cast<int8_t *>(kq_lds);
    float *sxd = reinterpret_cast<float *>(kq_lds + (size_t)ns * NC * KQ_XS);
    uint32_t *sxm = reinterpret_cast<uint32_t *>(sxd + (size_t)ns * NCP);
    float *xw = xch + (threadIdx.x >> 6) * X::FLOATS;
    if (T0 == T1 || sg.type == T0)
        kq_wave_run<T0, NC, KSW, PF, HAS45, HAS6, IS, FULL>(G, sg, wg, sxq, sxd, sxm, xw);
    else
        kq_wave_run<T1, NC, KSW, PF, HAS45, HAS6, IS, FULL>(G, sg, wg, sxq, sxd, sxm, xw);
}

// ------------------------------------------------------------------------------------ the lane-half kernel
// A matrix of few rows (the 5120-row down projections: 1280 tiles of 4 rows) gives the wave-split kernel about one
// wave per SIMD, which then waits on its own latencies for most of the launch. Here a pair of waves of one
// work-group shares each tile: wave h of the pair computes reference lane j + 4h (j = 0..3, lane pair j's thread
// block) of every super-block, and the h = 1 wave also the Q4_K/Q5_K min lanes. The 8 lane chains are independent
// until the final reduction (kdot.rs:1-18), so the two waves need no hand-off while they stream K; once at the end
// they meet (a work-group barrier) and the h = 0 wave forms ((l0+l4)+(l2+l6))+((l1+l5)+(l3+l7)) [+ (m0+m2)+(m1+m3)]
// from both waves' chains. Each wave loads and unpacks only its lane's codes (half the bytes of a tile): a launch
// has twice the waves, each with about half the work per round.

// This wave's half of one super-block's weight bytes (load_w): the codes of lane j + 4h, the row's scale record, and
// for Q5_K / Q6_K the high bits of that lane.
template <int TYPE>
__device__ __forceinline__ void load_w_half(WRegs<TYPE> &w, const MfArgs &a, uint32_t tile, int r, int j, int h) {
    const uint32_t jr = (uint32_t)(j * 4 + r), hh = (uint32_t)h;
    w.qa0 = ld_nt4(a.qa + (tile * 512u + jr * 16u + hh * 256u));
    w.sc = ld_nt4(a.sc + (tile * 64u + (uint32_t)r * 16u));
    if constexpr (TYPE == AQ_TYPE_Q5_K) {
        w.qb.x = ld_nt1(a.qb + (tile * 128u + jr * 8u + hh * 4u));
    } else if constexpr (TYPE == AQ_TYPE_Q6_K) {
        const uint2 q = ld_nt2(a.qb + (tile * 256u + jr * 16u + hh * 8u));
        w.qb.x = q.x;
        w.qb.y = q.y;
        w.d6 = ld_nth(a.dm + (tile * 8u + (uint32_t)r * 2u));
    }
}

// One super-block's products for one thread of a lane-half wave: pr = the lane chain's product (dx*dw)*float(sum)
// of lane l = j + 4h, per column; with `mins` (uniform) also pm = the min lane j's product. The integers and the
// f32 operations are those sb_products_split (Q4_K/Q5_K) and sb_products (Q6_K) compute for the same lanes
// (kdot.rs:37-140). With IS the integers are returned too (is: lane l's sum, ism: the min product).
template <int TYPE, int NC, int XS = 256, bool IS = false>
__device__ __forceinline__ void sb_half_products(const WRegs<TYPE> &wv, const int8_t *xq, const float *xd,
                                                 const uint32_t *xm, int ncp, int j, int r, int h, bool mins,
                                                 float *pr, float *pm, int *is = nullptr, int *ism = nullptr) {
    constexpr int NCG = (NC + 3) / 4;
    const uint32_t w[4] = {wv.qa0.x, wv.qa0.y, wv.qa0.z, wv.qa0.w}; // lane l's codes
    const int xo = j * 64 + h * 32;                                   // lane l's 32 activation codes in a record
    if constexpr (TYPE == AQ_TYPE_Q6_K) {
        const uint32_t qh[2] = {wv.qb.x, wv.qb.y};
        const uint32_t sw[4] = {wv.sc.x, wv.sc.y, wv.sc.z, wv.sc.w};
        uint32_t code[8];
        int scl[8];
#pragma unroll
        for (int hh = 0; hh < 2; hh++)
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int s = hh * 4 + kk;
                const int li = kk < 2 ? hh * 2 + kk : hh * 2 + kk - 2, sh = kk < 2 ? 0 : 4;
                code[s] = ((w[li] >> sh) & 0x0F0F0F0Fu) | (((qh[hh] >> (2 * kk)) & 0x03030303u) << 4);
                // group hh*8 + 2kk + h: word hh*2 + kk/2, byte 2(kk&1) + h
                scl[s] = (int)(int8_t)(sw[hh * 2 + (kk >> 1)] >> (8 * (2 * (kk & 1) + h)));
            }
        // the -32 fold scales of lane l: groups 2l, 2l+1 = bytes 2(j&1), 2(j&1)+1 of word 2h + j/2
        const uint32_t ow = h ? ((j >> 1) ? sw[3] : sw[2]) : ((j >> 1) ? sw[1] : sw[0]);
        const int osa = sbyte(ow, 2 * (j & 1)), osb = sbyte(ow, 2 * (j & 1) + 1);
        const uint32_t osp = ((uint32_t)osa & 0xFFFFu) | ((uint32_t)osb << 16);
        const float dw = h2f(wv.d6);
#pragma unroll
        for (int cg = 0; cg < NCG; cg++) {
            const int cA = cg * 4 + r < NC ? cg * 4 + r : 0;
            const uint4 *xp = reinterpret_cast<const uint4 *>(xq + cA * XS + xo);
            const uint4 va = xp[0], vb = xp[1];
            const uint32_t x[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
            int s0[4] = {0, 0, 0, 0};
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const v4i d = mfma(x[s], code[s]);
#pragma unroll
                for (int c = 0; c < 4; c++)
                    if (cg * 4 + c < NC) s0[c] += __mul24(scl[s], d[c]);
            }
            const float4 dx4 = *reinterpret_cast<const float4 *>(xd + cg * 4);
            const float dxs[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
            const uint4 m = *reinterpret_cast<const uint4 *>(xm + (j + 4 * h) * ncp + cg * 4);
            const uint32_t mw[4] = {m.x, m.y, m.z, m.w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int col = cg * 4 + c;
                if (col < NC) {
                    const float dd = dxs[c] * dw;
                    const int i0 = s0[c] - 32 * sdot2(osp, mw[c]);
                    pr[col] = dd * (float)i0;
                    if constexpr (IS) {
                        is[col] = i0;
                        ism[col] = 0;
                    }
                }
            }
        }
    } else {
        constexpr int DB = TYPE == AQ_TYPE_Q4_K ? 3 : 2, ND = TYPE == AQ_TYPE_Q4_K ? 2 : 3;
        uint4 xh[2];
        float4 dxh;
        uint4 mh;
        if constexpr (NCG == 1) { // the activation reads first: their LDS latency passes under the unpacking
            const uint4 *xp = reinterpret_cast<const uint4 *>(xq + (r < NC ? r : 0) * XS + xo);
            xh[0] = xp[0];
            xh[1] = xp[1];
            dxh = *reinterpret_cast<const float4 *>(xd);
            mh = *reinterpret_cast<const uint4 *>(xm + j * ncp);
            __builtin_amdgcn_sched_barrier(0);
        }
        const uint32_t q0 = wv.sc.y, q1 = wv.sc.z, q2 = wv.sc.w;
        const uint32_t sc_lo = q0 & 0x3F3F3F3Fu, mn_lo = q1 & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (q2 & 0x0F0F0F0Fu) | ((q0 >> 2) & 0x30303030u);
        const uint32_t mn_hi = ((q2 >> 4) & 0x0F0F0F0Fu) | ((q1 >> 2) & 0x30303030u);
        const uint32_t mnw = j < 2 ? mn_lo : mn_hi;
        const uint32_t mnp = __builtin_amdgcn_perm(0u, mnw, (uint32_t)(2 * (j & 1)) | 0x0C00u |
                                                              ((uint32_t)(2 * (j & 1) + 1) << 16) | 0x0C000000u);
        uint32_t dig[ND][4];
        kq_digits<DB, ND>(sc_lo, sc_hi, dig);
        uint32_t code[8];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            code[2 * q] = w[q] & 0x0F0F0F0Fu;
            code[2 * q + 1] = (w[q] >> 4) & 0x0F0F0F0Fu;
        }
        if constexpr (TYPE == AQ_TYPE_Q5_K) {
#pragma unroll
            for (int s = 0; s < 8; s++) code[s] |= ((wv.qb.x >> s) & 0x01010101u) << 4;
        }
        const float dw = h2f(wv.sc.x & 0xFFFF), dminw = h2f(wv.sc.x >> 16);
#pragma unroll
        for (int cg = 0; cg < NCG; cg++) {
            const uint4 *xp = reinterpret_cast<const uint4 *>(xq + (cg * 4 + r < NC ? cg * 4 + r : 0) * XS + xo);
            const uint4 va = NCG == 1 ? xh[0] : xp[0], vb = NCG == 1 ? xh[1] : xp[1];
            const uint32_t x[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
            v4i acc[ND];
#pragma unroll
            for (int i = 0; i < ND; i++) acc[i] = (v4i){0, 0, 0, 0};
#pragma unroll
            for (int s = 0; s < 8; s++) {
#pragma unroll
                for (int i = 0; i < ND; i++) {
                    const u16x2 dp = as_u16x2(dig[i][s >> 1]);
                    const u16x2 d2 = (s & 1) ? (u16x2){dp.y, dp.y} : (u16x2){dp.x, dp.x};
                    acc[i] = mfma_acc(x[s], as_u32(as_u16x2(code[s]) * d2), acc[i]);
                }
            }
            const float4 dx4 = NCG == 1 ? dxh : *reinterpret_cast<const float4 *>(xd + cg * 4);
            const float dxs[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
            const uint4 m0 = NCG == 1 ? mh : *reinterpret_cast<const uint4 *>(xm + j * ncp + cg * 4);
            const uint32_t mw0[4] = {m0.x, m0.y, m0.z, m0.w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int col = cg * 4 + c;
                if (col < NC) {
                    int s0 = acc[ND - 1][c];
#pragma unroll
                    for (int i = ND - 2; i >= 0; i--) s0 = (s0 << DB) + acc[i][c];
                    const float dd = dxs[c] * dw;
                    pr[col] = dd * (float)s0;
                    if constexpr (IS) is[col] = s0;
                }
            }
            // the min lanes only in the h = 1 wave: one uniform branch over the group's columns (the empty asm keeps
            // the compiler from computing them in both waves and selecting), then one unconditional store of each
            // result, which keeps pm in registers
            float pv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            int iv[4] = {0, 0, 0, 0};
            if (mins) {
                __asm__ volatile("");
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    if (cg * 4 + c < NC) {
                        iv[c] = sdot2z(mnp, mw0[c]);
                        pv[c] = (-dxs[c] * dminw) * (float)iv[c];
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int col = cg * 4 + c;
                if (col < NC) {
                    pm[col] = pv[c];
                    if constexpr (IS) ism[col] = iv[c];
                }
            }
        }
    }
}

// Chains of the h = 1 wave of a pair: lane j + 4 per column, and for Q4_K/Q5_K the min lane j per column (the h = 0
// wave runs the first NC).
template <int TYPE, int NC>
constexpr int kq_lh_nch() { return (TYPE == AQ_TYPE_Q6_K ? 1 : 2) * NC; }

// One wave of a lane-half pair: the pair's tile is wg * 2 + wid / 2 (4 rows; past the last one the rows are clamped
// and nothing is stored), its lane half h = wid % 2. The round structure is kq_wave_run's with KSW = 4 and one
// tile per wave: the K slices' products reach the chain owners by register transposes, in super-block order; the
// wave's LDS slot holds only the final chains.
template <int TYPE, int NC, int PF, bool HAS45, bool HAS6, bool IS, bool FULL>
__device__ __forceinline__ void kq_lh_run(const KqGroup &G, const KqSeg &sg, int wg, int8_t *sxq, float *sxd,
                                          uint32_t *sxm, float *xch) {
    constexpr int KSW = 4, NI = 16;
    constexpr int NCP = (NC + 3) / 4 * 4;
    constexpr bool Q6 = TYPE == AQ_TYPE_Q6_K;
    constexpr int NP = (HAS45 ? 4 : 0) + (HAS6 ? 8 : 0), POFF = Q6 && HAS45 ? 4 : 0;
    constexpr int NCH = kq_lh_nch<TYPE, NC>();
    constexpr int NO = (NCH + KSW - 1) / KSW;
    using X = KqXch<NCH, KSW, true>;
    MfArgs a{};
    a.qa = sg.qa;
    a.qb = sg.qb;
    a.sc = sg.sc;
    a.dm = sg.dm;
    a.rows = sg.rows;
    a.nb = G.nb;
    const int nb = G.nb;
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int h = wid & 1;
    const bool mins = !Q6 && h == 1;
    const int nch = mins ? NCH : NC; // chains of this wave (uniform)
    const int b = lane >> 2, r = lane & 3, j = b & 3, ks = b >> 2;
    const int idx = j * 4 + r; // chain owner index within the wave
    float *xw = xch + wid * X::FLOATS;
    const int chk = G.chk;
    const int tile = wg * 2 + (wid >> 1);
    const int row = tile * 4 + r < a.rows ? tile * 4 + r : a.rows - 1;
    const int nr = (nb + KSW - 1) / KSW; // rounds
    int prd = 0;
    const uint32_t ptile = (uint32_t)(row >> 2) * (uint32_t)nb + (uint32_t)ks, plast = ptile - ks + nb - 1;
    const int prr = row & 3;
    auto issue = [&](WRegs<TYPE> &wv) {
        const uint32_t tl = ptile + (uint32_t)(prd * KSW);
        load_w_half<TYPE>(wv, a, tl < plast ? tl : plast, prr, j, h);
        prd++;
    };
    WRegs<TYPE> wr[PF];
    const int ns0 = chk < nb ? chk : nb;
    if (ns0 * NC <= KQ_STAGE_REGS) { // uniform
        KqStageRegs<HAS45, HAS6> R;
        kq_stage_load<NC>(G, R, ns0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < PF; p++) issue(wr[p]);
        __builtin_amdgcn_sched_barrier(0);
        kq_stage_store<NC>(R, sxq, sxd, sxm, ns0);
    } else {
#pragma unroll
        for (int p = 0; p < PF; p++) issue(wr[p]);
        kq_stage<NC, HAS45, HAS6>(G, sxq, sxd, sxm, 0, ns0);
    }
    __syncthreads();
    int s0 = 0; // first super-block of the staged chunk
    float acc[NO];
#pragma unroll
    for (int i = 0; i < NO; i++) acc[i] = 0.0f;
    int crd = 0; // round
    auto round_body = [&](WRegs<TYPE> &wv, const bool prefetch) { // FULL as in kq_wave_run
        const int sb = crd * KSW + ks;
        const int sbc = FULL || sb < nb ? sb : nb - 1;
        float pr[2][NC];
#pragma unroll
        for (int c = 0; c < NC; c++) pr[1][c] = 0.0f;
        const int ls = sbc - s0; // LDS slot
        const int8_t *xq = sxq + (size_t)ls * NC * KQ_XS;
        const float *xd = sxd + ls * NCP;
        const uint32_t *xm = sxm + (ls * NP + POFF) * NCP;
        int ip[2][IS ? NC : 1];
        sb_half_products<TYPE, NC, KQ_XS, IS>(wv, xq, xd, xm, NCP, j, r, h, mins, pr[0], pr[1], ip[0], ip[1]);
        if constexpr (IS) { // the exact integers of this (row, super-block): lane j + 4h, and the min lane j
            const int orow = tile * 4 + r;
            if (sb < nb && orow < a.rows) {
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    const size_t o = ((size_t)c * a.rows + orow) * nb + sb;
                    G.isl[o * 8 + j + 4 * h] = ip[0][c];
                    if (!Q6 && h == 1) G.ism[o * 4 + j] = ip[1][c];
                    if (Q6 && h == 0) G.ism[o * 4 + j] = 0;
                }
            }
        }
#pragma unroll
        for (int k = 0; k < NCH; k++) __asm__ volatile("" : "+v"(pr[k / NC][k % NC]));
        if (prefetch) {
            __builtin_amdgcn_sched_barrier(0);
            issue(wv);
            __builtin_amdgcn_sched_barrier(0);
        }
        // super-blocks in this round (uniform)
        const int live = FULL ? KSW : nb - crd * KSW < KSW ? nb - crd * KSW : KSW;
        // chains in groups of four by register transposes (xpose4, the last group padded with zeros): the owner of
        // chain 4m + ks then holds its four products in super-block order
#pragma unroll
        for (int m = 0; m < (NCH + 3) / 4; m++) {
            if (4 * m < nch) { // uniform
                float q[4];
#pragma unroll
                for (int u = 0; u < 4; u++) q[u] = 4 * m + u < nch ? pr[(4 * m + u) / NC][(4 * m + u) % NC] : 0.0f;
                xpose4(q[0], q[1], q[2], q[3]);
                acc[m] += q[0];
                if (live > 1) acc[m] += q[1];
                if (live > 2) acc[m] += q[2];
                if (live > 3) acc[m] += q[3];
            }
        }
        crd++;
    };
    auto next_chunk = [&]() {
        if (crd * KSW >= s0 + chk) { // uniform across the work-group
            __syncthreads();
            s0 += chk;
            kq_stage<NC, HAS45, HAS6>(G, sxq, sxd, sxm, s0, nb - s0 < chk ? nb - s0 : chk);
            __syncthreads();
        }
    };
    const int nfull = nr / PF * PF;
    for (int i = 0; i < nfull; i += PF) {
        next_chunk();
#pragma unroll
        for (int p = 0; p < PF; p++) round_body(wr[p], true);
    }
    if (nfull < nr) next_chunk();
#pragma unroll
    for (int p = 0; p < PF; p++)
        if (nfull + p < nr) round_body(wr[p], false);
    // the final chains to the wave's slot [chain][owner]; the pair meets; the h = 0 wave reduces both halves
#pragma unroll
    for (int m = 0; m < NO; m++) {
        const int k = ks + KSW * m;
        if (k < nch) xw[k * NI + idx] = acc[m];
    }
    __syncthreads();
    if (h == 0 && lane < 4 * NC) {
        const int col = lane >> 2, rw = lane & 3;
        const float *x1 = xw + X::FLOATS; // the partner's slot (wave wid + 1)
        float a0[4];
#pragma unroll
        for (int jj = 0; jj < 4; jj++) a0[jj] = xw[col * NI + 4 * jj + rw] + x1[col * NI + 4 * jj + rw];
        float v = (a0[0] + a0[2]) + (a0[1] + a0[3]);
        if constexpr (!Q6) {
            const float *m = x1 + (NC + col) * NI + rw;
            v = v + ((m[0] + m[8]) + (m[4] + m[12]));
        }
        const int orow = tile * 4 + rw;
        if (orow < a.rows) {
            const size_t o = (size_t)col * a.rows + orow;
            sg.y[o] = sg.resid ? sg.resid[o] + v : v;
        }
    }
}

template <int T, int NC, int PF, bool IS, bool FULL>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NC <= 4 ? 4 : 1)))
kq_lh_kernel(KqGroup G) {
    constexpr bool HAS6 = T == AQ_TYPE_Q6_K, HAS45 = !HAS6;
    constexpr int NCP = (NC + 3) / 4 * 4;
    using X = KqXch<kq_lh_nch<T, NC>(), 4, true>;
    extern __shared__ __align__(16) uint8_t kq_lds[];
    __shared__ float xch[4 * X::FLOATS];
    const int ns = G.chk < G.nb ? G.chk : G.nb;
    int8_t *sxq = reinterpret_cast<int8_t *>(kq_lds);
    float *sxd = reinterpret_cast<float *>(kq_lds + (size_t)ns * NC * KQ_XS);
    uint32_t *sxm = reinterpret_cast<uint32_t *>(sxd + (size_t)ns * NCP);
    kq_lh_run<T, NC, PF, HAS45, HAS6, IS, FULL>(G, G.seg[0], (int)blockIdx.x, sxq, sxd, sxm, xch);
}

constexpr int KQ_LDS_MAX = 160 * 1024 - 512; // a CU's LDS, less a margin
// Prefetch depth in rounds. Deeper rings cost a wave per SIMD, and measured slower even where every tile has a
// resident wave (the down projections: 4 rounds 3-9% slower than 2).
constexpr int KQ_PF = 2;

template <int NC, int KSW>
constexpr size_t kq_xch_bytes() { return (size_t)4 * KqXch<3 * NC, KSW, kq_xp<NC, KSW>()>::FLOATS * 4; }

// Host mirror of the kernel's LDS use: the four waves' exchange slots, and the staging per super-block.
inline size_t kq_xch_bytes_rt(int nc, int ksw) {
    if (ksw == 1) return 4 * 4;
    if (ksw == 4) return (size_t)4 * 3 * nc * 16 * 4; // final chains only (register transposes)
    const int nch = 3 * nc, ni = 64 / ksw;
    const int s = nch * ni + (((ni - nch * ni) % 64) + 64) % 64;
    return (size_t)4 * ksw * s * 4;
}
inline size_t kq_sb_lds_bytes(int nc, bool has45, bool has6) {
    const int ncp = (nc + 3) / 4 * 4, np = (has45 ? 4 : 0) + (has6 ? 8 : 0);
    return (size_t)nc * KQ_XS + (size_t)ncp * 4 + (size_t)np * ncp * 4;
}

// K slices per wave: four (tiles of 4 rows, so work divides finely over the waves), two for K below 4 super-blocks
// and for the lm_head-sized matrices (at least KQ_TALL_ROWS rows: tiles of 8 rows, a long stream either way) at more
// than one column. Measured (MI355X, Q6_K 248320 x 5120, the current kernels): N = 4 199-201 us with two slices
// against 202-207 with four; N = 1 176.3 against 172.9 us (four passes of 400 launches each, alternated), so the
// matvec takes four. Every shorter matrix is slower with two (Q4_K 10240 x 5120 N = 4 13.3 vs 10.5 us, Q6_K
// 5120 x 17408 34.1 vs 28.1 us, an earlier build).
constexpr int KQ_TALL_ROWS = 131072;
inline int kq_pick_ksw(int nb, int rows, size_t ncols) { return nb < 4 || (rows >= KQ_TALL_ROWS && ncols > 1) ? 2 : 4; }

// Work-groups of `fn` (256 threads, `lds` dynamic bytes) resident on the whole device at once.
inline int kq_capacity(const void *fn, size_t lds) {
    static std::mutex mu;
    static std::map<std::pair<const void *, size_t>, int> cache;
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_pair(fn, lds);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, lds) != hipSuccess)
        return 0;
    return cache[key] = per_cu * cus;
}

// Super-blocks per activation staging chunk: all of K when the work-group's LDS stays within the budget that
// leaves room for two work-groups per CU, else the largest multiple of KSW * PF that does (the waves then meet at a
// barrier between chunks). Measured on the 5120-row matrices with K = 17408 (N = 4, 1280 tiles, 320 work-groups):
// a 76 KB budget (chunks of 48 super-blocks, one re-staging) 24.6 / 28.3 us for Q4_K / Q6_K, a 52 KB one (three
// work-groups per CU, chunks of 32) 25.1 / 29.4 us.
inline int kq_pick_chunk(int nb, int nc, bool has45, bool has6, int ksw, int pf, size_t budget = (size_t)76 * 1024,
                         size_t x = 0) {
    if (x == 0) x = kq_xch_bytes_rt(nc, ksw);
    const size_t per = kq_sb_lds_bytes(nc, has45, has6);
    if (x + per * nb <= budget) return nb;
    const int unit = ksw * pf;
    const int c = (int)((budget - x) / per) / unit * unit;
    return c < unit ? unit : c;
}

// Grid. One tile per wave, work-groups past the resident ones starting as others end, when there are at most
// KQ_PERSIST_MIN tiles per resident wave, when the staging is chunked, when F32 segments are present (their
// work-groups end early and free their slots) or when there are more than KQ_DYN tiles per resident wave (the
// dispatcher then balances the long stream over CUs that run at unequal speed). Otherwise a persistent grid: the
// resident work-groups shared between the segments by weight bytes, then trimmed so that every wave of a segment
// streams the same number of tiles (no wave runs a tile more than the others while the rest of the device idles).
// Measured (MI355X, N = 4): Q4_K 17408 x 5120 alone (1.06 tiles per resident wave) 18.7 us with one tile per wave
// against 20.3 us persistent (two tiles each on half the slots); gate + up in one launch (2.1 per resident wave)
// faster persistent.
constexpr int KQ_DYN = 8;
constexpr double KQ_PERSIST_MIN = 1.5;
// The launch shape of kq_wave_kernel<T0, T1, NC, KSW, PF> for group G: staging chunk and LDS bytes, tiles and F32
// work-groups, and the work-groups resident at once (less the F32 ones).
struct KqPlan {
    int chk;
    size_t lds;
    long tiles, f32_wgs, cap;
    double bytes;
};
template <int T0, int T1, int NC, int KSW, int PF, bool IS, bool FULL>
int kq_plan(const KqGroup &G, KqPlan &P) {
    constexpr int RW = 16 / KSW; // rows per tile
    constexpr bool HAS6 = T0 == AQ_TYPE_Q6_K || T1 == AQ_TYPE_Q6_K;
    constexpr bool HAS45 = T0 != AQ_TYPE_Q6_K || T1 != AQ_TYPE_Q6_K;
    P.chk = kq_pick_chunk(G.nb, NC, HAS45, HAS6, KSW, PF);
    P.lds = kq_sb_lds_bytes(NC, HAS45, HAS6) * (size_t)(P.chk < G.nb ? P.chk : G.nb);
    constexpr size_t xch = kq_xch_bytes<NC, KSW>();
    AQ_REQUIRE(P.lds + xch <= (size_t)KQ_LDS_MAX, "kq_mfma: activation staging exceeds LDS");
    const void *fn = reinterpret_cast<const void *>(&kq_wave_kernel<T0, T1, NC, KSW, PF, IS, FULL>);
    if (P.lds > 64 * 1024) {
        static bool raised = false; // once per instantiation: allow dynamic LDS up to the CU's size
        if (!raised) {
            AQ_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(KQ_LDS_MAX - xch)));
            raised = true;
        }
    }
    P.tiles = 0;
    P.f32_wgs = 0;
    P.bytes = 0.0;
    for (int i = 0; i < G.nseg; i++) {
        const KqSeg &sg = G.seg[i];
        if (sg.type == AQ_TYPE_F32) {
            AQ_REQUIRE((size_t)NC * ((G.xcol + 31) / 32) * 4 <= P.lds, "kq_mfma: F32 partials exceed the LDS");
            P.f32_wgs += sg.rows; // one row per work-group, partials in the staging LDS
            continue;
        }
        const long t = (sg.rows + RW - 1) / RW;
        P.tiles += t;
        P.bytes += (double)t * block_bytes(sg.type);
    }
    P.cap = kq_capacity(fn, P.lds) - P.f32_wgs;
    return 0;
}

template <int T0, int T1, int NC, int KSW, int PF, bool IS, bool FULL>
int launch_wave_pf(KqGroup G, const KqPlan &P, hipStream_t stream) {
    constexpr int RW = 16 / KSW; // rows per tile
    G.chk = P.chk;
    const long cap = P.cap;
    const bool persistent = G.chk >= G.nb && P.f32_wgs == 0 && cap >= G.nseg &&
                            (double)P.tiles > KQ_PERSIST_MIN * 4 * cap && P.tiles <= KQ_DYN * 4 * cap;
    // the F32 segments' work-groups take the lowest indices: dispatched first, they are done early and free their
    // slots for the K-quant work-groups past the resident ones
    std::stable_partition(G.seg, G.seg + G.nseg, [](const KqSeg &sg) { return sg.type == AQ_TYPE_F32; });
    int wgs = 0;
    for (int i = 0; i < G.nseg; i++) {
        KqSeg &sg = G.seg[i];
        long n;
        if (sg.type == AQ_TYPE_F32) {
            n = sg.rows;
        } else {
            const long t = (sg.rows + RW - 1) / RW, need = (t + 3) / 4;
            n = need;
            if (persistent) {
                n = (long)((double)cap * ((double)t * block_bytes(sg.type)) / P.bytes);
                n = n < 1 ? 1 : (n > need ? need : n);
                const long per = (t + 4 * n - 1) / (4 * n); // tiles per wave
                n = (t + 4 * per - 1) / (4 * per);
            }
        }
        sg.nwg = (int)n;
        wgs += (int)n;
        sg.wg_end = wgs;
    }
    hipLaunchKernelGGL((kq_wave_kernel<T0, T1, NC, KSW, PF, IS, FULL>), dim3((unsigned)wgs), dim3(256), P.lds, stream,
                       G);
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "kq_wave launch");
}

// Lane-half launches (kq_lh_kernel): one K-quant matrix of at most KQ_LH_MAX_ROWS rows, N <= 4. One tile per wave
// pair, two pairs per work-group; the staging budget leaves room for three work-groups per CU, so the 5120-row
// matrices (640 work-groups) are resident in one pass.
constexpr int KQ_LH_MAX_ROWS = 8192;
constexpr size_t KQ_LH_BUDGET = (size_t)52 * 1024;
constexpr int KQ_LH_PF = 2; // weight ring depth in rounds
inline bool kq_use_lh(const KqGroup &G, size_t ncols) {
    return G.nseg == 1 && is_kquant(G.seg[0].type) && G.seg[0].rows <= KQ_LH_MAX_ROWS && G.nb >= 4 && ncols <= 8;
}
template <int T, int NC, bool IS, bool FULL>
int launch_lh_f(KqGroup G, hipStream_t stream) {
    constexpr bool HAS6 = T == AQ_TYPE_Q6_K, HAS45 = !HAS6;
    constexpr size_t xch = (size_t)4 * KqXch<kq_lh_nch<T, NC>(), 4, true>::FLOATS * 4;
    G.chk = kq_pick_chunk(G.nb, NC, HAS45, HAS6, 4, KQ_LH_PF, KQ_LH_BUDGET, xch);
    const size_t lds = kq_sb_lds_bytes(NC, HAS45, HAS6) * (size_t)(G.chk < G.nb ? G.chk : G.nb);
    AQ_REQUIRE(lds + xch <= (size_t)KQ_LDS_MAX, "kq_mfma: activation staging exceeds LDS");
    if (lds > 64 * 1024) {
        static bool raised = false; // once per instantiation: allow dynamic LDS up to the CU's size
        if (!raised) {
            AQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&kq_lh_kernel<T, NC, KQ_LH_PF, IS, FULL>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)(KQ_LDS_MAX - xch)));
            raised = true;
        }
    }
    const long tiles = (G.seg[0].rows + 3) / 4, nwg = (tiles + 1) / 2;
    G.seg[0].nwg = (int)nwg;
    G.seg[0].wg_end = (int)nwg;
    hipLaunchKernelGGL((kq_lh_kernel<T, NC, KQ_LH_PF, IS, FULL>), dim3((unsigned)nwg), dim3(256), lds, stream, G);
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "kq_lh launch");
}
// K in whole rounds (nb a multiple of 4: every K of the 27B shape) takes the kernel without partial-round guards
template <int T, int NC, bool IS = false>
int launch_lh(const KqGroup &G, hipStream_t stream) {
    return G.nb % 4 == 0 ? launch_lh_f<T, NC, IS, true>(G, stream) : launch_lh_f<T, NC, IS, false>(G, stream);
}
template <int T>
int launch_lh_t(const KqGroup &G, size_t ncols, hipStream_t stream) {
    switch (ncols) {
    case 1: return launch_lh<T, 1>(G, stream);
    case 2: return launch_lh<T, 2>(G, stream);
    case 3: return launch_lh<T, 3>(G, stream);
    case 4: return launch_lh<T, 4>(G, stream);
    case 5: return launch_lh<T, 5>(G, stream);
    case 6: return launch_lh<T, 6>(G, stream);
    case 7: return launch_lh<T, 7>(G, stream);
    case 8: return launch_lh<T, 8>(G, stream);
    default: return fail(AQ_EINVAL, "kq_lh: ncols must be 1..8");
    }
}

template <int T0, int T1, int NC, int KSW, bool IS, bool FULL>
int launch_wave_ksf(const KqGroup &G, hipStream_t stream) {
    KqPlan P;
    const int rc = kq_plan<T0, T1, NC, KSW, KQ_PF, IS, FULL>(G, P);
    if (rc) return rc;
    return launch_wave_pf<T0, T1, NC, KSW, KQ_PF, IS, FULL>(G, P, stream);
}
// K in whole rounds (nb a multiple of KSW) takes the kernel without partial-round guards
template <int T0, int T1, int NC, int KSW, bool IS = false>
int launch_wave_ks(const KqGroup &G, hipStream_t stream) {
    return G.nb % KSW == 0 ? launch_wave_ksf<T0, T1, NC, KSW, IS, true>(G, stream)
                           : launch_wave_ksf<T0, T1, NC, KSW, IS, false>(G, stream);
}

template <int T0, int T1, int NC>
int launch_wave_nc(const KqGroup &G, int rows, hipStream_t stream) {
    if (kq_pick_ksw(G.nb, rows, NC) == 2) return launch_wave_ks<T0, T1, NC, 2>(G, stream);
    return launch_wave_ks<T0, T1, NC, 4>(G, stream);
}

template <int T0, int T1>
int launch_wave_t(const KqGroup &G, int rows, size_t ncols, hipStream_t stream) {
    switch (ncols) {
    case 1: return launch_wave_nc<T0, T1, 1>(G, rows, stream);
    case 2: return launch_wave_nc<T0, T1, 2>(G, rows, stream);
    case 3: return launch_wave_nc<T0, T1, 3>(G, rows, stream);
    case 4: return launch_wave_nc<T0, T1, 4>(G, rows, stream);
    case 5: return launch_wave_nc<T0, T1, 5>(G, rows, stream);
    case 6: return launch_wave_nc<T0, T1, 6>(G, rows, stream);
    case 7: return launch_wave_nc<T0, T1, 7>(G, rows, stream);
    case 8: return launch_wave_nc<T0, T1, 8>(G, rows, stream);
    default: return fail(AQ_EINVAL, "kq_mfma: ncols must be 1..8");
    }
}

// One launch over segments [i0, i1), of types T0 and T1 (F32 segments aside).
template <int T0, int T1>
int launch_run_t(const Weight *const *ws, float *const *ys, const float *const *resids, int i0, int i1, const Act &x,
                 size_t ncols, hipStream_t stream) {
    KqGroup G{};
    G.nseg = i1 - i0;
    G.nb = (int)ws[i0]->nb;
    G.xqs = x.qs;
    G.xd = x.d;
    G.xbs = x.bs;
    G.xq8s = x.q8s;
    G.xcol = x.n;
    G.xf = x.f32;
    int rows = 0;
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
        if (w.type != AQ_TYPE_F32) rows += (int)w.rows;
    }
    if constexpr (T0 == T1) {
        if (kq_use_lh(G, ncols)) return launch_lh_t<T0>(G, ncols, stream);
    }
    return launch_wave_t<T0, T1>(G, rows, ncols, stream);
}

// The integer check: the production grid and kernel of one K-quant matrix of type T (the K slices the production
// launch would pick), with the integer outputs on; y receives the usual f32 outputs.

template <int T, int NC>
int launch_isums_nc(const Weight &w, const Act &x, float *y, int32_t *lanes, int32_t *mins, hipStream_t stream) {
    KqGroup G{};
    G.nseg = 1;
    G.nb = (int)w.nb;
    G.xqs = x.qs;
    G.xd = x.d;
    G.xbs = x.bs;
    G.xq8s = x.q8s;
    G.xcol = x.n;
    G.xf = x.f32;
    G.isl = lanes;
    G.ism = mins;
    KqSeg &sg = G.seg[0];
    sg.qa = w.qa;
    sg.qb = w.qb;
    sg.sc = w.sc;
    sg.dm = w.dm;
    sg.y = y;
    sg.resid = nullptr;
    sg.rows = (int)w.rows;
    sg.type = w.type;
    if (kq_use_lh(G, NC)) return launch_lh<T, NC, true>(G, stream);
    if (kq_pick_ksw(G.nb, sg.rows, NC) == 2) return launch_wave_ks<T, T, NC, 2, true>(G, stream);
    return launch_wave_ks<T, T, NC, 4, true>(G, stream);
}

template <int T>
int launch_isums_t(const Weight &w, const Act &x, size_t ncols, float *y, int32_t *lanes, int32_t *mins,
                   hipStream_t stream) {
    switch (ncols) {
    case 1: return launch_isums_nc<T, 1>(w, x, y, lanes, mins, stream);
    case 4: return launch_isums_nc<T, 4>(w, x, y, lanes, mins, stream);
    case 8: return launch_isums_nc<T, 8>(w, x, y, lanes, mins, stream);
    default: return fail(AQ_EINVAL, "kq isums: ncols must be 1, 4 or 8");
    }
}

} // namespace

// One launch per type pair; each is instantiated in its own source file (kq_pair_*.hip) so they build in parallel.
#define AQ_KQ_RUN_DECL(NAME)                                                                                        \
    int NAME(const Weight *const *ws, float *const *ys, const float *const *resids, int i0, int i1, const Act &x, \
             size_t ncols, hipStream_t stream);
AQ_KQ_RUN_DECL(kq_run_q4q4)
AQ_KQ_RUN_DECL(kq_run_q5q5)
AQ_KQ_RUN_DECL(kq_run_q6q6)
AQ_KQ_RUN_DECL(kq_run_q4q5)
AQ_KQ_RUN_DECL(kq_run_q4q6)
AQ_KQ_RUN_DECL(kq_run_q5q6)
#undef AQ_KQ_RUN_DECL
// The matmul of one K-quant matrix with its exact integers written out (kq_isums.hip).
int kq_isums_run(const Weight &w, const Act &x, size_t ncols, float *y, int32_t *lanes, int32_t *mins,
                 hipStream_t stream);

} // namespace aq
