// kq_gemm.hip — weight x activation products over many columns (a prompt chunk's rows: model.rs:443-461 prefill,
// where every projection is a matmul over the chunk's tokens, matvec.rs:369-393). Each output equals the single-
// column dot bit for bit: the integer lane sums are exact and each output's f32 chains advance super-block by
// super-block (block by block for Q8_0 / Q4_0) in the reference's order.
//
// K-quants x Q8_K (kdot.rs:37-140, 176-333) on v_mfma_i32_16x16x32_i8. The reference's lane l of a super-block is
// the 32 elements 32s + 4l + b (s = sub-block, b = 0..3), and its sum is sum_s sc[s] * sum_b q * x. One matrix-core
// product over K = 32 covers exactly lane l: k-group g of the operands (lanes 16g .. 16g + 15) takes sub-blocks 2g and
// 2g + 1, four elements each. Q4_K / Q5_K (v_mfma_i32_16x16x32_i8): the scale goes into the weight operand as digits
// small enough that digit * code fits an int8 (6-bit scales in two base-8 digits, codes <= 15; three base-4 digits,
// codes <= 31), the digit products chained through the accumulator (c = digit_hi product; c = c * base + next
// digit's product ...). Q6_K (v_mfma_f32_16x16x32_f16): the signed 8-bit group scale sc = 16 hi + lo goes into two
// f16 weight operands q * lo and q * hi (unsigned codes <= 63: both exact in f16), the activation codes as f16, both
// sums exact in f32, taken to i32 as 16 * hi_sum + lo_sum, and the reference's -32 offset taken from the activation's
// 16-element group sums into lane l exactly as kdot.rs:125-129 does (the reference's lane split of it). Either
// way the result is the exact lane sum for a 16-row x 16-column tile. The f32 part then runs per output in the lanes
// that hold it (4 rows x 1 column per lane): acc[l] += (dx * d) * f32(sumi[l]), accm[i] += (-dx * dmin) *
// f32(prod[i]), no FMA, and reduce8(acc) [+ reduce4(accm)] at the end.
//
// Q8_0 / Q4_0 x Q8_0 (dot.rs:29-66): one product over K = 32 is one block's exact i32 sum for the tile (Q4_0: the
// unsigned codes, less 8 * the activation block's code sum), then acc += (dw * dx) * f32(isum) per output.
//
// Work: a wave owns 16 rows x 16 columns for all of K (its super-block's loads issued one step ahead); a 256-thread
// work-group the same 16 rows x 64 columns. Rows and columns past the ends are read clamped and not written.
#include "aq_common.h"

#include <atomic>

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
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
// Bytes of x times a small factor f, per byte (every product < 256, so no carry leaves its byte): one packed 16-bit
// multiply with f in both halves.
__device__ __forceinline__ uint32_t mul_bytes(uint32_t x, uint32_t f) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, x) * __builtin_bit_cast(u16x2, f * 0x00010001u));
}

// f16 operands of the matrix-core f16 product (Q6_K). Small integers are exact in f16 (|v| <= 2048, and multiples of
// 2^k up to 2048 * 2^k), the products of two f16 are exact in f32 and every partial sum of a lane (an integer below
// 2^24 in magnitude) is exact in f32, so v_mfma_f32_16x16x32_f16 returns the exact integer lane sums as floats.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint32_t h2bits(float a, float b) {
    return __builtin_bit_cast(uint32_t, f16x2{(_Float16)a, (_Float16)b});
}
// Unsigned bytes 0, 1 (k = 0) or 2, 3 (k = 1) of w as the f16 pair (1024 + byte): the byte under an exponent of 2^10.
__device__ __forceinline__ uint32_t magic_pair(uint32_t w, int k) {
    return __builtin_amdgcn_perm(0x64646464u, w, k == 0 ? 0x04010400u : 0x04030402u);
}
// a * b + c on f16 pairs, one rounding (v_pk_fma_f16): exact whenever the result is representable.
__device__ __forceinline__ uint32_t h2fma(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b),
                                                                  __builtin_bit_cast(f16x2, c)));
}
// Eight signed activation codes (bytes of x, in k order) as f16: (1024 + 128 + x) - 1152.
__device__ __forceinline__ f16x8 codes_f16(uint64_t x) {
    const uint32_t w0 = (uint32_t)x ^ 0x80808080u, w1 = (uint32_t)(x >> 32) ^ 0x80808080u;
    const f16x2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const f16x2 p0 = __builtin_bit_cast(f16x2, magic_pair(w0, 0)) + off, p1 = __builtin_bit_cast(f16x2, magic_pair(w0, 1)) + off;
    const f16x2 p2 = __builtin_bit_cast(f16x2, magic_pair(w1, 0)) + off, p3 = __builtin_bit_cast(f16x2, magic_pair(w1, 1)) + off;
    return __builtin_bit_cast(f16x8, uint4{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
                                           __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3)});
}
__device__ __forceinline__ f32x4 mma_f16(f16x8 a, f16x8 b) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
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
// Signed bytes k, k + 1 of w (k = 0 or 2) as an i16 pair: a byte permute of (w << 8, w) whose sign-fill selectors
// (10 / 11: bit 15 / 31 of the first source, 8 / 9: of the second) supply each byte's sign.
__device__ __forceinline__ uint32_t i8pair(uint32_t w, uint32_t w8, int k) {
    return __builtin_amdgcn_perm(w8, w, k == 0 ? 0x08010A00u : 0x09030B02u);
}


// ---- LDS staging ----
// Operands reach the LDS by direct global-to-LDS copies (global_load_lds_*: each active lane's 16 or 4 bytes land at
// m0 + 16 * lane or m0 + 4 * lane), issued GEMM_STAGES - 1 steps ahead into a ring of GEMM_STAGES buffers, so the
// loads' latency is covered without holding the data in registers. Every wave issues the same number of copies per
// step (a whole wave never skips one), so its count of outstanding vector-memory operations says which step has
// landed; a work-group barrier after the wait makes every wave's copies of that step visible and, at the same
// time, frees the buffer read one step earlier for the next copies.
constexpr int GEMM_STAGES = 3;

__device__ __forceinline__ void dma16(uint32_t lds, const void *g) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(g) : "memory", "m0");
}
__device__ __forceinline__ void dma4(uint32_t lds, const void *g) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(lds), "v"(g) : "memory", "m0");
}
// Wait until at most N of this wave's vector-memory operations are outstanding (and its LDS operations are done),
// then meet the work-group; one asm statement, so no memory access moves across it.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}
__device__ __forceinline__ uint32_t uni(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }

// One super-block step of a K-quant work-group (16 rows, 4 waves x 16 columns) in the LDS, in 16-byte units:
//   weight codes: unit c * 4 + k = byte chunk c of row tile k (rows r0 + 4k .. + 3) — the four tiles interleaved,
//     qa (32 chunks a tile), then qb (Q5_K 8, Q6_K 16 chunks a tile);
//   scale records: unit W_UNITS - 16 + i = row r0 + i's 16-byte record; Q6_K then the 4 tiles' f16 d (8 B each);
//   per wave: codes unit q * 16 + c = byte chunk q of column c's super-block (c = 0..15); f32 dx per column;
//     Q4_K / Q5_K the 8 sub-block sums (16 B) per column, Q6_K the 16 group sums (32 B).
template <int T>
struct KqStage { // every W_UNITS / 4 <= 64: one weight copy per wave
    static constexpr int QB_UNITS = T == AQ_TYPE_Q4_K ? 0 : (T == AQ_TYPE_Q5_K ? 32 : 64);
    static constexpr int W_UNITS = 128 + QB_UNITS + 16;
    static constexpr int WL = W_UNITS / 4; // weight units per wave
    static constexpr int WB = W_UNITS * 16 + (T == AQ_TYPE_Q6_K ? 32 : 0);
    static constexpr int XSUM = T == AQ_TYPE_Q6_K ? 512 : 256;
    static constexpr int XB = 4096 + 64 + XSUM;
    static constexpr int BYTES = WB + 4 * XB;
    static constexpr int NDMA = T == AQ_TYPE_Q6_K ? 8 : 7; // copies per wave per step
};

template <int T>
__device__ __forceinline__ void kq_issue(const GemmArgs &a, uint32_t buf, size_t sb, int r0, int c0w, int wave,
                                         int lane) {
    using S = KqStage<T>;
    const size_t nb = (size_t)a.nb;
    if (lane < S::WL) {
        const int u = wave * S::WL + lane;
        const uint8_t *src;
        if (u < 128) {
            src = a.qa + kq_tile((size_t)min(r0 + 4 * (u & 3), a.rows - 1), sb, nb) * 512 + (size_t)(u >> 2) * 16;
        } else if (u < 128 + S::QB_UNITS) {
            const int v = u - 128;
            src = a.qb + kq_tile((size_t)min(r0 + 4 * (v & 3), a.rows - 1), sb, nb) * (S::QB_UNITS * 4) +
                  (size_t)(v >> 2) * 16;
        } else {
            src = a.sc + kq_sc_off((size_t)min(r0 + u - 128 - S::QB_UNITS, a.rows - 1), sb, nb);
        }
        dma16(uni(buf + (uint32_t)(wave * S::WL * 16)), src);
    }
    if constexpr (T == AQ_TYPE_Q6_K) {
        if (lane < 2) {
            const int d = 2 * wave + lane; // tile d >> 1, its rows 2 (d & 1) .. + 1
            dma4(uni(buf + (uint32_t)(S::W_UNITS * 16 + wave * 8)),
                 a.dm + kq_tile((size_t)min(r0 + 4 * (d >> 1), a.rows - 1), sb, nb) * 8 + 4 * (d & 1));
        }
    }
    const uint32_t xw = buf + (uint32_t)(S::WB + wave * S::XB);
    const size_t col = (size_t)min(c0w + (lane & 15), a.ncols - 1);
    const int8_t *xs = a.xq + col * a.n + sb * 256;
#pragma unroll
    for (int i = 0; i < 4; i++) dma16(uni(xw + (uint32_t)(i * 1024)), xs + (size_t)(i * 4 + (lane >> 4)) * 16);
    if (lane < 16) dma4(uni(xw + 4096), a.xd + col * nb + sb);
    if constexpr (T == AQ_TYPE_Q6_K) {
        if (lane < 32) {
            const size_t c2 = (size_t)min(c0w + (lane >> 1), a.ncols - 1);
            dma16(uni(xw + 4160), a.xbs + (c2 * nb + sb) * 16 + 8 * (lane & 1));
        }
    } else {
        if (lane < 16) dma16(uni(xw + 4160), a.xq8s + (col * nb + sb) * 8);
    }
}

// K-quant x Q8_K: a work-group owns 16 rows x 64 columns, wave w the 16 x 16 tile of columns c0 + 16w; lane
// (li = lane & 15, g = lane >> 4) feeds weight row li / column li into the products (k-group g = sub-blocks 2g,
// 2g + 1 of each lane slot) and owns the outputs of rows 4g .. 4g + 3 in column li.
template <int T>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) kq_gemm_kernel(GemmArgs a) {
    using S = KqStage<T>;
    constexpr int ND = T == AQ_TYPE_Q4_K ? 2 : (T == AQ_TYPE_Q5_K ? 3 : 4); // digits
    constexpr int BASE = T == AQ_TYPE_Q4_K ? 8 : (T == AQ_TYPE_Q5_K ? 4 : 5);
    extern __shared__ __align__(16) uint8_t gm_lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, li = lane & 15, k4 = li >> 2, r4 = li & 3;
    const int r0 = (int)blockIdx.x * 16;
    const int c0w = (int)blockIdx.y * 64 + wave * 16;
    const bool live = c0w < a.ncols; // a wave past the last column copies and waits but computes nothing
    const int nb = a.nb;
    const uint32_t lds0 = (uint32_t)(uintptr_t)gm_lds;

    float acc[4][8], accm[4][4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
        for (int l = 0; l < 8; l++) acc[j][l] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) accm[j][i] = 0.0f;
    }
#pragma unroll
    for (int s = 0; s < GEMM_STAGES - 1; s++)
        if (s < nb) kq_issue<T>(a, lds0 + (uint32_t)(s * S::BYTES), (size_t)s, r0, c0w, wave, lane);

    for (int sb = 0; sb < nb; sb++) {
        if (sb + GEMM_STAGES - 2 < nb) wait_vm_barrier<(GEMM_STAGES - 2) * S::NDMA>();
        else wait_vm_barrier<0>();
        if (sb + GEMM_STAGES - 1 < nb)
            kq_issue<T>(a, lds0 + (uint32_t)(((sb + GEMM_STAGES - 1) % GEMM_STAGES) * S::BYTES),
                        (size_t)(sb + GEMM_STAGES - 1), r0, c0w, wave, lane);
        if (!live) continue;
        const uint8_t *W = gm_lds + (sb % GEMM_STAGES) * S::BYTES;
        const uint8_t *X = W + S::WB + wave * S::XB;
        const uint8_t *SC = W + (S::W_UNITS - 16) * 16;

        // every LDS operand of the step, read up front: the weight codes of row li (lane slots 0..7), the column's
        // activation codes, the scale records of row li and of the output rows 4g .. 4g + 3, dx and the sums
        uint32_t wa[8], wb[8], wh[8];
        uint64_t bx[8];
#pragma unroll
        for (int l = 0; l < 8; l++) {
            const int h = l >> 2, p = l & 3;
            const int cq = h * 16 + p * 4 + r4; // the lane's qa chunk in its row tile
            if constexpr (T == AQ_TYPE_Q6_K) {
                const uint2 w = *reinterpret_cast<const uint2 *>(W + (cq * 4 + k4) * 16 + 8 * (g >> 1));
                wa[l] = w.x;
                wb[l] = w.y;
                wh[l] = *reinterpret_cast<const uint32_t *>(W + 2048 + ((p * 4 + r4) * 4 + k4) * 16 + h * 8 + 4 * (g >> 1));
            } else {
                wa[l] = *reinterpret_cast<const uint32_t *>(W + (cq * 4 + k4) * 16 + 4 * g);
                if constexpr (T == AQ_TYPE_Q5_K) {
                    const int e = p * 4 + r4;
                    wh[l] = *reinterpret_cast<const uint32_t *>(W + 2048 + ((e >> 1) * 4 + k4) * 16 + (e & 1) * 8 + h * 4);
                }
            }
            bx[l] = *reinterpret_cast<const uint64_t *>(X + ((lane_slot(l) * 2 + (g >> 1)) * 16 + li) * 16 + 8 * (g & 1));
        }
        const uint4 sa = *reinterpret_cast<const uint4 *>(SC + li * 16);
        uint4 se[4];
#pragma unroll
        for (int j = 0; j < 4; j++) se[j] = *reinterpret_cast<const uint4 *>(SC + (4 * g + j) * 16);
        const float dx = *reinterpret_cast<const float *>(X + 4096 + 4 * li);
        uint4 xs0, xs1;
        uint2 d6;
        if constexpr (T == AQ_TYPE_Q6_K) {
            d6 = *reinterpret_cast<const uint2 *>(W + S::W_UNITS * 16 + 8 * g);
            xs0 = *reinterpret_cast<const uint4 *>(X + 4160 + 32 * li);
            xs1 = *reinterpret_cast<const uint4 *>(X + 4160 + 32 * li + 16);
        } else {
            xs0 = *reinterpret_cast<const uint4 *>(X + 4160 + 16 * li);
        }

        // the weight operand's scales: Q4_K / Q5_K as digits of the scales of sub-blocks 2g and 2g + 1; Q6_K as f16
        // factor pairs of its group scales sc = 16 hi + lo (lo in 0..15, hi in -8..7): (1024 + q) * f - 1024 * f =
        // q * f, exact (|.| <= 945). Group scale k of the word: 0 = sub-block 2g lanes 0-3, 1 = lanes 4-7, 2 and 3
        // the same for sub-block 2g + 1.
        int dga[ND], dgb[ND], dgc[ND], dgd[ND];
        uint32_t flo[4], clo[4], fhi[4], chi[4];
        if constexpr (T == AQ_TYPE_Q6_K) {
            const uint32_t sw = g == 0 ? sa.x : g == 1 ? sa.y : g == 2 ? sa.z : sa.w;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int sc = (int8_t)(sw >> (8 * k)), lo = sc & 15, hi = sc >> 4;
                flo[k] = h2bits((float)lo, (float)lo);
                clo[k] = h2bits((float)(-1024 * lo), (float)(-1024 * lo));
                fhi[k] = h2bits((float)hi, (float)hi);
                chi[k] = h2bits((float)(-1024 * hi), (float)(-1024 * hi));
            }
        } else {
            // 6-bit scales of sub-blocks 2g, 2g + 1 (quant.rs:45-51): bytes 2g, 2g + 1 of the low or high word
            const uint32_t sc_lo = sa.y & 0x3F3F3F3Fu;
            const uint32_t sc_hi = (sa.w & 0x0F0F0F0Fu) | ((sa.y >> 2) & 0x30303030u);
            const uint32_t scw = g < 2 ? sc_lo : sc_hi;
            const int sca = (int)((scw >> (16 * (g & 1))) & 0xFF), scb = (int)((scw >> (16 * (g & 1) + 8)) & 0xFF);
            constexpr int BB = T == AQ_TYPE_Q4_K ? 3 : 2;
#pragma unroll
            for (int i = 0; i < ND; i++) {
                dga[i] = dgc[i] = (sca >> (BB * i)) & ((1 << BB) - 1);
                dgb[i] = dgd[i] = (scb >> (BB * i)) & ((1 << BB) - 1);
            }
        }

        // the codes of sub-blocks 2g (lo) and 2g + 1 (hi) per lane slot, as unsigned bytes
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int l = 0; l < 8; l++) {
            if constexpr (T == AQ_TYPE_Q6_K) {
                const int sh = 4 * (g & 1);
                lo[l] = ((wa[l] >> sh) & 0x0F0F0F0Fu) | (((wh[l] >> sh) & 0x03030303u) << 4);
                hi[l] = ((wb[l] >> sh) & 0x0F0F0F0Fu) | (((wh[l] >> (sh + 2)) & 0x03030303u) << 4);
            } else {
                lo[l] = wa[l] & 0x0F0F0F0Fu;
                hi[l] = (wa[l] >> 4) & 0x0F0F0F0Fu;
                if constexpr (T == AQ_TYPE_Q5_K) {
                    lo[l] |= ((wh[l] >> (2 * g)) & 0x01010101u) << 4;
                    hi[l] |= ((wh[l] >> (2 * g + 1)) & 0x01010101u) << 4;
                }
            }
        }

        // the exact lane sums of the tile: c[l][j] = lane l's sum for output row 4g + j of this lane's column.
        // Q4_K / Q5_K: int8 products digit by digit over all eight lane slots (eight independent products in flight).
        // Q6_K: two f16 products per lane slot (the lo and hi scale parts; each sum exact in f32, |.| < 2^22), taken
        // to i32 and combined there as 16 hi + lo, before the reference's -32 group-sum term (kdot.rs:97-140).
        v4i c[8];
        if constexpr (T == AQ_TYPE_Q6_K) {
#pragma unroll
            for (int l = 0; l < 8; l++) {
                const int ka = l < 4 ? 0 : 1, kb = l < 4 ? 2 : 3;
                const uint32_t la = magic_pair(lo[l], 0), lb = magic_pair(lo[l], 1);
                const uint32_t ha = magic_pair(hi[l], 0), hb = magic_pair(hi[l], 1);
                const f16x8 alo = __builtin_bit_cast(
                    f16x8, uint4{h2fma(la, flo[ka], clo[ka]), h2fma(lb, flo[ka], clo[ka]), h2fma(ha, flo[kb], clo[kb]),
                                 h2fma(hb, flo[kb], clo[kb])});
                const f16x8 ahi = __builtin_bit_cast(
                    f16x8, uint4{h2fma(la, fhi[ka], chi[ka]), h2fma(lb, fhi[ka], chi[ka]), h2fma(ha, fhi[kb], chi[kb]),
                                 h2fma(hb, fhi[kb], chi[kb])});
                const f16x8 b = codes_f16(bx[l]);
                const f32x4 dl = mma_f16(alo, b), dh = mma_f16(ahi, b);
#pragma unroll
                for (int e = 0; e < 4; e++) c[l][e] = 16 * (int)dh[e] + (int)dl[e];
            }
        } else {
#pragma unroll
            for (int i = ND - 1; i >= 0; i--) {
#pragma unroll
                for (int l = 0; l < 8; l++) {
                    const int *da = l < 4 ? dga : dgc, *db = l < 4 ? dgb : dgd;
                    const uint32_t alo = mul_bytes(lo[l], (uint32_t)da[i]), ahi = mul_bytes(hi[l], (uint32_t)db[i]);
                    v4i cin = {0, 0, 0, 0};
                    if (i < ND - 1) {
#pragma unroll
                        for (int e = 0; e < 4; e++) cin[e] = c[l][e] * BASE;
                    }
                    c[l] = mma(pack2(alo, ahi), bx[l], cin);
                }
            }
        }

        // the f32 chains of the lane's four outputs (kdot.rs:37-140), in super-block order
        if constexpr (T == AQ_TYPE_Q6_K) {
            const uint32_t bsw[8] = {xs0.x, xs0.y, xs0.z, xs0.w, xs1.x, xs1.y, xs1.z, xs1.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t sw[4] = {se[j].x, se[j].y, se[j].z, se[j].w};
                const float d = dx * h2f((j < 2 ? d6.x : d6.y) >> (16 * (j & 1)));
#pragma unroll
                for (int l = 0; l < 8; l++) {
                    // kdot.rs:125-129: lane l less 32 * (bs[2l] sc[2l] + bs[2l + 1] sc[2l + 1])
                    const int off = sdot2(bsw[l], i8pair(sw[l >> 1], sw[l >> 1] << 8, 2 * (l & 1)));
                    acc[j][l] += d * (float)(c[l][j] - 32 * off);
                }
            }
        } else {
            const uint32_t q8w[4] = {xs0.x, xs0.y, xs0.z, xs0.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float d = dx * h2f(se[j].x), dmin = -dx * h2f(se[j].x >> 16);
                // the 8 mins as bytes (quant.rs:45-51): sub-blocks 0..3 from bytes 4..7, 4..7 from bytes 8..11 + 4..7
                const uint32_t mlo = se[j].z & 0x3F3F3F3Fu;
                const uint32_t mhi = ((se[j].w >> 4) & 0x0F0F0F0Fu) | ((se[j].z >> 2) & 0x30303030u);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t m2 = __builtin_amdgcn_perm(0u, i < 2 ? mlo : mhi, (i & 1) ? 0x0C030C02u : 0x0C010C00u);
                    accm[j][i] += dmin * (float)sdot2(m2, q8w[i]); // m[2i] q8s[2i] + m[2i+1] q8s[2i+1]
                }
#pragma unroll
                for (int l = 0; l < 8; l++) acc[j][l] += d * (float)c[l][j];
            }
        }
    }

    const int ocol = c0w + li;
    if (live && ocol < a.ncols) {
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

// One step of a Q8_0 / Q4_0 work-group = 8 blocks (256 elements), in 16-byte units: codes unit q * 16 + i = byte
// chunk q of row r0 + i's 8 blocks (Q8_0: 16 chunks, Q4_0: 8), then row i's 8 f16 d at unit NQ + i; per wave the
// activation codes as for the K-quants, then each column's 8 f32 d (32 B) and, for Q4_0, its 8 i32 code sums.
template <int T>
struct Q8Stage {
    static constexpr int QC = T == AQ_TYPE_Q8_0 ? 16 : 8; // code chunks per row
    static constexpr int W_UNITS = 16 * QC + 16;
    static constexpr int WL = W_UNITS / 4;          // weight units per wave
    static constexpr int WI = (WL + 63) / 64;       // copies they take
    static constexpr int WB = W_UNITS * 16;
    static constexpr int XB = 4096 + 512 + (T == AQ_TYPE_Q4_0 ? 512 : 0);
    static constexpr int BYTES = WB + 4 * XB;
    static constexpr int NDMA = WI + 5 + (T == AQ_TYPE_Q4_0 ? 1 : 0);
};

template <int T>
__device__ __forceinline__ void q8_issue(const GemmArgs &a, uint32_t buf, size_t st, int r0, int c0w, int wave,
                                         int lane) {
    using S = Q8Stage<T>;
    const size_t nb = (size_t)a.nb; // 32-blocks per row
#pragma unroll
    for (int i = 0; i < S::WI; i++) {
        if (i * 64 + lane < S::WL) { // every copy has active lanes: WL > 64 (WI - 1)
            const int u = wave * S::WL + i * 64 + lane;
            const uint8_t *src;
            if (u < 16 * S::QC) {
                const size_t row = (size_t)min(r0 + (u & 15), a.rows - 1);
                src = a.qa + (row * nb + st * 8) * (S::QC * 2) + (size_t)(u >> 4) * 16;
            } else {
                const size_t row = (size_t)min(r0 + u - 16 * S::QC, a.rows - 1);
                src = a.dm + (row * nb + st * 8) * 2;
            }
            dma16(uni(buf + (uint32_t)((wave * S::WL + i * 64) * 16)), src);
        }
    }
    const uint32_t xw = buf + (uint32_t)(S::WB + wave * S::XB);
    const size_t col = (size_t)min(c0w + (lane & 15), a.ncols - 1);
    const int8_t *xs = a.xq + col * a.n + st * 256;
#pragma unroll
    for (int i = 0; i < 4; i++) dma16(uni(xw + (uint32_t)(i * 1024)), xs + (size_t)(i * 4 + (lane >> 4)) * 16);
    const size_t c2 = (size_t)min(c0w + (lane >> 1), a.ncols - 1);
    if (lane < 32) dma16(uni(xw + 4096), a.xd + c2 * nb + st * 8 + 4 * (lane & 1));
    if constexpr (T == AQ_TYPE_Q4_0) {
        if (lane < 32) dma16(uni(xw + 4608), a.xs0 + c2 * nb + st * 8 + 4 * (lane & 1));
    }
}

// Q8_0 / Q4_0 weights x Q8_0 activations: the same work-group and lane roles; one product over K = 32 per block.
template <int T>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) q8_gemm_kernel(GemmArgs a) {
    using S = Q8Stage<T>;
    extern __shared__ __align__(16) uint8_t gm_lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, li = lane & 15;
    const int r0 = (int)blockIdx.x * 16;
    const int c0w = (int)blockIdx.y * 64 + wave * 16;
    const bool live = c0w < a.ncols;
    const int nst = a.nb / 8; // steps
    const uint32_t lds0 = (uint32_t)(uintptr_t)gm_lds;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < GEMM_STAGES - 1; s++)
        if (s < nst) q8_issue<T>(a, lds0 + (uint32_t)(s * S::BYTES), (size_t)s, r0, c0w, wave, lane);

    for (int st = 0; st < nst; st++) {
        if (st + GEMM_STAGES - 2 < nst) wait_vm_barrier<(GEMM_STAGES - 2) * S::NDMA>();
        else wait_vm_barrier<0>();
        if (st + GEMM_STAGES - 1 < nst)
            q8_issue<T>(a, lds0 + (uint32_t)(((st + GEMM_STAGES - 1) % GEMM_STAGES) * S::BYTES),
                        (size_t)(st + GEMM_STAGES - 1), r0, c0w, wave, lane);
        if (!live) continue;
        const uint8_t *W = gm_lds + (st % GEMM_STAGES) * S::BYTES;
        const uint8_t *X = W + S::WB + wave * S::XB;
        uint4 dwr[4];
#pragma unroll
        for (int j = 0; j < 4; j++) dwr[j] = *reinterpret_cast<const uint4 *>(W + (16 * S::QC + 4 * g + j) * 16);
#pragma unroll
        for (int b = 0; b < 8; b++) {
            uint64_t wa;
            if constexpr (T == AQ_TYPE_Q8_0) {
                wa = *reinterpret_cast<const uint64_t *>(W + ((2 * b + (g >> 1)) * 16 + li) * 16 + 8 * (g & 1));
            } else {
                // elements 8g .. 8g + 7: bytes 8 (g & 1) .., low nibbles for g < 2, high for g >= 2
                const uint64_t w = *reinterpret_cast<const uint64_t *>(W + (b * 16 + li) * 16 + 8 * (g & 1));
                wa = (w >> (4 * (g >> 1))) & 0x0F0F0F0F0F0F0F0Full;
            }
            const uint64_t bx =
                *reinterpret_cast<const uint64_t *>(X + ((2 * b + (g >> 1)) * 16 + li) * 16 + 8 * (g & 1));
            const float dx = *reinterpret_cast<const float *>(X + 4096 + 32 * li + 4 * b);
            int off = 0;
            if constexpr (T == AQ_TYPE_Q4_0) // dot.rs:48-66: codes less 8
                off = 8 * *reinterpret_cast<const int32_t *>(X + 4608 + 32 * li + 4 * b);
            v4i c = {0, 0, 0, 0};
            c = mma(wa, bx, c);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t dww = (b >> 1) == 0 ? dwr[j].x : (b >> 1) == 1 ? dwr[j].y : (b >> 1) == 2 ? dwr[j].z : dwr[j].w;
                acc[j] += (h2f(dww >> (16 * (b & 1))) * dx) * (float)(c[j] - off);
            }
        }
    }
    const int ocol = c0w + li;
    if (live && ocol < a.ncols) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int row = r0 + 4 * g + j;
            if (row >= a.rows) continue;
            const size_t o = (size_t)ocol * a.rows + row;
            a.y[o] = a.resid ? a.resid[o] + acc[j] : acc[j];
        }
    }
}

template <typename K>
int launch_staged(K kernel, int bytes, const GemmArgs &ga, hipStream_t stream, const char *what) {
    const dim3 grid((unsigned)((ga.rows + 15) / 16), (unsigned)((ga.ncols + 63) / 64));
    const size_t lds = (size_t)bytes * GEMM_STAGES;
    if (lds > 64 * 1024) { // once per kernel and process: allow the ring's dynamic LDS (up to the CU's 160 KB)
        static std::atomic<bool> raised{false};
        if (!raised.load()) {
            const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return fail(AQ_EHIP, what);
            raised.store(true);
        }
    }
    hipLaunchKernelGGL(kernel, grid, dim3(256), lds, stream, ga);
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, what);
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
        case AQ_TYPE_Q4_K:
            return launch_staged(kq_gemm_kernel<AQ_TYPE_Q4_K>, KqStage<AQ_TYPE_Q4_K>::BYTES, ga, stream, "kq_gemm launch");
        case AQ_TYPE_Q5_K:
            return launch_staged(kq_gemm_kernel<AQ_TYPE_Q5_K>, KqStage<AQ_TYPE_Q5_K>::BYTES, ga, stream, "kq_gemm launch");
        default:
            return launch_staged(kq_gemm_kernel<AQ_TYPE_Q6_K>, KqStage<AQ_TYPE_Q6_K>::BYTES, ga, stream, "kq_gemm launch");
        }
    }
    AQ_REQUIRE(w.type == AQ_TYPE_Q8_0 || w.type == AQ_TYPE_Q4_0, "gemm: weight type");
    AQ_REQUIRE(w.cols % 256 == 0, "gemm: Q8_0 / Q4_0 columns must be a multiple of 256");
    ga.xq = x.q0;
    ga.xd = x.d0;
    ga.xs0 = x.s0;
    if (w.type == AQ_TYPE_Q8_0)
        return launch_staged(q8_gemm_kernel<AQ_TYPE_Q8_0>, Q8Stage<AQ_TYPE_Q8_0>::BYTES, ga, stream, "q8_gemm launch");
    return launch_staged(q8_gemm_kernel<AQ_TYPE_Q4_0>, Q8Stage<AQ_TYPE_Q4_0>::BYTES, ga, stream, "q8_gemm launch");
}

} // namespace aq
