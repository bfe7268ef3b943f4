// quant_dev.h — device building blocks shared by the quantise, norm, activation and model kernels: the Q8_K and
// Q8_0 activation quantisers as device functions, and the reference's scalar activations.
#pragma once

#include "aq_common.h"
#include "aq_math.h"

namespace aq {

__device__ __forceinline__ float f16_to_f32(uint16_t bits) {
    _Float16 f;
    __builtin_memcpy(&f, &bits, 2);
    return (float)f;
}

// act.rs:7-9 `silu`, 12-14 `sigmoid`, 33-40 `softplus` (threshold 20), same operation order; exp and log1p from
// aq_math.h (the same bits as the CPU oracle's).
__device__ __forceinline__ float exp_f(float x) { return aq_expf(x); }
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + exp_f(-x)); }
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + exp_f(-x)); }
__device__ __forceinline__ float softplus_f(float x) { return x > 20.0f ? x : aq_log1pf(exp_f(x)); }

// Sequential sum acc + x[start] + x[start+stride] + ... over [start, end), in that order, reading 16 values
// ahead so the chain waits on adds, not on each load. SQUARE: the terms are x*x (each product rounded).
template <bool SQUARE>
__device__ __forceinline__ float seq_sum(const float *x, int start, int end, int stride, float acc) {
    int i = start;
    if (i + 15 * stride < end) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; u++) v[u] = x[i + u * stride];
        i += 16 * stride;
        for (; i + 15 * stride < end; i += 16 * stride) { // next batch in flight while this one is summed
            float w[16];
#pragma unroll
            for (int u = 0; u < 16; u++) w[u] = x[i + u * stride];
#pragma unroll
            for (int u = 0; u < 16; u++) acc += SQUARE ? v[u] * v[u] : v[u];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = w[u];
        }
#pragma unroll
        for (int u = 0; u < 16; u++) acc += SQUARE ? v[u] * v[u] : v[u];
    }
    for (; i < end; i += stride) acc += SQUARE ? x[i] * x[i] : x[i];
    return acc;
}

// Work-group copy of n floats from global memory into LDS, every load of a thread issued before the first wait
// (a plain strided loop waits for each load before issuing the next): batches of 8 predicated loads, float4
// when n and both pointers allow.
__device__ __forceinline__ void copy_rows_in(float *dst, const float *src, int n, int tid, int nthreads) {
    if ((n & 3) == 0 && ((uintptr_t)src & 15) == 0 && ((uintptr_t)dst & 15) == 0) {
        const int n4 = n >> 2;
        const float4 *s4 = reinterpret_cast<const float4 *>(src);
        float4 *d4 = reinterpret_cast<float4 *>(dst);
        for (int i = tid; i < n4; i += 8 * nthreads) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = s4[min(i + u * nthreads, n4 - 1)]; // clamped: always in range
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (i + u * nthreads < n4) d4[i + u * nthreads] = v[u];
        }
        return;
    }
    for (int i = tid; i < n; i += 8 * nthreads) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = src[min(i + u * nthreads, n - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (i + u * nthreads < n) dst[i + u * nthreads] = v[u];
    }
}

// rmsnorm.rs reduce8 / reduce4 pairings.
__device__ __forceinline__ float reduce8_f(const float *l) {
    return ((l[0] + l[4]) + (l[2] + l[6])) + ((l[1] + l[5]) + (l[3] + l[7]));
}

// Cross-lane steps on the DPP network (full rate, no LDS round trip).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_mov(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, ROW_MASK, 0xF, false);
}
// Wave-wide max / min of ints (order-free, so exact); the result is uniform.
__device__ __forceinline__ int wave_max_i32(int v) {
    v = max(v, dpp_mov<0xB1>(v));       // quad_perm [1,0,3,2]
    v = max(v, dpp_mov<0x4E>(v));       // quad_perm [2,3,0,1]
    v = max(v, dpp_mov<0x124>(v));      // row_ror:4
    v = max(v, dpp_mov<0x128>(v));      // row_ror:8 (every lane of a row holds the row's max)
    v = max(v, dpp_mov<0x142, 0xA>(v)); // row_bcast:15 into rows 1 and 3
    v = max(v, dpp_mov<0x143, 0xC>(v)); // row_bcast:31 into rows 2 and 3
    return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ int wave_min_i32(int v) {
    v = min(v, dpp_mov<0xB1>(v));
    v = min(v, dpp_mov<0x4E>(v));
    v = min(v, dpp_mov<0x124>(v));
    v = min(v, dpp_mov<0x128>(v));
    v = min(v, dpp_mov<0x142, 0xA>(v));
    v = min(v, dpp_mov<0x143, 0xC>(v));
    return __builtin_amdgcn_readlane(v, 63);
}

// One Q8_K block (256 values) quantised by one wave: lane i holds x[4i..4i+3]. Q8KRow::quantize_scalar_into
// (q8k.rs:76-114): max = the first element with the largest |x|, iscale = -127/max, q = min(127,
// round_ties_even(iscale*x)), d = 1/iscale (0 for an all-zero block), bsums per 16, q8s per 32. The largest |x|
// (a max, order-free) and then its first index (a min over lanes) come from DPP reductions. Writes the block at
// (qs_blk, *d_out, bs_blk[16], q8s_blk[8]) in the kernels' lane-slot code order.
__device__ __forceinline__ void q8k_block_wave(const float x[4], int lane, int8_t *qs_blk, float *d_out,
                                               int16_t *bs_blk, int16_t *q8s_blk) {
    float la = fabsf(x[0]);
#pragma unroll
    for (int j = 1; j < 4; j++) la = fmaxf(la, fabsf(x[j]));
    const int amax_bits = wave_max_i32(__float_as_int(la)); // |x| >= 0: int order is float order
    const float amax = __int_as_float(amax_bits);
    int first = 0x7fffffff;
#pragma unroll
    for (int j = 3; j >= 0; j--)
        if (__float_as_int(fabsf(x[j])) == amax_bits) first = lane * 4 + j;
    const int idx = wave_min_i32(first);
    const float pick = (idx & 3) == 0 ? x[0] : (idx & 3) == 1 ? x[1] : (idx & 3) == 2 ? x[2] : x[3];
    const float maxv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pick), idx >> 2));
    int q[4] = {0, 0, 0, 0};
    if (amax != 0.0f) {
        const float iscale = -127.0f / maxv;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int qi = (int)__builtin_rintf(iscale * x[j]);
            q[j] = qi < 127 ? qi : 127;
        }
        if (lane == 0) *d_out = 1.0f / iscale;
    } else if (lane == 0) {
        *d_out = 0.0f;
    }
    const int s = lane >> 3, l = lane & 7;
    const uint32_t packed = (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) | ((uint32_t)(uint8_t)q[2] << 16) |
                            ((uint32_t)(uint8_t)q[3] << 24);
    *reinterpret_cast<uint32_t *>(qs_blk + lane_slot(l) * 32 + s * 4) = packed;
    int sum = q[0] + q[1] + q[2] + q[3];
    sum += dpp_mov<0xB1>(sum); // quad: the 16 values of a group
    sum += dpp_mov<0x4E>(sum);
    if ((lane & 3) == 0) bs_blk[lane >> 2] = (int16_t)sum;
    const int s32 = sum + dpp_mov<0x12C>(sum); // row_ror:12 = lane i + 4: the next quad, a 32-value sub-block
    if ((lane & 7) == 0) q8s_blk[lane >> 3] = (int16_t)s32;
}

// Store block `blk` of column `col` of a Q8_K activation.
__device__ __forceinline__ void q8k_block_store(const Act &a, size_t col, size_t blk, const float x[4], int lane) {
    const size_t m = col * a.nb + blk;
    q8k_block_wave(x, lane, a.qs + col * a.n + blk * 256, a.d + m, a.bs + m * 16, a.q8s + m * 8);
}

// Max / sum of ints over each 32-lane half of a wave (order-free, so exact): every lane gets its half's value. The
// lanes of a half that is used must all be active.
__device__ __forceinline__ int half_max_i32(int v, int lane) {
    v = max(v, dpp_mov<0xB1>(v));
    v = max(v, dpp_mov<0x4E>(v));
    v = max(v, dpp_mov<0x124>(v));
    v = max(v, dpp_mov<0x128>(v));
    v = max(v, dpp_mov<0x142, 0xA>(v)); // row_bcast:15 into rows 1 and 3: lanes 31 and 63 hold their half's max
    const int lo = __builtin_amdgcn_readlane(v, 31), hi = __builtin_amdgcn_readlane(v, 63);
    return lane < 32 ? lo : hi;
}
__device__ __forceinline__ int half_sum_i32(int v, int lane) {
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x124>(v);
    v += dpp_mov<0x128>(v);
    v += dpp_mov<0x142, 0xA>(v);
    const int lo = __builtin_amdgcn_readlane(v, 31), hi = __builtin_amdgcn_readlane(v, 63);
    return lane < 32 ? lo : hi;
}

// One Q8_0 block (32 values) per 32-lane half of a wave, lane l of the half holding element l: the d, id, codes
// and code sum of q8_0_block_store below (a NaN is passed over by the maximum as there). `lane` is the wave lane.
__device__ __forceinline__ void q8_0_block_half(const Act &a, size_t col, size_t blk, float v, int lane) {
    const float av = fabsf(v);
    const int key = half_max_i32(av > 0.0f ? __float_as_int(av) : 0, lane); // |v| >= 0: int order is float order
    const float dd = __int_as_float(key) / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    const float r = roundf(v * id);
    const int qi = r > 127.0f ? 127 : (r < -128.0f ? -128 : (int)r);
    const int sum = half_sum_i32(qi, lane);
    const int l = lane & 31;
    a.q0[col * a.n + blk * 32 + l] = (int8_t)qi;
    if (l == 0) {
        const _Float16 hd = (_Float16)dd;
        uint16_t hbits;
        __builtin_memcpy(&hbits, &hd, 2);
        const size_t m = col * a.nb32 + blk;
        a.d0[m] = (float)hd;
        a.h0[m] = hbits;
        a.s0[m] = sum;
    }
}

// One Q8_0 block (32 values) by one lane. Q8Row::quantize_scalar_into (q8.rs:81-121): d = amax/127 -> f16
// (round to nearest even), id = d != 0 ? 1/d : 0 from the unrounded d, q = round_half_away(x*id) saturated.
__device__ __forceinline__ void q8_0_block_store(const Act &a, size_t col, size_t blk, const float *v) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) {
        const float av = fabsf(v[i]);
        if (av > amax) amax = av;
    }
    const float dd = amax / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    const _Float16 hd = (_Float16)dd;
    uint16_t hbits;
    __builtin_memcpy(&hbits, &hd, 2);
    int sum = 0;
    uint32_t words[8];
    for (int i = 0; i < 8; i++) {
        uint32_t w = 0;
        for (int j = 0; j < 4; j++) {
            const float r = roundf(v[4 * i + j] * id);
            const int qi = r > 127.0f ? 127 : (r < -128.0f ? -128 : (int)r);
            sum += qi;
            w |= (uint32_t)(uint8_t)qi << (8 * j);
        }
        words[i] = w;
    }
    uint4 *dst = reinterpret_cast<uint4 *>(a.q0 + col * a.n + blk * 32);
    dst[0] = make_uint4(words[0], words[1], words[2], words[3]);
    dst[1] = make_uint4(words[4], words[5], words[6], words[7]);
    const size_t m = col * a.nb32 + blk;
    a.d0[m] = (float)hd;
    a.h0[m] = hbits;
    a.s0[m] = sum;
}

} // namespace aq
