// quantize.hip — activation quantisers on the device: Q8_K (the K-quant weights' activation form) and Q8_0
// (the Q8_0 / Q4_0 weights' form), bit-exact with the reference's scalar quantisers.
#include "aq_common.h"

namespace aq {
namespace {

// One wave per 256-element block; lane i owns elements 4i..4i+3 (sub-block s = i/8, lane l = i%8).
// Q8KRow::quantize_scalar_into (q8k.rs:76-114): max = the first element with the largest |x| (strict >
// scan), iscale = -127/max, q = min(127, round_ties_even(iscale*x)), d = 1/iscale, bsums per 16, q8s per 32.
__global__ void __launch_bounds__(256) q8k_quantize_kernel(const float *__restrict__ src, size_t src_stride,
                                                           int8_t *__restrict__ qs, float *__restrict__ dout,
                                                           int16_t *__restrict__ bs, int16_t *__restrict__ q8s,
                                                           size_t n, size_t nblocks_total) {
    const int lane = threadIdx.x & 63;
    const size_t blk = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblocks_total) return;
    const size_t nb = n / 256;
    const size_t col = blk / nb, b = blk % nb;
    const float4 v = *reinterpret_cast<const float4 *>(src + col * src_stride + b * 256 + lane * 4);
    float x[4] = {v.x, v.y, v.z, v.w};
    // (|x|, index) max with the first index winning ties
    float amax = 0.0f;
    int idx = 0x7fffffff;
    float maxv = 0.0f;
    for (int j = 0; j < 4; j++) {
        float a = fabsf(x[j]);
        if (a > amax) {
            amax = a;
            idx = lane * 4 + j;
            maxv = x[j];
        }
    }
    for (int off = 32; off >= 1; off >>= 1) {
        float oa = __shfl_xor(amax, off);
        int oi = __shfl_xor(idx, off);
        float om = __shfl_xor(maxv, off);
        if (oa > amax || (oa == amax && oi < idx)) {
            amax = oa;
            idx = oi;
            maxv = om;
        }
    }
    const size_t qbase = col * n + b * 256;
    const size_t mbase = col * nb + b;
    int q[4];
    if (amax == 0.0f) {
        q[0] = q[1] = q[2] = q[3] = 0;
    } else {
        const float iscale = -127.0f / maxv;
        for (int j = 0; j < 4; j++) {
            int qi = (int)__builtin_rintf(iscale * x[j]);
            q[j] = qi < 127 ? qi : 127;
        }
        if (lane == 0) dout[mbase] = 1.0f / iscale;
    }
    if (amax == 0.0f && lane == 0) dout[mbase] = 0.0f;
    const int s = lane >> 3, l = lane & 7;
    const uint32_t packed = (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) | ((uint32_t)(uint8_t)q[2] << 16) |
                            ((uint32_t)(uint8_t)q[3] << 24);
    *reinterpret_cast<uint32_t *>(qs + qbase + lane_slot(l) * 32 + s * 4) = packed;
    int sum = q[0] + q[1] + q[2] + q[3];
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2); // group of 16 = 4 lanes
    if ((lane & 3) == 0) bs[mbase * 16 + (lane >> 2)] = (int16_t)sum;
    int s32 = sum + __shfl_xor(sum, 4); // sub-block of 32 = 8 lanes
    if ((lane & 7) == 0) q8s[mbase * 8 + (lane >> 3)] = (int16_t)s32;
}

// One lane per 32-block. Q8Row::quantize_scalar_into (q8.rs:81-121): d = amax/127 -> f16 (RNE),
// id = d != 0 ? 1/d : 0 from the unrounded d, q = round_half_away(x*id) saturated to i8.
__global__ void __launch_bounds__(256) q8_0_quantize_kernel(const float *__restrict__ src, size_t src_stride,
                                                            int8_t *__restrict__ q0, float *__restrict__ d0,
                                                            uint16_t *__restrict__ h0, int32_t *__restrict__ s0,
                                                            size_t n, size_t nblocks_total) {
    const size_t blk = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= nblocks_total) return;
    const size_t nb = n / 32;
    const size_t col = blk / nb, b = blk % nb;
    const float *x = src + col * src_stride + b * 32;
    float v[32];
    for (int i = 0; i < 8; i++) {
        float4 t = *reinterpret_cast<const float4 *>(x + 4 * i);
        v[4 * i] = t.x;
        v[4 * i + 1] = t.y;
        v[4 * i + 2] = t.z;
        v[4 * i + 3] = t.w;
    }
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) {
        float a = fabsf(v[i]);
        if (a > amax) amax = a;
    }
    const float dd = amax / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    const _Float16 hd = (_Float16)dd; // v_cvt_f16_f32: round to nearest even, as half::f16::from_f32
    uint16_t hbits;
    __builtin_memcpy(&hbits, &hd, 2);
    int sum = 0;
    uint32_t words[8];
    for (int i = 0; i < 8; i++) {
        uint32_t w = 0;
        for (int j = 0; j < 4; j++) {
            float r = roundf(v[4 * i + j] * id);
            int qi = r > 127.0f ? 127 : (r < -128.0f ? -128 : (int)r);
            sum += qi;
            w |= (uint32_t)(uint8_t)qi << (8 * j);
        }
        words[i] = w;
    }
    uint4 *dst = reinterpret_cast<uint4 *>(q0 + col * n + b * 32);
    dst[0] = make_uint4(words[0], words[1], words[2], words[3]);
    dst[1] = make_uint4(words[4], words[5], words[6], words[7]);
    const size_t m = col * nb + b;
    d0[m] = (float)hd;
    h0[m] = hbits;
    s0[m] = sum;
}

} // namespace

int launch_q8k_quantize(const Act &a, size_t ncols, const float *src, size_t src_stride, hipStream_t stream) {
    const size_t total = ncols * a.nb;
    if (total == 0) return 0;
    const unsigned grid = (unsigned)((total + 3) / 4);
    hipLaunchKernelGGL(q8k_quantize_kernel, dim3(grid), dim3(256), 0, stream, src, src_stride, a.qs, a.d, a.bs,
                       a.q8s, a.n, total);
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "q8k_quantize launch");
}

int launch_q8_0_quantize(const Act &a, size_t ncols, const float *src, size_t src_stride, hipStream_t stream) {
    const size_t total = ncols * a.nb32;
    if (total == 0) return 0;
    const unsigned grid = (unsigned)((total + 255) / 256);
    hipLaunchKernelGGL(q8_0_quantize_kernel, dim3(grid), dim3(256), 0, stream, src, src_stride, a.q0, a.d0, a.h0,
                       a.s0, a.n, total);
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "q8_0_quantize launch");
}

} // namespace aq
