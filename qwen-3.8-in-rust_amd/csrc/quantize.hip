// quantize.hip — activation quantisers on the device: Q8_K (the K-quant weights' activation form) and Q8_0
// (the Q8_0 / Q4_0 weights' form), bit-exact with the reference's scalar quantisers.
#include "quant_dev.h"

namespace aq {
namespace {

// One wave per 256-element block of one column; lane i owns elements 4i..4i+3 (q8k_block_wave).
__global__ void __launch_bounds__(256) q8k_quantize_kernel(const float *__restrict__ src, size_t src_stride, Act a,
                                                           size_t nblocks_total) {
    const int lane = threadIdx.x & 63;
    const size_t blk = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblocks_total) return;
    const size_t col = blk / a.nb, b = blk % a.nb;
    const float4 v = *reinterpret_cast<const float4 *>(src + col * src_stride + b * 256 + lane * 4);
    const float x[4] = {v.x, v.y, v.z, v.w};
    q8k_block_store(a, col, b, x, lane);
}

__global__ void __launch_bounds__(256) q8_0_quantize_kernel(const float *__restrict__ src, size_t src_stride, Act a,
                                                            size_t nblocks_total) {
    // one lane per element, a half wave per 32-block (a half is past the end as a whole or not at all)
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x, blk = e / 32;
    if (blk >= nblocks_total) return;
    const size_t col = blk / a.nb32, b = blk % a.nb32;
    q8_0_block_half(a, col, b, src[col * src_stride + b * 32 + (e & 31)], (int)(threadIdx.x & 63));
}

} // namespace

int launch_q8k_quantize(const Act &a, size_t ncols, const float *src, size_t src_stride, hipStream_t stream) {
    const size_t total = ncols * a.nb;
    if (total == 0) return 0;
    const unsigned grid = (unsigned)((total + 3) / 4);
    hipLaunchKernelGGL(q8k_quantize_kernel, dim3(grid), dim3(256), 0, stream, src, src_stride, a, total);
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "q8k_quantize launch");
}

int launch_q8_0_quantize(const Act &a, size_t ncols, const float *src, size_t src_stride, hipStream_t stream) {
    const size_t total = ncols * a.nb32;
    if (total == 0) return 0;
    const unsigned grid = (unsigned)((total * 32 + 255) / 256);
    hipLaunchKernelGGL(q8_0_quantize_kernel, dim3(grid), dim3(256), 0, stream, src, src_stride, a, total);
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "q8_0_quantize launch");
}

} // namespace aq
