// synth.hip — synthetic tensors on the host (threads) and on the device (one thread per block), from the
// shared generator in synth.h, so both produce the same ggml bytes.
#include <algorithm>
#include <thread>
#include <vector>

#include "aq_common.h"
#include "synth.h"

namespace aq {

int weight_from_ggml(Weight &w, int type, size_t rows, size_t cols, const void *ggml, bool ggml_on_device, int device,
                     hipStream_t stream);
void free_weight(Weight &w);

namespace {

__global__ void synth_blocks_kernel(aq_synth_spec s, float scale, uint8_t *out, size_t nblocks, int bbytes) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    synth_block(s, i, scale, out + i * bbytes);
}

__global__ void synth_f32_kernel(aq_synth_spec s, float scale, float *out, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = synth_value(s, i, scale);
}

int check_spec(const aq_synth_spec *s) {
    AQ_REQUIRE(s, "synth: null spec");
    AQ_REQUIRE(block_bytes(s->ggml_type) > 0, "synth: unsupported type");
    AQ_REQUIRE(s->rows > 0 && s->cols > 0, "synth: empty shape");
    AQ_REQUIRE(s->cols % block_elems(s->ggml_type) == 0, "synth: cols not a multiple of the block size");
    AQ_REQUIRE(s->dist <= 2, "synth: unknown distribution");
    return 0;
}

} // namespace

// Device generation into a ggml-layout buffer `out` (device memory).
int synth_device(const aq_synth_spec &s, uint8_t *out, hipStream_t stream) {
    const float scale = synth_scale(s);
    if (s.ggml_type == AQ_TYPE_F32) {
        const size_t n = (size_t)s.rows * s.cols;
        hipLaunchKernelGGL(synth_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, s, scale,
                           (float *)out, n);
    } else {
        const size_t nblocks = (size_t)s.rows * s.cols / block_elems(s.ggml_type);
        hipLaunchKernelGGL(synth_blocks_kernel, dim3((unsigned)((nblocks + 127) / 128)), dim3(128), 0, stream, s, scale,
                           out, nblocks, block_bytes(s.ggml_type));
    }
    return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "synth launch");
}

} // namespace aq

using namespace aq;

extern "C" {

int aq_synth_host(const aq_synth_spec *spec, void *ggml_out, int threads) {
    int rc = check_spec(spec);
    if (rc) return rc;
    AQ_REQUIRE(ggml_out, "aq_synth_host: null output");
    const aq_synth_spec s = *spec;
    const float scale = synth_scale(s);
    unsigned nt = threads > 0 ? (unsigned)threads : std::max(1u, std::thread::hardware_concurrency());
    if (s.ggml_type == AQ_TYPE_F32) {
        float *o = (float *)ggml_out;
        const size_t n = (size_t)s.rows * s.cols;
        for (size_t i = 0; i < n; i++) o[i] = synth_value(s, i, scale);
        return 0;
    }
    const size_t nblocks = (size_t)s.rows * s.cols / block_elems(s.ggml_type);
    const int bb = block_bytes(s.ggml_type);
    nt = (unsigned)std::min<size_t>(nt, std::max<size_t>(1, nblocks / 64));
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < nt; t++)
        pool.emplace_back([&, t]() {
            const size_t a = nblocks * t / nt, b = nblocks * (t + 1) / nt;
            for (size_t i = a; i < b; i++) synth_block(s, i, scale, (uint8_t *)ggml_out + i * bb);
        });
    for (auto &th : pool) th.join();
    return 0;
}

int aq_weight_synth(aq_ctx *ctx, const aq_synth_spec *spec, aq_weight **out) {
    AQ_REQUIRE(ctx && out, "aq_weight_synth: null argument");
    int rc = check_spec(spec);
    if (rc) return rc;
    AQ_HIP(hipSetDevice(ctx->device));
    const size_t bytes = (size_t)spec->rows * (spec->cols / block_elems(spec->ggml_type)) * block_bytes(spec->ggml_type);
    void *tmp = nullptr;
    if (dev_malloc(&tmp, bytes) != hipSuccess) return fail(AQ_ENOMEM, "aq_weight_synth: staging");
    rc = synth_device(*spec, (uint8_t *)tmp, ctx->stream);
    aq_weight *w = nullptr;
    if (rc == 0) {
        w = new aq_weight();
        w->ctx = ctx;
        rc = weight_from_ggml(w->w, spec->ggml_type, spec->rows, spec->cols, tmp, true, ctx->device, ctx->stream);
    }
    if (hipStreamSynchronize(ctx->stream) != hipSuccess && rc == 0) rc = fail(AQ_EHIP, "aq_weight_synth: sync");
    (void)hipFree(tmp);
    if (rc) {
        if (w) {
            free_weight(w->w);
            delete w;
        }
        return rc;
    }
    *out = w;
    return 0;
}

} // extern "C"
