// runtime.hip — lifecycle, device memory, weights, activation buffers and the operator-level C-ABI
// (include/aq.h). Every entry point validates its arguments and returns an AQ_E* code instead of aborting.
#include <atomic>
#include <cstring>
#include <mutex>
#include <vector>

#include "aq_common.h"
#include "ops.h"

namespace aq {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }

namespace {
std::atomic<bool> g_q8_fine{false};
std::atomic<uint64_t> g_dev_allocs{0}, g_pinned_allocs{0};
} // namespace

hipError_t dev_malloc_raw(void **p, size_t bytes) {
    g_dev_allocs.fetch_add(1, std::memory_order_relaxed);
    return hipMalloc(p, bytes);
}

hipError_t pinned_malloc(void **p, size_t bytes) {
    g_pinned_allocs.fetch_add(1, std::memory_order_relaxed);
    return hipHostMalloc(p, bytes, hipHostMallocDefault);
}
bool q8_fine() { return g_q8_fine.load(std::memory_order_relaxed); }
void set_q8_fine(bool on) { g_q8_fine.store(on, std::memory_order_relaxed); }

// Every error return passes here: it also clears HIP's per-thread last error, so that a failed runtime call whose
// code this library already reported (an allocation that ran out of memory, say) is not reported again by the
// launch check of a later, unrelated call.
int fail(int code, const std::string &msg) {
    set_error(msg);
    (void)hipGetLastError();
    return code;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// The allocation-free argmax's partial results: a file-scope device array, one copy per GPU, held until the
// process ends. Rows of at most AQ_NOALLOC_MAX_N values, at most AQ_NOALLOC_MAX_ROWS rows per call.
constexpr size_t AQ_NOALLOC_MAX_N = (size_t)1 << 20, AQ_NOALLOC_MAX_ROWS = 16;
constexpr size_t AQ_NOALLOC_SCRATCH = 128 * 1024;
static __device__ __align__(256) uint8_t scratch[AQ_NOALLOC_SCRATCH];
// Its address on each device (hipGetSymbolAddress with that device current, at aq_init); host code uses these,
// never the array's name, which in host code is only a stand-in.
static std::mutex g_scratch_mu;
static std::vector<void *> g_scratch_ptr;

static int scratch_setup(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if ((size_t)device < g_scratch_ptr.size() && g_scratch_ptr[device]) return 0;
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
        return fail(AQ_EHIP, std::string("aq_init: hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    if (g_scratch_ptr.size() <= (size_t)device) g_scratch_ptr.resize(device + 1, nullptr);
    g_scratch_ptr[device] = ptr;
    return 0;
}

static void *scratch_ptr(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return (size_t)device < g_scratch_ptr.size() ? g_scratch_ptr[device] : nullptr;
}

// Allocate the planes of a weight (layouts in aq_common.h).
static int alloc_weight(Weight &w, int type, size_t rows, size_t cols, int device) {
    const int be = block_elems(type);
    AQ_REQUIRE(block_bytes(type) > 0, "weight: unsupported ggml type " + std::to_string(type));
    AQ_REQUIRE(rows > 0 && cols > 0, "weight: empty shape");
    AQ_REQUIRE(cols % be == 0, "weight: cols " + std::to_string(cols) + " is not a multiple of the block size " +
                                   std::to_string(be));
    w.type = type;
    w.rows = rows;
    w.cols = cols;
    w.nb = cols / be;
    w.device = device;
    switch (type) {
    case AQ_TYPE_Q4_K: w.qa_bytes = 128; w.qb_bytes = 0; w.sc_bytes = 16; w.dm_bytes = 0; break;
    case AQ_TYPE_Q5_K: w.qa_bytes = 128; w.qb_bytes = 32; w.sc_bytes = 16; w.dm_bytes = 0; break;
    case AQ_TYPE_Q6_K: w.qa_bytes = 128; w.qb_bytes = 64; w.sc_bytes = 16; w.dm_bytes = 2; break;
    case AQ_TYPE_Q8_0: w.qa_bytes = 32; w.qb_bytes = 0; w.sc_bytes = 0; w.dm_bytes = 2; break;
    case AQ_TYPE_Q4_0: w.qa_bytes = 16; w.qb_bytes = 0; w.sc_bytes = 0; w.dm_bytes = 2; break;
    default: w.qa_bytes = 4; w.qb_bytes = 0; w.sc_bytes = 0; w.dm_bytes = 0; break;
    }
    const size_t nbl = (is_kquant(type) ? (rows + 3) / 4 * 4 : rows) * w.nb; // K-quant tiles hold 4 rows
    const size_t sa = align256(nbl * w.qa_bytes), sb = align256(nbl * w.qb_bytes), ss = align256(nbl * w.sc_bytes),
                 sd = align256(nbl * w.dm_bytes);
    w.total = sa + sb + ss + sd;
    void *p = nullptr;
    if (dev_malloc(&p, w.total) != hipSuccess) return fail(AQ_ENOMEM, "weight: hipMalloc of " + std::to_string(w.total) + " bytes");
    w.base = (uint8_t *)p;
    w.qa = w.base;
    w.qb = w.qb_bytes ? w.base + sa : nullptr;
    w.sc = w.sc_bytes ? w.base + sa + sb : nullptr;
    w.dm = w.dm_bytes ? w.base + sa + sb + ss : nullptr;
    return 0;
}

int weight_from_ggml(Weight &w, int type, size_t rows, size_t cols, const void *ggml, bool ggml_on_device,
                     int device, hipStream_t stream) {
    int rc = alloc_weight(w, type, rows, cols, device);
    if (rc) return rc;
    const size_t bytes = rows * (cols / block_elems(type)) * block_bytes(type);
    const uint8_t *src = (const uint8_t *)ggml;
    void *tmp = nullptr;
    if (!ggml_on_device) {
        if (dev_malloc(&tmp, bytes) != hipSuccess) return fail(AQ_ENOMEM, "weight: staging hipMalloc");
        AQ_HIP(hipMemcpyAsync(tmp, ggml, bytes, hipMemcpyHostToDevice, stream));
        src = (const uint8_t *)tmp;
    }
    rc = launch_repack(w, src, true, stream);
    if (tmp) {
        AQ_HIP(hipStreamSynchronize(stream));
        AQ_HIP(hipFree(tmp));
    }
    return rc;
}

void free_weight(Weight &w) {
    if (w.base) (void)hipFree(w.base);
    w.base = nullptr;
}

int alloc_act(Act &a, size_t n, size_t ncols, int device) {
    AQ_REQUIRE(n > 0 && ncols > 0, "act: empty shape");
    a.n = n;
    a.ncols = ncols;
    a.nb = n / 256;
    a.nb32 = n / 32;
    a.device = device;
    const size_t f = align256(ncols * n * 4), q = align256(ncols * n), d = align256(ncols * a.nb * 4 + 4),
                 bs = align256(ncols * a.nb * 32 + 4), q8s = align256(ncols * a.nb * 16 + 4), q0 = align256(ncols * n),
                 d0 = align256(ncols * a.nb32 * 4), h0 = align256(ncols * a.nb32 * 2), s0 = align256(ncols * a.nb32 * 4);
    const size_t total = f + q + d + bs + q8s + q0 + d0 + h0 + s0;
    void *p = nullptr;
    if (dev_malloc(&p, total) != hipSuccess) return fail(AQ_ENOMEM, "act: hipMalloc");
    if (hipMemset(p, 0, total) != hipSuccess) return fail(AQ_EHIP, "act: hipMemset");
    // The clear runs on the null stream, which the context's non-blocking stream does not wait for.
    if (hipDeviceSynchronize() != hipSuccess) return fail(AQ_EHIP, "act: clear sync");
    uint8_t *b = (uint8_t *)p;
    a.base = p;
    a.f32 = (float *)b;
    b += f;
    a.qs = (int8_t *)b;
    b += q;
    a.d = (float *)b;
    b += d;
    a.bs = (int16_t *)b;
    b += bs;
    a.q8s = (int16_t *)b;
    b += q8s;
    a.q0 = (int8_t *)b;
    b += q0;
    a.d0 = (float *)b;
    b += d0;
    a.h0 = (uint16_t *)b;
    b += h0;
    a.s0 = (int32_t *)b;
    return 0;
}

void free_act(Act &a) {
    if (a.base) (void)hipFree(a.base);
    a.base = nullptr;
}

// The read floor (measurement only): a plain streaming read of n4 float4s, grid-stride, one partial sum per
// work-group into partials[blockIdx.x] — the least time any kernel needs to read that many bytes on the device.
constexpr int READ_FLOOR_WGS = 2048;
__global__ void __launch_bounds__(256) read_floor_kernel(const float4 *p, size_t n4, float *partials) {
    float acc = 0.0f;
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
        const float4 v = p[i];
        acc += (v.x + v.y) + (v.z + v.w);
    }
    __shared__ float red[256];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int off = 128; off >= 1; off >>= 1) {
        if ((int)threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
        __syncthreads();
    }
    if (threadIdx.x == 0) partials[blockIdx.x] = red[0];
}

} // namespace aq

using namespace aq;

// ================================================================================================== C-ABI
extern "C" {

const char *aq_last_error(void) { return g_last_error.c_str(); }

#ifndef AQ_BUILD_HASH
#define AQ_BUILD_HASH "unstamped"
#endif
const char *aq_build_hash(void) { return AQ_BUILD_HASH; }

int aq_device_count(int *out) {
    AQ_REQUIRE(out, "aq_device_count: null out");
    int n = 0;
    AQ_HIP(hipGetDeviceCount(&n));
    *out = n;
    return 0;
}

int aq_init(int device, aq_ctx **out) {
    AQ_REQUIRE(out, "aq_init: null out");
    int n = 0;
    AQ_HIP(hipGetDeviceCount(&n));
    AQ_REQUIRE(device >= 0 && device < n, "aq_init: device " + std::to_string(device) + " of " + std::to_string(n));
    AQ_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    AQ_HIP(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(AQ_EUNSUP, std::string("aq_init: this build targets gfx950, device is ") + prop.gcnArchName);
    const int rc = scratch_setup(device); // the device is current
    if (rc) return rc;
    aq_ctx *c = new aq_ctx();
    c->device = device;
    AQ_HIP(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    AQ_HIP(hipEventCreate(&c->ev0));
    AQ_HIP(hipEventCreate(&c->ev1));
    *out = c;
    return 0;
}

int aq_ctx_free(aq_ctx *ctx) {
    if (!ctx) return 0;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipEventDestroy(ctx->ev0);
    (void)hipEventDestroy(ctx->ev1);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return 0;
}

int aq_synchronize(aq_ctx *ctx) {
    AQ_REQUIRE(ctx, "aq_synchronize: null ctx");
    AQ_HIP(hipSetDevice(ctx->device));
    AQ_HIP(hipStreamSynchronize(ctx->stream));
    return 0;
}

int aq_dev_alloc(aq_ctx *ctx, size_t nbytes, void **dev_out) {
    AQ_REQUIRE(ctx && dev_out, "aq_dev_alloc: null argument");
    AQ_HIP(hipSetDevice(ctx->device));
    void *p = nullptr;
    if (dev_malloc(&p, nbytes ? nbytes : 1) != hipSuccess) return fail(AQ_ENOMEM, "aq_dev_alloc");
    *dev_out = p;
    return 0;
}

int aq_dev_free(aq_ctx *ctx, void *dev) {
    AQ_REQUIRE(ctx, "aq_dev_free: null ctx");
    if (dev) AQ_HIP(hipFree(dev));
    return 0;
}

int aq_memcpy_htod(aq_ctx *ctx, void *dev, const void *host, size_t nbytes) {
    AQ_REQUIRE(ctx && dev && host, "aq_memcpy_htod: null argument");
    AQ_HIP(hipMemcpyAsync(dev, host, nbytes, hipMemcpyHostToDevice, ctx->stream));
    AQ_HIP(hipStreamSynchronize(ctx->stream));
    return 0;
}

int aq_memcpy_dtod(aq_ctx *ctx, void *dst, const void *src, size_t nbytes) {
    AQ_REQUIRE(ctx && dst && src, "aq_memcpy_dtod: null argument");
    AQ_HIP(hipSetDevice(ctx->device));
    AQ_HIP(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToDevice, ctx->stream));
    AQ_HIP(hipStreamSynchronize(ctx->stream));
    return 0;
}

int aq_memcpy_dtoh(aq_ctx *ctx, void *host, const void *dev, size_t nbytes) {
    AQ_REQUIRE(ctx && dev && host, "aq_memcpy_dtoh: null argument");
    AQ_HIP(hipMemcpyAsync(host, dev, nbytes, hipMemcpyDeviceToHost, ctx->stream));
    AQ_HIP(hipStreamSynchronize(ctx->stream));
    return 0;
}

int aq_weight_upload(aq_ctx *ctx, int ggml_type, size_t rows, size_t cols, const void *ggml_bytes, aq_weight **out) {
    AQ_REQUIRE(ctx && ggml_bytes && out, "aq_weight_upload: null argument");
    AQ_HIP(hipSetDevice(ctx->device));
    aq_weight *w = new aq_weight();
    w->ctx = ctx;
    int rc = weight_from_ggml(w->w, ggml_type, rows, cols, ggml_bytes, false, ctx->device, ctx->stream);
    if (rc == 0) rc = hipStreamSynchronize(ctx->stream) == hipSuccess ? 0 : fail(AQ_EHIP, "aq_weight_upload: sync");
    if (rc) {
        free_weight(w->w);
        delete w;
        return rc;
    }
    *out = w;
    return 0;
}

int aq_weight_free(aq_weight *w) {
    if (!w) return 0;
    (void)hipSetDevice(w->w.device);
    free_weight(w->w);
    delete w;
    return 0;
}

int aq_weight_download(const aq_weight *w, void *ggml_bytes_out) {
    AQ_REQUIRE(w && ggml_bytes_out, "aq_weight_download: null argument");
    aq_ctx *ctx = w->ctx;
    AQ_HIP(hipSetDevice(ctx->device));
    const size_t bytes = w->w.rows * w->w.nb * block_bytes(w->w.type);
    void *tmp = nullptr;
    if (dev_malloc(&tmp, bytes) != hipSuccess) return fail(AQ_ENOMEM, "aq_weight_download: staging");
    Weight copy = w->w;
    int rc = launch_repack(copy, (const uint8_t *)tmp, false, ctx->stream);
    if (rc == 0) {
        AQ_HIP(hipMemcpyAsync(ggml_bytes_out, tmp, bytes, hipMemcpyDeviceToHost, ctx->stream));
        AQ_HIP(hipStreamSynchronize(ctx->stream));
    }
    (void)hipFree(tmp);
    return rc;
}

int aq_act_new(aq_ctx *ctx, size_t n, size_t ncols, aq_act **out) {
    AQ_REQUIRE(ctx && out, "aq_act_new: null argument");
    AQ_REQUIRE(ncols >= 1 && ncols <= 64, "aq_act_new: ncols must be 1..64");
    AQ_HIP(hipSetDevice(ctx->device));
    aq_act *a = new aq_act();
    a->ctx = ctx;
    int rc = alloc_act(a->a, n, ncols, ctx->device);
    if (rc) {
        delete a;
        return rc;
    }
    *out = a;
    return 0;
}

int aq_act_free(aq_act *a) {
    if (!a) return 0;
    (void)hipSetDevice(a->a.device);
    free_act(a->a);
    delete a;
    return 0;
}

int aq_act_set_f32(aq_act *a, const float *host, size_t ncols) {
    AQ_REQUIRE(a && host, "aq_act_set_f32: null argument");
    AQ_REQUIRE(ncols <= a->a.ncols, "aq_act_set_f32: more columns than the buffer holds");
    AQ_HIP(hipSetDevice(a->ctx->device));
    AQ_HIP(hipMemcpyAsync(a->a.f32, host, ncols * a->a.n * 4, hipMemcpyHostToDevice, a->ctx->stream));
    AQ_HIP(hipStreamSynchronize(a->ctx->stream));
    return 0;
}

static int act_quantize(aq_act *a, int weight_type, size_t ncols, hipStream_t stream) {
    AQ_REQUIRE(a, "aq_act_quantize: null act");
    AQ_REQUIRE(ncols >= 1 && ncols <= a->a.ncols, "aq_act_quantize: ncols out of range");
    AQ_HIP(hipSetDevice(a->ctx->device));
    if (is_kquant(weight_type) && !q8_fine()) {
        AQ_REQUIRE(a->a.n % 256 == 0, "aq_act_quantize: Q8_K needs n % 256 == 0 (matvec.rs:73-77)");
        return launch_q8k_quantize(a->a, ncols, a->a.f32, a->a.n, stream);
    }
    if (is_kquant(weight_type) || weight_type == AQ_TYPE_Q8_0 || weight_type == AQ_TYPE_Q4_0) {
        AQ_REQUIRE(a->a.n % 32 == 0, "aq_act_quantize: Q8_0 needs n % 32 == 0");
        return launch_q8_0_quantize(a->a, ncols, a->a.f32, a->a.n, stream);
    }
    if (weight_type == AQ_TYPE_F32) return 0;
    return fail(AQ_EUNSUP, "aq_act_quantize: unsupported weight type");
}

int aq_act_quantize(aq_act *a, int weight_type, size_t ncols) {
    return act_quantize(a, weight_type, ncols, a ? a->ctx->stream : nullptr);
}

int aq_act_quantize_on(aq_act *a, int weight_type, size_t ncols, void *stream) {
    return act_quantize(a, weight_type, ncols, stream ? (hipStream_t)stream : (a ? a->ctx->stream : nullptr));
}

int aq_act_get_q8k(const aq_act *a, void *ggml_out, size_t ncols) {
    AQ_REQUIRE(a && ggml_out, "aq_act_get_q8k: null argument");
    AQ_REQUIRE(ncols <= a->a.ncols && a->a.n % 256 == 0, "aq_act_get_q8k: shape");
    const Act &x = a->a;
    AQ_HIP(hipSetDevice(a->ctx->device));
    std::vector<int8_t> qs(ncols * x.n);
    std::vector<float> d(ncols * x.nb);
    std::vector<int16_t> bs(ncols * x.nb * 16);
    AQ_HIP(hipMemcpyAsync(qs.data(), x.qs, qs.size(), hipMemcpyDeviceToHost, a->ctx->stream));
    AQ_HIP(hipMemcpyAsync(d.data(), x.d, d.size() * 4, hipMemcpyDeviceToHost, a->ctx->stream));
    AQ_HIP(hipMemcpyAsync(bs.data(), x.bs, bs.size() * 2, hipMemcpyDeviceToHost, a->ctx->stream));
    AQ_HIP(hipStreamSynchronize(a->ctx->stream));
    uint8_t *o = (uint8_t *)ggml_out;
    for (size_t c = 0; c < ncols; c++)
        for (size_t b = 0; b < x.nb; b++) {
            uint8_t *blk = o + (c * x.nb + b) * 292;
            std::memcpy(blk, &d[c * x.nb + b], 4);
            const int8_t *src = qs.data() + c * x.n + b * 256;
            for (int s = 0; s < 8; s++)
                for (int l = 0; l < 8; l++)
                    for (int j = 0; j < 4; j++) blk[4 + 32 * s + 4 * l + j] = (uint8_t)src[lane_slot(l) * 32 + s * 4 + j];
            std::memcpy(blk + 260, &bs[(c * x.nb + b) * 16], 32);
        }
    return 0;
}

int aq_act_get_q8_0(const aq_act *a, void *ggml_out, size_t ncols) {
    AQ_REQUIRE(a && ggml_out, "aq_act_get_q8_0: null argument");
    AQ_REQUIRE(ncols <= a->a.ncols && a->a.n % 32 == 0, "aq_act_get_q8_0: shape");
    const Act &x = a->a;
    AQ_HIP(hipSetDevice(a->ctx->device));
    std::vector<int8_t> q(ncols * x.n);
    std::vector<uint16_t> h(ncols * x.nb32);
    AQ_HIP(hipMemcpyAsync(q.data(), x.q0, q.size(), hipMemcpyDeviceToHost, a->ctx->stream));
    AQ_HIP(hipMemcpyAsync(h.data(), x.h0, h.size() * 2, hipMemcpyDeviceToHost, a->ctx->stream));
    AQ_HIP(hipStreamSynchronize(a->ctx->stream));
    uint8_t *o = (uint8_t *)ggml_out;
    for (size_t i = 0; i < ncols * x.nb32; i++) {
        std::memcpy(o + i * 34, &h[i], 2);
        std::memcpy(o + i * 34 + 2, q.data() + i * 32, 32);
    }
    return 0;
}

static int check_matmul(const aq_weight *w, const aq_act *x, size_t ncols, const void *y) {
    AQ_REQUIRE(w && x && y, "aq_matmul: null argument");
    AQ_REQUIRE(x->a.n == w->w.cols, "aq_matmul: activation length " + std::to_string(x->a.n) + " != weight cols " +
                                        std::to_string(w->w.cols) + " (matvec.rs:338-339)");
    AQ_REQUIRE(ncols >= 1 && ncols <= x->a.ncols && ncols <= 64, "aq_matmul: ncols must be 1..min(64, act columns)");
    AQ_REQUIRE(w->ctx == x->ctx, "aq_matmul: weight and activation belong to different contexts");
    return 0;
}

int aq_matmul(aq_ctx *ctx, const aq_weight *w, const aq_act *x, size_t ncols, float *y_dev) {
    AQ_REQUIRE(ctx, "aq_matmul: null ctx");
    int rc = check_matmul(w, x, ncols, y_dev);
    if (rc) return rc;
    AQ_HIP(hipSetDevice(ctx->device));
    rc = launch_matmul_many(w->w, x->a, ncols, y_dev, nullptr, ctx->stream);
    if (rc) return rc;
    AQ_HIP(hipStreamSynchronize(ctx->stream));
    return 0;
}

int aq_matmul_on(aq_ctx *ctx, const aq_weight *w, const aq_act *x, size_t ncols, float *y_dev, void *stream) {
    AQ_REQUIRE(ctx, "aq_matmul_on: null ctx");
    int rc = check_matmul(w, x, ncols, y_dev);
    if (rc) return rc;
    AQ_HIP(hipSetDevice(ctx->device));
    return launch_matmul_many(w->w, x->a, ncols, y_dev, nullptr, stream ? (hipStream_t)stream : ctx->stream);
}

int aq_set_q8_fine(int on) {
    set_q8_fine(on != 0);
    return 0;
}

int aq_q8_fine(void) { return q8_fine() ? 1 : 0; }

int aq_alloc_counts(uint64_t *device_allocs, uint64_t *pinned_host_allocs) {
    if (device_allocs) *device_allocs = g_dev_allocs.load(std::memory_order_relaxed);
    if (pinned_host_allocs) *pinned_host_allocs = g_pinned_allocs.load(std::memory_order_relaxed);
    return 0;
}

int aq_kq_isums(aq_ctx *ctx, const aq_weight *w, const aq_act *x, size_t ncols, int32_t *lanes_dev,
                int32_t *mins_dev) {
    if (q8_fine()) return fail(AQ_EUNSUP, "aq_kq_isums: the integer lanes are the Q8_K kernel's; q8-fine is on");
    AQ_REQUIRE(ctx && w && x && lanes_dev && mins_dev, "aq_kq_isums: null argument");
    AQ_REQUIRE(is_kquant(w->w.type), "aq_kq_isums: K-quant weights only");
    AQ_REQUIRE(x->a.n == w->w.cols, "aq_kq_isums: activation length");
    AQ_REQUIRE(ncols >= 1 && ncols <= x->a.ncols, "aq_kq_isums: ncols");
    AQ_HIP(hipSetDevice(ctx->device));
    void *y = nullptr;
    if (dev_malloc(&y, ncols * w->w.rows * 4) != hipSuccess) return fail(AQ_ENOMEM, "aq_kq_isums: outputs");
    int rc = kq_isums_run(w->w, x->a, ncols, (float *)y, lanes_dev, mins_dev, ctx->stream);
    if (!rc && hipStreamSynchronize(ctx->stream) != hipSuccess) rc = fail(AQ_EHIP, "aq_kq_isums: sync");
    (void)hipFree(y);
    return rc;
}

int aq_argmax(aq_ctx *ctx, const float *x_dev, size_t n, size_t t, uint32_t *ids_dev) {
    AQ_REQUIRE(ctx && x_dev && ids_dev, "aq_argmax: null argument");
    AQ_REQUIRE(n >= 1 && t >= 1 && n <= 0xFFFFFFFEull, "aq_argmax: empty or over-long rows");
    AQ_HIP(hipSetDevice(ctx->device));
    void *scratch = nullptr;
    if (dev_malloc(&scratch, argmax_scratch_bytes(n, t)) != hipSuccess) return fail(AQ_ENOMEM, "aq_argmax: scratch");
    int rc = launch_argmax(x_dev, n, n, t, ids_dev, scratch, ctx->stream);
    if (!rc && hipStreamSynchronize(ctx->stream) != hipSuccess) rc = fail(AQ_EHIP, "aq_argmax: sync");
    (void)hipFree(scratch);
    return rc;
}

int aq_argmax_noalloc(aq_ctx *ctx, const float *x_dev, size_t n, size_t t, uint32_t *ids_dev) {
    AQ_REQUIRE(ctx && x_dev && ids_dev, "aq_argmax_noalloc: null argument");
    AQ_REQUIRE(n >= 1 && t >= 1, "aq_argmax_noalloc: empty rows");
    AQ_REQUIRE(n <= AQ_NOALLOC_MAX_N && t <= AQ_NOALLOC_MAX_ROWS,
               "aq_argmax_noalloc: at most " + std::to_string(AQ_NOALLOC_MAX_ROWS) + " rows of at most " +
                   std::to_string(AQ_NOALLOC_MAX_N) + " values (got " + std::to_string(t) + " x " +
                   std::to_string(n) + ")");
    static_assert((AQ_NOALLOC_MAX_ROWS * ((AQ_NOALLOC_MAX_N + 2047) / 2048) * 4 + 255) / 256 * 256 +
                          AQ_NOALLOC_MAX_ROWS * ((AQ_NOALLOC_MAX_N + 2047) / 2048) * 4 <=
                      AQ_NOALLOC_SCRATCH,
                  "the argmax partials of the largest call fit the scratch array");
    AQ_REQUIRE(argmax_scratch_bytes(n, t) <= AQ_NOALLOC_SCRATCH, "aq_argmax_noalloc: scratch too small");
    void *sp = scratch_ptr(ctx->device);
    AQ_REQUIRE(sp, "aq_argmax_noalloc: the device's scratch address is not set up (aq_init)");
    AQ_HIP(hipSetDevice(ctx->device));
    int rc = launch_argmax(x_dev, n, n, t, ids_dev, sp, ctx->stream);
    if (!rc && hipStreamSynchronize(ctx->stream) != hipSuccess) rc = fail(AQ_EHIP, "aq_argmax_noalloc: sync");
    return rc;
}

int aq_matmul_time(aq_ctx *ctx, const aq_weight *const *ws, size_t nw, const aq_act *x, size_t ncols, float *y_dev,
                   int iters, double *us_per_launch) {
    AQ_REQUIRE(ctx && ws && nw > 0 && us_per_launch && iters > 0, "aq_matmul_time: bad argument");
    for (size_t i = 0; i < nw; i++) {
        int rc = check_matmul(ws[i], x, ncols, y_dev);
        if (rc) return rc;
        AQ_REQUIRE(ws[i]->w.rows == ws[0]->w.rows, "aq_matmul_time: weights of different shapes");
    }
    AQ_HIP(hipSetDevice(ctx->device));
    AQ_HIP(hipEventRecord(ctx->ev0, ctx->stream));
    for (int i = 0; i < iters; i++) {
        int rc = launch_matmul_many(ws[i % nw]->w, x->a, ncols, y_dev, nullptr, ctx->stream);
        if (rc) return rc;
    }
    AQ_HIP(hipEventRecord(ctx->ev1, ctx->stream));
    AQ_HIP(hipEventSynchronize(ctx->ev1));
    float ms = 0.0f;
    AQ_HIP(hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1));
    *us_per_launch = (double)ms * 1000.0 / iters;
    return 0;
}

int aq_matmul_time_each(aq_ctx *ctx, const aq_weight *const *ws, size_t nw, const aq_act *x, size_t ncols, float *y_dev,
                        int iters, float *us_each) {
    AQ_REQUIRE(ctx && ws && nw > 0 && us_each && iters > 0 && iters <= 4096, "aq_matmul_time_each: bad argument");
    for (size_t i = 0; i < nw; i++) {
        int rc = check_matmul(ws[i], x, ncols, y_dev);
        if (rc) return rc;
        AQ_REQUIRE(ws[i]->w.rows == ws[0]->w.rows, "aq_matmul_time_each: weights of different shapes");
    }
    AQ_HIP(hipSetDevice(ctx->device));
    std::vector<hipEvent_t> ev((size_t)iters + 1, nullptr);
    int rc = 0;
    for (auto &e : ev)
        if (!rc && hipEventCreate(&e) != hipSuccess) rc = fail(AQ_EHIP, "aq_matmul_time_each: event");
    // one event between consecutive launches: launch i's time is the interval between events i and i + 1
    for (int i = 0; !rc && i < iters; i++) {
        if (hipEventRecord(ev[i], ctx->stream) != hipSuccess) rc = fail(AQ_EHIP, "aq_matmul_time_each: record");
        if (!rc) rc = launch_matmul_many(ws[i % nw]->w, x->a, ncols, y_dev, nullptr, ctx->stream);
    }
    if (!rc && hipEventRecord(ev[iters], ctx->stream) != hipSuccess) rc = fail(AQ_EHIP, "aq_matmul_time_each: record");
    if (!rc && hipEventSynchronize(ev[iters]) != hipSuccess) rc = fail(AQ_EHIP, "aq_matmul_time_each: sync");
    for (int i = 0; !rc && i < iters; i++) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, ev[i], ev[i + 1]) != hipSuccess) rc = fail(AQ_EHIP, "aq_matmul_time_each: time");
        us_each[i] = ms * 1000.0f;
    }
    for (auto &e : ev)
        if (e) (void)hipEventDestroy(e);
    return rc;
}

int aq_read_floor_time(aq_ctx *ctx, const void *const *bufs_dev, size_t nbuf, size_t bytes, float *partials_dev,
                       int iters, double *us_per_launch) {
    AQ_REQUIRE(ctx && bufs_dev && nbuf > 0 && partials_dev && us_per_launch && iters > 0,
               "aq_read_floor_time: bad argument");
    AQ_REQUIRE(bytes >= 16 && bytes % 16 == 0, "aq_read_floor_time: bytes must be a positive multiple of 16");
    for (size_t i = 0; i < nbuf; i++)
        AQ_REQUIRE(bufs_dev[i] && ((uintptr_t)bufs_dev[i] & 15) == 0, "aq_read_floor_time: buffers must be 16-aligned");
    AQ_HIP(hipSetDevice(ctx->device));
    const size_t n4 = bytes / 16;
    auto launch = [&](int i) {
        hipLaunchKernelGGL(read_floor_kernel, dim3(READ_FLOOR_WGS), dim3(256), 0, ctx->stream,
                           reinterpret_cast<const float4 *>(bufs_dev[(size_t)i % nbuf]), n4, partials_dev);
        return hipGetLastError() == hipSuccess ? 0 : fail(AQ_EHIP, "read_floor launch");
    };
    AQ_HIP(hipEventRecord(ctx->ev0, ctx->stream));
    for (int i = 0; i < iters; i++) {
        const int rc = launch(i);
        if (rc) return rc;
    }
    AQ_HIP(hipEventRecord(ctx->ev1, ctx->stream));
    AQ_HIP(hipEventSynchronize(ctx->ev1));
    float ms = 0.0f;
    AQ_HIP(hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1));
    *us_per_launch = (double)ms * 1000.0 / iters;
    return 0;
}

} // extern "C"
