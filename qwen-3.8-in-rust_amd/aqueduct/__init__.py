"""Python binding of libaq.so, the MI355X speculative-decode library (C-ABI in include/aq.h).

Mirrors the reference engine's operator and model entry points (crates/core/src/kernels/matvec.rs, model.rs,
spec.rs) for tests and benchmarks. There is no fallback: if libaq.so is missing or the device is not a gfx950
GPU, every call raises AqError.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libaq.so")

F32, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 2, 8, 12, 13, 14
BLOCK = {F32: (1, 4), Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}


# status codes of include/aq.h
AQ_EINVAL, AQ_EHIP, AQ_ENOMEM, AQ_EUNSUP, AQ_ESTATE = -1, -2, -3, -4, -5


class AqError(RuntimeError):
    """A failed libaq call; `code` is its AQ_E* status."""

    def __init__(self, msg, code=None):
        super().__init__(msg)
        self.code = code


def row_bytes(t, cols):
    bs, ts = BLOCK[t]
    return cols // bs * ts


class AqTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("ggml_type", C.c_int32), ("rows", C.c_int64), ("cols", C.c_int64),
                ("data", C.c_void_p), ("nbytes", C.c_size_t)]


class AqModelConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("n_layer", "hidden", "ffn", "vocab", "n_head", "n_head_kv", "head_dim",
                                          "rope_dim")] + [("rope_theta", C.c_float), ("rms_eps", C.c_float)] + \
               [(n, C.c_uint32) for n in ("full_attention_interval", "dn_n_k_heads", "dn_n_v_heads", "dn_head_dim_k",
                                          "dn_head_dim_v", "dn_conv_kernel", "has_mtp")]


class AqSpecStats(C.Structure):
    _fields_ = [("rounds", C.c_uint64), ("drafted", C.c_uint64), ("accepted", C.c_uint64), ("emitted", C.c_uint64),
                ("hist", C.c_uint64 * 17), ("verify_ms", C.c_double), ("commit_ms", C.c_double),
                ("refeed_ms", C.c_double), ("chain_ms", C.c_double)]


_lib = None


def source_hash():
    """The stamp a library built from the sources beside this package carries (build_lib.source_hash)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("aq_build_lib", os.path.join(os.path.dirname(HERE), "build_lib.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.source_hash()


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise AqError(f"{LIB_PATH} is not built: run __graft_entry__.build() (hipcc, gfx950)")
    L = C.CDLL(LIB_PATH)
    L.aq_build_hash.restype = C.c_char_p
    L.aq_build_hash.argtypes = []
    built, want = L.aq_build_hash().decode(), source_hash()
    if built != want:
        raise AqError(f"{LIB_PATH} was built from other sources (stamp {built}, sources {want}): rebuild it with "
                      "__graft_entry__.build()")
    P, sz, i = C.c_void_p, C.c_size_t, C.c_int
    sigs = {
        "aq_last_error": (C.c_char_p, []),
        "aq_device_count": (i, [C.POINTER(C.c_int)]),
        "aq_init": (i, [i, C.POINTER(P)]),
        "aq_ctx_free": (i, [P]),
        "aq_synchronize": (i, [P]),
        "aq_dev_alloc": (i, [P, sz, C.POINTER(P)]),
        "aq_dev_free": (i, [P, P]),
        "aq_memcpy_htod": (i, [P, P, P, sz]),
        "aq_memcpy_dtoh": (i, [P, P, P, sz]),
        "aq_memcpy_dtod": (i, [P, P, P, sz]),
        "aq_weight_upload": (i, [P, i, sz, sz, P, C.POINTER(P)]),
        "aq_weight_free": (i, [P]),
        "aq_weight_download": (i, [P, P]),
        "aq_act_new": (i, [P, sz, sz, C.POINTER(P)]),
        "aq_act_free": (i, [P]),
        "aq_act_set_f32": (i, [P, P, sz]),
        "aq_act_quantize": (i, [P, i, sz]),
        "aq_act_get_q8k": (i, [P, P, sz]),
        "aq_act_get_q8_0": (i, [P, P, sz]),
        "aq_matmul": (i, [P, P, P, sz, P]),
        "aq_kq_isums": (i, [P, P, P, sz, P, P]),
        "aq_sampler_new": (i, [P, P, C.c_uint32, C.POINTER(P)]),
        "aq_sampler_free": (i, [P]),
        "aq_sampler_reseed": (i, [P, C.c_uint64]),
        "aq_sampler_get_rng": (i, [P, P]),
        "aq_sampler_process": (i, [P, P, C.POINTER(C.c_uint32)]),
        "aq_sampler_kept": (i, [P, P, P, sz, C.POINTER(sz)]),
        "aq_sampler_draw": (i, [P, C.POINTER(C.c_uint32)]),
        "aq_sampler_sample": (i, [P, P, C.POINTER(C.c_uint32)]),
        "aq_sampler_write_dense": (i, [P, P]),
        "aq_sampler_accept_or_resample": (i, [P, P, P, C.c_uint32, C.POINTER(C.c_int), C.POINTER(C.c_uint32)]),
        "aq_prefill_sampled": (i, [P, P, P, sz, P, P]),
        "aq_forward_token_sampled": (i, [P, P, C.c_uint32, P, P]),
        "aq_spec_prefill_sampled": (i, [P, P, P, sz, P]),
        "aq_spec_round_sampled": (i, [P, P, C.c_uint32, P, P, P]),
        "aq_alloc_counts": (i, [C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
        "aq_set_q8_fine": (i, [i]),
        "aq_q8_fine": (i, []),
        "aq_argmax": (i, [P, P, sz, sz, P]),
        "aq_argmax_noalloc": (i, [P, P, sz, sz, P]),
        "aq_gguf_open": (i, [C.c_char_p, C.POINTER(P)]),
        "aq_gguf_close": (i, [P]),
        "aq_gguf_info": (i, [P, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                             C.POINTER(C.c_uint64)]),
        "aq_gguf_tensor": (i, [P, C.c_uint64, C.POINTER(C.c_char_p), C.POINTER(C.c_int32), C.POINTER(C.c_int64),
                               C.POINTER(C.c_int64), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), C.POINTER(P)]),
        "aq_gguf_get_u32": (i, [P, C.c_char_p, C.POINTER(C.c_uint32)]),
        "aq_gguf_get_f32": (i, [P, C.c_char_p, C.POINTER(C.c_float)]),
        "aq_gguf_get_str": (i, [P, C.c_char_p, C.POINTER(C.c_char_p)]),
        "aq_gguf_model_config": (i, [P, P]),
        "aq_model_load_gguf": (i, [P, C.c_char_p, C.POINTER(P), P]),
        "aq_gguf_layout": (i, [P, sz, C.c_uint32, P]),
        "aq_gguf_write_synth": (i, [C.c_char_p, P, i, C.c_uint64, i]),
        "aq_matmul_time": (i, [P, P, sz, P, sz, P, i, C.POINTER(C.c_double)]),
        "aq_matmul_time_each": (i, [P, P, sz, P, sz, P, i, P]),
        "aq_read_floor_time": (i, [P, P, sz, sz, P, i, C.POINTER(C.c_double)]),
        "aq_act_quantize_on": (i, [P, i, sz, P]),
        "aq_matmul_on": (i, [P, P, P, sz, P, P]),
        "aq_synth_host": (i, [P, P, i]),
        "aq_weight_synth": (i, [P, P, C.POINTER(P)]),
        "aq_model_plan": (i, [P, i, C.c_uint64, P, sz, C.POINTER(sz)]),
        "aq_model_load": (i, [P, P, P, sz, C.POINTER(P)]),
        "aq_model_synth": (i, [P, P, i, C.c_uint64, C.POINTER(P)]),
        "aq_model_free": (i, [P]),
        "aq_model_get_bytes": (i, [P, P]),
        "aq_state_new": (i, [P, C.c_uint32, C.c_uint32, C.POINTER(P)]),
        "aq_state_free": (i, [P]),
        "aq_prefill": (i, [P, P, sz, P, P]),
        "aq_forward_token": (i, [P, C.c_uint32, P, P]),
        "aq_spec_prefill": (i, [P, P, sz, P]),
        "aq_spec_round": (i, [P, C.c_uint32, P, P, P]),
        "aq_spec_set_drafts": (i, [P, P, sz]),
        "aq_spec_get_drafts": (i, [P, P, sz]),
        "aq_spec_logits_row": (i, [P, sz, P]),
        "aq_spec_get_stats": (i, [P, P]),
        "aq_state_pos": (i, [P, P]),
        "aq_state_export": (i, [P, P, sz, C.POINTER(sz)]),
        "aq_layer_run": (i, [P, P, P, sz, i, P, sz, C.c_uint32, P, P, P, P, P, C.c_uint32, P]),
        "aq_eval_math": (i, [P, i, P, P, sz]),
        "aq_deltanet_verify_commit": (i, [P, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, sz, sz, P, P, P, P, P,
                                          P, P]),
        "aq_deltanet_verify_commit_dev": (i, [P, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, sz, sz, P, P, P, P,
                                              P, P, P]),
    }
    for name, (res, args) in sigs.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def check(rc):
    if rc != 0:
        raise AqError(f"libaq error {rc}: {lib().aq_last_error().decode()}", rc)


def ptr(a):
    return None if a is None else a.ctypes.data


class Context:
    """aq_ctx: one device, one HIP stream."""

    def __init__(self, device=0):
        h = C.c_void_p()
        check(lib().aq_init(device, C.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().aq_ctx_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def sync(self):
        check(lib().aq_synchronize(self.h))


class DeviceBuffer:
    def __init__(self, ctx: Context, nbytes):
        self.ctx = ctx
        self.nbytes = nbytes
        p = C.c_void_p()
        check(lib().aq_dev_alloc(ctx.h, nbytes, C.byref(p)))
        self.p = p

    def free(self):
        if getattr(self, "p", None):
            lib().aq_dev_free(self.ctx.h, self.p)
            self.p = None

    def __del__(self):
        self.free()

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        check(lib().aq_memcpy_htod(self.ctx.h, self.p, ptr(arr), arr.nbytes))

    def copy_from(self, other, nbytes):
        check(lib().aq_memcpy_dtod(self.ctx.h, self.p, other.p, nbytes))

    def download(self, dtype, count):
        out = np.zeros(count, dtype)
        check(lib().aq_memcpy_dtoh(self.ctx.h, ptr(out), self.p, out.nbytes))
        return out


class Weight:
    """A weight matrix on the device (the reference's WeightMat, matvec.rs:49-119)."""

    def __init__(self, ctx: Context, ggml_type, rows, cols, data):
        data = np.ascontiguousarray(data, dtype=np.uint8) if ggml_type != F32 else \
            np.ascontiguousarray(data).view(np.uint8)
        assert data.nbytes == rows * row_bytes(ggml_type, cols)
        self.ctx, self.type, self.rows, self.cols = ctx, ggml_type, rows, cols
        h = C.c_void_p()
        check(lib().aq_weight_upload(ctx.h, ggml_type, rows, cols, ptr(data), C.byref(h)))
        self.h = h

    def free(self):
        if getattr(self, "h", None):
            lib().aq_weight_free(self.h)
            self.h = None

    def __del__(self):
        self.free()

    def download(self):
        out = np.zeros(self.rows * row_bytes(self.type, self.cols), np.uint8)
        check(lib().aq_weight_download(self.h, ptr(out)))
        return out


class Act:
    """Activation rows on the device with their quantised forms (the reference's ActBuf)."""

    def __init__(self, ctx: Context, n, ncols):
        self.ctx, self.n, self.ncols = ctx, n, ncols
        h = C.c_void_p()
        check(lib().aq_act_new(ctx.h, n, ncols, C.byref(h)))
        self.h = h

    def free(self):
        if getattr(self, "h", None):
            lib().aq_act_free(self.h)
            self.h = None

    def __del__(self):
        self.free()

    def set(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, self.n)
        check(lib().aq_act_set_f32(self.h, ptr(x), x.shape[0]))
        return x.shape[0]

    def quantize(self, weight_type, ncols):
        check(lib().aq_act_quantize(self.h, weight_type, ncols))

    def q8k(self, ncols):
        out = np.zeros(ncols * self.n // 256 * 292, np.uint8)
        check(lib().aq_act_get_q8k(self.h, ptr(out), ncols))
        return out.reshape(ncols, -1)

    def q8_0(self, ncols):
        out = np.zeros(ncols * self.n // 32 * 34, np.uint8)
        check(lib().aq_act_get_q8_0(self.h, ptr(out), ncols))
        return out.reshape(ncols, -1)


def matmul(ctx: Context, w: Weight, x: Act, ncols, y: DeviceBuffer = None):
    """y[c, r] = W[r] . x[c] (matvec.rs:336 / 377); returns host f32 [ncols, rows]."""
    own = y is None
    if own:
        y = DeviceBuffer(ctx, ncols * w.rows * 4)
    check(lib().aq_matmul(ctx.h, w.h, x.h, ncols, y.p))
    out = y.download(np.float32, ncols * w.rows).reshape(ncols, w.rows)
    if own:
        y.free()
    return out


class AqSamplerConfig(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float), ("min_p", C.c_float),
                ("seed", C.c_uint64)]


def sampler_config(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, seed=0):
    return AqSamplerConfig(temperature, top_k, top_p, min_p, seed)


class Sampler:
    """aq_sampler: the reference's Sampler (sample.rs:148-303) on the device."""

    def __init__(self, ctx: Context, cfg, vocab):
        self.ctx, self.cfg, self.vocab = ctx, cfg, vocab
        h = C.c_void_p()
        check(lib().aq_sampler_new(ctx.h, C.byref(cfg), vocab, C.byref(h)))
        self.h = h

    def free(self):
        if getattr(self, "h", None):
            lib().aq_sampler_free(self.h)
            self.h = None

    def __del__(self):
        self.free()

    def reseed(self, seed):
        check(lib().aq_sampler_reseed(self.h, seed))

    def rng(self):
        out = np.zeros(4, np.uint64)
        check(lib().aq_sampler_get_rng(self.h, ptr(out)))
        return out

    def process(self, logits: DeviceBuffer):
        n = C.c_uint32()
        check(lib().aq_sampler_process(self.h, logits.p, C.byref(n)))
        return self.kept()

    def kept(self):
        n = C.c_size_t()
        check(lib().aq_sampler_kept(self.h, None, None, 0, C.byref(n)))
        ids, probs = np.zeros(n.value, np.uint32), np.zeros(n.value, np.float32)
        check(lib().aq_sampler_kept(self.h, ptr(ids), ptr(probs), n.value, C.byref(n)))
        return ids, probs

    def draw(self):
        t = C.c_uint32()
        check(lib().aq_sampler_draw(self.h, C.byref(t)))
        return t.value

    def sample(self, logits: DeviceBuffer):
        t = C.c_uint32()
        check(lib().aq_sampler_sample(self.h, logits.p, C.byref(t)))
        return t.value

    def write_dense(self, out: DeviceBuffer):
        check(lib().aq_sampler_write_dense(self.h, out.p))

    def accept_or_resample(self, target: DeviceBuffer, q: DeviceBuffer, d):
        ok, t = C.c_int(), C.c_uint32()
        check(lib().aq_sampler_accept_or_resample(self.h, target.p, q.p, d, C.byref(ok), C.byref(t)))
        return bool(ok.value), t.value


def alloc_counts():
    """(device allocations, pinned host allocations) the library has made so far (aq_alloc_counts)."""
    d, h = C.c_uint64(), C.c_uint64()
    check(lib().aq_alloc_counts(C.byref(d), C.byref(h)))
    return d.value, h.value


class q8_fine:
    """The q8-fine switch (aq_set_q8_fine; matvec.rs:133 `set_q8_fine`) on inside the block, restored after."""

    def __init__(self, on=True):
        self.on = on

    def __enter__(self):
        self.prev = lib().aq_q8_fine()
        check(lib().aq_set_q8_fine(1 if self.on else 0))
        return self

    def __exit__(self, *exc):
        check(lib().aq_set_q8_fine(self.prev))


def kq_isums(ctx: Context, w: Weight, x: Act, ncols=1):
    """The kernel's exact integers (aq_kq_isums): lanes [ncols, rows, nb, 8], mins [ncols, rows, nb, 4]."""
    nb = w.cols // 256
    lanes = DeviceBuffer(ctx, ncols * w.rows * nb * 8 * 4)
    mins = DeviceBuffer(ctx, ncols * w.rows * nb * 4 * 4)
    check(lib().aq_kq_isums(ctx.h, w.h, x.h, ncols, lanes.p, mins.p))
    return (lanes.download(np.int32, ncols * w.rows * nb * 8).reshape(ncols, w.rows, nb, 8),
            mins.download(np.int32, ncols * w.rows * nb * 4).reshape(ncols, w.rows, nb, 4))


def argmax(ctx: Context, x):
    """Per-row argmax on the device (aq_argmax, model.rs:505-513): x [t, n] f32 -> t ids."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    t, n = x.shape
    xb = DeviceBuffer(ctx, x.nbytes)
    ib = DeviceBuffer(ctx, t * 4)
    xb.upload(x)
    check(lib().aq_argmax(ctx.h, xb.p, n, t, ib.p))
    return ib.download(np.uint32, t).tolist()


def matmul_time(ctx: Context, ws, x: Act, ncols, y: DeviceBuffer, iters):
    arr = (C.c_void_p * len(ws))(*[w.h.value for w in ws])
    us = C.c_double()
    check(lib().aq_matmul_time(ctx.h, arr, len(ws), x.h, ncols, y.p, iters, C.byref(us)))
    return us.value


def matmul_time_each(ctx: Context, ws, x: Act, ncols, y: DeviceBuffer, iters):
    """Per-launch device times (us) of `iters` launches cycling over `ws` (aq_matmul_time_each)."""
    arr = (C.c_void_p * len(ws))(*[w.h.value for w in ws])
    out = np.zeros(iters, np.float32)
    check(lib().aq_matmul_time_each(ctx.h, arr, len(ws), x.h, ncols, y.p, iters, ptr(out)))
    return out


def quantize_on(a, weight_type, ncols, stream):
    """aq_act_quantize on a caller's HIP stream (an integer hipStream_t, e.g. torch.cuda.Stream().cuda_stream),
    queued without waiting."""
    check(lib().aq_act_quantize_on(a.h, weight_type, ncols, C.c_void_p(stream)))


def matmul_on(ctx: Context, w, a, ncols, y: DeviceBuffer, stream):
    """aq_matmul into the device buffer y on a caller's HIP stream, queued without waiting."""
    check(lib().aq_matmul_on(ctx.h, w.h, a.h, ncols, y.p, C.c_void_p(stream)))


def read_floor_time(ctx: Context, nbytes, iters=1000, nbuf=8):
    """Mean device time (us) of a plain streaming read of `nbytes` (rounded down to 16), cycling over `nbuf`
    buffers so the 256 MB MALL cannot serve it (aq_read_floor_time): the least time any kernel needs to read that
    many bytes on this device."""
    nbytes = nbytes // 16 * 16
    bufs = [DeviceBuffer(ctx, nbytes) for _ in range(nbuf)]
    part = DeviceBuffer(ctx, 2048 * 4)
    arr = (C.c_void_p * nbuf)(*[b.p.value for b in bufs])
    us = C.c_double()
    check(lib().aq_read_floor_time(ctx.h, arr, nbuf, nbytes, part.p, 50, C.byref(us)))  # warm-up
    check(lib().aq_read_floor_time(ctx.h, arr, nbuf, nbytes, part.p, iters, C.byref(us)))
    for b in bufs:
        b.free()
    part.free()
    return us.value


class AqSynthSpec(C.Structure):
    _fields_ = [("ggml_type", C.c_int32), ("rows", C.c_int64), ("cols", C.c_int64), ("seed", C.c_uint64),
                ("dist", C.c_uint32), ("a", C.c_float), ("b", C.c_float)]


NORMAL, UNIFORM, CONST = 0, 1, 2


def synth_spec(ggml_type, rows, cols, seed, dist=NORMAL, a=0.0, b=0.02):
    return AqSynthSpec(ggml_type, rows, cols, seed, dist, a, b)


def synth_host(spec: AqSynthSpec, threads=0):
    """ggml bytes of a synthetic tensor (aq_synth_host); F32 comes back as float32."""
    n = spec.rows * row_bytes(spec.ggml_type, spec.cols)
    out = np.zeros(n, np.uint8)
    check(lib().aq_synth_host(C.byref(spec), ptr(out), threads))
    return out.view(np.float32) if spec.ggml_type == F32 else out


class SynthWeight(Weight):
    """A synthetic weight generated directly on the device (aq_weight_synth)."""

    def __init__(self, ctx: Context, spec: AqSynthSpec):
        self.ctx, self.type, self.rows, self.cols = ctx, spec.ggml_type, spec.rows, spec.cols
        h = C.c_void_p()
        check(lib().aq_weight_synth(ctx.h, C.byref(spec), C.byref(h)))
        self.h = h


def device_count():
    n = C.c_int()
    check(lib().aq_device_count(C.byref(n)))
    return n.value


# ------------------------------------------------------------------------------------------------ model level
MIX_Q4_K_M, MIX_TINY = 0, 1


class AqTensorPlan(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("spec", AqSynthSpec)]


class AqModelBytes(C.Structure):
    _fields_ = [("main", C.c_uint64), ("mtp_block", C.c_uint64), ("lm_head", C.c_uint64), ("embed_row", C.c_uint64)]


def config(**kw):
    c = AqModelConfig()
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def tiny_config():
    """The tiny hybrid of the correctness config: 3 DeltaNet layers + 1 attention layer + the MTP block."""
    return config(n_layer=4, hidden=256, ffn=768, vocab=4096, n_head=4, n_head_kv=2, head_dim=64, rope_dim=16,
                  rope_theta=1e7, rms_eps=1e-6, full_attention_interval=4, dn_n_k_heads=2, dn_n_v_heads=4,
                  dn_head_dim_k=64, dn_head_dim_v=64, dn_conv_kernel=4, has_mtp=1)


def config_27b():
    """The 27B hybrid's shapes (docs/model-facts.md:22-123 of the reference)."""
    return config(n_layer=64, hidden=5120, ffn=17408, vocab=248320, n_head=24, n_head_kv=4, head_dim=256,
                  rope_dim=64, rope_theta=1e7, rms_eps=1e-6, full_attention_interval=4, dn_n_k_heads=16,
                  dn_n_v_heads=48, dn_head_dim_k=128, dn_head_dim_v=128, dn_conv_kernel=4, has_mtp=1)


def model_plan(cfg, mix, seed):
    """[(name, AqSynthSpec)] of a synthetic model (aq_model_plan)."""
    n = C.c_size_t()
    check(lib().aq_model_plan(C.byref(cfg), mix, seed, None, 0, C.byref(n)))
    arr = (AqTensorPlan * n.value)()
    check(lib().aq_model_plan(C.byref(cfg), mix, seed, arr, n.value, C.byref(n)))
    return [(e.name.decode(), AqSynthSpec(e.spec.ggml_type, e.spec.rows, e.spec.cols, e.spec.seed, e.spec.dist,
                                          e.spec.a, e.spec.b)) for e in arr]


def plan_tensors(plan, threads=0):
    """Host ggml bytes of every plan entry: [(name, type, rows, cols, data)]."""
    return [(name, sp.ggml_type, sp.rows, sp.cols, synth_host(sp, threads)) for name, sp in plan]


def tensor_table(tensors):
    arr = (AqTensor * len(tensors))()
    keep = []
    for i, (name, t, rows, cols, data) in enumerate(tensors):
        data = np.ascontiguousarray(data)
        nb = name.encode()
        keep += [nb, data]
        arr[i] = AqTensor(nb, t, rows, cols, data.ctypes.data, data.nbytes)
    return arr, keep


class Model:
    """aq_model: the whole model resident in device memory (the reference's Model, model.rs)."""

    def __init__(self, ctx: Context, cfg, tensors=None, mix=None, seed=None):
        self.ctx, self.cfg = ctx, cfg
        h = C.c_void_p()
        if tensors is not None:
            table, keep = tensor_table(tensors)
            check(lib().aq_model_load(ctx.h, C.byref(cfg), table, len(tensors), C.byref(h)))
        else:
            check(lib().aq_model_synth(ctx.h, C.byref(cfg), mix, seed, C.byref(h)))
        self.h = h

    def free(self):
        if getattr(self, "h", None):
            lib().aq_model_free(self.h)
            self.h = None

    def __del__(self):
        self.free()

    def bytes(self):
        b = AqModelBytes()
        check(lib().aq_model_get_bytes(self.h, C.byref(b)))
        return {"main": b.main, "mtp_block": b.mtp_block, "lm_head": b.lm_head, "embed_row": b.embed_row}


class State:
    """aq_state: one sequence (the reference's State + spec buffers, model.rs / spec.rs)."""

    def __init__(self, model: Model, spec_k=0, max_pos=512):
        self.model, self.k = model, spec_k
        h = C.c_void_p()
        check(lib().aq_state_new(model.h, spec_k, max_pos, C.byref(h)))
        self.h = h

    def free(self):
        if getattr(self, "h", None):
            lib().aq_state_free(self.h)
            self.h = None

    def __del__(self):
        self.free()

    @property
    def pos(self):
        p = C.c_uint32()
        check(lib().aq_state_pos(self.h, C.byref(p)))
        return p.value

    def forward_token(self, tok, want_logits=False, sampler=None):
        lg = np.zeros(self.model.cfg.vocab, np.float32) if want_logits else None
        a = C.c_uint32()
        if sampler is None:
            check(lib().aq_forward_token(self.h, tok, ptr(lg), C.byref(a)))
        else:
            check(lib().aq_forward_token_sampled(self.h, sampler.h, tok, ptr(lg), C.byref(a)))
        return (a.value, lg) if want_logits else a.value

    def prefill(self, ids, want_logits=False, sampler=None):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        lg = np.zeros(self.model.cfg.vocab, np.float32) if want_logits else None
        a = C.c_uint32()
        if sampler is None:
            check(lib().aq_prefill(self.h, ptr(ids), ids.size, ptr(lg), C.byref(a)))
        else:
            check(lib().aq_prefill_sampled(self.h, sampler.h, ptr(ids), ids.size, ptr(lg), C.byref(a)))
        return (a.value, lg) if want_logits else a.value

    def spec_prefill(self, ids, sampler=None):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        x = C.c_uint32()
        if sampler is None:
            check(lib().aq_spec_prefill(self.h, ptr(ids), ids.size, C.byref(x)))
        else:
            check(lib().aq_spec_prefill_sampled(self.h, sampler.h, ptr(ids), ids.size, C.byref(x)))
        return x.value

    def spec_round(self, x_p, sampler=None):
        em = np.zeros(self.k + 1, np.uint32)
        n, m = C.c_uint32(), C.c_uint32()
        if sampler is None:
            check(lib().aq_spec_round(self.h, x_p, ptr(em), C.byref(n), C.byref(m)))
        else:
            check(lib().aq_spec_round_sampled(self.h, sampler.h, x_p, ptr(em), C.byref(n), C.byref(m)))
        return m.value, em[: n.value].tolist()

    def set_drafts(self, d):
        d = np.ascontiguousarray(d, dtype=np.uint32)
        check(lib().aq_spec_set_drafts(self.h, ptr(d), d.size))

    def drafts(self):
        d = np.zeros(self.k, np.uint32)
        check(lib().aq_spec_get_drafts(self.h, ptr(d), self.k))
        return d.tolist()

    def logits_row(self, i):
        out = np.zeros(self.model.cfg.vocab, np.float32)
        check(lib().aq_spec_logits_row(self.h, i, ptr(out)))
        return out

    def stats(self):
        st = AqSpecStats()
        check(lib().aq_spec_get_stats(self.h, C.byref(st)))
        return {"rounds": st.rounds, "drafted": st.drafted, "accepted": st.accepted, "emitted": st.emitted,
                "hist": list(st.hist), "verify_ms": st.verify_ms, "commit_ms": st.commit_ms,
                "refeed_ms": st.refeed_ms, "chain_ms": st.chain_ms}

    def export(self):
        n = C.c_size_t()
        check(lib().aq_state_export(self.h, None, 0, C.byref(n)))
        out = np.zeros(n.value, np.float32)
        check(lib().aq_state_export(self.h, ptr(out), out.size, C.byref(n)))
        return out


def layer_run(ctx: Context, cfg, tensors, kind, x, start_pos, conv=None, rec=None, k_cache=None, v_cache=None,
              kv_len=0, kv_cap=0):
    """One decoder piece (aq_layer_run); conv/rec/k_cache/v_cache are updated in place. Returns (y, kv_len)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    t = x.shape[0]
    y = np.zeros_like(x)
    table, keep = tensor_table(tensors)
    kl = C.c_uint32(kv_len)
    check(lib().aq_layer_run(ctx.h, C.byref(cfg), table, len(tensors), kind, ptr(x), t, start_pos, ptr(conv),
                             ptr(rec), ptr(k_cache), ptr(v_cache), C.byref(kl), kv_cap, ptr(y)))
    return y, kl.value


def deltanet_verify_commit(ctx: Context, nk, nv, dk, dv, keep, q, k, v, g, beta, state: DeviceBuffer):
    """The isolated recurrence with rollback (aq_deltanet_verify_commit): returns out [t, nv*dv]."""
    q, k, v, g, beta = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v, g, beta))
    t = q.shape[0]
    out = np.zeros((t, nv * dv), np.float32)
    check(lib().aq_deltanet_verify_commit(ctx.h, nk, nv, dk, dv, t, keep, ptr(q), ptr(k), ptr(v), ptr(g), ptr(beta),
                                          state.p, ptr(out)))
    return out


def deltanet_verify_commit_dev(ctx: Context, nk, nv, dk, dv, t, keep, q, k, v, g, beta, state, out):
    """aq_deltanet_verify_commit_dev: the same on DeviceBuffers (q, k, v, g, beta, state, out), nothing allocated."""
    check(lib().aq_deltanet_verify_commit_dev(ctx.h, nk, nv, dk, dv, t, keep, q.p, k.p, v.p, g.p, beta.p, state.p,
                                              out.p))


def eval_math(ctx: Context, fn, x):
    """The device's activations elementwise (aq_eval_math): fn 0 exp, 1 log1p, 2 silu, 3 sigmoid, 4 softplus."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros_like(x)
    check(lib().aq_eval_math(ctx.h, fn, ptr(x), ptr(y), x.size))
    return y


# ------------------------------------------------------------------------------------------------ GGUF files
class Gguf:
    """A GGUF v3 file (aq_gguf_open): metadata reads, the tensor index, the derived model config."""

    def __init__(self, path):
        h = C.c_void_p()
        check(lib().aq_gguf_open(os.fsencode(path), C.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().aq_gguf_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def info(self):
        a, d, nt, nk = C.c_uint32(), C.c_uint64(), C.c_uint64(), C.c_uint64()
        check(lib().aq_gguf_info(self.h, C.byref(a), C.byref(d), C.byref(nt), C.byref(nk)))
        return {"alignment": a.value, "data_offset": d.value, "n_tensors": nt.value, "n_kv": nk.value}

    def tensors(self, with_data=False):
        """[(name, type, rows, cols, rel_offset, nbytes[, bytes])] in file order."""
        out = []
        for i in range(self.info()["n_tensors"]):
            nm, t, r, c, off, nb, dp = (C.c_char_p(), C.c_int32(), C.c_int64(), C.c_int64(), C.c_uint64(),
                                        C.c_uint64(), C.c_void_p())
            check(lib().aq_gguf_tensor(self.h, i, C.byref(nm), C.byref(t), C.byref(r), C.byref(c), C.byref(off),
                                       C.byref(nb), C.byref(dp)))
            e = (nm.value.decode(), t.value, r.value, c.value, off.value, nb.value)
            if with_data:
                e += (np.ctypeslib.as_array((C.c_uint8 * nb.value).from_address(dp.value)).copy(),)
            out.append(e)
        return out

    def get_u32(self, key):
        v = C.c_uint32()
        check(lib().aq_gguf_get_u32(self.h, key.encode(), C.byref(v)))
        return v.value

    def get_f32(self, key):
        v = C.c_float()
        check(lib().aq_gguf_get_f32(self.h, key.encode(), C.byref(v)))
        return v.value

    def get_str(self, key):
        v = C.c_char_p()
        check(lib().aq_gguf_get_str(self.h, key.encode(), C.byref(v)))
        return v.value.decode()

    def model_config(self):
        c = AqModelConfig()
        check(lib().aq_gguf_model_config(self.h, C.byref(c)))
        return c


def gguf_write_synth(path, cfg, mix, seed, threads=0):
    check(lib().aq_gguf_write_synth(os.fsencode(path), C.byref(cfg), mix, seed, threads))


def gguf_layout(plan_entries, alignment=32):
    """Data-section offsets of [(name, AqSynthSpec)] written in this order."""
    arr = (AqTensorPlan * len(plan_entries))()
    for i, (name, sp) in enumerate(plan_entries):
        arr[i].name = name.encode()
        arr[i].spec = sp
    out = np.zeros(len(plan_entries), np.uint64)
    check(lib().aq_gguf_layout(arr, len(plan_entries), alignment, ptr(out)))
    return out


def model_load_gguf(ctx: Context, path):
    """(Model, config) of a GGUF file (aq_model_load_gguf)."""
    m = Model.__new__(Model)
    m.ctx = ctx
    cfg = AqModelConfig()
    h = C.c_void_p()
    check(lib().aq_model_load_gguf(ctx.h, os.fsencode(path), C.byref(h), C.byref(cfg)))
    m.h, m.cfg = h, cfg
    return m, cfg
