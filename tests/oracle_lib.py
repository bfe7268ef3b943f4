"""ctypes binding of the CPU oracle (oracle/liboracle.so). Test infrastructure only: the checker, never the
thing under test. Builds the library on first use if it is missing."""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "oracle", "liboracle.so")

F32, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 2, 8, 12, 13, 14
TYPE_BY_NAME = {"F32": F32, "Q4_0": Q4_0, "Q8_0": Q8_0, "Q4_K": Q4_K, "Q5_K": Q5_K, "Q6_K": Q6_K}
BLOCK = {F32: (1, 4), Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}


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


def tensor_table(tensors):
    """tensors: list of (name, type, rows, cols, numpy uint8/float32 array). Returns (array, keepalive)."""
    arr = (AqTensor * len(tensors))()
    keep = []
    for i, (name, t, rows, cols, data) in enumerate(tensors):
        data = np.ascontiguousarray(data)
        nb = name.encode()
        keep += [nb, data]
        arr[i] = AqTensor(nb, t, rows, cols, data.ctypes.data, data.nbytes)
    return arr, keep


_lib = None


def eval_math(fn, x, restated=False):
    """fn 0 exp, 1 log1p, 2 silu, 3 sigmoid, 4 softplus: the platform libm's (the reference's arithmetic), or
    with restated=True aq_math.h's restatement (the device's arithmetic) compiled for the host."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros_like(x)
    lib().or_eval_math(fn, x.ctypes.data, y.ctypes.data, x.size, int(restated))
    return y


def math_sweep(fn, first=0, count=1 << 32, stride=1):
    """Restatement vs platform libm over f32 bit patterns first, first+stride, ...: (mismatches, first bad)."""
    fb = C.c_uint32()
    bad = lib().or_math_sweep(fn, first, count, stride, C.byref(fb))
    return int(bad), fb.value


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        import importlib.util
        spec = importlib.util.spec_from_file_location("build_oracle", os.path.join(ROOT, "oracle", "build_oracle.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    L = C.CDLL(LIB_PATH)
    P = C.c_void_p
    sz = C.c_size_t
    sigs = {
        "or_f16_to_f32": (C.c_float, [C.c_uint16]),
        "or_f32_to_f16": (C.c_uint16, [C.c_float]),
        "or_q8k_quantize": (None, [P, sz, P]),
        "or_q8_0_quantize": (None, [P, sz, P]),
        "or_dequant": (C.c_int, [C.c_int, P, sz, P]),
        "or_row_bytes": (sz, [C.c_int, sz]),
        "or_dot_q8k": (C.c_float, [C.c_int, P, P, sz]),
        "or_dot_q8k_t": (None, [C.c_int, P, P, sz, sz, P]),
        "or_kq_isums": (None, [C.c_int, P, P, sz, P, P]),
        "or_kq_isums_mat": (None, [C.c_int, P, sz, P, sz, P, P]),
        "or_dot_q8": (C.c_float, [C.c_int, P, P, sz]),
        "or_dot_f32": (C.c_float, [P, P, sz]),
        "or_matmul": (None, [C.c_int, P, sz, sz, P, sz, P, C.c_int]),
        "or_set_q8_fine": (None, [C.c_int]),
        "or_q8_fine": (C.c_int, []),
        "or_set_simd": (None, [C.c_int]),
        "or_simd": (C.c_int, []),
        "or_rmsnorm": (None, [P, P, C.c_float, P, sz]),
        "or_rmsnorm_gated": (None, [P, P, P, C.c_float, P, sz]),
        "or_softmax": (None, [P, P, sz]),
        "or_silu": (C.c_float, [C.c_float]),
        "or_eval_math": (None, [C.c_int, P, P, sz, C.c_int]),
        "or_math_sweep": (C.c_uint64, [C.c_int, C.c_uint32, C.c_uint64, C.c_uint32, C.POINTER(C.c_uint32)]),
        "or_sigmoid": (C.c_float, [C.c_float]),
        "or_softplus": (C.c_float, [C.c_float]),
        "or_swiglu": (None, [P, P, P, sz]),
        "or_inv_freq": (None, [sz, C.c_float, P]),
        "or_cos_sin": (None, [C.c_uint32, P, sz, P, P]),
        "or_apply_rope": (None, [P, sz, sz, sz, P, P]),
        "or_conv1d_step": (None, [P, P, sz, P, P, sz, C.c_int]),
        "or_l2norm": (None, [P, sz, C.c_float]),
        "or_gate_g": (C.c_float, [C.c_float, C.c_float, C.c_float]),
        "or_deltanet_step": (None, [P, P, P, C.c_float, C.c_float, P, P, sz, sz]),
        "or_model_new": (P, [P, P, sz, C.c_int]),
        "or_model_free": (None, [P]),
        "or_state_new": (P, [P, C.c_uint32, C.c_uint32]),
        "or_state_free": (None, [P]),
        "or_forward_token": (C.c_uint32, [P, P, C.c_uint32, P]),
        "or_prefill": (C.c_uint32, [P, P, P, sz, P]),
        "or_spec_prefill": (C.c_uint32, [P, P, P, sz]),
        "or_spec_round": (C.c_uint32, [P, P, C.c_uint32, P, P]),
        "or_spec_set_drafts": (None, [P, P, sz]),
        "or_forward_token_s": (C.c_uint32, [P, P, P, C.c_uint32, P]),
        "or_prefill_s": (C.c_uint32, [P, P, P, P, sz, P]),
        "or_spec_prefill_s": (C.c_uint32, [P, P, P, P, sz]),
        "or_spec_round_s": (C.c_uint32, [P, P, P, C.c_uint32, P, P]),
        "or_rng_seed": (None, [C.c_uint64, P]),
        "or_rng_next": (C.c_uint64, [P]),
        "or_rng_f32": (C.c_float, [P]),
        "or_sampler_new": (P, [P, sz]),
        "or_sampler_free": (None, [P]),
        "or_sampler_reseed": (None, [P, C.c_uint64]),
        "or_sampler_rng": (None, [P, P]),
        "or_sampler_is_greedy": (C.c_int, [P]),
        "or_sampler_process": (sz, [P, P]),
        "or_sampler_kept": (sz, [P, P, P]),
        "or_sampler_draw": (C.c_uint32, [P]),
        "or_sampler_sample": (C.c_uint32, [P, P]),
        "or_sampler_write_dense": (None, [P, P]),
        "or_sampler_accept_or_resample": (C.c_int, [P, P, P, C.c_uint32, P]),
        "or_spec_get_drafts": (None, [P, P]),
        "or_spec_logits_row": (None, [P, sz, P]),
        "or_state_pos": (C.c_uint32, [P]),
        "or_state_export": (sz, [P, P]),
        "or_layer_run": (C.c_int, [P, P, sz, C.c_int, P, sz, C.c_uint32, P, P, P, P, P, C.c_uint32, P]),
    }
    for name, (res, args) in sigs.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def ptr(a):
    return None if a is None else a.ctypes.data


# ------------------------------------------------------------------------------------------- thin wrappers

def q8k_quantize(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 256 * 292, np.uint8)
    lib().or_q8k_quantize(ptr(x), x.size, ptr(out))
    return out


def q8_0_quantize(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 32 * 34, np.uint8)
    lib().or_q8_0_quantize(ptr(x), x.size, ptr(out))
    return out


def dequant(t, raw, n):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.zeros(n, np.float32)
    assert lib().or_dequant(t, ptr(raw), n, ptr(out)) == 0
    return out


def dot_q8k(t, wrow, xq, n):
    return lib().or_dot_q8k(t, ptr(np.ascontiguousarray(wrow)), ptr(np.ascontiguousarray(xq)), n)


def kq_isums(t, wrow, xq, n):
    nb = n // 256
    lanes = np.zeros(nb * 8, np.int32)
    mins = np.zeros(nb * 4, np.int32)
    lib().or_kq_isums(t, ptr(np.ascontiguousarray(wrow)), ptr(np.ascontiguousarray(xq)), n, ptr(lanes), ptr(mins))
    return lanes, mins


def kq_isums_mat(t, w, rows, xq, n):
    """or_kq_isums of every row: lanes [rows, nb, 8], mins [rows, nb, 4]."""
    nb = n // 256
    lanes = np.zeros((rows, nb, 8), np.int32)
    mins = np.zeros((rows, nb, 4), np.int32)
    lib().or_kq_isums_mat(t, ptr(np.ascontiguousarray(w)), rows, ptr(np.ascontiguousarray(xq)), n, ptr(lanes),
                          ptr(mins))
    return lanes, mins


def dot_q8k_t(t, wrow, xqs, n):
    xqs = [np.ascontiguousarray(x) for x in xqs]
    arr = (C.c_void_p * len(xqs))(*[x.ctypes.data for x in xqs])
    out = np.zeros(len(xqs), np.float32)
    lib().or_dot_q8k_t(t, ptr(np.ascontiguousarray(wrow)), arr, len(xqs), n, ptr(out))
    return out


def dot_q8(t, wrow, xq, n):
    return lib().or_dot_q8(t, ptr(np.ascontiguousarray(wrow)), ptr(np.ascontiguousarray(xq)), n)


class q8_fine:
    """Context manager: the oracle's process-wide q8-fine switch (matvec.rs:133 set_q8_fine) on inside the block."""

    def __init__(self, on=True):
        self.on = on

    def __enter__(self):
        self.prev = lib().or_q8_fine()
        lib().or_set_q8_fine(1 if self.on else 0)
        return self

    def __exit__(self, *exc):
        lib().or_set_q8_fine(self.prev)


class simd:
    """Context manager: the oracle's AVX2 dots (oracle_simd.c, bit-identical to the scalar ones) on inside the block."""

    def __init__(self, on=True):
        self.on = on

    def __enter__(self):
        self.prev = lib().or_simd()
        lib().or_set_simd(1 if self.on else 0)
        return self

    def __exit__(self, *exc):
        lib().or_set_simd(self.prev)


def matmul(t, w, rows, cols, x, threads=4):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
    y = np.zeros((x.shape[0], rows), np.float32)
    lib().or_matmul(t, ptr(np.ascontiguousarray(w)), rows, cols, ptr(x), x.shape[0], ptr(y), threads)
    return y


class Model:
    """The oracle model over a tensor table (borrowed: the table's arrays are kept alive here)."""

    def __init__(self, cfg: AqModelConfig, tensors, threads=8):
        self.cfg = cfg
        self.table, self.keep = tensor_table(tensors)
        self.h = lib().or_model_new(C.byref(cfg), self.table, len(tensors), threads)
        assert self.h, "oracle model load failed"

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_model_free(self.h)
            self.h = None


class AqSamplerConfig(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float), ("min_p", C.c_float),
                ("seed", C.c_uint64)]


def sampler_config(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, seed=0):
    return AqSamplerConfig(temperature, top_k, top_p, min_p, seed)


class Sampler:
    """The oracle's Sampler (sample.rs:148-303)."""

    def __init__(self, cfg, vocab):
        self.vocab = vocab
        self.cfg = cfg
        self.h = lib().or_sampler_new(C.byref(cfg), vocab)

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_sampler_free(self.h)
            self.h = None

    def reseed(self, seed):
        lib().or_sampler_reseed(self.h, seed)

    def rng(self):
        out = np.zeros(4, np.uint64)
        lib().or_sampler_rng(self.h, ptr(out))
        return out

    def process(self, logits):
        logits = np.ascontiguousarray(logits, np.float32)
        n = lib().or_sampler_process(self.h, ptr(logits))
        ids, probs = np.zeros(n, np.uint32), np.zeros(n, np.float32)
        lib().or_sampler_kept(self.h, ptr(ids), ptr(probs))
        return ids, probs

    def kept(self):
        n = lib().or_sampler_kept(self.h, None, None)
        ids, probs = np.zeros(n, np.uint32), np.zeros(n, np.float32)
        lib().or_sampler_kept(self.h, ptr(ids), ptr(probs))
        return ids, probs

    def draw(self):
        return lib().or_sampler_draw(self.h)

    def sample(self, logits):
        return lib().or_sampler_sample(self.h, ptr(np.ascontiguousarray(logits, np.float32)))

    def write_dense(self):
        out = np.zeros(self.vocab, np.float32)
        lib().or_sampler_write_dense(self.h, ptr(out))
        return out

    def accept_or_resample(self, target, q, d):
        tok = C.c_uint32(0)
        ok = lib().or_sampler_accept_or_resample(self.h, ptr(np.ascontiguousarray(target, np.float32)),
                                                 ptr(np.ascontiguousarray(q, np.float32)), d, C.byref(tok))
        return bool(ok), tok.value


def rng_seed(seed):
    s = np.zeros(4, np.uint64)
    lib().or_rng_seed(seed, ptr(s))
    return s


def _sp(sampler):
    return None if sampler is None else sampler.h


class State:
    def __init__(self, model: Model, spec_k=0, max_pos=512):
        self.model = model
        self.k = spec_k
        self.h = lib().or_state_new(model.h, spec_k, max_pos)

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_state_free(self.h)
            self.h = None

    @property
    def pos(self):
        return lib().or_state_pos(self.h)

    def forward_token(self, tok, want_logits=False, sampler=None):
        lg = np.zeros(self.model.cfg.vocab, np.float32) if want_logits else None
        a = lib().or_forward_token_s(self.model.h, self.h, _sp(sampler), tok, ptr(lg))
        return (a, lg) if want_logits else a

    def prefill(self, ids, want_logits=False, sampler=None):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        lg = np.zeros(self.model.cfg.vocab, np.float32) if want_logits else None
        a = lib().or_prefill_s(self.model.h, self.h, _sp(sampler), ptr(ids), ids.size, ptr(lg))
        return (a, lg) if want_logits else a

    def spec_prefill(self, ids, sampler=None):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        return lib().or_spec_prefill_s(self.model.h, self.h, _sp(sampler), ptr(ids), ids.size)

    def spec_round(self, x_p, sampler=None):
        em = np.zeros(self.k + 1, np.uint32)
        n = C.c_uint32(0)
        m = lib().or_spec_round_s(self.model.h, self.h, _sp(sampler), x_p, ptr(em), C.byref(n))
        return m, em[: n.value].tolist()

    def set_drafts(self, d):
        d = np.ascontiguousarray(d, dtype=np.uint32)
        lib().or_spec_set_drafts(self.h, ptr(d), d.size)

    def drafts(self):
        d = np.zeros(self.k, np.uint32)
        lib().or_spec_get_drafts(self.h, ptr(d))
        return d.tolist()

    def logits_row(self, i):
        out = np.zeros(self.model.cfg.vocab, np.float32)
        lib().or_spec_logits_row(self.h, i, ptr(out))
        return out

    def export(self):
        n = lib().or_state_export(self.h, None)
        out = np.zeros(n, np.float32)
        lib().or_state_export(self.h, ptr(out))
        return out
