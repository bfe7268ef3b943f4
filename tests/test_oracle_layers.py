"""The oracle's layers against the reference's HF layer fixtures (tests/golden/layers, hidden 64, F32 weights in
GGUF layout), as tests/layers.rs:109-271 checks them: prefill of t rows, then one cached step; budget
k * sqrt(width) * eps * max|ref| with the fixture's k."""
import ctypes as C
import json
import math
import os

import numpy as np

import oracle_lib as O

DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "layers")
EPS = float(np.finfo(np.float32).eps)

with open(os.path.join(DIR, "manifest.json")) as f:
    M = json.load(f)
CFG = M["config"]
K = M["budget_k"]


def arr(field):
    return np.load(os.path.join(DIR, field["file"]), allow_pickle=False).astype(np.float32)


def case(name):
    return next(c for c in M["cases"] if c["case"] == name)


def config():
    c = O.AqModelConfig()
    c.n_layer, c.hidden, c.ffn, c.vocab = 1, CFG["hidden_size"], CFG["intermediate_size"], CFG["vocab_size"]
    c.n_head, c.n_head_kv, c.head_dim = CFG["num_attention_heads"], CFG["num_key_value_heads"], CFG["head_dim"]
    c.rope_dim = int(CFG["head_dim"] * CFG["rope_parameters"]["partial_rotary_factor"])
    c.rope_theta, c.rms_eps = CFG["rope_parameters"]["rope_theta"], CFG["rms_norm_eps"]
    c.full_attention_interval = 4
    c.dn_n_k_heads, c.dn_n_v_heads = CFG["linear_num_key_heads"], CFG["linear_num_value_heads"]
    c.dn_head_dim_k, c.dn_head_dim_v = CFG["linear_key_head_dim"], CFG["linear_value_head_dim"]
    c.dn_conv_kernel, c.has_mtp = CFG["linear_conv_kernel_dim"], 0
    return c


def tensors(c):
    out = []
    for name, f in c["weights"].items():
        a = arr(f)
        rows, cols = (a.shape[0], a.shape[1]) if a.ndim == 2 else (1, a.size)
        out.append(("blk.0." + name, O.F32, rows, cols, a))
    return out


def check(label, got, want, width):
    bud = K * math.sqrt(width) * EPS * float(np.abs(want).max())
    d = float(np.abs(got.astype(np.float64) - want.astype(np.float64)).max())
    assert d <= bud, f"{label}: {d:e} > {bud:e}"


class Runner:
    def __init__(self, c, kind):
        self.cfg = config()
        self.table, self.keep = O.tensor_table(tensors(c))
        self.kind = kind
        cd = 2 * self.cfg.dn_n_k_heads * self.cfg.dn_head_dim_k + self.cfg.dn_n_v_heads * self.cfg.dn_head_dim_v
        self.conv = np.zeros(cd * (self.cfg.dn_conv_kernel - 1), np.float32)
        self.rec = np.zeros(self.cfg.dn_n_v_heads * self.cfg.dn_head_dim_k * self.cfg.dn_head_dim_v, np.float32)
        self.cap = 16
        stride = self.cfg.n_head_kv * self.cfg.head_dim
        self.kc = np.zeros(self.cap * stride, np.float32)
        self.vc = np.zeros(self.cap * stride, np.float32)
        self.kv_len = C.c_uint32(0)

    def run(self, x, start):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.cfg.hidden)
        y = np.zeros_like(x)
        rc = O.lib().or_layer_run(C.byref(self.cfg), self.table, len(self.keep) // 2, self.kind, O.ptr(x), x.shape[0],
                                  start, O.ptr(self.conv), O.ptr(self.rec), O.ptr(self.kc), O.ptr(self.vc),
                                  C.byref(self.kv_len), self.cap, O.ptr(y))
        assert rc == 0
        return y


def hf_conv_window(field, kernel):
    a = arr(field)
    return np.ascontiguousarray(a[:, a.shape[1] - (kernel - 1):]).ravel()


def test_gated_deltanet_prefill_and_step():
    c = case("deltanet_layer")
    r = Runner(c, 0)
    hidden = CFG["hidden_size"]
    width = max(hidden, c["head_k"] * c["head_v"])
    y = r.run(arr(c["prefill"]["x"]), 0)
    check("deltanet prefill", y, arr(c["prefill"]["y"]).reshape(y.shape), width)
    check("deltanet prefill vs sequential", y, arr(c["prefill"]["y_seq"]).reshape(y.shape), width)
    check("deltanet rec state", r.rec, arr(c["prefill"]["rec_state"]).ravel(), width)
    check("deltanet conv window", r.conv, hf_conv_window(c["prefill"]["conv_state"], 4), hidden)
    y1 = r.run(arr(c["step"]["x"]), c["t"])
    check("deltanet step", y1, arr(c["step"]["y"]).reshape(y1.shape), width)
    check("deltanet step rec", r.rec, arr(c["step"]["rec_state"]).ravel(), width)
    check("deltanet step conv", r.conv, hf_conv_window(c["step"]["conv_state"], 4), hidden)


def test_gqa_attention_prefill_and_step():
    c = case("attention_layer")
    r = Runner(c, 1)
    hidden, t = CFG["hidden_size"], c["t"]
    nkv, hd = c["n_head_kv"], c["head_dim"]
    width = max(hidden, hd, t)
    y = r.run(arr(c["prefill"]["x"]), 0)
    check("attention prefill", y, arr(c["prefill"]["y"]).reshape(y.shape), width)
    stride = nkv * hd
    k_ours = r.kc[: t * stride].reshape(t, nkv, hd).transpose(1, 0, 2)
    v_ours = r.vc[: t * stride].reshape(t, nkv, hd).transpose(1, 0, 2)
    check("attention K cache", k_ours, arr(c["prefill"]["k_cache"]).reshape(k_ours.shape), hidden)
    check("attention V cache", v_ours, arr(c["prefill"]["v_cache"]).reshape(v_ours.shape), hidden)
    y1 = r.run(arr(c["step"]["x"]), c["step"]["position"])
    check("attention step", y1, arr(c["step"]["y"]).reshape(y1.shape), width)


def test_mlp_matches_hf():
    c = case("mlp_layer")
    r = Runner(c, 2)
    y = r.run(arr(c["prefill"]["x"]), 0)
    check("mlp", y, arr(c["prefill"]["y"]).reshape(y.shape), CFG["intermediate_size"])


def test_decoder_layers_prefill_and_step():
    hidden, inter = CFG["hidden_size"], CFG["intermediate_size"]
    for kind, code in (("linear_attention", 3), ("full_attention", 4)):
        c = case(f"decoder_{kind}")
        width = max(hidden, inter)
        r = Runner(c, code)
        x = arr(c["prefill"]["x"])
        # token by token (tests/layers.rs:253-257) ...
        ys = np.concatenate([r.run(x[i], i) for i in range(c["t"])])
        check(f"decoder {kind} prefill", ys, arr(c["prefill"]["y"]).reshape(ys.shape), width)
        y1 = r.run(arr(c["step"]["x"]), c["step"]["position"])
        check(f"decoder {kind} step", y1, arr(c["step"]["y"]).reshape(y1.shape), width)
        # ... and batched: row i of the batch equals the token path bit for bit (layers/mod.rs:332-334)
        rb = Runner(c, code)
        yb = rb.run(x, 0)
        assert np.array_equal(yb.view(np.uint32), ys.view(np.uint32))
