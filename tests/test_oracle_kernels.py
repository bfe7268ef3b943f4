"""The CPU oracle against the reference's own golden fixtures (tests/golden/, copied from the reference's
tests/fixtures/). Budgets follow the reference's tests exactly: k * sqrt(width) * eps * max|ref| (tests/kernels.rs:49-51),
the K-quant term-magnitude budget (tests/common/mod.rs:108-131), bit-exact where the manifest says `exact`."""
import json
import math
import os
import zlib

import numpy as np
import pytest

import oracle_lib as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
EPS = float(np.finfo(np.float32).eps)


class Fx:
    def __init__(self, group, sub="kernels"):
        self.dir = os.path.join(GOLD, sub, group) if sub else os.path.join(GOLD, group)
        with open(os.path.join(self.dir, "manifest.json")) as f:
            self.m = json.load(f)

    @property
    def cases(self):
        return self.m["cases"]

    @property
    def k(self):
        return self.m["budget_k"]

    def arr(self, field):
        return np.load(os.path.join(self.dir, field["file"]), allow_pickle=False).astype(np.float32).ravel()

    def raw(self, field):
        with open(os.path.join(self.dir, field["file"]), "rb") as f:
            return np.frombuffer(f.read(), np.uint8)


def budget(k, width, max_abs):
    return k * math.sqrt(width) * EPS * max_abs


def max_diff(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    fin = np.isfinite(got) & np.isfinite(want)
    d = np.zeros_like(got)
    d[fin] = np.abs(got[fin] - want[fin])
    nf = ~fin
    same = (np.isnan(got) & np.isnan(want)) | (got == want)
    d[nf & ~same] = np.inf
    return float(d.max()) if d.size else 0.0


def check_rows(got, want, width, k):
    for r in range(got.size // width):
        g, w = got[r * width:(r + 1) * width], want[r * width:(r + 1) * width]
        fin = w[np.isfinite(w)]
        ma = float(np.abs(fin).max()) if fin.size else 0.0
        assert max_diff(g, w) <= budget(k, width, ma), f"row {r}"


def kquant_terms_budget(t, wrow, w_deq, x_deq, k):
    """tests/common/mod.rs:112-131: k * eps * sum_j (|main_j| + |min_j|) |x_j|."""
    width = w_deq.size
    nsb = width // 256
    bb = wrow.size // nsb
    mags = 0.0
    for sb in range(nsb):
        wb = wrow[sb * bb:(sb + 1) * bb]
        dmin = 0.0 if t == O.Q6_K else float(np.frombuffer(wb[2:4].tobytes(), np.float16)[0])
        for s in range(8):
            if t == O.Q6_K:
                m = 0
            else:
                q = wb[4:16]
                m = (q[s + 4] & 63) if s < 4 else ((q[s + 4] >> 4) | ((q[s] >> 6) << 4))
            mp = dmin * m
            j = slice(sb * 256 + s * 32, sb * 256 + (s + 1) * 32)
            mags += float(np.sum((np.abs(w_deq[j].astype(np.float64) + mp) + abs(mp)) * np.abs(x_deq[j].astype(np.float64))))
    return k * EPS * mags


def q8k_dequant(raw, n):
    out = np.zeros(n, np.float32)
    for b in range(n // 256):
        blk = raw[b * 292:(b + 1) * 292]
        d = np.frombuffer(blk[:4].tobytes(), np.float32)[0]
        out[b * 256:(b + 1) * 256] = d * blk[4:260].view(np.int8).astype(np.float32)
    return out


# ------------------------------------------------------------------------------------------------- f16

def test_f16_roundtrip_exact():
    """quant.rs:264-270 unit test values, plus every f16 bit pattern against numpy's IEEE conversion."""
    L = O.lib()
    assert L.or_f16_to_f32(0x3C00) == 1.0
    assert L.or_f16_to_f32(0xC000) == -2.0
    assert L.or_f16_to_f32(0x0001) == np.float32(5.9604645e-8)
    assert L.or_f16_to_f32(0x7BFF) == 65504.0
    allbits = np.arange(65536, dtype=np.uint16)
    ref = allbits.view(np.float16).astype(np.float32)
    got = np.array([L.or_f16_to_f32(int(b)) for b in allbits], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    # f32 -> f16: round to nearest even against numpy on random and boundary values
    rng = np.random.default_rng(1)
    xs = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-8, 5, 20000),
                         np.array([65504.0, 65520.0, 65519.99, 6.1035156e-05, 5.96e-8, 2.98e-8, 0.0, -0.0], np.float32)]
                        ).astype(np.float32)
    got = np.array([L.or_f32_to_f16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, xs.astype(np.float16).view(np.uint16))


# --------------------------------------------------------------------------------------------- quantisers

def test_q8k_quantiser_bit_exact():
    """tests/q8k.rs:143-170: every fixture row (12 hostile rows x widths 256/512/5120) byte-identical."""
    fx = Fx("q8k_quantize")
    assert fx.m["exact"] is True
    n = 0
    for c in fx.cases:
        width = c["width"]
        x = fx.arr(c["x"]).reshape(-1, width)
        raw = fx.raw(c["raw"])
        bpr = width // 256 * 292
        for r in range(x.shape[0]):
            got = O.q8k_quantize(x[r])
            assert np.array_equal(got, raw[r * bpr:(r + 1) * bpr]), f"{c['case']} row {r} ({c['rows'][r]})"
            n += 1
    assert n == 36


def test_q8k_fixture_discriminates_rounding():
    """The ties_even row breaks a round-half-away quantiser (tests/q8k.rs:117-121): planted on the CPU."""
    fx = Fx("q8k_quantize")
    c = fx.cases[0]
    x = fx.arr(c["x"]).reshape(-1, 256)[c["rows"].index("ties_even")]
    raw = fx.raw(c["raw"])[c["rows"].index("ties_even") * 292:][:292]
    amax_i = int(np.argmax(np.abs(x)))
    iscale = np.float32(-127.0) / x[amax_i]
    wrong = np.minimum(np.sign(iscale * x) * np.floor(np.abs(iscale * x) + 0.5), 127).astype(np.int8)
    assert not np.array_equal(wrong.view(np.uint8), raw[4:260])
    assert np.array_equal(O.q8k_quantize(x), raw)


def test_q8_0_quantiser_bit_exact():
    """tests/kernels.rs:190-211: Q8_0 bytes and dequantised values exact."""
    fx = Fx("q8_quantize")
    for c in fx.cases:
        width = c["width"]
        x = fx.arr(c["x"]).reshape(-1, width)
        raw = fx.raw(c["raw"])
        deq = fx.arr(c["deq"]).reshape(-1, width)
        rb = width // 32 * 34
        for r in range(x.shape[0]):
            got = O.q8_0_quantize(x[r])
            assert np.array_equal(got, raw[r * rb:(r + 1) * rb]), f"{c['case']} row {r}"
            assert np.array_equal(O.dequant(O.Q8_0, got, width).view(np.uint32), deq[r].view(np.uint32))


# ----------------------------------------------------------------------------------------------- dequant

def test_dequant_prefix_hostile_and_full_tensor_crc():
    """tests/dequant.rs:35-156: prefix blocks and hostile blocks exact; full tensors (real GGUF rows shipped
    with the fixture) by the CRC-32 of their f32 stream."""
    d = os.path.join(GOLD, "dequant")
    with open(os.path.join(d, "manifest.json")) as f:
        m = json.load(f)
    for name, t in m["types"].items():
        tid = O.TYPE_BY_NAME[name]
        p = t["prefix"]
        raw = np.fromfile(os.path.join(d, p["raw_bin"]), np.uint8)
        want = np.load(os.path.join(d, p["npy"]), allow_pickle=False).astype(np.float32).ravel()
        got = O.dequant(tid, raw, p["n_elements"])
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{name} prefix"
        full = t["full"]
        if full.get("raw_bin") and os.path.exists(os.path.join(d, full["raw_bin"])):
            raw = np.fromfile(os.path.join(d, full["raw_bin"]), np.uint8)
            got = O.dequant(tid, raw, full["n_elements"])
            assert zlib.crc32(got.astype("<f4").tobytes()) == full["digest"]["crc32"], f"{name} full-tensor crc"
            head = np.load(os.path.join(d, full["head_npy"]), allow_pickle=False).astype(np.float32).ravel()
            assert np.array_equal(got[:head.size].view(np.uint32), head.view(np.uint32))
    for h in m["hostile"]:
        tid = O.TYPE_BY_NAME[h["ggml_type"]]
        raw = np.fromfile(os.path.join(d, h["raw_bin"]), np.uint8)
        want = np.load(os.path.join(d, h["npy"]), allow_pickle=False).astype(np.float32).ravel()
        got = O.dequant(tid, raw, h["n_elements"])
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), h["label"]


def test_dequant_fixture_discriminates_nibble_order():
    """A Q4_K unpack with low/high nibbles swapped fails the hostile block (tests/dequant.rs:127-156)."""
    d = os.path.join(GOLD, "dequant")
    raw = np.fromfile(os.path.join(d, "hostile_q4_k.bin"), np.uint8).copy()
    want = np.load(os.path.join(d, "hostile_q4_k.npy"), allow_pickle=False).astype(np.float32).ravel()
    swapped = raw.copy()
    swapped[16:144] = ((raw[16:144] & 0x0F) << 4) | (raw[16:144] >> 4)
    assert not np.array_equal(O.dequant(O.Q4_K, swapped, 256), want)


# ---------------------------------------------------------------------------------------------- dots

def test_kquant_q8k_dots_within_f64_budget():
    """tests/q8k.rs:174-216: x_deq re-quantised to Q8_K; |dot - f64 reference| <= term-magnitude budget."""
    fx = Fx("dot")
    k = fx.k
    seen = 0
    for c in fx.cases:
        t = O.TYPE_BY_NAME[c["ggml_type"]]
        if t not in (O.Q4_K, O.Q5_K, O.Q6_K):
            continue
        width, n_rows = c["width"], c["n_rows"]
        w_raw = fx.raw(c["w_raw"])
        x_deq = fx.arr(c["x_deq"]).reshape(n_rows, width)
        rb = O.row_bytes(t, width)
        for r in range(n_rows):
            wrow = w_raw[r * rb:(r + 1) * rb]
            xq = O.q8k_quantize(x_deq[r])
            wd = O.dequant(t, wrow, width)
            xd = q8k_dequant(xq, width)
            ref = float(np.dot(wd.astype(np.float64), xd.astype(np.float64)))
            bud = kquant_terms_budget(t, wrow, wd, xd, k)
            got = O.dot_q8k(t, wrow, xq, width)
            assert abs(got - ref) <= bud, f"{c['case']} row {r}: {got} vs {ref} (budget {bud})"
            seen += 1
    assert seen >= 21


def test_dot_kernels_q8_activation_within_budget():
    """tests/kernels.rs:213-249 for the Q8_0-activation kernels (Q8_0, Q4_0 weights): fixture Q8_0 rows."""
    fx = Fx("dot")
    for c in fx.cases:
        t = O.TYPE_BY_NAME[c["ggml_type"]]
        if t not in (O.Q8_0, O.Q4_0):
            continue
        width, n_rows = c["width"], c["n_rows"]
        w_raw, x_raw = fx.raw(c["w_raw"]), fx.raw(c["x_raw"])
        wrb, xrb = O.row_bytes(t, width), width // 32 * 34
        for r in range(n_rows):
            got = O.dot_q8(t, w_raw[r * wrb:(r + 1) * wrb], x_raw[r * xrb:(r + 1) * xrb], width)
            bud = budget(fx.k, width, c["max_abs_term"][r])
            assert abs(got - c["ref_f64"][r]) <= bud, f"{c['case']} row {r}"


def test_f32_dot_within_budget():
    """F32 weights x f32 activations (matvec.rs:270-279 -> dot.rs:180-200) on the F32 dot fixture."""
    fx = Fx("dot")
    for c in fx.cases:
        if c["ggml_type"] != "F32":
            continue
        width, n_rows = c["width"], c["n_rows"]
        w = fx.arr(c["w_deq"]).reshape(n_rows, width)
        x = fx.arr(c["x_deq"]).reshape(n_rows, width)
        for r in range(n_rows):
            got = O.lib().or_dot_f32(O.ptr(np.ascontiguousarray(w[r])), O.ptr(np.ascontiguousarray(x[r])), width)
            assert abs(got - c["ref_f64"][r]) <= budget(fx.k, width, c["max_abs_term"][r])


def test_blocked_dot_equals_single_rows_bitwise():
    """tests/matmul_t.rs:137-253: out[i] == dot_q8k(w, xs[i]) bit for bit, every tile 1..16."""
    fx = Fx("dot")
    rng = np.random.default_rng(7)
    for c in fx.cases:
        t = O.TYPE_BY_NAME[c["ggml_type"]]
        if t not in (O.Q4_K, O.Q5_K, O.Q6_K) or c["width"] != 5120:
            continue
        width = c["width"]
        wrow = fx.raw(c["w_raw"])[: O.row_bytes(t, width)]
        xs = [O.q8k_quantize(rng.standard_normal(width).astype(np.float32) * s) for s in (1, 0.01, 100) * 6]
        single = np.array([O.dot_q8k(t, wrow, x, width) for x in xs], np.float32)
        for tile in (1, 2, 3, 4, 7, 8, 16):
            got = O.dot_q8k_t(t, wrow, xs[:tile], width)
            assert np.array_equal(got.view(np.uint32), single[:tile].view(np.uint32))


def test_kquant_integer_lanes_match_brute_force():
    """The exact integer part (the bit-exact contract of the GPU kernel) restated by brute force from the
    dequantisation formula: sum over lane l of sc*q*x equals the oracle's lane, and the f32 dot rebuilt from
    the lanes with the documented order equals the oracle's dot."""
    rng = np.random.default_rng(3)
    for t in (O.Q4_K, O.Q5_K, O.Q6_K):
        width = 512
        wrow = rng.integers(0, 256, O.row_bytes(t, width), dtype=np.uint8)
        bb = O.row_bytes(t, 256)
        for sb in range(width // 256):  # finite f16 scales
            for off in ((0, 2) if t != O.Q6_K else (208,)):
                wrow[sb * bb + off + 1] = (wrow[sb * bb + off + 1] & 0x83) | 0x20
        x = rng.standard_normal(width).astype(np.float32)
        xq = O.q8k_quantize(x)
        lanes, mins = O.kq_isums(t, wrow, xq, width)
        codes = xq.reshape(-1, 292)[:, 4:260].view(np.int8).astype(np.int64)
        for sb in range(width // 256):
            wb = wrow[sb * bb:(sb + 1) * bb]
            if t == O.Q6_K:
                sc = wb[192:208].view(np.int8).astype(np.int64)
                q = np.zeros(256, np.int64)
                for half in range(2):
                    ql, qh = wb[half * 64:half * 64 + 64], wb[128 + half * 32:128 + half * 32 + 32]
                    for kk in range(4):
                        lo = (ql[(kk & 1) * 32:(kk & 1) * 32 + 32] >> (4 * (kk >> 1))) & 0xF
                        hi = (qh >> (2 * kk)) & 3
                        q[half * 128 + kk * 32:half * 128 + kk * 32 + 32] = (lo | (hi << 4)).astype(np.int64) - 32
                prod = sc[np.arange(256) // 16] * q * codes[sb]
                # the -32 offset lands in lanes by group (kdot.rs:125-129); the +32*q part by position
                e = np.arange(256)
                pos_part = sc[e // 16] * (q + 32) * codes[sb]
                want = np.zeros(8, np.int64)
                np.add.at(want, (e % 32) // 4, pos_part)
                bs = codes[sb].reshape(16, 16).sum(axis=1)
                for i in range(8):
                    want[i] -= 32 * (bs[2 * i] * sc[2 * i] + bs[2 * i + 1] * sc[2 * i + 1])
                assert int(prod.sum()) == int(want.sum())
            else:
                sc, mn = np.zeros(8, np.int64), np.zeros(8, np.int64)
                s12 = wb[4:16].astype(np.int64)
                for j in range(8):
                    if j < 4:
                        sc[j], mn[j] = s12[j] & 63, s12[j + 4] & 63
                    else:
                        sc[j] = (s12[j + 4] & 0xF) | ((s12[j - 4] >> 6) << 4)
                        mn[j] = (s12[j + 4] >> 4) | ((s12[j] >> 6) << 4)
                qlo = wb[16:144] if t == O.Q4_K else wb[48:176]
                q = np.zeros(256, np.int64)
                for s in range(8):
                    nib = (qlo[(s // 2) * 32:(s // 2) * 32 + 32] >> (4 * (s % 2))) & 0xF
                    q[s * 32:(s + 1) * 32] = nib
                    if t == O.Q5_K:
                        q[s * 32:(s + 1) * 32] += ((wb[16:48] >> s) & 1).astype(np.int64) * 16
                e = np.arange(256)
                want = np.zeros(8, np.int64)
                np.add.at(want, (e % 32) // 4, sc[e // 32] * q * codes[sb])
                q8s = codes[sb].reshape(8, 32).sum(axis=1)
                want_m = np.array([mn[2 * i] * q8s[2 * i] + mn[2 * i + 1] * q8s[2 * i + 1] for i in range(4)])
                assert np.array_equal(mins[sb * 4:(sb + 1) * 4], want_m)
            assert np.array_equal(lanes[sb * 8:(sb + 1) * 8], want), f"type {t} sb {sb}"


def test_matvec_fixture_within_budget():
    """tests/kernels.rs:251-291: the reference matvec fixture (Q8_0 activation rows), thread invariance."""
    fx = Fx("matvec")
    for c in fx.cases:
        t = O.TYPE_BY_NAME[c["ggml_type"]]
        rows, width = c["n_rows"], c["width"]
        w = fx.raw(c["w_raw"])
        xr = fx.raw(c["x_raw"])
        rb = O.row_bytes(t, width)
        xd = O.dequant(O.Q8_0, xr, width)
        for r in range(rows):
            wrow = w[r * rb:(r + 1) * rb]
            if t in (O.Q8_0, O.Q4_0):
                got = O.dot_q8(t, wrow, xr, width)
                bud = budget(fx.k, width, c["max_abs_term"][r])
            elif t == O.F32:
                got = O.lib().or_dot_f32(O.ptr(np.ascontiguousarray(wrow.view(np.float32))), O.ptr(xd), width)
                bud = budget(fx.k, width, c["max_abs_term"][r])
            else:
                continue  # K-quant rows take Q8_K activations here; covered by the dot fixture test
            assert abs(got - c["ref_f64"][r]) <= bud, f"{c['case']} row {r}"
        if t != O.F32:
            y1 = O.matmul(t, w, rows, width, xd[None, :], threads=1)
            y5 = O.matmul(t, w, rows, width, xd[None, :], threads=5)
            assert np.array_equal(y1.view(np.uint32), y5.view(np.uint32))


# -------------------------------------------------------------------------------------- row kernels

def test_rmsnorm_matches_hf():
    fx = Fx("rmsnorm")
    L = O.lib()
    for c in fx.cases:
        width = c["width"]
        x = fx.arr(c["x"]).reshape(-1, width)
        w = fx.arr(c["w_gguf"])
        want = fx.arr(c["y"])
        got = np.zeros_like(x)
        for r in range(x.shape[0]):
            xr = np.ascontiguousarray(x[r])
            yr = np.zeros(width, np.float32)
            if c["kind"] == "rmsnorm":
                L.or_rmsnorm(O.ptr(xr), O.ptr(w), c["eps"], O.ptr(yr), width)
            else:
                gate = np.ascontiguousarray(fx.arr(c["gate"]).reshape(-1, width)[r])
                L.or_rmsnorm_gated(O.ptr(xr), O.ptr(gate), O.ptr(w), c["eps"], O.ptr(yr), width)
            got[r] = yr
        check_rows(got.ravel(), want, width, fx.k)


def test_act_matches_torch():
    fx = Fx("act")
    L = O.lib()
    for c in fx.cases:
        want = fx.arr(c["y"])
        if c["kind"] == "silu":
            got = np.array([L.or_silu(float(v)) for v in fx.arr(c["x"])], np.float32)
        else:
            g, u = fx.arr(c["gate"]), fx.arr(c["up"])
            got = np.zeros_like(g)
            L.or_swiglu(O.ptr(g), O.ptr(u), O.ptr(got), g.size)
        floor = fx.k * EPS * float(np.finfo(np.float32).tiny)
        for gv, wv in zip(got, want):
            if not np.isfinite(wv):
                assert gv == wv or (np.isnan(gv) and np.isnan(wv))
                continue
            bud = max(fx.k * EPS * abs(float(wv)), 0.0 if wv == 0 else floor)
            assert abs(float(gv) - float(wv)) <= bud


def test_softmax_matches_torch():
    fx = Fx("softmax")
    L = O.lib()
    for c in fx.cases:
        want = fx.arr(c["y"])
        if c["kind"] == "softmax":
            width = c["width"]
            x = fx.arr(c["x"]).reshape(-1, width)
            got = np.zeros_like(x)
            for r in range(x.shape[0]):
                xr = np.ascontiguousarray(x[r])
                yr = np.zeros(width, np.float32)
                L.or_softmax(O.ptr(xr), O.ptr(yr), width)
                got[r] = yr
        else:
            width = c["t"]
            s = fx.arr(c["scores"]).reshape(width, width)
            got = np.zeros_like(s)
            for r in range(width):
                xr = np.ascontiguousarray(s[r, :r + 1])
                yr = np.zeros(r + 1, np.float32)
                L.or_softmax(O.ptr(xr), O.ptr(yr), r + 1)
                got[r, :r + 1] = yr
        check_rows(got.ravel(), want, width, fx.k)


def test_rope_tables_and_rotation_match_hf():
    fx = Fx("rope")
    L = O.lib()
    for c in fx.cases:
        hd, rd, theta = c["head_dim"], c["rope_dim"], c["theta"]
        pos = c["positions"]
        inv = np.zeros(rd // 2, np.float32)
        L.or_inv_freq(rd, theta, O.ptr(inv))
        inv_hf = fx.arr(c["inv_freq"])
        assert np.max(np.abs(inv.view(np.int32).astype(np.int64) - inv_hf.view(np.int32).astype(np.int64))) <= 1
        cos_hf, sin_hf = fx.arr(c["cos"]).reshape(-1, rd), fx.arr(c["sin"]).reshape(-1, rd)
        for ti, p in enumerate(pos):
            cs, sn = np.zeros(rd, np.float32), np.zeros(rd, np.float32)
            L.or_cos_sin(p, O.ptr(inv_hf), rd // 2, O.ptr(cs), O.ptr(sn))
            assert max_diff(cs, cos_hf[ti]) <= budget(fx.k, 1, 1.0)
            assert max_diff(sn, sin_hf[ti]) <= budget(fx.k, 1, 1.0)
        for name, out, heads in (("q", "q_out", 4), ("k", "k_out", 2)):
            x = fx.arr(c[name]).reshape(heads, len(pos), hd)
            want = fx.arr(c[out]).reshape(heads, len(pos), hd)
            got = x.copy()
            for h in range(heads):
                for ti in range(len(pos)):
                    v = np.ascontiguousarray(got[h, ti])
                    L.or_apply_rope(O.ptr(v), hd, hd, rd, O.ptr(np.ascontiguousarray(cos_hf[ti])),
                                    O.ptr(np.ascontiguousarray(sin_hf[ti])))
                    got[h, ti] = v
            assert max_diff(got, want) <= budget(fx.k, 2, c["max_abs"])
            assert np.array_equal(got[..., rd:].view(np.uint32), x[..., rd:].view(np.uint32))


def test_conv1d_step_and_prefill_match_hf():
    fx = Fx("conv1d")
    L = O.lib()
    for c in fx.cases:
        ch, kern = c["channels"], c["kernel"]
        w = fx.arr(c["w"])
        want = fx.arr(c["out"])
        bud = budget(fx.k, kern, c["max_abs"])
        if c["kind"] == "conv_step":
            st = fx.arr(c["state"]).copy()
            xn = fx.arr(c["x_new"])
            out = np.zeros(ch, np.float32)
            L.or_conv1d_step(O.ptr(st), O.ptr(w), kern, O.ptr(xn), O.ptr(out), ch, 1)
            assert max_diff(out, want) <= bud
            assert np.array_equal(st.view(np.uint32), fx.arr(c["new_state"]).view(np.uint32))
        else:
            t = c["t"]
            x = fx.arr(c["x"]).reshape(ch, t)
            st = np.zeros(ch * (kern - 1), np.float32)
            got = np.zeros((ch, t), np.float32)
            for step in range(t):
                xin = np.ascontiguousarray(x[:, step])
                o = np.zeros(ch, np.float32)
                L.or_conv1d_step(O.ptr(st), O.ptr(w), kern, O.ptr(xin), O.ptr(o), ch, 1)
                got[:, step] = o
            assert max_diff(got.ravel(), want) <= bud


def test_deltanet_step_matches_hf():
    fx = Fx("deltanet")
    L = O.lib()
    for c in fx.cases:
        heads, dk, dv = c["heads"], c["dk"], c["dv"]
        q, k, v = fx.arr(c["q"]), fx.arr(c["k"]), fx.arr(c["v"])
        a, b, big_a, dt = fx.arr(c["a"]), fx.arr(c["b"]), fx.arr(c["ssm_a"]), fx.arr(c["dt_bias"])
        g_hf, beta_hf = fx.arr(c["g"]), fx.arr(c["beta"])
        g = np.array([L.or_gate_g(float(a[h]), float(dt[h]), float(big_a[h])) for h in range(heads)], np.float32)
        beta = np.array([L.or_sigmoid(float(b[h])) for h in range(heads)], np.float32)
        assert max_diff(g, g_hf) <= budget(fx.k, 1, float(np.abs(g_hf).max()))
        assert max_diff(beta, beta_hf) <= budget(fx.k, 1, 1.0)
        state = fx.arr(c["state"]).copy()
        out = np.zeros(heads * dv, np.float32)
        scale = np.float32(1.0) / np.sqrt(np.float32(dk))
        for h in range(heads):
            qn = np.ascontiguousarray(q[h * dk:(h + 1) * dk])
            kn = np.ascontiguousarray(k[h * dk:(h + 1) * dk])
            L.or_l2norm(O.ptr(qn), dk, 1e-6)
            L.or_l2norm(O.ptr(kn), dk, 1e-6)
            qn = (qn * scale).astype(np.float32)
            s = np.ascontiguousarray(state[h * dk * dv:(h + 1) * dk * dv])
            o = np.zeros(dv, np.float32)
            L.or_deltanet_step(O.ptr(qn), O.ptr(kn), O.ptr(np.ascontiguousarray(v[h * dv:(h + 1) * dv])),
                               float(g_hf[h]), float(beta_hf[h]), O.ptr(s), O.ptr(o), dk, dv)
            state[h * dk * dv:(h + 1) * dk * dv] = s
            out[h * dv:(h + 1) * dv] = o
        assert max_diff(out, fx.arr(c["out"])) <= budget(fx.k, dk, c["max_abs"])
        assert max_diff(state, fx.arr(c["new_state"])) <= budget(fx.k, dk, c["max_abs"])
