"""The oracle's AVX2 dots (oracle/oracle_simd.c: the form bench.py's cpu_baseline times) against its scalar ones.

The reference's CPU path runs hand-written AVX2 kernels that are bit-identical to its scalar kernels (avx2.rs:1-20,
checked by its tests/avx2.rs on every kernel fixture and on random rows). The same property here: with the simd
switch on, every K-quant x Q8_K dot (every tile width 1..16), every Q8_0 / Q4_0 dot, the row-parallel matmul and a
whole model's logits equal the scalar forms bit for bit — on the reference's dot fixtures, on random rows with
extreme codes (activation codes of -128, the largest weight codes of each type, negative Q6_K scales) and on a
K of 17408 (68 super-blocks). The scalar forms are the ones the fixtures pin (test_oracle_kernels.py)."""
import json
import os

import numpy as np
import pytest

import oracle_lib as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "kernels", "dot")


def both(fn):
    """fn() with the switch off, then on: the two results."""
    with O.simd(False):
        a = fn()
    with O.simd(True):
        b = fn()
    return a, b


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


def fixture_cases():
    with open(os.path.join(GOLD, "manifest.json")) as f:
        m = json.load(f)

    def raw(field):
        with open(os.path.join(GOLD, field["file"]), "rb") as f:
            return np.frombuffer(f.read(), np.uint8)

    def arr(field):
        return np.load(os.path.join(GOLD, field["file"]), allow_pickle=False).astype(np.float32).ravel()

    return m["cases"], raw, arr


def random_weight_rows(rng, t, n_rows, width):
    """Random bytes with finite f16 scales; every code value of the type is reachable."""
    rb = O.row_bytes(t, width)
    w = rng.integers(0, 256, n_rows * rb, dtype=np.uint8).reshape(n_rows, rb)
    bb = {O.Q4_K: 144, O.Q5_K: 176, O.Q6_K: 210, O.Q8_0: 34, O.Q4_0: 18}[t]
    nblk = rb // bb
    h = (rng.uniform(-1, 1, (n_rows, nblk, 2)) * 0.05).astype(np.float16).view(np.uint8).reshape(n_rows, nblk, 4)
    blocks = w.reshape(n_rows, nblk, bb)
    if t == O.Q6_K:
        blocks[:, :, 208:210] = h[:, :, 0:2]
    elif t in (O.Q4_K, O.Q5_K):
        blocks[:, :, 0:4] = h
    else:
        blocks[:, :, 0:2] = h[:, :, 0:2]
    return w


def extreme_q8k(rng, width):
    """Q8_K rows (ggml wire layout) from scaled normals, one with codes forced to -128 / 127 in places."""
    out = [O.q8k_quantize((rng.standard_normal(width) * s).astype(np.float32)) for s in (1.0, 0.01, 100.0)]
    planted = out[0].copy()
    for b in range(width // 256):
        codes = planted[b * 292 + 4:b * 292 + 260].view(np.int8)
        codes[::7] = -128
        codes[3::11] = 127
    out.append(planted)
    return out


@pytest.mark.parametrize("t", [O.Q4_K, O.Q5_K, O.Q6_K])
def test_kquant_q8k_simd_equals_scalar_on_fixtures(t):
    cases, raw, arr = fixture_cases()
    rng = np.random.default_rng(11)
    seen = 0
    for c in cases:
        if O.TYPE_BY_NAME[c["ggml_type"]] != t:
            continue
        width, n_rows = c["width"], c["n_rows"]
        w_raw = raw(c["w_raw"])
        x_deq = arr(c["x_deq"]).reshape(n_rows, width)
        rb = O.row_bytes(t, width)
        for r in range(n_rows):
            wrow = w_raw[r * rb:(r + 1) * rb]
            xs = [O.q8k_quantize(x_deq[r])] + extreme_q8k(rng, width) * 3
            for tile in (1, 2, 4, 7, 8, 16):
                a, b = both(lambda: O.dot_q8k_t(t, wrow, xs[:tile], width))
                assert same_bits(a, b), f"{c['case']} row {r} tile {tile}"
            seen += 1
    assert seen >= 3


@pytest.mark.parametrize("t", [O.Q4_K, O.Q5_K, O.Q6_K])
@pytest.mark.parametrize("width", [256, 17408])
def test_kquant_q8k_simd_equals_scalar_random(t, width):
    rng = np.random.default_rng(5 + t + width)
    w = random_weight_rows(rng, t, 6, width)
    xs = extreme_q8k(rng, width) * 4
    for r in range(w.shape[0]):
        for tile in (1, 3, 4, 8, 16):
            a, b = both(lambda: O.dot_q8k_t(t, w[r], xs[:tile], width))
            assert same_bits(a, b), f"row {r} tile {tile}"


def test_kquant_simd_discriminates():
    """A planted mistake shows: the simd form with one code bit flipped is not the scalar form."""
    rng = np.random.default_rng(3)
    w = random_weight_rows(rng, O.Q4_K, 1, 256)[0]
    xs = extreme_q8k(rng, 256)
    with O.simd(False):
        a = O.dot_q8k_t(O.Q4_K, w, xs, 256)
    w2 = w.copy()
    w2[16] ^= 0x01
    with O.simd(True):
        b = O.dot_q8k_t(O.Q4_K, w2, xs, 256)
    assert not same_bits(a, b)


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_0])
def test_q8_0_q4_0_simd_equals_scalar(t):
    cases, raw, arr = fixture_cases()
    seen = 0
    for c in cases:
        if O.TYPE_BY_NAME[c["ggml_type"]] != t:
            continue
        width, n_rows = c["width"], c["n_rows"]
        w_raw, x_raw = raw(c["w_raw"]), raw(c["x_raw"])
        wrb, xrb = O.row_bytes(t, width), width // 32 * 34
        for r in range(n_rows):
            wr, xr = w_raw[r * wrb:(r + 1) * wrb], x_raw[r * xrb:(r + 1) * xrb]
            a, b = both(lambda: O.dot_q8(t, wr, xr, width))
            assert same_bits(a, b), f"{c['case']} row {r}"
            seen += 1
    assert seen >= 2
    rng = np.random.default_rng(9 + t)
    for width in (32, 6144):
        w = random_weight_rows(rng, t, 4, width)
        if t == O.Q8_0:  # weight codes of -128 too
            w.reshape(4, -1, 34)[:, :, 2::9] = 0x80
        for s in (1.0, 0.01, 100.0):
            xq = O.q8_0_quantize((rng.standard_normal(width) * s).astype(np.float32)).copy()
            xq.reshape(-1, 34)[:, 2::5] = 0x80  # activation codes of -128
            for r in range(4):
                a, b = both(lambda: O.dot_q8(t, w[r], xq, width))
                assert same_bits(a, b), f"width {width} scale {s} row {r}"


@pytest.mark.parametrize("t", [O.Q4_K, O.Q5_K, O.Q6_K, O.Q8_0, O.Q4_0, O.F32])
def test_matmul_simd_equals_scalar(t):
    """The row-parallel matmul (matvec.rs:483-539) over 1, 4 and 20 columns (a 16-column tile and a 4-column one)."""
    rng = np.random.default_rng(21 + t)
    rows, cols = 37, 1024
    if t == O.F32:
        w = rng.standard_normal((rows, cols)).astype(np.float32).view(np.uint8).ravel()
    else:
        w = random_weight_rows(rng, t, rows, cols).ravel()
    for n in (1, 4, 20):
        x = rng.standard_normal((n, cols)).astype(np.float32)
        a, b = both(lambda: O.matmul(t, w, rows, cols, x, threads=4))
        assert same_bits(a, b), f"columns {n}"


def test_tiny_model_logits_simd_equal_scalar():
    """A whole model: the tiny hybrid's prefill and 6 greedy steps, every logit, with the switch off and on."""
    import aqueduct as aq
    cfg = aq.tiny_config()
    tensors = aq.plan_tensors(aq.model_plan(cfg, aq.MIX_TINY, 20260905))
    ocfg = O.AqModelConfig()
    for name, _ in O.AqModelConfig._fields_:
        setattr(ocfg, name, getattr(cfg, name))
    om = O.Model(ocfg, tensors, threads=4)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, 12).astype(np.uint32)

    def run():
        st = O.State(om, 0, 64)
        tok, lg = st.prefill(prompt, want_logits=True)
        out = [lg]
        for _ in range(6):
            tok, lg = st.forward_token(tok, want_logits=True)
            out.append(lg)
        return np.stack(out)

    a, b = both(run)
    assert same_bits(a, b)
