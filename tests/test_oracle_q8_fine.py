"""The oracle's `--q8-fine` K-quant x Q8_0 dots (dot.rs:69-160) and its process-wide switch (matvec.rs:127-160).

* The reference's own tests of these kernels: tests/kernels.rs:213-249 (`dot_kernels_within_budget` runs `dot_q8` on
  every fixture type, K-quants included, against the fixture's Q8_0 activation rows) and :251-291 (the matvec
  fixture): |dot - f64 reference| within the K-quant term-magnitude budget (tests/common/mod.rs:108-131).
* The budget tells plausible mistakes apart: the same f64 dot with one mistake planted in the weights' decoded
  values (the Q6_K -32 offset dropped, its two group scales swapped, the Q4_K/Q5_K mins dropped, added with the wrong
  sign, or taken from the neighbouring sub-block) lands outside it on the fixture rows; the correct decoding, rebuilt
  here from codes and scales and equal to the pinned dequantiser, lands inside.
* The switch: on, the oracle's matmul of K-quant weights equals its per-row `dot_q8` bit for bit (matvec.rs:282-292
  `one_row` -> `dot_q8`) and is thread-invariant; off, it is the Q8_K blocked path again.
* The integer part is exact: with every activation scale and weight scale a power of two and small codes, each f32
  product and sum is exact, so the dot equals the integer sum of q_w * q_x * scales computed in Python integers
  (what fixes the lane sums, the -32 fold and the min term independently of their f32 order).
The placement of the -32 offset in lanes 0 and 4 (rather than spread over lanes 0..7) changes only f32 rounding, which
no fixture of the reference records for this form: that placement follows dot.rs:145-146 by reading.
"""
import numpy as np
import pytest

import oracle_lib as O
from test_oracle_kernels import Fx, kquant_terms_budget

KQ = (O.Q4_K, O.Q5_K, O.Q6_K)


def f16(b, off):
    return float(np.frombuffer(b[off:off + 2].tobytes(), np.float16)[0])


def scale_min_k4(s, q):
    if s < 4:
        return int(q[s] & 63), int(q[s + 4] & 63)
    return int((q[s + 4] & 0xF) | ((q[s - 4] >> 6) << 4)), int((q[s + 4] >> 4) | ((q[s] >> 6) << 4))


def decode(t, wrow, width):
    """Per element: (code, scale, min, the weight's d, dmin) of a K-quant row, from the ggml bytes (quant.rs:65-219,
    docs/quant-layouts.md). Codes are unsigned; Q6_K's value is d * sc * (code - 32)."""
    nsb = width // 256
    bb = {O.Q4_K: 144, O.Q5_K: 176, O.Q6_K: 210}[t]
    code = np.zeros(width, np.int64)
    sc = np.zeros(width, np.int64)
    mn = np.zeros(width, np.int64)
    d = np.zeros(width)
    dmin = np.zeros(width)
    for sb in range(nsb):
        wb = wrow[sb * bb:(sb + 1) * bb]
        base = sb * 256
        if t == O.Q6_K:
            d[base:base + 256] = f16(wb, 208)
            for e in range(256):
                g, l = divmod(e, 128)
                k, li = divmod(l, 32)
                byte = wb[g * 64 + (k & 1) * 32 + li]
                lo = (byte & 0xF) if k < 2 else (byte >> 4)
                hi = (wb[128 + g * 32 + li] >> (2 * k)) & 3
                code[base + e] = lo | (hi << 4)
                sc[base + e] = np.int8(wb[192 + g * 8 + 2 * k + li // 16])
            continue
        d[base:base + 256], dmin[base:base + 256] = f16(wb, 0), f16(wb, 2)
        qoff = 48 if t == O.Q5_K else 16
        for s in range(8):
            scs, ms = scale_min_k4(s, wb[4:16])
            for j in range(32):
                byte = wb[qoff + (s // 2) * 32 + j]
                c = (byte & 0xF) if s % 2 == 0 else (byte >> 4)
                if t == O.Q5_K and wb[16 + j] & (1 << s):
                    c += 16
                code[base + s * 32 + j] = c
                sc[base + s * 32 + j] = scs
                mn[base + s * 32 + j] = ms
    return code, sc, mn, d, dmin


def values(t, dec, mutant=None):
    """The decoded weights in f64, with an optional planted mistake."""
    code, sc, mn, d, dmin = dec
    if t == O.Q6_K:
        if mutant == "q6_offset_dropped":
            return d * sc * code
        if mutant == "q6_scales_swapped":
            sw = sc.reshape(-1, 2, 16)[:, ::-1, :].reshape(-1)
            return d * sw * (code - 32)
        return d * sc * (code - 32)
    m = mn.astype(np.float64) * dmin
    if mutant == "mins_dropped":
        return d * sc * code
    if mutant == "mins_sign":
        return d * sc * code + m
    if mutant == "mins_neighbour":
        return d * sc * code - m.reshape(-1, 2, 32)[:, ::-1, :].reshape(-1)
    return d * sc * code - m


MUTANTS = {O.Q4_K: ("mins_dropped", "mins_sign", "mins_neighbour"), O.Q5_K: ("mins_dropped", "mins_sign",
                                                                             "mins_neighbour"),
           O.Q6_K: ("q6_offset_dropped", "q6_scales_swapped")}


def kq_cases(group):
    fx = Fx(group)
    for c in fx.cases:
        t = O.TYPE_BY_NAME[c["ggml_type"]]
        if t in KQ:
            yield fx, c, t


def test_q8_fine_dots_within_budget_on_the_dot_fixture():
    seen = 0
    for fx, c, t in kq_cases("dot"):
        width, n_rows = c["width"], c["n_rows"]
        w_raw, x_raw = fx.raw(c["w_raw"]), fx.raw(c["x_raw"])
        wrb, xrb = O.row_bytes(t, width), width // 32 * 34
        for r in range(n_rows):
            wrow, xrow = w_raw[r * wrb:(r + 1) * wrb], x_raw[r * xrb:(r + 1) * xrb]
            got = O.dot_q8(t, wrow, xrow, width)
            xd = O.dequant(O.Q8_0, xrow, width)
            bud = kquant_terms_budget(t, wrow, O.dequant(t, wrow, width), xd, fx.k)
            assert abs(got - c["ref_f64"][r]) <= bud, f"{c['case']} row {r}: {got} vs {c['ref_f64'][r]} ({bud})"
            seen += 1
    assert seen >= 21


def test_the_budget_catches_planted_mistakes():
    caught = {t: set() for t in KQ}
    for fx, c, t in kq_cases("dot"):
        width = c["width"]
        w_raw, x_raw = fx.raw(c["w_raw"]), fx.raw(c["x_raw"])
        wrb, xrb = O.row_bytes(t, width), width // 32 * 34
        r = c["rows"].index("random") if "random" in c["rows"] else 0
        wrow, xrow = w_raw[r * wrb:(r + 1) * wrb], x_raw[r * xrb:(r + 1) * xrb]
        xd = O.dequant(O.Q8_0, xrow, width).astype(np.float64)
        wd = O.dequant(t, wrow, width)
        dec = decode(t, wrow, width)
        assert np.array_equal(values(t, dec).astype(np.float32), wd), c["case"]  # the decoding is the pinned one
        bud = kquant_terms_budget(t, wrow, wd, xd.astype(np.float32), fx.k)
        assert abs(float(values(t, dec) @ xd) - c["ref_f64"][r]) <= bud
        for mu in MUTANTS[t]:
            if abs(float(values(t, dec, mu) @ xd) - c["ref_f64"][r]) > bud:
                caught[t].add(mu)
    for t in KQ:
        assert caught[t] == set(MUTANTS[t]), (t, caught[t])


def test_q8_fine_matvec_fixture_and_the_switch():
    for fx, c, t in kq_cases("matvec"):
        rows, width = c["n_rows"], c["width"]
        w, xr = fx.raw(c["w_raw"]), fx.raw(c["x_raw"])
        rb = O.row_bytes(t, width)
        xd = O.dequant(O.Q8_0, xr, width)
        per_row = np.array([O.dot_q8(t, w[r * rb:(r + 1) * rb], xr, width) for r in range(rows)], np.float32)
        for r in range(rows):
            bud = kquant_terms_budget(t, w[r * rb:(r + 1) * rb], O.dequant(t, w[r * rb:(r + 1) * rb], width), xd,
                                      fx.k)
            assert abs(float(per_row[r]) - c["ref_f64"][r]) <= bud, f"{c['case']} row {r}"
        # the fixture's activation row re-quantises to itself, so the matmul sees the same Q8_0 row
        assert np.array_equal(np.frombuffer(O.q8_0_quantize(xd), np.uint8), xr)
        with O.q8_fine():
            y1 = O.matmul(t, w, rows, width, xd[None, :], threads=1)[0]
            y5 = O.matmul(t, w, rows, width, xd[None, :], threads=5)[0]
        assert np.array_equal(y1.view(np.uint32), per_row.view(np.uint32)), c["case"]
        assert np.array_equal(y5.view(np.uint32), y1.view(np.uint32))
        yk = O.matmul(t, w, rows, width, xd[None, :], threads=2)[0]
        want = np.array([O.dot_q8k(t, w[r * rb:(r + 1) * rb], O.q8k_quantize(xd), width) for r in range(rows)],
                        np.float32)
        assert np.array_equal(yk.view(np.uint32), want.view(np.uint32)), "switch off: the Q8_K path"
    assert O.lib().or_q8_fine() == 0


def exact_case(t, seed, width=512):
    """A K-quant row and a Q8_0 activation row whose dot is exact in f32: every scale a power of two, codes small."""
    rng = np.random.default_rng(seed)
    nsb = width // 256
    bb = {O.Q4_K: 144, O.Q5_K: 176, O.Q6_K: 210}[t]
    w = rng.integers(0, 256, nsb * bb, dtype=np.uint8)
    for sb in range(nsb):
        wb = w[sb * bb:(sb + 1) * bb]
        if t == O.Q6_K:
            wb[208:210] = np.frombuffer(np.float16(2.0 ** -int(rng.integers(4, 8))).tobytes(), np.uint8)
            wb[192:208] = rng.choice(np.array([1, 2, 4, 8, -1, -2, -4, -8], np.int8), 16).view(np.uint8)
        else:
            wb[0:2] = np.frombuffer(np.float16(2.0 ** -int(rng.integers(4, 8))).tobytes(), np.uint8)
            wb[2:4] = np.frombuffer(np.float16(2.0 ** -int(rng.integers(4, 8))).tobytes(), np.uint8)
            # 6-bit scales and mins as powers of two (1, 2, 4, 8, 16, 32)
            sc = 2 ** rng.integers(0, 6, 8)
            mn = 2 ** rng.integers(0, 6, 8)
            q = np.zeros(12, np.uint8)
            for s in range(4):
                q[s] = sc[s] & 63 | ((sc[s + 4] >> 4) << 6)
                q[s + 4] = mn[s] & 63 | ((mn[s + 4] >> 4) << 6)
                q[s + 8] = (sc[s + 4] & 0xF) | ((mn[s + 4] & 0xF) << 4)
            wb[4:16] = q
    nb = width // 32
    x = np.zeros(nb * 34, np.uint8)
    for b in range(nb):
        x[b * 34:b * 34 + 2] = np.frombuffer(np.float16(2.0 ** -int(rng.integers(2, 6))).tobytes(), np.uint8)
        x[b * 34 + 2:b * 34 + 34] = rng.integers(-8, 9, 32).astype(np.int8).view(np.uint8)
    return w, x


@pytest.mark.parametrize("t", KQ)
def test_q8_fine_integer_content_is_exact(t):
    from fractions import Fraction
    width = 512
    for seed in range(6):
        w, x = exact_case(t, seed, width)
        code, sc, mn, d, dmin = decode(t, w, width)
        xs = np.array([f16(x, b * 34) for b in range(width // 32)])
        xq = np.concatenate([x[b * 34 + 2:b * 34 + 34].view(np.int8) for b in range(width // 32)]).astype(np.int64)
        want = Fraction(0)
        for e in range(width):
            dx = Fraction(xs[e // 32])
            if t == O.Q6_K:
                want += Fraction(d[e]) * int(sc[e]) * (int(code[e]) - 32) * int(xq[e]) * dx
            else:
                want += (Fraction(d[e]) * int(sc[e]) * int(code[e]) - Fraction(dmin[e]) * int(mn[e])) * int(xq[e]) * dx
        got = O.dot_q8(t, w, x, width)
        assert Fraction(float(got)) == want, (t, seed, got, float(want))
