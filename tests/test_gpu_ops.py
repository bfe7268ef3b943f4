"""GPU parity of the operator-level path (gfx950) against the CPU oracle, through the C-ABI.

Bar: bit-exact for the integer / byte work (Q8_K and Q8_0 quantisation, weight repack round trip, the K-quant
integer lane sums) and bit-exact fp32 for every matmul, because the kernels reproduce the reference's
accumulation order (kdot.rs:1-18, dot.rs:29-66, 180-200); plus the identity contract: column c of an N-column
(verify) call equals the 1-column call on that column bit for bit (kdot.rs:164-173)."""
import json
import os
import sys

import numpy as np
import pytest

import aqueduct as aq
import oracle_lib as O

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "kernels")


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = aq.Context(0)
    yield c
    c.close()


def fixture(group):
    d = os.path.join(GOLD, group)
    with open(os.path.join(d, "manifest.json")) as f:
        return d, json.load(f)


def npy(d, field):
    return np.load(os.path.join(d, field["file"]), allow_pickle=False).astype(np.float32)


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_q8k_quantize_matches_fixture_bytes(ctx):
    d, m = fixture("q8k_quantize")
    for c in m["cases"]:
        width = c["width"]
        x = npy(d, c["x"]).reshape(-1, width)
        raw = np.fromfile(os.path.join(d, c["raw"]["file"]), np.uint8).reshape(x.shape[0], -1)
        say(f"q8k {c['case']}: {x.shape[0]} rows")
        for r0 in range(0, x.shape[0], 8):
            rows = x[r0:r0 + 8]
            a = aq.Act(ctx, width, rows.shape[0])
            a.set(rows)
            a.quantize(aq.Q4_K, rows.shape[0])
            got = a.q8k(rows.shape[0])
            for i in range(rows.shape[0]):
                assert np.array_equal(got[i], raw[r0 + i]), f"{c['case']} row {r0 + i} ({c['rows'][r0 + i]})"
            a.free()


def test_q8_0_quantize_matches_fixture_bytes(ctx):
    d, m = fixture("q8_quantize")
    for c in m["cases"]:
        width = c["width"]
        x = npy(d, c["x"]).reshape(-1, width)
        raw = np.fromfile(os.path.join(d, c["raw"]["file"]), np.uint8).reshape(x.shape[0], -1)
        say(f"q8_0 {c['case']}")
        for r0 in range(0, x.shape[0], 8):
            rows = x[r0:r0 + 8]
            a = aq.Act(ctx, width, rows.shape[0])
            a.set(rows)
            a.quantize(aq.Q8_0, rows.shape[0])
            got = a.q8_0(rows.shape[0])
            for i in range(rows.shape[0]):
                assert np.array_equal(got[i], raw[r0 + i]), f"{c['case']} row {r0 + i}"
            a.free()


def test_quantize_random_rows_match_oracle(ctx):
    rng = np.random.default_rng(11)
    n, ncols = 17408, 8
    x = (rng.standard_normal((ncols, n)) * np.array([1, 1e-3, 1e3, 1, 5, 0.1, 1, 20])[:, None]).astype(np.float32)
    x[3, 256:512] = 0.0  # an all-zero block
    say("random q8k/q8_0 rows 8 x 17408")
    a = aq.Act(ctx, n, ncols)
    a.set(x)
    a.quantize(aq.Q6_K, ncols)
    a.quantize(aq.Q8_0, ncols)
    gk, g0 = a.q8k(ncols), a.q8_0(ncols)
    for c in range(ncols):
        assert np.array_equal(gk[c], O.q8k_quantize(x[c])), f"q8k column {c}"
        assert np.array_equal(g0[c], O.q8_0_quantize(x[c])), f"q8_0 column {c}"


@pytest.mark.parametrize("t", [aq.Q4_K, aq.Q5_K, aq.Q6_K, aq.Q8_0, aq.Q4_0, aq.F32])
def test_weight_repack_round_trip_and_device_synth(ctx, t):
    rows, cols = 96, 1536
    spec = aq.synth_spec(t, rows, cols, seed=77 + t, b=0.02)
    host = aq.synth_host(spec)
    say(f"repack/synth type {t}")
    w = aq.Weight(ctx, t, rows, cols, host)
    assert np.array_equal(w.download(), host.view(np.uint8))
    sw = aq.SynthWeight(ctx, spec)
    assert np.array_equal(sw.download(), host.view(np.uint8)), "device synth differs from host synth"


def kquant_dot_rows():
    d, m = fixture("dot")
    for c in m["cases"]:
        t = O.TYPE_BY_NAME[c["ggml_type"]]
        yield d, c, t


def test_kquant_isums_bit_exact_on_fixture_rows(ctx):
    for d, c, t in kquant_dot_rows():
        if t not in (aq.Q4_K, aq.Q5_K, aq.Q6_K):
            continue
        width, n_rows = c["width"], c["n_rows"]
        w_raw = np.fromfile(os.path.join(d, c["w_raw"]["file"]), np.uint8).reshape(n_rows, -1)
        x_deq = npy(d, c["x_deq"]).reshape(n_rows, width)
        say(f"isums {c['case']}")
        w = aq.Weight(ctx, t, n_rows, width, w_raw)
        for r in range(n_rows):
            a = aq.Act(ctx, width, 1)
            a.set(x_deq[r])
            a.quantize(t, 1)
            lanes, mins = aq.kq_isums(ctx, w, a)
            want_l, want_m = O.kq_isums(t, w_raw[r], O.q8k_quantize(x_deq[r]), width)
            assert np.array_equal(lanes[0, r].ravel(), want_l), f"{c['case']} row {r} lanes"
            assert np.array_equal(mins[0, r].ravel(), want_m), f"{c['case']} row {r} mins"
            y = aq.matmul(ctx, w, a, 1)
            want = O.dot_q8k(t, w_raw[r], O.q8k_quantize(x_deq[r]), width)
            assert bits_equal(y[0, r], want), f"{c['case']} row {r}: {y[0, r]} vs {want}"
            a.free()
        w.free()


def test_q8_weight_dots_bit_exact_on_fixture_rows(ctx):
    for d, c, t in kquant_dot_rows():
        if t not in (aq.Q8_0, aq.Q4_0, aq.F32):
            continue
        width, n_rows = c["width"], c["n_rows"]
        say(f"q8 dots {c['case']}")
        if t == aq.F32:
            wf = npy(d, c["w_deq"]).reshape(n_rows, width)
            xf = npy(d, c["x_deq"]).reshape(n_rows, width)
            w = aq.Weight(ctx, t, n_rows, width, wf)
            a = aq.Act(ctx, width, 1)
            for r in range(n_rows):
                a.set(xf[r])
                y = aq.matmul(ctx, w, a, 1)
                want = O.lib().or_dot_f32(O.ptr(np.ascontiguousarray(wf[r])), O.ptr(np.ascontiguousarray(xf[r])), width)
                assert bits_equal(y[0, r], want), f"{c['case']} row {r}"
            continue
        w_raw = np.fromfile(os.path.join(d, c["w_raw"]["file"]), np.uint8).reshape(n_rows, -1)
        x_deq = npy(d, c["x_deq"]).reshape(n_rows, width)
        w = aq.Weight(ctx, t, n_rows, width, w_raw)
        a = aq.Act(ctx, width, 1)
        for r in range(n_rows):
            a.set(x_deq[r])
            a.quantize(t, 1)
            y = aq.matmul(ctx, w, a, 1)
            want = O.dot_q8(t, w_raw[r], O.q8_0_quantize(x_deq[r]), width)
            assert bits_equal(y[0, r], want), f"{c['case']} row {r}: {y[0, r]} vs {want}"


@pytest.mark.parametrize("t,rows,cols", [(aq.Q4_K, 17408, 5120), (aq.Q6_K, 5120, 17408), (aq.Q5_K, 1024, 5120)])
def test_kquant_isums_full_shapes_on_the_matmul_kernel(ctx, t, rows, cols):
    """Config 2's integer contract on the kernel the product runs: the exact i32 lane sums and min products of every
    (row, super-block) from kq_wave_kernel (its integer-output instance, same grid), N = 1 and each column of N = 4,
    equal the reference's sumi / prod (kdot.rs:37-140) from the oracle."""
    say(f"isums full shape type {t} {rows}x{cols}")
    spec = aq.synth_spec(t, rows, cols, seed=4048 + t, b=0.02)
    host = aq.synth_host(spec).view(np.uint8)
    w = aq.SynthWeight(ctx, spec)
    x = np.random.default_rng(31 + t).standard_normal((4, cols)).astype(np.float32)
    a = aq.Act(ctx, cols, 4)
    a.set(x)
    a.quantize(t, 4)
    for n in (1, 4):
        lanes, mins = aq.kq_isums(ctx, w, a, n)
        for c in range(n):
            want_l, want_m = O.kq_isums_mat(t, host, rows, O.q8k_quantize(x[c]), cols)
            bad = int(np.sum(lanes[c] != want_l))
            assert bad == 0, f"N={n} column {c}: {bad} lane sums differ"
            assert np.array_equal(mins[c], want_m), f"N={n} column {c}: min products differ"


@pytest.mark.parametrize("t,rows,cols", [(aq.Q4_K, 17408, 5120), (aq.Q6_K, 5120, 17408), (aq.Q5_K, 1024, 5120),
                                         (aq.Q4_K, 12288, 5120), (aq.Q4_K, 5120, 6144), (aq.Q6_K, 10240, 5120),
                                         (aq.Q5_K, 5120, 6144), (aq.Q4_K, 1000, 512),
                                         (aq.Q8_0, 5120, 6144), (aq.Q4_0, 1024, 5120), (aq.Q4_0, 512, 17408),
                                         (aq.F32, 48, 5120)])
def test_matmul_full_shapes_bit_exact_and_column_identity(ctx, t, rows, cols):
    """Config 2 (N = 1) and config 3 (N = k+1 for k in 1, 3, 5, 7) at the real shapes: every output equals the
    oracle bit for bit, and each column of an N-column call equals the 1-column call."""
    say(f"full-shape matmul type {t} {rows}x{cols}")
    spec = aq.synth_spec(t, rows, cols, seed=2024 + t, b=0.02)
    host = aq.synth_host(spec)
    w = aq.SynthWeight(ctx, spec)
    rng = np.random.default_rng(t)
    x = rng.standard_normal((8, cols)).astype(np.float32)
    a = aq.Act(ctx, cols, 8)
    a.set(x)
    a.quantize(t, 8)
    y1 = np.stack([aq.matmul(ctx, w, _single(ctx, x[c], t), 1)[0] for c in range(8)])
    want = O.matmul(t, host.view(np.uint8), rows, cols, x, threads=8)
    assert bits_equal(y1, want), f"N=1 vs oracle: {np.sum(y1.view(np.uint32) != want.view(np.uint32))} mismatches"
    for n in (2, 4, 6, 8):
        yn = aq.matmul(ctx, w, a, n)
        assert bits_equal(yn, y1[:n]), f"N={n} columns differ from N=1"


@pytest.mark.parametrize("t,rows,cols", [(aq.Q4_K, 37, 1280), (aq.Q5_K, 4, 1024), (aq.Q6_K, 4099, 1536),
                                         (aq.Q4_K, 8192, 1024), (aq.Q6_K, 6, 2304)])
def test_lane_half_edge_shapes_bit_exact(ctx, t, rows, cols):
    """Single K-quant matrices of at most 8192 rows take the lane-half kernel (a pair of waves per tile of 4 rows):
    row counts that are not a multiple of 4 (the last tile's rows clamped, nothing stored past the matrix), a single
    pair, super-block counts that leave a partial last round (5, 6, 9 of 4 per round), and every column count 1..8:
    each output equals the oracle bit for bit, and the integer lane sums equal the reference's at N = 1 and 4."""
    say(f"lane-half edge shape type {t} {rows}x{cols}")
    spec = aq.synth_spec(t, rows, cols, seed=77 + rows + t, b=0.02)
    host = aq.synth_host(spec)
    w = aq.SynthWeight(ctx, spec)
    x = np.random.default_rng(rows + cols).standard_normal((8, cols)).astype(np.float32)
    a = aq.Act(ctx, cols, 8)
    a.set(x)
    a.quantize(t, 8)
    want = O.matmul(t, host.view(np.uint8), rows, cols, x, threads=8)
    for n in range(1, 9):
        yn = aq.matmul(ctx, w, a, n)
        bad = int(np.sum(yn.view(np.uint32) != want[:n].view(np.uint32)))
        assert bad == 0, f"N={n}: {bad} outputs differ from the oracle"
    for n in (1, 4):
        lanes, mins = aq.kq_isums(ctx, w, a, n)
        for c in range(n):
            want_l, want_m = O.kq_isums_mat(t, host.view(np.uint8), rows, O.q8k_quantize(x[c]), cols)
            assert np.array_equal(lanes[c], want_l), f"N={n} column {c}: lane sums differ"
            assert np.array_equal(mins[c], want_m), f"N={n} column {c}: min products differ"
    a.free()
    w.free()


_single_cache = {}


def _single(ctx, xrow, t):
    a = aq.Act(ctx, xrow.size, 1)
    a.set(xrow)
    a.quantize(t, 1)
    _single_cache.setdefault("keep", []).append(a)
    return a


def test_read_floor_time(ctx):
    """The measurement helper aq_read_floor_time (the plain streaming read bench.py reports beside the dominant
    kernel): a positive time that grows with the bytes read, and a clear error for a size that is not whole
    16-byte loads."""
    say("read floor timing")
    t_small = aq.read_floor_time(ctx, 1 << 20, iters=50, nbuf=2)
    t_big = aq.read_floor_time(ctx, 64 << 20, iters=50, nbuf=2)
    assert 0.0 < t_small < t_big
    buf, part = aq.DeviceBuffer(ctx, 4096), aq.DeviceBuffer(ctx, 2048 * 4)
    arr = (aq.C.c_void_p * 1)(buf.p.value)
    us = aq.C.c_double()
    rc = aq.lib().aq_read_floor_time(ctx.h, arr, 1, 4000 + 8, part.p, 1, aq.C.byref(us))
    assert rc != 0 and "multiple of 16" in aq.lib().aq_last_error().decode()
    buf.free()
    part.free()
