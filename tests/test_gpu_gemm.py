"""The many-column matrix-core kernels (kq_gemm.hip: a prompt chunk's matmuls, model.rs:443-461 / matvec.rs:369-393)
through aq_matmul with 9..64 columns.

Bar: bit-exact. Every column equals the single-column kernel's output on that column (itself bit-exact to the
oracle, tests/test_gpu_ops.py) at the model's shapes, and equals the oracle directly on smaller ones, for Q4_K,
Q5_K, Q6_K (x Q8_K) and Q8_0, Q4_0 (x Q8_0), with row and column counts that are not multiples of the tiles."""
import os
import sys

import numpy as np
import pytest

import oracle_lib as O

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "qwen-3.8-in-rust_amd"))
import aqueduct as aq  # noqa: E402

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def ctx():
    return aq.Context(0)


def run(ctx, t, rows, cols, ncols, seed):
    spec = aq.synth_spec(t, rows, cols, seed=seed, b=0.02)
    host = aq.synth_host(spec).view(np.uint8)
    w = aq.SynthWeight(ctx, spec)
    x = (np.random.default_rng(seed).standard_normal((ncols, cols)) * 1.5).astype(np.float32)
    x[ncols // 2] *= 0.0  # an all-zero column (scales 0)
    a = aq.Act(ctx, cols, ncols)
    a.set(x)
    a.quantize(t, ncols)
    y = aq.matmul(ctx, w, a, ncols)
    return host, w, a, x, y


@pytest.mark.parametrize("t", [aq.Q4_K, aq.Q5_K, aq.Q6_K, aq.Q8_0, aq.Q4_0])
@pytest.mark.parametrize("rows,cols,ncols", [(37, 256, 9), (100, 512, 33), (130, 768, 64)])
def test_gemm_equals_oracle_small(ctx, t, rows, cols, ncols):
    print(f"case gemm type {t} {rows}x{cols} N={ncols}", flush=True)
    host, w, a, x, y = run(ctx, t, rows, cols, ncols, 300 + t + rows)
    want = O.matmul(t, host, rows, cols, x, threads=8)
    bad = int(np.sum(bits(y) != bits(want)))
    assert bad == 0, f"{bad} outputs differ from the oracle"


@pytest.mark.parametrize("t,rows,cols", [(aq.Q4_K, 17408, 5120), (aq.Q6_K, 5120, 17408), (aq.Q5_K, 1024, 6144),
                                         (aq.Q6_K, 10240, 5120), (aq.Q8_0, 5120, 6144), (aq.Q4_0, 1024, 10240)])
def test_gemm_columns_equal_single_column_kernel(ctx, t, rows, cols):
    ncols = 64
    print(f"case gemm full shape type {t} {rows}x{cols} N={ncols}", flush=True)
    host, w, a, x, y = run(ctx, t, rows, cols, ncols, 900 + t)
    keep = []
    for c in range(ncols):
        a1 = aq.Act(ctx, cols, 1)
        a1.set(x[c])
        a1.quantize(t, 1)
        keep.append(a1)
        y1 = aq.matmul(ctx, w, a1, 1)[0]
        assert np.array_equal(bits(y[c]), bits(y1)), f"column {c}: {int(np.sum(bits(y[c]) != bits(y1)))} differ"
    for a1 in keep:
        a1.free()
    # and a few columns straight against the oracle
    want = O.matmul(t, host, rows, cols, x[[0, ncols // 2, ncols - 1]], threads=8)
    assert np.array_equal(bits(y[[0, ncols // 2, ncols - 1]]), bits(want))


@pytest.mark.parametrize("t", [aq.Q8_0, aq.Q4_0])
def test_rows_not_a_multiple_of_256_take_column_pieces(ctx, t):
    rows, cols, ncols = 45, 160, 20
    print(f"case gemm pieces type {t} {rows}x{cols} N={ncols}", flush=True)
    host, w, a, x, y = run(ctx, t, rows, cols, ncols, 77 + t)
    want = O.matmul(t, host, rows, cols, x, threads=8)
    assert np.array_equal(bits(y), bits(want))


@pytest.mark.parametrize("t", [aq.Q4_K, aq.Q6_K])
def test_many_columns_under_q8_fine_equal_the_oracle(ctx, t):
    """Under the q8-fine switch (Q8_0-grain activations for K-quant weights, dot.rs:69-160) a 33-column product runs
    as 8-column pieces of the q8-fine kernel; every column equals the oracle's q8-fine dot."""
    rows, cols, ncols = 130, 512, 33
    print(f"case q8-fine many columns type {t}", flush=True)
    with aq.q8_fine(), O.q8_fine():
        host, w, a, x, y = run(ctx, t, rows, cols, ncols, 555 + t)
        want = O.matmul(t, host, rows, cols, x, threads=8)
    assert np.array_equal(bits(y), bits(want))


@pytest.mark.parametrize("ncols", [9, 33, 64])
def test_f32_many_columns_equal_the_oracle(ctx, ncols):
    """F32 weights (the DeltaNet ssm_alpha / ssm_beta projections) over a prompt chunk's columns: one launch, eight
    columns per work-group along the grid's second dimension (dot.rs:180-200 per column)."""
    rows, cols = 48, 5120
    print(f"case f32 many columns N={ncols}", flush=True)
    host, w, a, x, y = run(ctx, aq.F32, rows, cols, ncols, 808 + ncols)
    want = O.matmul(aq.F32, host, rows, cols, x, threads=8)
    assert np.array_equal(bits(y), bits(want))


@pytest.mark.parametrize("t,rows,cols,ncols", [(aq.Q4_K, 1024, 5120, 4), (aq.Q6_K, 520, 2048, 33),
                                               (aq.Q8_0, 300, 1024, 1)])
def test_quantize_and_matmul_on_a_caller_stream(ctx, t, rows, cols, ncols):
    """aq_act_quantize_on / aq_matmul_on queued on a stream the caller created (here through the HIP runtime this
    process already has loaded, the one libaq uses) give the synchronous calls' bits."""
    print(f"case caller stream type {t} {rows}x{cols} N={ncols}", flush=True)
    hip = aq.C.CDLL("libamdhip64.so.7")  # already mapped by libaq: the same runtime instance
    spec = aq.synth_spec(t, rows, cols, seed=31 + t)
    w = aq.SynthWeight(ctx, spec)
    x = (np.random.default_rng(5).standard_normal((ncols, cols)) * 1.5).astype(np.float32)
    a_sync = aq.Act(ctx, cols, ncols)
    a_sync.set(x)
    a_sync.quantize(t, ncols)
    want = aq.matmul(ctx, w, a_sync, ncols)
    a = aq.Act(ctx, cols, ncols)
    a.set(x)
    y = aq.DeviceBuffer(ctx, ncols * rows * 4)
    s = aq.C.c_void_p()
    assert hip.hipStreamCreate(aq.C.byref(s)) == 0
    try:
        aq.quantize_on(a, t, ncols, s.value)
        aq.matmul_on(ctx, w, a, ncols, y, s.value)
        assert hip.hipStreamSynchronize(s) == 0
    finally:
        hip.hipStreamDestroy(s)
    got = y.download(np.float32, ncols * rows).reshape(ncols, rows)
    assert np.array_equal(bits(got), bits(want))
    for o in (y, a, a_sync):
        o.free()
