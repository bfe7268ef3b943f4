"""aq_argmax_noalloc (the allocation-free variant of aq_argmax, whose partial results live in a fixed device array)
against aq_argmax, through the C-ABI: two calls in a row, the second with a smaller input, then the size limit."""
import ctypes as C

import numpy as np
import pytest

import aqueduct as aq

pytestmark = pytest.mark.gpu


def test_argmax_noalloc_equals_argmax_on_consecutive_calls():
    ctx = aq.Context(0)
    L = aq.lib()
    rng = np.random.default_rng(17)
    for t, n in ((16, 1 << 20), (3, 4099)):  # the largest accepted call, then a smaller one
        print(f"case argmax_noalloc t={t} n={n}", flush=True)
        x = rng.standard_normal((t, n)).astype(np.float32)
        x[0, [7, n - 1]] = 50.0  # a tie: the first wins
        x[1, 0] = np.nan  # a NaN at index 0: the answer is 0
        x[2, : n // 2] = -np.inf
        xb = aq.DeviceBuffer(ctx, x.nbytes)
        xb.upload(x)
        ia, ib = aq.DeviceBuffer(ctx, t * 4), aq.DeviceBuffer(ctx, t * 4)
        aq.check(L.aq_argmax(ctx.h, xb.p, n, t, ia.p))
        aq.check(L.aq_argmax_noalloc(ctx.h, xb.p, n, t, ib.p))
        a, b = ia.download(np.uint32, t), ib.download(np.uint32, t)
        assert np.array_equal(a, b), f"t={t} n={n}: noalloc {b} vs argmax {a}"
        assert a[0] == 7 and a[1] == 0
        for r in range(3, t):
            assert a[r] == int(np.argmax(x[r]))
    xb = aq.DeviceBuffer(ctx, 64)
    ib = aq.DeviceBuffer(ctx, 64)
    assert L.aq_argmax_noalloc(ctx.h, xb.p, (1 << 20) + 1, 1, ib.p) == -1  # past the limit: refused, nothing runs
    assert b"at most" in L.aq_last_error()
    assert L.aq_argmax_noalloc(ctx.h, xb.p, 16, 17, ib.p) == -1
