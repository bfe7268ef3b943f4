"""exp and log1p of the activations: the device's restatement (aq_math.h) against the functions the reference calls.

The reference's f32 `exp` / `ln_1p` (act.rs:7-40, softmax.rs:22-49, deltanet.rs:43-86) are GNU libc's `expf` /
`log1pf`. aq_math.h restates the two glibc 2.35 algorithms; the oracle calls the platform libm itself.

* exhaustive: every one of the 2^32 f32 bit patterns gives the same bits from the restatement (compiled for the host)
  as from the platform libm, for exp and log1p; strided sweeps for silu / sigmoid / softplus built on them. The
  sweep is sensitive to the algorithm's details: associating fdlibm's final correction term as (c + k*ln2_lo)
  instead of (k*ln2_lo + c) gives 14,404 mismatching arguments, evaluating expf's x*32/ln2 unfused gives 2;
* the platform libm is the function it claims to be: within one ulp of double-precision exp / log1p rounded once;
* special values (0, +-inf, NaN, -1, the overflow and underflow edges, subnormal results);
* on the device (gpu): aq_eval_math equals the platform libm bit for bit over 2^24 arguments spread over all
  exponents, and over the ranges the activations see.
"""
import math
import os
import sys

import numpy as np
import pytest

import oracle_lib as O

EXP, LOG1P, SILU, SIGMOID, SOFTPLUS = 0, 1, 2, 3, 4


@pytest.mark.parametrize("fn", [EXP, LOG1P])
def test_restatement_equals_platform_libm_on_every_f32(fn):
    bad, first = O.math_sweep(fn)
    assert bad == 0, f"fn {fn}: {bad} of 2^32 arguments differ from libm, first bit pattern {first:#010x}"


@pytest.mark.parametrize("fn", [SILU, SIGMOID, SOFTPLUS])
def test_activations_equal_platform_libm_strided(fn):
    bad, first = O.math_sweep(fn, first=12345, count=(1 << 32) // 61, stride=61)
    assert bad == 0, f"fn {fn}: {bad} arguments differ from libm, first bit pattern {first:#010x}"


def exp_args(n, seed=1):
    rng = np.random.default_rng(seed)
    a = rng.uniform(-104.0, 89.0, n).astype(np.float32)
    b = rng.uniform(-2.0, 2.0, n).astype(np.float32)
    bits = rng.integers(0, 2**31, n, dtype=np.uint32).view(np.float32)  # positive floats of every exponent
    bits = bits[np.isfinite(bits) & (bits < 89.0)]
    return np.concatenate([a, b, bits, -bits])


def ulps(a, b):
    ia, ib = a.view(np.int32).astype(np.int64), b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def test_platform_libm_is_within_one_ulp_of_the_exact_values():
    x = exp_args(100_000)
    want = np.empty_like(x)
    for i, v in enumerate(x.tolist()):
        try:
            want[i] = np.float32(math.exp(v))
        except OverflowError:
            want[i] = np.float32(np.inf)
    got = O.eval_math(EXP, x)
    fin = np.isfinite(want) & np.isfinite(got)
    assert np.array_equal(np.isfinite(want), np.isfinite(got))
    d = ulps(got[fin], want[fin])
    assert d.max() <= 1 and np.mean(d != 0) < 1e-3
    rng = np.random.default_rng(2)
    u = np.concatenate([O.eval_math(EXP, rng.uniform(-30.0, 20.0, 100_000).astype(np.float32)),
                        rng.uniform(-0.999, 0.0, 20_000).astype(np.float32)])
    want = np.array([np.float32(math.log1p(v)) for v in u.tolist()], np.float32)
    d = ulps(O.eval_math(LOG1P, u), want)
    assert d.max() <= 1 and np.mean(d != 0) < 5e-2  # fdlibm log1pf: ~2% of arguments one ulp off


def test_special_values():
    x = np.float32([0.0, -0.0, np.inf, -np.inf, np.nan, 88.72283, 88.7229, -87.33654, -103.97, -104.0, 1.0])
    for restated in (False, True):
        y = O.eval_math(EXP, x, restated=restated)
        assert y[0] == 1.0 and y[1] == 1.0 and y[2] == np.inf and y[3] == 0.0 and np.isnan(y[4])
        assert np.isfinite(y[5]) and y[6] == np.inf
        assert y[7] > 0 and y[8] > 0 and y[8] < np.finfo(np.float32).tiny  # subnormal result
        assert y[9] == 0.0
        u = np.float32([0.0, -0.0, -1.0, np.inf, np.nan, -2.0, 1e-30, 2**-29, 2**30])
        l = O.eval_math(LOG1P, u, restated=restated)
        assert l[0] == 0.0 and l[1] == 0.0 and np.signbit(l[1]) and l[2] == -np.inf and l[3] == np.inf
        assert np.isnan(l[4]) and np.isnan(l[5]) and l[6] == np.float32(1e-30)
        assert abs(float(l[8]) - 30 * math.log(2)) < 1e-5


def device_args():
    """2^24 f32 patterns spread over every exponent and sign, plus the activations' working ranges."""
    pats = (np.arange(1 << 24, dtype=np.uint64) * 256 + 77).astype(np.uint32).view(np.float32)
    rng = np.random.default_rng(5)
    acts = np.concatenate([rng.standard_normal(1 << 20).astype(np.float32) * 8,
                           rng.uniform(-104.0, 89.0, 1 << 20).astype(np.float32)])
    return np.concatenate([pats, acts])


@pytest.mark.gpu
def test_device_math_equals_platform_libm_bitwise():
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                    "qwen-3.8-in-rust_amd"))
    import aqueduct as aq

    ctx = aq.Context(0)
    x = device_args()
    for fn in (EXP, LOG1P, SILU, SIGMOID, SOFTPLUS):
        print(f"case math fn {fn}", flush=True)
        d, h = aq.eval_math(ctx, fn, x), O.eval_math(fn, x)
        same = (d.view(np.uint32) == h.view(np.uint32)) | (np.isnan(d) & np.isnan(h))
        bad = np.flatnonzero(~same)
        assert bad.size == 0, f"fn {fn}: {bad.size} differ, e.g. x={x[bad[:4]]} dev={d[bad[:4]]} libm={h[bad[:4]]}"
