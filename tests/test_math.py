"""exp and log1p of the activations (aq_math.h), pinned against the mathematics and libm, and the device's copy
of them against the CPU's, bit for bit.

* against double-precision libm rounded once to f32 (math.exp / math.log1p, i.e. the correctly rounded f32 value
  up to double's error): no mismatch on millions of arguments over the whole range the activations use;
* special values (0, +-inf, NaN, over/underflow edges, subnormal results);
* against the platform's f32 expf / log1pf (what the reference calls): every difference is one ulp, and rare;
* on the device (gpu): aq_eval_math equals the oracle's evaluation bit for bit.
"""
import math
import os
import sys

import numpy as np
import pytest

import oracle_lib as O

EXP, LOG1P, SILU, SIGMOID, SOFTPLUS = 0, 1, 2, 3, 4


def exp_args(n, seed=1):
    rng = np.random.default_rng(seed)
    a = rng.uniform(-104.0, 89.0, n).astype(np.float32)
    b = rng.uniform(-2.0, 2.0, n).astype(np.float32)
    bits = rng.integers(0, 2**31, n, dtype=np.uint32).view(np.float32)  # positive floats of every exponent
    bits = bits[np.isfinite(bits) & (bits < 89.0)]
    return np.concatenate([a, b, bits, -bits])


def ref_exp(x):
    out = np.empty_like(x)
    for i, v in enumerate(x.tolist()):
        try:
            out[i] = np.float32(math.exp(v))
        except OverflowError:
            out[i] = np.float32(np.inf)
    return out


def test_exp_matches_double_libm_rounded_once():
    x = exp_args(300_000)
    got = O.eval_math(EXP, x)
    want = ref_exp(x)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{bad.size} mismatches, e.g. x={x[bad[:5]]} got={got[bad[:5]]} want={want[bad[:5]]}"


def test_log1p_matches_double_libm_rounded_once():
    rng = np.random.default_rng(2)
    e = O.eval_math(EXP, rng.uniform(-30.0, 20.0, 200_000).astype(np.float32))  # softplus's argument range
    u = np.concatenate([e, rng.uniform(-0.999, 0.0, 50_000).astype(np.float32),
                        np.float32([0.0, 1e-30, 1e-10, 2**-29, 2**-28, 1.0, 2**29, 4.8e8])])
    got = O.eval_math(LOG1P, u)
    want = np.array([np.float32(math.log1p(v)) for v in u.tolist()], np.float32)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{bad.size} mismatches, e.g. u={u[bad[:5]]} got={got[bad[:5]]} want={want[bad[:5]]}"


def test_special_values():
    x = np.float32([0.0, -0.0, np.inf, -np.inf, np.nan, 88.72283, 88.7229, -87.33654, -103.97, -104.0, 1.0])
    y = O.eval_math(EXP, x)
    assert y[0] == 1.0 and y[1] == 1.0 and y[2] == np.inf and y[3] == 0.0 and np.isnan(y[4])
    assert np.isfinite(y[5]) and y[6] == np.inf
    assert y[7] > 0 and y[8] > 0 and y[8] < np.finfo(np.float32).tiny  # subnormal result
    assert y[10] == np.float32(math.e)
    u = np.float32([0.0, -1.0, np.inf, np.nan, -2.0])
    l = O.eval_math(LOG1P, u)
    assert l[0] == 0.0 and l[1] == -np.inf and l[2] == np.inf and np.isnan(l[3]) and np.isnan(l[4])


def test_platform_libm_differs_by_one_ulp_at_most_and_rarely():
    x = exp_args(200_000, seed=3)
    ours, libm = O.eval_math(EXP, x), O.eval_math(EXP, x, libm=True)
    diff = np.abs(ours.view(np.int32).astype(np.int64) - libm.view(np.int32).astype(np.int64))
    fin = np.isfinite(ours)
    assert diff[fin].max() <= 1
    frac = float(np.mean(diff[fin] != 0))
    print(f"expf: platform libm differs on {frac:.2e} of arguments")
    assert frac < 1e-3


@pytest.mark.gpu
def test_device_math_equals_oracle_bitwise():
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                    "qwen-3.8-in-rust_amd"))
    import aqueduct as aq

    ctx = aq.Context(0)
    x = exp_args(200_000, seed=4)
    rng = np.random.default_rng(5)
    acts = np.concatenate([x[np.abs(x) < 40], rng.standard_normal(100_000).astype(np.float32) * 8])
    u = O.eval_math(EXP, rng.uniform(-30.0, 20.0, 100_000).astype(np.float32))
    for fn, arg in ((EXP, x), (LOG1P, u), (SILU, acts), (SIGMOID, acts), (SOFTPLUS, acts)):
        print(f"case math fn {fn}", flush=True)
        d, h = aq.eval_math(ctx, fn, arg), O.eval_math(fn, arg)
        assert np.array_equal(d.view(np.uint32), h.view(np.uint32)), f"fn {fn}: device differs from the oracle"
