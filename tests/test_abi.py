"""CPU-side checks of the product library: it builds, loads, exports every symbol include/aq.h declares, refuses
bad arguments with an error code instead of aborting, and its synthetic-tensor generator is deterministic and
produces valid blocks of the intended distribution (no GPU needed)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import aqueduct as aq
import oracle_lib as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "aq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(aq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = aq.lib()
    names = declared_symbols()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"libaq.so lacks {missing}"


def test_errors_are_codes_not_aborts():
    L = aq.lib()
    assert L.aq_init(0, None) == -1
    assert b"null" in L.aq_last_error()
    spec = aq.synth_spec(aq.Q4_K, 2, 300, 1)  # cols not a multiple of 256
    out = np.zeros(16, np.uint8)
    assert L.aq_synth_host(C.byref(spec), out.ctypes.data, 1) == -1
    assert b"multiple" in L.aq_last_error()


@pytest.mark.parametrize("t", [aq.Q4_K, aq.Q5_K, aq.Q6_K, aq.Q8_0, aq.Q4_0])
def test_synth_quantisers_deterministic_and_faithful(t):
    rows, cols = 64, 1024
    spec = aq.synth_spec(t, rows, cols, seed=1234, b=0.02)
    a = aq.synth_host(spec, threads=1)
    b = aq.synth_host(spec, threads=5)
    assert np.array_equal(a, b), "thread count changed the bytes"
    spec2 = aq.synth_spec(t, rows, cols, seed=1235, b=0.02)
    assert not np.array_equal(a, aq.synth_host(spec2))
    deq = O.dequant(t, a, rows * cols)
    assert np.all(np.isfinite(deq))
    # the generator's own values: Irwin-Hall(4) normal of sigma 0.02
    f = aq.synth_host(aq.synth_spec(aq.F32, rows, cols, seed=1234, b=0.02))
    assert abs(float(f.std()) - 0.02) < 0.001 and abs(float(f.mean())) < 0.001
    assert float(np.abs(f).max()) <= 0.02 * 3.4642
    # quantisation error small against the scale
    rel = float(np.sqrt(np.mean((deq - f) ** 2))) / 0.02
    limit = {aq.Q4_K: 0.15, aq.Q5_K: 0.08, aq.Q6_K: 0.05, aq.Q8_0: 0.02, aq.Q4_0: 0.15}[t]
    assert rel < limit, f"rms quantisation error {rel:.3f} of sigma"


def test_synth_uniform_and_const():
    u = aq.synth_host(aq.synth_spec(aq.F32, 1, 4096, 9, aq.UNIFORM, -0.5, 0.5))
    assert u.min() >= -0.5 and u.max() < 0.5 and abs(float(u.mean())) < 0.03
    c = aq.synth_host(aq.synth_spec(aq.F32, 1, 48, 9, aq.CONST, 1.0, 0.0))
    assert np.all(c == 1.0)
