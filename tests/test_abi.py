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
    # the generator's own values: normal of sigma 0.02
    f = aq.synth_host(aq.synth_spec(aq.F32, rows, cols, seed=1234, b=0.02))
    assert abs(float(f.std()) - 0.02) < 0.001 and abs(float(f.mean())) < 0.001
    # quantisation error small against the scale
    rel = float(np.sqrt(np.mean((deq - f) ** 2))) / 0.02
    limit = {aq.Q4_K: 0.15, aq.Q5_K: 0.08, aq.Q6_K: 0.05, aq.Q8_0: 0.02, aq.Q4_0: 0.15}[t]
    assert rel < limit, f"rms quantisation error {rel:.3f} of sigma"


def test_synth_normal_is_normal():
    """N(a, b): moments, tails and the whole CDF of a million draws (scipy's normal as the yardstick), and the
    inverse CDF's accuracy at fixed points where Phi^-1 is known to many digits."""
    from scipy import stats
    n = 1 << 20
    f = aq.synth_host(aq.synth_spec(aq.F32, 1, n, seed=77, b=0.02)).astype(np.float64) / 0.02
    assert abs(f.mean()) < 0.005 and abs(f.std() - 1.0) < 0.005
    assert abs(stats.kurtosis(f)) < 0.03 and abs(stats.skew(f)) < 0.01  # Irwin-Hall(4) would give -0.3
    assert abs(np.mean(np.abs(f) > 3.0) / (2 * stats.norm.sf(3.0)) - 1.0) < 0.1
    assert np.max(np.abs(f)) > 4.0
    assert stats.kstest(f, "norm").pvalue > 1e-3
    g = aq.synth_host(aq.synth_spec(aq.F32, 1, 4096, seed=5, a=1.5, b=0.25)).astype(np.float64)
    assert abs(g.mean() - 1.5) < 0.02 and abs(g.std() - 0.25) < 0.01
    # value i is Phi^-1(p_i) * sigma with p_i from the element's splitmix64 draw: check against scipy's ppf
    m64 = (1 << 64) - 1

    def splitmix(x):
        x = (x + 0x9E3779B97F4A7C15) & m64
        x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & m64
        x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & m64
        return x ^ (x >> 31)

    h = aq.synth_host(aq.synth_spec(aq.F32, 1, 4096, seed=77, b=0.02)).astype(np.float64)
    ps = np.array([((splitmix(77 ^ ((i * 0xD1B54A32D192ED03) & m64)) >> 11) + 0.5) * 2.0 ** -53 for i in range(4096)])
    want = stats.norm.ppf(ps) * 0.02
    assert np.max(np.abs(h - want) / np.abs(want)) < 2e-7
    assert np.sum((ps < 0.02425) | (ps > 0.97575)) > 100  # the tail branch is exercised


def test_synth_uniform_and_const():
    u = aq.synth_host(aq.synth_spec(aq.F32, 1, 4096, 9, aq.UNIFORM, -0.5, 0.5))
    assert u.min() >= -0.5 and u.max() < 0.5 and abs(float(u.mean())) < 0.03
    c = aq.synth_host(aq.synth_spec(aq.F32, 1, 48, 9, aq.CONST, 1.0, 0.0))
    assert np.all(c == 1.0)


def c_decls():
    """{name: parameter count} of every function include/aq.h declares."""
    text = open(os.path.join(ROOT, "include", "aq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(aq_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        p = params.strip()
        out[name] = 0 if p in ("", "void") else p.count(",") + 1
    return out


def test_integration_rust_binding_matches_the_header():
    """INTEGRATION.md's ffi.rs: every `pub fn` is a function aq.h declares, with as many parameters; the raw types
    it uses are imported; every libaq entry point the integration table routes a reference function to is declared
    in the binding (a maintainer can paste the block as written)."""
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = re.search(r"```rust\n#!\[allow\(non_camel_case_types\)\]\n(.*?)```", doc, flags=re.S).group(1)
    decl = c_decls()
    fns = dict(re.findall(r"pub fn (aq_[a-z0-9_]+)\(([^)]*)\)", block, flags=re.S))
    assert len(fns) >= 40
    for name, params in fns.items():
        assert name in decl, f"ffi.rs declares {name}, which aq.h does not"
        n = 0 if not params.strip() else params.count(":")
        assert n == decl[name], f"{name}: {n} parameters in ffi.rs, {decl[name]} in aq.h"
    imported = set(re.search(r"use std::os::raw::\{([^}]*)\}", block).group(1).replace(" ", "").split(","))
    for ty in ("c_char", "c_int", "c_void"):
        if re.search(rf"\b{ty}\b", block.split("\n", 2)[-1]):
            assert ty in imported, f"ffi.rs uses {ty} without importing it"
    table = doc[doc.index("## 3."):]
    table = table[: table.index("\n\n", table.index("|---|"))]
    routed = set(re.findall(r"`(aq_[a-z0-9_]+)", table)) & set(decl)  # functions, not the structs named there
    missing = sorted(n for n in routed if n not in fns)
    assert not missing, f"the table routes to {missing}, which ffi.rs does not declare"
