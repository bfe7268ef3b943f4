"""The oracle's MTP draft head and speculative loop against a closed form (CPU only).

The reference's MTP fixtures need the tiny GGUF that is not available offline, so the composition of the draft head
(mtp.rs:95-137, spec.rs:192-272, docs/mtp.md:57-93) is pinned by weights that reduce it to pinned primitives: every
layer's output projections zero (each layer the identity) and an F32 `eh_proj` that selects the hidden half, the
embedding half, or their sum (tests/mtp_closed_form.py). The oracle's spec_prefill and spec_round must then emit the
closed form's tokens and drafts round after round; the same checks reject each plausible mistake (halves swapped,
the chain fed the pre-norm hidden, the chain re-embedding the wrong token)."""
import numpy as np
import pytest

import aqueduct as aq
import oracle_lib as O
from mtp_closed_form import ClosedForm, collapsed_tensors, run_trace

SEED = 424242
K = 3
ROUNDS = 16


@pytest.fixture(scope="module")
def base():
    cfg = aq.tiny_config()
    return cfg, aq.plan_tensors(aq.model_plan(cfg, aq.MIX_TINY, SEED))


def ocfg(cfg):
    c = O.AqModelConfig()
    for name, _ in O.AqModelConfig._fields_:
        setattr(c, name, getattr(cfg, name))
    return c


def oracle_trace(cfg, tensors, prompt, rounds, cf):
    om = O.Model(ocfg(cfg), tensors, threads=4)
    return run_trace(O.State(om, K, 128), cf, prompt, rounds)


CASES = [("h", "random"), ("e", "random"), ("sum", "random"), ("e", "matched")]


@pytest.mark.parametrize("eh_mode,norm_mode", CASES)
def test_oracle_spec_loop_equals_closed_form(base, eh_mode, norm_mode):
    cfg, tensors = base
    ts = collapsed_tensors(tensors, cfg, eh_mode, SEED + 1, norm_mode)
    prompt = np.random.default_rng(SEED).integers(0, cfg.vocab, 16).astype(np.uint32)
    cf = ClosedForm(cfg, ts, eh_mode, K)
    got = oracle_trace(cfg, ts, prompt, ROUNDS, cf)
    want = run_trace(cf, cf, prompt, ROUNDS)
    for r, (g, w) in enumerate(zip(got, want)):
        assert g == w, f"round {r}: oracle {g} closed form {w}"
    ms = [m for m, _, _ in got[1:]]
    assert set(ms[1::2]) == set(range(K + 1)), ms  # forced rounds: every acceptance count
    if norm_mode == "matched":  # the MTP predicts the main model: its own drafts are accepted
        assert sum(ms[0::2]) >= ROUNDS // 2


@pytest.mark.parametrize("mutant", ClosedForm.MUTANTS)
def test_closed_form_rejects_plausible_mistakes(base, mutant):
    """Each mistake changes some draft in one of the cases, so the check above would catch it."""
    cfg, tensors = base
    prompt = np.random.default_rng(SEED).integers(0, cfg.vocab, 16).astype(np.uint32)
    differs = False
    for eh_mode, norm_mode in CASES[:3]:
        ts = collapsed_tensors(tensors, cfg, eh_mode, SEED + 1, norm_mode)
        cf = ClosedForm(cfg, ts, eh_mode, K)
        bad = ClosedForm(cfg, ts, eh_mode, K, mutant=mutant)
        right, wrong = run_trace(cf, cf, prompt, 4), run_trace(bad, bad, prompt, 4)
        differs |= right != wrong
    assert differs, f"mutant {mutant} is indistinguishable"
