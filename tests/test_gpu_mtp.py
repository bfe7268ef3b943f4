"""The device's MTP draft head and speculative loop against the closed form of tests/mtp_closed_form.py: identity
layers and a selection `eh_proj` reduce the draft head (mtp.rs:95-137, spec.rs:192-272, 326-433) to primitives the
reference's fixtures pin; the device must emit the closed form's tokens and drafts in every round, including forced
rounds that cycle the acceptance count through 0..k."""
import numpy as np
import pytest

import aqueduct as aq
import oracle_lib as O  # noqa: F401  (the closed form's primitives)
from mtp_closed_form import ClosedForm, collapsed_tensors, run_trace

SEED = 424242
K = 3
ROUNDS = 16
CASES = [("h", "random"), ("e", "random"), ("sum", "random"), ("e", "matched")]

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    return aq.Context(0)


@pytest.mark.parametrize("eh_mode,norm_mode", CASES)
def test_device_spec_loop_equals_closed_form(ctx, eh_mode, norm_mode):
    print(f"case mtp closed form {eh_mode} {norm_mode}", flush=True)
    cfg = aq.tiny_config()
    tensors = aq.plan_tensors(aq.model_plan(cfg, aq.MIX_TINY, SEED))
    ts = collapsed_tensors(tensors, cfg, eh_mode, SEED + 1, norm_mode)
    prompt = np.random.default_rng(SEED).integers(0, cfg.vocab, 16).astype(np.uint32)
    cf = ClosedForm(cfg, ts, eh_mode, K)
    gm = aq.Model(ctx, cfg, tensors=ts)
    got = run_trace(aq.State(gm, K, 128), cf, prompt, ROUNDS)
    want = run_trace(cf, cf, prompt, ROUNDS)
    for r, (g, w) in enumerate(zip(got, want)):
        assert g == w, f"round {r}: device {g} closed form {w}"
    ms = [m for m, _, _ in got[1:]]
    assert set(ms[1::2]) == set(range(K + 1)), ms
