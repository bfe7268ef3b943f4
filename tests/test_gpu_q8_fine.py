"""The q8-fine path on the device (kq_q8f.hip) against the CPU oracle, through the C-ABI: K-quant weights x Q8_0
activations (dot.rs:69-160) under the process-wide switch (matvec.rs:127-160, aq_set_q8_fine).

Bar: bit-exact fp32, as for the production kernels (the device keeps the reference's per-sub-block order):
* the reference's dot fixture rows (tests/kernels.rs:213-249: K-quant rows x the fixture's Q8_0 activation rows);
* synthetic matrices at the model's shapes and at small ragged ones, N = 1..8 columns, each column of an N-column
  call equal to the 1-column call;
* the tiny hybrid model with the switch on: prefill and greedy tokens give the oracle's logits bit for bit (the
  oracle under its own switch), and greedy --spec 3 emits the plain ids round by round as the oracle does;
* the switch routes: the activation is quantised to Q8_0 for K-quant weights while it is on, Q8_K when off, and the
  integer-lane export refuses to run under it.
"""
import os
import sys

import numpy as np
import pytest

import oracle_lib as O

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "qwen-3.8-in-rust_amd"))
import aqueduct as aq  # noqa: E402

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "kernels", "dot")
KQ = (aq.Q4_K, aq.Q5_K, aq.Q6_K)
SEED = 20260905


def say(msg):
    print(msg, flush=True)


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.fixture(scope="module")
def ctx():
    c = aq.Context(0)
    yield c
    c.close()


@pytest.fixture(autouse=True)
def switch_off_after():
    yield
    aq.lib().aq_set_q8_fine(0)
    O.lib().or_set_q8_fine(0)


def test_fixture_rows_bit_exact(ctx):
    import json
    with open(os.path.join(GOLD, "manifest.json")) as f:
        m = json.load(f)
    seen = 0
    with aq.q8_fine():
        for c in m["cases"]:
            t = O.TYPE_BY_NAME[c["ggml_type"]]
            if t not in KQ:
                continue
            width, n_rows = c["width"], c["n_rows"]
            say(f"q8-fine fixture {c['case']}")
            w_raw = np.fromfile(os.path.join(GOLD, c["w_raw"]["file"]), np.uint8).reshape(n_rows, -1)
            x_raw = np.fromfile(os.path.join(GOLD, c["x_raw"]["file"]), np.uint8).reshape(n_rows, -1)
            x_deq = np.load(os.path.join(GOLD, c["x_deq"]["file"]), allow_pickle=False).astype(np.float32)
            x_deq = x_deq.reshape(n_rows, width)
            w = aq.Weight(ctx, t, n_rows, width, w_raw)
            a = aq.Act(ctx, width, 1)
            for r in range(n_rows):
                a.set(x_deq[r])
                a.quantize(t, 1)  # Q8_0 under the switch: the fixture's own activation bytes
                assert np.array_equal(a.q8_0(1)[0], x_raw[r]), f"{c['case']} row {r}: activation bytes"
                y = aq.matmul(ctx, w, a, 1)
                want = O.dot_q8(t, w_raw[r], x_raw[r], width)
                assert bits_equal(y[0, r], want), f"{c['case']} row {r}: {y[0, r]} vs {want}"
                seen += 1
            a.free()
            w.free()
    assert seen >= 21


def _single(ctx, xrow, t, keep):
    a = aq.Act(ctx, xrow.size, 1)
    a.set(xrow)
    a.quantize(t, 1)
    keep.append(a)
    return a


@pytest.mark.parametrize("t,rows,cols", [(aq.Q4_K, 37, 256), (aq.Q5_K, 100, 768), (aq.Q6_K, 68, 512),
                                         (aq.Q4_K, 17408, 5120), (aq.Q6_K, 5120, 17408), (aq.Q5_K, 1024, 5120),
                                         (aq.Q6_K, 10240, 5120), (aq.Q4_K, 5120, 6144)])
def test_matmul_bit_exact_and_column_identity(ctx, t, rows, cols):
    say(f"q8-fine matmul type {t} {rows}x{cols}")
    spec = aq.synth_spec(t, rows, cols, seed=811 + t + rows, b=0.02)
    host = aq.synth_host(spec).view(np.uint8)
    w = aq.SynthWeight(ctx, spec)
    x = np.random.default_rng(rows + t).standard_normal((8, cols)).astype(np.float32)
    keep = []
    with aq.q8_fine(), O.q8_fine():
        a = aq.Act(ctx, cols, 8)
        a.set(x)
        a.quantize(t, 8)
        want = O.matmul(t, host, rows, cols, x, threads=8)
        y1 = np.stack([aq.matmul(ctx, w, _single(ctx, x[c], t, keep), 1)[0] for c in range(8)])
        bad = int(np.sum(y1.view(np.uint32) != want.view(np.uint32)))
        assert bad == 0, f"N=1 vs oracle: {bad} mismatches"
        for n in (2, 3, 4, 5, 8):
            assert bits_equal(aq.matmul(ctx, w, a, n), y1[:n]), f"N={n} columns differ from N=1"
    for a1 in keep:
        a1.free()


def test_switch_routes_the_activation_and_refuses_isums(ctx):
    t, rows, cols = aq.Q4_K, 64, 512
    spec = aq.synth_spec(t, rows, cols, seed=5, b=0.02)
    host = aq.synth_host(spec).view(np.uint8)
    w = aq.SynthWeight(ctx, spec)
    x = np.random.default_rng(5).standard_normal(cols).astype(np.float32)
    a = aq.Act(ctx, cols, 1)
    a.set(x)
    a.quantize(t, 1)
    assert np.array_equal(a.q8k(1)[0], O.q8k_quantize(x))
    y_k = aq.matmul(ctx, w, a, 1)[0]
    with aq.q8_fine():
        assert aq.lib().aq_q8_fine() == 1
        a.quantize(t, 1)
        assert np.array_equal(a.q8_0(1)[0], O.q8_0_quantize(x))
        y_f = aq.matmul(ctx, w, a, 1)[0]
        with pytest.raises(aq.AqError, match="q8-fine"):
            aq.kq_isums(ctx, w, a, 1)
    assert aq.lib().aq_q8_fine() == 0
    assert bits_equal(y_k, O.matmul(t, host, rows, cols, x[None, :])[0])
    with O.q8_fine():
        assert bits_equal(y_f, O.matmul(t, host, rows, cols, x[None, :])[0])
    assert not bits_equal(y_k, y_f)  # the two activation forms round differently


@pytest.fixture(scope="module")
def tiny(ctx):
    cfg = aq.tiny_config()
    plan = aq.model_plan(cfg, aq.MIX_TINY, SEED)
    tensors = aq.plan_tensors(plan)
    gm = aq.Model(ctx, cfg, tensors=tensors)
    ocfg = O.AqModelConfig()
    for name, _ in O.AqModelConfig._fields_:
        setattr(ocfg, name, getattr(cfg, name))
    om = O.Model(ocfg, tensors, threads=8)
    prompt = np.random.default_rng(SEED).integers(0, cfg.vocab, 16).astype(np.uint32)
    yield dict(cfg=cfg, gm=gm, om=om, prompt=prompt)
    gm.free()


def plain_run(state, prompt, n):
    tok, lg = state.prefill(prompt, want_logits=True)
    ids, lgs = [tok], [lg]
    for _ in range(n - 1):
        tok, lg = state.forward_token(ids[-1], want_logits=True)
        ids.append(tok)
        lgs.append(lg)
    return ids, lgs


def spec_run(state, prompt, n):
    x = state.spec_prefill(prompt)
    out, rounds = [x], []
    while len(out) < n:
        drafts = state.drafts()
        m, em = state.spec_round(out[-1])
        rounds.append((drafts, m, em))
        out += em
    return out[:n], rounds


def test_tiny_model_under_the_switch_matches_oracle(ctx, tiny):
    say("case tiny plain greedy, q8-fine")
    base_ids, base_lg = plain_run(aq.State(tiny["gm"], 0, 128), tiny["prompt"], 4)
    with aq.q8_fine(), O.q8_fine():
        gids, glg = plain_run(aq.State(tiny["gm"], 0, 128), tiny["prompt"], 24)
        oids, olg = plain_run(O.State(tiny["om"], 0, 128), tiny["prompt"], 24)
        exact = sum(bits_equal(g, o) for g, o in zip(glg, olg))
        say(f"tiny q8-fine: {exact}/24 steps bit-identical; ids {gids[:8]}")
        assert gids == oids
        assert exact == 24
        say("case tiny spec 3, q8-fine")
        gs = aq.State(tiny["gm"], 3, 160)
        os_ = O.State(tiny["om"], 3, 160)
        sids, srounds = spec_run(gs, tiny["prompt"], 24)
        tids, trounds = spec_run(os_, tiny["prompt"], 24)
        assert sids == gids, "greedy --spec 3 must emit the plain ids"
        assert sids == tids
        assert [r[:2] for r in srounds] == [r[:2] for r in trounds], "drafts and acceptance differ from the oracle"
    assert not bits_equal(base_lg[0], glg[0]), "the switch must change the activation form"
