"""The 27B-shaped model (64 layers: 48 Gated-DeltaNet + 16 gated GQA, hidden 5120, FFN 17408, vocab 248,320, MTP)
in the Q4_K_M mix, generated on the device, against the CPU oracle holding the same bytes:

* prefill of a 4-token seeded prompt: the last row's logits within 1e-3 of the oracle's (relative to the largest
  |logit|), the same argmax, and every per-layer state tensor (DeltaNet recurrent state and conv window, K/V cache)
  within 1e-3;
* greedy decoding: device plain ids == device --spec 3 ids == oracle --spec 3 ids over 6 tokens, round by round
  the oracle's drafts and accepted counts (tests/spec_identity.rs:34-119 at the full shape).

The oracle is the checker only (a C restatement of the reference's CPU path, oracle/); it runs on the host cores
at ~4 s per 27B token, so the sample stays short.
"""
import os
import sys

import numpy as np
import pytest

import oracle_lib as O

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "qwen-3.8-in-rust_amd"))
import aqueduct as aq  # noqa: E402

pytestmark = pytest.mark.gpu

SEED = 20260905
NTOK = 6


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.fixture(scope="module")
def big():
    ctx = aq.Context(0)
    cfg = aq.config_27b()
    plan = aq.model_plan(cfg, aq.MIX_Q4_K_M, SEED)
    print("case 27B: generating the model on the device and the same bytes on the host", flush=True)
    gm = aq.Model(ctx, cfg, mix=aq.MIX_Q4_K_M, seed=SEED)
    threads = min(16, os.cpu_count() or 1)
    tensors = aq.plan_tensors(plan, threads)
    ocfg = O.AqModelConfig()
    for name, _ in O.AqModelConfig._fields_:
        setattr(ocfg, name, getattr(cfg, name))
    om = O.Model(ocfg, tensors, threads=threads)
    prompt = np.random.default_rng(SEED + 2).integers(0, cfg.vocab, 4).astype(np.uint32)
    yield dict(ctx=ctx, cfg=cfg, gm=gm, om=om, prompt=prompt)
    del om, tensors
    gm.free()


def test_27b_prefill_logits_and_state_match_oracle(big):
    print("case 27B prefill", flush=True)
    gs = aq.State(big["gm"], 0, 32)
    os_ = O.State(big["om"], 0, 32)
    tg, lg = gs.prefill(big["prompt"], want_logits=True)
    to, lo = os_.prefill(big["prompt"], want_logits=True)
    r = rel(lg, lo)
    print(f"27B prefill: argmax device {tg} oracle {to}, logits max rel {r:.3e}, "
          f"bit-identical {np.array_equal(lg, lo)}", flush=True)
    assert lg.shape == lo.shape == (big["cfg"].vocab,)
    assert tg == to == int(np.argmax(lo))
    assert r <= 1e-3
    se, so = gs.export(), os_.export()
    assert se.size == so.size
    rs = rel(se, so)
    print(f"27B prefill: state ({se.size} floats) max rel {rs:.3e}, bit-identical {np.array_equal(se, so)}",
          flush=True)
    assert rs <= 1e-3


def test_27b_spec3_ids_equal_plain_and_oracle(big):
    print("case 27B greedy plain vs --spec 3", flush=True)
    gp = aq.State(big["gm"], 0, 64)
    plain = [gp.prefill(big["prompt"])]
    while len(plain) < NTOK:
        plain.append(gp.forward_token(plain[-1]))
    gs = aq.State(big["gm"], 3, 64)
    os_ = O.State(big["om"], 3, 64)
    g = [gs.spec_prefill(big["prompt"])]
    o = [os_.spec_prefill(big["prompt"])]
    assert g == o
    while len(g) < NTOK:
        gd, od = gs.drafts(), os_.drafts()
        m, em = gs.spec_round(g[-1])
        mo, emo = os_.spec_round(o[-1])
        print(f"27B round: drafts {gd} accepted {m} emitted {em}", flush=True)
        assert gd == od and (m, em) == (mo, emo)
        g += em
        o += emo
    print(f"27B ids: plain {plain}, spec {g[:NTOK]}", flush=True)
    assert g[:NTOK] == plain
