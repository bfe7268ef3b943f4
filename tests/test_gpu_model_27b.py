"""The 27B-shaped model (64 layers: 48 Gated-DeltaNet + 16 gated GQA, hidden 5120, FFN 17408, vocab 248,320, MTP)
in the Q4_K_M mix, generated on the device, against the CPU oracle holding the same bytes:

* prefill of a 4-token seeded prompt: the last row's logits bit-identical to the oracle's (the north star asks for
  1e-3 relative; both sides evaluate the reference's glibc expf / log1pf, so they agree exactly), the same argmax,
  and every per-layer state tensor (DeltaNet recurrent state and conv window, K/V cache) bit-identical;
* greedy decoding: device plain ids == device --spec 3 ids == oracle --spec 3 ids over 6 tokens, round by round
  the oracle's drafts and accepted counts (tests/spec_identity.rs:34-119 at the full shape);
* forced drafts accepted up to position m = 1, 2, 3, 0: after every round the device state equals the plain
  state at the same position bit for bit, and the oracle's (tests/spec_identity.rs:136-170 at the full shape);
* config 4 as the bench runs it (a 64-token prompt, then 12 --spec 3 rounds and 4 forced rounds accepting 3, 1, 2, 0):
  drafts, accepted counts and emitted ids equal the oracle's round by round, and the whole state after the last
  round is bit-identical;
* sampled --spec 3 (top-k 40 / top-p 0.95, and temperature 1.2 over the whole vocabulary): accepted counts, emitted
  ids, drafts and the generator state equal the oracle's round by round, the final state bit-identical;
* --q8-fine: the prefill's logits and state bit-identical, then 3 --spec 3 rounds equal to the oracle's.

The oracle is the checker only (a C restatement of the reference's CPU path, oracle/); with its scalar dots it runs
at ~4 s per 27B token on the host cores, so those samples stay short; the config-4 sample runs its AVX2 dots.
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
    assert np.array_equal(lg, lo)
    se, so = gs.export(), os_.export()
    assert se.size == so.size
    rs = rel(se, so)
    print(f"27B prefill: state ({se.size} floats) max rel {rs:.3e}, bit-identical {np.array_equal(se, so)}",
          flush=True)
    assert rs <= 1e-3
    assert np.array_equal(se, so)


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


def test_27b_forced_drafts_rollback_state(big):
    print("case 27B forced drafts", flush=True)
    vocab = big["cfg"].vocab
    gp = aq.State(big["gm"], 0, 64)
    plain = [gp.prefill(big["prompt"])]
    while len(plain) < 16:
        plain.append(gp.forward_token(plain[-1]))
    gs = aq.State(big["gm"], 3, 64)
    os_ = O.State(big["om"], 3, 64)
    out = [gs.spec_prefill(big["prompt"])]
    assert out[0] == os_.spec_prefill(big["prompt"]) == plain[0]
    for r, n_ok in enumerate([1, 2, 3, 0]):
        j = len(out)
        d = [plain[j + i] if i < n_ok else (plain[j + i] + 1) % vocab for i in range(3)]
        gs.set_drafts(d)
        os_.set_drafts(d)
        m, em = gs.spec_round(out[-1])
        mo, emo = os_.spec_round(out[-1])
        print(f"27B forced round {r}: m {m} emitted {em}", flush=True)
        assert (m, em) == (mo, emo) and m == n_ok and em == plain[j:j + len(em)]
        out += em
        ref = aq.State(big["gm"], 0, 64)
        ref.prefill(big["prompt"])
        for tok in out[:-1]:
            ref.forward_token(tok)
        a, b = gs.export(), ref.export()
        assert gs.pos == ref.pos
        assert np.array_equal(a[: b.size], b), f"round {r}: spec state differs from the plain state"
        assert np.array_equal(a, os_.export()), f"round {r}: spec state differs from the oracle's"
        assert gs.drafts() == os_.drafts()


def test_27b_config4_prompt_spec3_rounds_match_oracle(big):
    """Config 4 as the bench runs it: a 64-token seeded prompt through the spec prefill (one 64-row chunk on the
    device), then 12 greedy --spec 3 rounds and 4 rounds whose drafts are forced to accept 3, 1, 2 and 0 tokens of
    the plain continuation; round by round the drafts, the accepted count and the emitted ids equal the oracle's
    (and the plain ids), and after the last round every per-layer state tensor is bit-identical. The oracle runs its AVX2
    dots here (bit-identical to its scalar ones, tests/test_oracle_simd.py), which makes this sample affordable."""
    print("case 27B config 4: 64-token prompt, 12 --spec 3 rounds vs the oracle", flush=True)
    prompt = np.random.default_rng(SEED).integers(0, big["cfg"].vocab, 64).astype(np.uint32)
    gs = aq.State(big["gm"], 3, 160)
    os_ = O.State(big["om"], 3, 160)
    with O.simd(True):
        g = [gs.spec_prefill(prompt)]
        o = [os_.spec_prefill(prompt)]
        assert g == o
        for r in range(12):
            gd, od = gs.drafts(), os_.drafts()
            m, em = gs.spec_round(g[-1])
            mo, emo = os_.spec_round(o[-1])
            print(f"27B config 4 round {r}: drafts {gd} accepted {m} emitted {em}", flush=True)
            assert gd == od and (m, em) == (mo, emo), f"round {r}"
            g += em
            o += emo
        # then forced rounds accepting 3, 1, 2, 0 drafts of the plain continuation (spec_identity.rs:136-170)
        gp = aq.State(big["gm"], 0, 160)
        plain = [gp.prefill(prompt)]
        while len(plain) < len(g) + 16:
            plain.append(gp.forward_token(plain[-1]))
        assert plain[:len(g)] == g
        vocab = big["cfg"].vocab
        for r, n_ok in enumerate([3, 1, 2, 0]):
            j = len(g)
            d = [plain[j + i] if i < n_ok else (plain[j + i] + 1) % vocab for i in range(3)]
            gs.set_drafts(d)
            os_.set_drafts(d)
            m, em = gs.spec_round(g[-1])
            mo, emo = os_.spec_round(o[-1])
            print(f"27B config 4 forced round {r}: accepted {m} emitted {em}", flush=True)
            assert (m, em) == (mo, emo) and m == n_ok and em == plain[j:j + len(em)], f"forced round {r}"
            g += em
            o += emo
    assert gs.pos == os_.pos
    se, so = gs.export(), os_.export()
    print(f"27B config 4: {len(g)} ids, state ({se.size} floats) bit-identical {np.array_equal(se, so)}", flush=True)
    assert np.array_equal(se, so)


@pytest.mark.parametrize("kw", [dict(temperature=1.0, top_k=40, top_p=0.95), dict(temperature=1.2)])
def test_27b_sampled_spec3_rounds_match_oracle(big, kw):
    """Sampled --spec 3 at the full shape (sample.rs:279 accept_or_resample via spec.rs:367-380, the sampler over
    the 248,320-entry vocabulary: top-k by sorted chunks, or with no top-k the whole row sorted): a 16-token prompt,
    then 8 rounds; round by round the accepted count, the emitted ids, the next drafts and the generator state equal
    the oracle's (with its AVX2 dots), and the state after the last round is bit-identical."""
    print(f"case 27B sampled --spec 3 {kw}", flush=True)
    vocab = big["cfg"].vocab
    prompt = np.random.default_rng(SEED + 5).integers(0, vocab, 16).astype(np.uint32)
    ds = aq.Sampler(big["ctx"], aq.sampler_config(**kw, seed=11), vocab)
    os_ = O.Sampler(O.sampler_config(**kw, seed=11), vocab)
    g, o = aq.State(big["gm"], 3, 96), O.State(big["om"], 3, 96)
    with O.simd(True):
        xg, xo = g.spec_prefill(prompt, sampler=ds), o.spec_prefill(prompt, sampler=os_)
        assert xg == xo and g.drafts() == o.drafts()
        for r in range(8):
            mg, eg = g.spec_round(xg, sampler=ds)
            mo, eo = o.spec_round(xo, sampler=os_)
            print(f"27B sampled round {r}: accepted {mg} emitted {eg}", flush=True)
            assert (mg, eg) == (mo, eo), f"round {r}: {(mg, eg)} vs {(mo, eo)}"
            assert g.drafts() == o.drafts(), f"round {r}: drafts"
            assert np.array_equal(ds.rng(), os_.rng()), f"round {r}: generator state"
            xg, xo = eg[-1], eo[-1]
    assert np.array_equal(g.export(), o.export())
    ds.free()


def test_27b_q8_fine_prefill_and_spec_rounds_match_oracle(big):
    """--q8-fine at the full shape (matvec.rs:129-160: K-quant weights against Q8_0-grain activations, dot.rs:69-160):
    the 4-token prompt's logits and every state tensor bit-identical to the oracle's, then a spec prefill and 3
    greedy --spec 3 rounds with the same drafts, accepted counts and emitted ids. The oracle runs its scalar
    q8-fine dots."""
    print("case 27B q8-fine prefill and --spec 3 rounds", flush=True)
    with aq.q8_fine(), O.q8_fine():
        gs, os_ = aq.State(big["gm"], 0, 32), O.State(big["om"], 0, 32)
        tg, lg = gs.prefill(big["prompt"], want_logits=True)
        to, lo = os_.prefill(big["prompt"], want_logits=True)
        print(f"27B q8-fine prefill: argmax {tg} / {to}, logits bit-identical {np.array_equal(lg, lo)}", flush=True)
        assert tg == to and np.array_equal(lg, lo)
        assert np.array_equal(gs.export(), os_.export())
        gs, os_ = aq.State(big["gm"], 3, 48), O.State(big["om"], 3, 48)
        g, o = [gs.spec_prefill(big["prompt"])], [os_.spec_prefill(big["prompt"])]
        assert g == o
        for r in range(3):
            gd, od = gs.drafts(), os_.drafts()
            m, em = gs.spec_round(g[-1])
            mo, emo = os_.spec_round(o[-1])
            print(f"27B q8-fine round {r}: drafts {gd} accepted {m} emitted {em}", flush=True)
            assert gd == od and (m, em) == (mo, emo), f"round {r}"
            g += em
            o += emo
        assert np.array_equal(gs.export(), os_.export())


def test_27b_prompt_chunks_equal_token_by_token_feed(big):
    """A 70-token prompt at the full shape: one chunk of 64 rows (every projection through the matrix-core prompt
    GEMM, csrc/kq_gemm.hip, attention over the whole chunk, the DeltaNet recurrence in 8-row pieces inside one launch)
    and one of 6; the last row's logits
    and every per-layer state tensor equal those of the same prompt fed one token at a time through the decode
    kernels (themselves bit-exact to the oracle above) — model.rs:443-461, prefill row i is forward_token on row i."""
    print("case 27B 70-token prompt in chunks vs one token at a time", flush=True)
    cfg = big["cfg"]
    prompt = np.random.default_rng(SEED + 7).integers(0, cfg.vocab, 70).astype(np.uint32)
    g = aq.State(big["gm"], 0, 96)
    tg, lg = g.prefill(prompt, want_logits=True)
    f = aq.State(big["gm"], 0, 96)
    f.prefill(prompt[:1])
    for tok in prompt[1:-1]:
        f.forward_token(int(tok))
    tf, lf = f.forward_token(int(prompt[-1]), want_logits=True)
    assert tf == tg and np.array_equal(lf.view(np.uint32), lg.view(np.uint32)), "chunked prefill logits differ"
    assert np.array_equal(g.export(), f.export()), "chunked prefill state differs"
    g.free()
    f.free()


def test_27b_config4_256_ids_plain_equal_spec3(big):
    """Config 4 over its full length: the 64-token seeded prompt, then 256 greedy ids from the device's plain loop
    and from its --spec 3 loop are identical (spec_identity.rs:34-119 at the full shape); the spec prefill and the
    first 4 rounds equal the oracle's (its AVX2 dots), and the spec state at the end equals a plain state that
    consumed the same tokens, bit for bit."""
    print("case 27B config 4: 256 greedy ids, plain vs --spec 3", flush=True)
    n = 256
    prompt = np.random.default_rng(SEED).integers(0, big["cfg"].vocab, 64).astype(np.uint32)
    max_pos = len(prompt) + n + 32
    gp = aq.State(big["gm"], 0, max_pos)
    plain = [gp.prefill(prompt)]
    while len(plain) < n:
        plain.append(gp.forward_token(plain[-1]))
    gs = aq.State(big["gm"], 3, max_pos)
    os_ = O.State(big["om"], 3, max_pos)
    g = [gs.spec_prefill(prompt)]
    with O.simd(True):
        o = [os_.spec_prefill(prompt)]
        assert g == o
        for r in range(4):
            gd, od = gs.drafts(), os_.drafts()
            m, em = gs.spec_round(g[-1])
            mo, emo = os_.spec_round(o[-1])
            assert gd == od and (m, em) == (mo, emo), f"round {r}"
            g += em
            o += emo
    del os_
    while len(g) < n:
        _, em = gs.spec_round(g[-1])
        g += em
    st = gs.stats()
    print(f"27B config 4: {n} ids, {st['rounds']} rounds, accepted {st['accepted']}", flush=True)
    assert g[:n] == plain, "--spec 3 ids differ from the plain ids"
    # the plain state that consumed what the spec state consumed
    consumed = gs.pos - len(prompt)
    ref = aq.State(big["gm"], 0, max_pos)
    ref.prefill(prompt)
    for tok in g[:consumed]:
        ref.forward_token(tok)
    a, b = gs.export(), ref.export()
    assert gs.pos == ref.pos and np.array_equal(a[: b.size], b)
