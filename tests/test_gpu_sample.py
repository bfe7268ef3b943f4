"""The device sampler (sample.hip) against the oracle's restatement of sample.rs, through the C-ABI.

Bar: identical results. The kept set (ids and probabilities, bit for bit), every draw, the accept/resample decisions and
the generator's state after each call equal the oracle's, for the configurations the reference runs (the
generation_config defaults temperature 1, top_k 20, top_p 0.95; min-p; no top-k; a top_k past the chunked selection;
top_k 1; greedy) on rows with planted ties, at the tiny vocabulary and at the 27B's 248,320.
* the reference's own distribution test (tests/sample.rs:47-74) on the device: chi-square of 20,000 accept/resample
  outcomes against p, the acceptance rate, seeded reproducibility;
* the tiny hybrid model's sampled loops (run.rs's sampled decode; spec.rs:229-433 with the rejection rule): every token,
  draft, accepted count, generator state and the whole carried state equal the oracle's round by round; top_k = 1
  gives the greedy loop's ids.
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

CONFIGS = [dict(temperature=1.0, top_k=20, top_p=0.95), dict(temperature=0.6, top_k=20, top_p=0.95, min_p=0.05),
           dict(temperature=1.3), dict(temperature=0.8, top_k=700, top_p=0.9), dict(temperature=0.9, top_k=512),
           dict(temperature=0.7, top_k=1), dict(temperature=0.0)]


def say(msg):
    print(msg, flush=True)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def ctx():
    return aq.Context(0)


def logits_rows(vocab, n, seed):
    rng = np.random.default_rng(seed)
    rows = (rng.standard_normal((n, vocab)) * 2.5).astype(np.float32)
    for r in range(n):  # ties at the top and across the top-k boundary
        top = np.argsort(-rows[r])[:30]
        rows[r, top[3]] = rows[r, top[2]]
        rows[r, rng.integers(0, vocab, 5)] = rows[r, top[19]]
        rows[r, rng.integers(0, vocab)] = -0.0
    return rows


@pytest.mark.parametrize("vocab", [4096, 248320])
@pytest.mark.parametrize("ci", range(len(CONFIGS)))
def test_process_draw_accept_equal_the_oracle(ctx, vocab, ci):
    kw = CONFIGS[ci]
    say(f"case sampler vocab {vocab} config {kw}")
    rows = logits_rows(vocab, 6, vocab + ci)
    cfg = dict(kw, seed=1234 + ci)
    ds = aq.Sampler(ctx, aq.sampler_config(**cfg), vocab)
    os_ = O.Sampler(O.sampler_config(**cfg), vocab)
    qsrc_d = aq.Sampler(ctx, aq.sampler_config(**dict(kw, temperature=max(kw.get("temperature", 1.0), 0.0) * 1.2,
                                                     seed=99)), vocab)
    qsrc_o = O.Sampler(O.sampler_config(**dict(kw, temperature=max(kw.get("temperature", 1.0), 0.0) * 1.2, seed=99)),
                       vocab)
    lb = aq.DeviceBuffer(ctx, vocab * 4)
    qb = aq.DeviceBuffer(ctx, vocab * 4)
    for r in range(rows.shape[0]):
        lb.upload(rows[r])
        ids, probs = ds.process(lb)
        oids, oprobs = os_.process(rows[r])
        assert np.array_equal(ids, oids), f"row {r}: kept ids differ"
        assert np.array_equal(bits(probs), bits(oprobs)), f"row {r}: kept probabilities differ"
        for _ in range(5):
            assert ds.draw() == os_.draw()
        assert ds.sample(lb) == os_.sample(rows[r])
        assert np.array_equal(ds.rng(), os_.rng())
        # a draft distribution from another row, a draft from it, the acceptance rule
        q_row = rows[(r + 1) % rows.shape[0]]
        lb.upload(q_row)
        qsrc_d.process(lb)
        qsrc_o.process(q_row)
        qsrc_d.write_dense(qb)
        q = qsrc_o.write_dense()
        assert np.array_equal(bits(qb.download(np.float32, vocab)), bits(q))
        lb.upload(rows[r])
        for d in [int(qsrc_o.draw()), int(oids[0]), int(np.argmin(rows[r]))]:
            got = ds.accept_or_resample(lb, qb, d)
            want = os_.accept_or_resample(rows[r], q, d)
            assert got == want, f"row {r} draft {d}: {got} vs {want}"
            assert np.array_equal(ds.rng(), os_.rng())
            kd, ko = ds.kept(), os_.kept()  # the processed set, or the residual after a rejection
            assert np.array_equal(kd[0], ko[0]) and np.array_equal(bits(kd[1]), bits(ko[1])), f"row {r} draft {d}"
    for b in (lb, qb):
        b.free()
    for s in (ds, qsrc_d):
        s.free()


def test_reference_distribution_test_on_the_device(ctx):
    """tests/sample.rs:47-74 with the device's accept_or_resample (drafts drawn on the host from q)."""
    n = 20_000
    p = [0.5, 0.3, 0.2]
    logits = np.log(np.asarray(p, np.float32)).astype(np.float32)
    lb, qb = aq.DeviceBuffer(ctx, 12), aq.DeviceBuffer(ctx, 12)
    lb.upload(logits)

    def hist(q, seed):
        ds = aq.Sampler(ctx, aq.sampler_config(temperature=1.0, seed=seed), 3)
        qb.upload(np.asarray(q, np.float32))
        rng = O.rng_seed(seed ^ 0xA5A5)
        counts, acc = np.zeros(3, np.int64), 0
        for _ in range(n):
            u = np.float32(O.lib().or_rng_f32(O.ptr(rng)))
            cum, d = np.float32(0), 2
            for i, qi in enumerate(np.asarray(q, np.float32)):
                cum = np.float32(cum + qi)
                if u < cum:
                    d = i
                    break
            ok, tok = ds.accept_or_resample(lb, qb, d)
            counts[tok] += 1
            acc += ok
        ds.free()
        return counts, acc

    for what, q in [("q != p", [0.2, 0.5, 0.3]), ("q == p", [0.5, 0.3, 0.2]), ("point-mass", [0.0, 1.0, 0.0])]:
        say(f"case distribution {what}")
        counts, acc = hist(q, 7)
        e = n * np.asarray(p)
        x = float(np.sum((counts - e) ** 2 / e))
        assert x < 13.82, f"{what}: chi2 {x}"
        assert abs(acc / n - sum(min(a, b) for a, b in zip(p, q))) < 0.02
    a, _ = hist([0.2, 0.5, 0.3], 11)
    b, _ = hist([0.2, 0.5, 0.3], 11)
    assert np.array_equal(a, b)


@pytest.fixture(scope="module")
def tiny(ctx):
    cfg = aq.tiny_config()
    tensors = aq.plan_tensors(aq.model_plan(cfg, aq.MIX_TINY, SEED))
    gm = aq.Model(ctx, cfg, tensors=tensors)
    ocfg = O.AqModelConfig()
    for name, _ in O.AqModelConfig._fields_:
        setattr(ocfg, name, getattr(cfg, name))
    om = O.Model(ocfg, tensors, threads=8)
    prompt = np.random.default_rng(SEED).integers(0, cfg.vocab, 16).astype(np.uint32)
    return dict(cfg=cfg, gm=gm, om=om, prompt=prompt)


@pytest.mark.parametrize("kw", [dict(temperature=1.0, top_k=20, top_p=0.95), dict(temperature=1.4),
                                dict(temperature=0.9, top_k=600, min_p=0.02)])
def test_tiny_sampled_plain_and_spec_equal_the_oracle(ctx, tiny, kw):
    vocab = tiny["cfg"].vocab
    say(f"case tiny sampled decode {kw}")
    ds = aq.Sampler(ctx, aq.sampler_config(**kw, seed=5), vocab)
    os_ = O.Sampler(O.sampler_config(**kw, seed=5), vocab)
    g, o = aq.State(tiny["gm"], 0, 128), O.State(tiny["om"], 0, 128)
    tg, to = g.prefill(tiny["prompt"], sampler=ds), o.prefill(tiny["prompt"], sampler=os_)
    for i in range(20):
        assert tg == to, f"plain token {i}"
        tg, to = g.forward_token(tg, sampler=ds), o.forward_token(to, sampler=os_)
    assert np.array_equal(ds.rng(), os_.rng())
    assert np.array_equal(g.export(), o.export())
    say(f"case tiny sampled spec 3 {kw}")
    ds.reseed(77)
    os_.reseed(77)
    g, o = aq.State(tiny["gm"], 3, 200), O.State(tiny["om"], 3, 200)
    xg, xo = g.spec_prefill(tiny["prompt"], sampler=ds), o.spec_prefill(tiny["prompt"], sampler=os_)
    assert xg == xo and g.drafts() == o.drafts()
    hist = np.zeros(4, np.int64)
    for r in range(16):
        mg, eg = g.spec_round(xg, sampler=ds)
        mo, eo = o.spec_round(xo, sampler=os_)
        assert (mg, eg) == (mo, eo), f"round {r}: {(mg, eg)} vs {(mo, eo)}"
        assert g.drafts() == o.drafts(), f"round {r}: drafts"
        assert np.array_equal(ds.rng(), os_.rng()), f"round {r}: generator state"
        hist[mg] += 1
        xg, xo = eg[-1], eo[-1]
    say(f"accepted-count histogram {hist.tolist()}")
    assert np.array_equal(g.export(), o.export())
    ds.free()


def test_tiny_top_k_1_sampled_spec_is_the_greedy_loop(ctx, tiny):
    vocab = tiny["cfg"].vocab
    ds = aq.Sampler(ctx, aq.sampler_config(temperature=0.8, top_k=1, seed=3), vocab)
    g, s = aq.State(tiny["gm"], 3, 160), aq.State(tiny["gm"], 3, 160)
    xg, xs = g.spec_prefill(tiny["prompt"]), s.spec_prefill(tiny["prompt"], sampler=ds)
    assert xg == xs
    for r in range(8):
        a, b = g.spec_round(xg), s.spec_round(xs, sampler=ds)
        assert a == b and g.drafts() == s.drafts(), f"round {r}"
        xg = xs = a[1][-1]
    assert np.array_equal(g.export(), s.export())
    ds.free()


def test_tiny_sampler_calls_right_after_a_sampled_round_see_its_draws(ctx, tiny):
    """A sampled round returns while its MTP re-feed and draft chain are still queued on the state's stream, and
    they draw from the sampler. Reading the generator state, or running an operator call on the sampler, right after
    the round (no drafts() call in between, which would synchronise) must see every draw of the round: the sampler
    orders its users by its last-use event. Checked against the oracle round by round, with a sampled operator call
    on the context stream between rounds."""
    vocab = tiny["cfg"].vocab
    say("case sampler used right after a sampled round")
    kw = dict(temperature=1.0, top_k=20, top_p=0.95)
    ds = aq.Sampler(ctx, aq.sampler_config(**kw, seed=21), vocab)
    os_ = O.Sampler(O.sampler_config(**kw, seed=21), vocab)
    g, o = aq.State(tiny["gm"], 3, 200), O.State(tiny["om"], 3, 200)
    xg, xo = g.spec_prefill(tiny["prompt"], sampler=ds), o.spec_prefill(tiny["prompt"], sampler=os_)
    assert xg == xo
    row = logits_rows(vocab, 1, SEED + 9)[0]
    dev_row = aq.DeviceBuffer(ctx, row.nbytes)
    dev_row.upload(row)
    for r in range(8):
        mg, eg = g.spec_round(xg, sampler=ds)
        mo, eo = o.spec_round(xo, sampler=os_)
        assert np.array_equal(ds.rng(), os_.rng()), f"round {r}: generator state read right after the round"
        assert (mg, eg) == (mo, eo), f"round {r}"
        # an operator call on the context stream while nothing has synchronised the state's stream
        tg = ds.sample(dev_row)
        to = os_.sample(row)
        assert tg == to and np.array_equal(ds.rng(), os_.rng()), f"round {r}: operator sample after the round"
        assert g.drafts() == o.drafts(), f"round {r}: drafts"
        xg, xo = eg[-1], eo[-1]
    assert np.array_equal(g.export(), o.export())
    ds.free()
