"""The oracle's sampler (oracle_sample.c, a restatement of sample.rs) against what pins it:

* the generators' published known answers: xoshiro256** from the state {1, 2, 3, 4} (Blackman & Vigna's reference
  implementation, the vector rand_xoshiro checks) and splitmix64 from 0; f32() takes the top 24 bits;
* the reference's own test, tests/sample.rs:47-74: 20,000 draws through accept_or_resample from a fixed 3-way
  target p with a 3-way draft q (q != p, q == p, a point mass) match p by chi-square (2 d.o.f., 13.82), the
  acceptance rate is sum min(p, q) within 0.02, the plain sampler matches p, and seeded runs reproduce;
* closed forms of `process` (sample.rs:181-236): the order (logit descending, ties by the lower id, also where
  top_k cuts through a tie), the top-p rule (a candidate stays while the mass before it is below top_p), the min-p
  rule, the softmax at a temperature against float64, greedy = first argmax, write_dense;
* the random stream the rule consumes: one draw per accept test, one more for a resample, none in greedy mode
  (what the device must reproduce draw for draw);
* a model-level special case: with top_k = 1 the sampled speculative loop (spec.rs:367-380) must emit the greedy
  ids, each round consuming exactly the draws the rule implies.
"""
import numpy as np
import pytest

import oracle_lib as O

XOSHIRO_1234 = [11520, 0, 1509978240, 1215971899390074240, 1216172134540287360, 607988272756665600,
                16172922978634559625, 8476171486693032832, 10595114339597558777, 2904607092377533576]
SPLITMIX_0 = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
N = 20_000
CHI2_TOL = 13.82


def test_generators_known_answers():
    s = np.array([1, 2, 3, 4], np.uint64)
    assert [int(O.lib().or_rng_next(O.ptr(s))) for _ in range(10)] == XOSHIRO_1234
    assert [int(v) for v in O.rng_seed(0)] == SPLITMIX_0
    s = O.rng_seed(99)
    ref = s.copy()
    for _ in range(100):
        u = O.lib().or_rng_f32(O.ptr(s))
        top = int(O.lib().or_rng_next(O.ptr(ref))) >> 40
        assert u == np.float32(top) * np.float32(2.0 ** -24) and 0.0 <= u < 1.0


def draw_from(state, q):
    u = np.float32(O.lib().or_rng_f32(O.ptr(state)))
    cum = np.float32(0)
    for i, qi in enumerate(q):
        cum = np.float32(cum + np.float32(qi))
        if u < cum:
            return i
    return len(q) - 1


def chi2(counts, p):
    e = N * np.asarray(p, np.float64)
    return float(np.sum((np.asarray(counts) - e) ** 2 / e))


def histogram(p, q, seed):
    logits = np.log(np.asarray(p, np.float32)).astype(np.float32)
    sp = O.Sampler(O.sampler_config(temperature=1.0, seed=seed), len(p))
    rng = O.rng_seed(seed ^ 0xA5A5)
    q = np.asarray(q, np.float32)
    counts, acc = np.zeros(len(p), np.int64), 0
    for _ in range(N):
        d = draw_from(rng, q)
        ok, tok = sp.accept_or_resample(logits, q, d)
        counts[tok] += 1
        acc += ok
    return counts, acc


def test_speculative_sampling_preserves_the_target_distribution():
    p = [0.5, 0.3, 0.2]
    for what, q in [("q != p", [0.2, 0.5, 0.3]), ("q == p", [0.5, 0.3, 0.2]), ("point-mass draft", [0.0, 1.0, 0.0])]:
        counts, acc = histogram(p, q, 7)
        x = chi2(counts, p)
        assert x < CHI2_TOL, f"{what}: chi2 {x}"
        exp = sum(min(a, b) for a, b in zip(p, q))
        assert abs(acc / N - exp) < 0.02, f"{what}: acceptance {acc / N} vs {exp}"
    logits = np.log(np.asarray(p, np.float32)).astype(np.float32)
    sp = O.Sampler(O.sampler_config(temperature=1.0, seed=7), 3)
    counts = np.bincount([sp.sample(logits) for _ in range(N)], minlength=3)
    assert chi2(counts, p) < CHI2_TOL
    a, _ = histogram(p, [0.2, 0.5, 0.3], 11)
    b, _ = histogram(p, [0.2, 0.5, 0.3], 11)
    assert np.array_equal(a, b)


def test_a_wrong_rule_fails_the_distribution_test():
    """The chi-square test can tell the rule apart from plausible mistakes (resampling from p instead of the
    residual; accepting with p(d) alone): simulated here with the same draws."""
    p = np.array([0.5, 0.3, 0.2])
    q = np.array([0.2, 0.5, 0.3])
    rng = np.random.default_rng(3)
    for mistake in ("resample_from_p", "accept_with_p"):
        counts = np.zeros(3, np.int64)
        for _ in range(N):
            d = rng.choice(3, p=q)
            acc_p = p[d] if mistake == "accept_with_p" else min(1.0, p[d] / q[d])
            if rng.random() < acc_p:
                counts[d] += 1
                continue
            r = p if mistake == "resample_from_p" else np.maximum(p - q, 0) / np.maximum(p - q, 0).sum()
            counts[rng.choice(3, p=r)] += 1
        assert chi2(counts, p) > CHI2_TOL, mistake


def test_process_order_ties_and_top_k():
    logits = np.array([1.0, 3.0, 3.0, -2.0, 3.0, 0.5, 2.0], np.float32)
    sp = O.Sampler(O.sampler_config(temperature=1.0, top_k=0), logits.size)
    ids, probs = sp.process(logits)
    assert ids.tolist() == [1, 2, 4, 6, 0, 5, 3]  # descending, ties by the lower id
    assert probs[0] == probs[1] == probs[2] and np.all(np.diff(probs) <= 0)
    sp = O.Sampler(O.sampler_config(temperature=1.0, top_k=2), logits.size)
    ids, probs = sp.process(logits)
    assert ids.tolist() == [1, 2] and probs.tolist() == [0.5, 0.5]  # top_k cuts the tie by id
    sp = O.Sampler(O.sampler_config(temperature=1.0, top_k=1), logits.size)
    assert sp.process(logits)[0].tolist() == [1] and sp.process(logits)[1].tolist() == [1.0]
    g = O.Sampler(O.sampler_config(temperature=0.0), logits.size)
    assert g.process(logits)[0].tolist() == [1] and g.sample(logits) == 1  # greedy: the first maximum


@pytest.mark.parametrize("temp", [0.3, 1.0, 2.5])
def test_process_softmax_closed_form(temp):
    rng = np.random.default_rng(int(temp * 10))
    logits = (rng.standard_normal(300) * 3).astype(np.float32)
    sp = O.Sampler(O.sampler_config(temperature=temp), logits.size)
    ids, probs = sp.process(logits)
    order = sorted(range(logits.size), key=lambda i: (-float(logits[i]), i))
    assert ids.tolist() == order
    z = logits.astype(np.float64)[order] / temp
    ref = np.exp(z - z.max())
    ref /= ref.sum()
    assert np.max(np.abs(probs - ref) / ref) < 2e-5
    assert abs(float(np.sum(probs.astype(np.float64))) - 1.0) < 1e-5
    dense = sp.write_dense()
    assert np.array_equal(dense[ids], probs) and np.count_nonzero(dense) == np.count_nonzero(probs)


def test_top_p_and_min_p_rules():
    p = np.array([0.5, 0.25, 0.125, 0.0625, 0.0625], np.float32)  # exact in f32, softmax of log p is near-exact
    logits = np.log(p).astype(np.float32)
    for top_p, want in [(0.5, 1), (0.6, 2), (0.75, 2), (0.8, 3), (0.9, 4), (0.95, 5), (1.0, 5)]:
        sp = O.Sampler(O.sampler_config(top_p=top_p), 5)
        ids, probs = sp.process(logits)
        assert ids.size == want, (top_p, ids.size)
        assert abs(float(probs.sum()) - 1.0) < 1e-6
    for min_p, want in [(0.0, 5), (0.1, 5), (0.2, 3), (0.3, 2), (0.9, 1)]:
        sp = O.Sampler(O.sampler_config(min_p=min_p), 5)
        assert sp.process(logits)[0].size == want, min_p


def advanced(seed, n):
    s = O.rng_seed(seed)
    for _ in range(n):
        O.lib().or_rng_next(O.ptr(s))
    return s


def test_accept_rule_consumes_one_draw_and_one_more_to_resample():
    rng = np.random.default_rng(5)
    vocab = 50
    for trial in range(40):
        logits = (rng.standard_normal(vocab) * 2).astype(np.float32)
        sp = O.Sampler(O.sampler_config(temperature=1.0, top_k=10, seed=trial), vocab)
        qs = O.Sampler(O.sampler_config(temperature=1.3, top_k=12, seed=1000 + trial), vocab)
        qs.process((rng.standard_normal(vocab) * 2).astype(np.float32))
        q = qs.write_dense()
        d = int(rng.integers(0, vocab))
        ok, tok = sp.accept_or_resample(logits, q, d)
        assert np.array_equal(sp.rng(), advanced(trial, 1 if ok else 2))
        if ok:
            assert tok == d
        else:
            ids, probs = O.Sampler(O.sampler_config(temperature=1.0, top_k=10), vocab).process(logits)
            assert tok in ids.tolist()
            assert probs[ids.tolist().index(tok)] > q[tok], "a resample comes from where p exceeds q"
    # q == p: always accepted; q(d) = 0: never
    logits = (rng.standard_normal(vocab)).astype(np.float32)
    sp = O.Sampler(O.sampler_config(temperature=1.0, top_k=8, seed=3), vocab)
    sp.process(logits)
    q = sp.write_dense()
    ids = sp.process(logits)[0]
    for d in ids.tolist():
        assert sp.accept_or_resample(logits, q, d) == (True, d)
    zero = [i for i in range(vocab) if q[i] == 0][:5]
    for d in zero:
        ok, tok = sp.accept_or_resample(logits, q, d)
        assert not ok and tok != d


def test_top_k_1_sampled_spec_is_greedy_spec():
    """With top_k = 1 every processed distribution is a point mass on the argmax: the sampled loop emits the greedy
    ids and drafts, and consumes, per round, k draws for the drafts plus one per accept test, one more on a rejection
    and one for the bonus (spec.rs:367-380, 192-203)."""
    import aqueduct as aq
    cfg = aq.tiny_config()
    tensors = aq.plan_tensors(aq.model_plan(cfg, aq.MIX_TINY, 4242))
    ocfg = O.AqModelConfig()
    for name, _ in O.AqModelConfig._fields_:
        setattr(ocfg, name, getattr(cfg, name))
    om = O.Model(ocfg, tensors, threads=8)
    prompt = np.random.default_rng(3).integers(0, cfg.vocab, 12).astype(np.uint32)
    k = 3
    g = O.State(om, k, 128)
    s = O.State(om, k, 128)
    sp = O.Sampler(O.sampler_config(temperature=0.8, top_k=1, seed=77), cfg.vocab)
    xg, xs = g.spec_prefill(prompt), s.spec_prefill(prompt, sampler=sp)
    assert xg == xs and g.drafts() == s.drafts()
    used = 1 + k
    assert np.array_equal(sp.rng(), advanced(77, used))
    for r in range(6):
        mg, eg = g.spec_round(xg)
        ms, es = s.spec_round(xs, sampler=sp)
        assert (mg, eg) == (ms, es) and g.drafts() == s.drafts(), f"round {r}"
        used += ms + (2 if ms < k else 1 + 1) + k
        assert np.array_equal(sp.rng(), advanced(77, used)), f"round {r}: draws consumed"
        xg = xs = eg[-1]
    assert np.array_equal(g.export(), s.export())
