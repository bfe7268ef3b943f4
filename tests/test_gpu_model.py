"""The device model path against the CPU oracle and the reference's layer fixtures.

* layer pieces (tests/layers.rs:109-271 fixtures, F32 weights): the device layer equals the oracle's and meets the
  fixture budget;
* the tiny hybrid (3 DeltaNet + 1 attention layer + MTP, Q4_K/Q6_K): prefill and 32 greedy tokens give the oracle's
  ids, logits within 1e-3 of the oracle's (relative to the largest |logit|);
* greedy --spec 3 emits exactly the plain ids (tests/spec_identity.rs:34-119) and matches the oracle round by round
  (drafts, accepted count);
* forced drafts: after every round the device state equals the plain path's state at the same position bit for
  bit, and the oracle's within tolerance (the reference's rollback contract, spec.rs:396-415);
* the isolated recurrence with rollback (the DeltaNet config: 32 V / 16 K heads x 128): outputs within 1e-4 of the
  oracle, the committed state bit-identical to a plain sequential run of the kept rows.
"""
import ctypes as C
import json
import math
import os
import sys

import numpy as np
import pytest

import oracle_lib as O

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "qwen-3.8-in-rust_amd"))
import aqueduct as aq  # noqa: E402

pytestmark = pytest.mark.gpu

DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "layers")
EPS = float(np.finfo(np.float32).eps)
SEED = 20260905


@pytest.fixture(scope="module")
def ctx():
    return aq.Context(0)


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


# ------------------------------------------------------------------------------------------ layer fixtures
with open(os.path.join(DIR, "manifest.json")) as f:
    M = json.load(f)
CFG = M["config"]
K = M["budget_k"]


def farr(field):
    return np.load(os.path.join(DIR, field["file"]), allow_pickle=False).astype(np.float32)


def fcase(name):
    return next(c for c in M["cases"] if c["case"] == name)


def fx_config(mod):
    c = mod.AqModelConfig()
    c.n_layer, c.hidden, c.ffn, c.vocab = 1, CFG["hidden_size"], CFG["intermediate_size"], CFG["vocab_size"]
    c.n_head, c.n_head_kv, c.head_dim = CFG["num_attention_heads"], CFG["num_key_value_heads"], CFG["head_dim"]
    c.rope_dim = int(CFG["head_dim"] * CFG["rope_parameters"]["partial_rotary_factor"])
    c.rope_theta, c.rms_eps = CFG["rope_parameters"]["rope_theta"], CFG["rms_norm_eps"]
    c.full_attention_interval = 4
    c.dn_n_k_heads, c.dn_n_v_heads = CFG["linear_num_key_heads"], CFG["linear_num_value_heads"]
    c.dn_head_dim_k, c.dn_head_dim_v = CFG["linear_key_head_dim"], CFG["linear_value_head_dim"]
    c.dn_conv_kernel, c.has_mtp = CFG["linear_conv_kernel_dim"], 0
    return c


def fx_tensors(c):
    out = []
    for name, f in c["weights"].items():
        a = farr(f)
        rows, cols = (a.shape[0], a.shape[1]) if a.ndim == 2 else (1, a.size)
        out.append(("blk.0." + name, aq.F32, rows, cols, a))
    return out


class Pair:
    """The same layer on the device and in the oracle, with their own carried state."""

    def __init__(self, ctx, c, kind):
        self.ctx, self.kind = ctx, kind
        self.tensors = fx_tensors(c)
        self.gcfg, self.ocfg = fx_config(aq), fx_config(O)
        self.otable, self.okeep = O.tensor_table(self.tensors)
        cfg = self.gcfg
        cd = 2 * cfg.dn_n_k_heads * cfg.dn_head_dim_k + cfg.dn_n_v_heads * cfg.dn_head_dim_v
        self.cap = 16
        stride = cfg.n_head_kv * cfg.head_dim
        z = lambda n: np.zeros(n, np.float32)  # noqa: E731
        self.g = dict(conv=z(cd * 3), rec=z(cfg.dn_n_v_heads * cfg.dn_head_dim_k * cfg.dn_head_dim_v),
                      kc=z(self.cap * stride), vc=z(self.cap * stride), len=0)
        self.o = dict(conv=z(cd * 3), rec=z(cfg.dn_n_v_heads * cfg.dn_head_dim_k * cfg.dn_head_dim_v),
                      kc=z(self.cap * stride), vc=z(self.cap * stride), len=C.c_uint32(0))

    def run(self, x, start):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.gcfg.hidden)
        g = self.g
        yg, g["len"] = aq.layer_run(self.ctx, self.gcfg, self.tensors, self.kind, x, start, g["conv"], g["rec"],
                                    g["kc"], g["vc"], g["len"], self.cap)
        o = self.o
        yo = np.zeros_like(x)
        rc = O.lib().or_layer_run(C.byref(self.ocfg), self.otable, len(self.tensors), self.kind, O.ptr(x), x.shape[0],
                                  start, O.ptr(o["conv"]), O.ptr(o["rec"]), O.ptr(o["kc"]), O.ptr(o["vc"]),
                                  C.byref(o["len"]), self.cap, O.ptr(yo))
        assert rc == 0
        return yg, yo


def budget_check(label, got, want, width):
    bud = K * math.sqrt(width) * EPS * float(np.abs(want).max())
    d = float(np.abs(got.astype(np.float64) - want.astype(np.float64)).max())
    assert d <= bud, f"{label}: {d:e} > {bud:e}"


def oracle_check(label, got, want, tol=1e-5):
    r = rel(got, want)
    print(f"{label}: device vs oracle rel {r:.3e}, bit-identical {np.array_equal(got, want)}", flush=True)
    assert r <= tol, f"{label}: device vs oracle {r:e}"


@pytest.mark.parametrize("name,kind", [("deltanet_layer", 0), ("attention_layer", 1), ("mlp_layer", 2),
                                       ("decoder_linear_attention", 3), ("decoder_full_attention", 4)])
def test_layer_pieces_match_oracle_and_fixtures(ctx, name, kind):
    print(f"case {name} kind {kind}", flush=True)
    c = fcase(name)
    p = Pair(ctx, c, kind)
    hidden, inter = CFG["hidden_size"], CFG["intermediate_size"]
    width = max(hidden, inter, 64)
    x = farr(c["prefill"]["x"])
    if kind >= 3:  # token by token, as tests/layers.rs:253-257
        ys = [p.run(x[i], i) for i in range(c["t"])]
        yg = np.concatenate([a for a, _ in ys])
        yo = np.concatenate([b for _, b in ys])
    else:
        yg, yo = p.run(x, 0)
    oracle_check(f"{name} prefill", yg, yo)
    budget_check(f"{name} prefill vs fixture", yg, farr(c["prefill"]["y"]).reshape(yg.shape), width)
    if kind in (0, 3):
        oracle_check(f"{name} rec", p.g["rec"], p.o["rec"])
        oracle_check(f"{name} conv", p.g["conv"], p.o["conv"])
    if kind in (1, 4):
        assert p.g["len"] == p.o["len"].value
        n = p.g["len"] * fx_config(aq).n_head_kv * CFG["head_dim"]
        oracle_check(f"{name} K cache", p.g["kc"][:n], p.o["kc"][:n])
        oracle_check(f"{name} V cache", p.g["vc"][:n], p.o["vc"][:n])
    if "step" in c:
        pos = c["step"].get("position", c["t"])
        yg1, yo1 = p.run(farr(c["step"]["x"]), pos)
        oracle_check(f"{name} step", yg1, yo1)
        budget_check(f"{name} step vs fixture", yg1, farr(c["step"]["y"]).reshape(yg1.shape), width)


def test_attention_past_the_lds_context(ctx):
    """A KV cache longer than the attention kernel's LDS holds scores for (16k positions less head_dim): the score
    rows go to device memory, with the same arithmetic, against the oracle."""
    c = fcase("attention_layer")
    print("case attention long context", flush=True)
    tensors = fx_tensors(c)
    gcfg, ocfg = fx_config(aq), fx_config(O)
    stride = gcfg.n_head_kv * gcfg.head_dim
    lds_positions = 65536 // 4 - gcfg.head_dim - 32
    base, t = lds_positions - 2, 4  # the launch's context, base + t, is past what the LDS holds
    cap = base + t
    rng = np.random.default_rng(3)
    kc = np.zeros(cap * stride, np.float32)
    vc = np.zeros(cap * stride, np.float32)
    kc[: base * stride] = rng.standard_normal(base * stride).astype(np.float32)
    vc[: base * stride] = rng.standard_normal(base * stride).astype(np.float32)
    x = rng.standard_normal((t, gcfg.hidden)).astype(np.float32)
    z = lambda n: np.zeros(n, np.float32)  # noqa: E731
    cd = 2 * gcfg.dn_n_k_heads * gcfg.dn_head_dim_k + gcfg.dn_n_v_heads * gcfg.dn_head_dim_v
    kg, vg = kc.copy(), vc.copy()
    yg, lg = aq.layer_run(ctx, gcfg, tensors, 1, x, base, z(cd * 3), z(1), kg, vg, base, cap)
    ko, vo = kc.copy(), vc.copy()
    lo = C.c_uint32(base)
    table, keep = O.tensor_table(tensors)
    yo = np.zeros_like(x)
    assert O.lib().or_layer_run(C.byref(ocfg), table, len(tensors), 1, O.ptr(x), t, base, O.ptr(z(cd * 3)),
                                O.ptr(z(1)), O.ptr(ko), O.ptr(vo), C.byref(lo), cap, O.ptr(yo)) == 0
    assert lg == lo.value == cap
    oracle_check("attention long context", yg, yo)
    assert np.array_equal(kg, ko) and np.array_equal(vg, vo)


# ---------------------------------------------------------------------------------------------- tiny model
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
    return dict(cfg=cfg, plan=plan, tensors=tensors, gm=gm, om=om, prompt=prompt)


def plain_run(state, prompt, n, want_logits=False):
    tok, lg = state.prefill(prompt, want_logits=True)
    ids, lgs = [tok], [lg]
    for _ in range(n - 1):
        tok, lg = state.forward_token(ids[-1], want_logits=True)
        ids.append(tok)
        lgs.append(lg)
    return ids, lgs


def test_tiny_synth_on_device_equals_host_upload(ctx, tiny):
    print("case tiny synth vs upload", flush=True)
    gs = aq.Model(ctx, tiny["cfg"], mix=aq.MIX_TINY, seed=SEED)
    a = aq.State(tiny["gm"], 0, 128)
    b = aq.State(gs, 0, 128)
    ta, la = a.prefill(tiny["prompt"], want_logits=True)
    tb, lb = b.prefill(tiny["prompt"], want_logits=True)
    assert ta == tb and np.array_equal(la, lb)
    assert tiny["gm"].bytes() == gs.bytes()


def test_tiny_model_loaded_from_gguf_equals_tensor_table(ctx, tiny, tmp_path):
    """aq_model_load_gguf (config derived from the file's metadata, tensors from the mapped file) against the same
    model loaded from host tensors: the same config and bit-identical logits and state."""
    print("case tiny model from a GGUF file", flush=True)
    p = tmp_path / "tiny.gguf"
    aq.gguf_write_synth(p, tiny["cfg"], aq.MIX_TINY, SEED, threads=4)
    gm, cfg = aq.model_load_gguf(ctx, p)
    assert all(getattr(cfg, n) == getattr(tiny["cfg"], n) for n, _ in aq.AqModelConfig._fields_)
    a, b = aq.State(tiny["gm"], 0, 64), aq.State(gm, 0, 64)
    ta, la = a.prefill(tiny["prompt"], want_logits=True)
    tb, lb = b.prefill(tiny["prompt"], want_logits=True)
    assert ta == tb and np.array_equal(la, lb)
    for _ in range(4):
        ta, tb = a.forward_token(ta), b.forward_token(tb)
        assert ta == tb
    assert np.array_equal(a.export(), b.export())


def test_tiny_plain_greedy_matches_oracle(ctx, tiny):
    print("case tiny plain greedy", flush=True)
    gs = aq.State(tiny["gm"], 0, 128)
    os_ = O.State(tiny["om"], 0, 128)
    gids, glg = plain_run(gs, tiny["prompt"], 32)
    oids, olg = plain_run(os_, tiny["prompt"], 32)
    worst = max(rel(g, o) for g, o in zip(glg, olg))
    exact = sum(np.array_equal(g, o) for g, o in zip(glg, olg))
    print(f"tiny plain: logits max rel {worst:.3e}, {exact}/32 steps bit-identical; ids {gids[:8]}...", flush=True)
    assert gids == oids
    assert worst <= 1e-3  # the north star's bound; with the reference's expf / log1pf on both sides, 0
    assert exact == 32, "logits differ from the oracle (which calls the platform libm, as the reference does)"
    se, so = gs.export(), os_.export()
    assert se.size == so.size
    assert np.array_equal(se, so)


def spec_run(state, prompt, n):
    x = state.spec_prefill(prompt)
    out, rounds = [x], []
    while len(out) < n:
        drafts = state.drafts()
        m, em = state.spec_round(out[-1])
        rounds.append((drafts, m, em))
        out += em
    return out[:n], rounds


def test_tiny_spec3_identity_and_oracle_rounds(ctx, tiny):
    print("case tiny spec 3", flush=True)
    gp = aq.State(tiny["gm"], 0, 160)
    plain, _ = plain_run(gp, tiny["prompt"], 32)
    gs = aq.State(tiny["gm"], 3, 160)
    os_ = O.State(tiny["om"], 3, 160)
    gids, grounds = spec_run(gs, tiny["prompt"], 32)
    oids, orounds = spec_run(os_, tiny["prompt"], 32)
    st = gs.stats()
    print(f"tiny spec: rounds {st['rounds']} accepted {st['accepted']} hist {st['hist'][:4]}", flush=True)
    assert gids == plain, "greedy --spec 3 must emit the plain ids"
    assert gids == oids
    assert [r[:2] for r in grounds] == [r[:2] for r in orounds], "drafts and acceptance differ from the oracle"


def test_tiny_forced_drafts_state_equals_plain(ctx, tiny):
    print("case tiny forced drafts", flush=True)
    gp = aq.State(tiny["gm"], 0, 160)
    plain, _ = plain_run(gp, tiny["prompt"], 40)
    gs = aq.State(tiny["gm"], 3, 160)
    os_ = O.State(tiny["om"], 3, 160)
    x = gs.spec_prefill(tiny["prompt"])
    assert x == os_.spec_prefill(tiny["prompt"]) == plain[0]
    out = [x]
    for r in range(8):
        j = len(out)  # plain[j:j+3] are the correct drafts for this round
        n_ok = r % 4  # every acceptance count m = 0..3 twice (spec_identity.rs:136-170)
        d = [plain[j + i] if i < n_ok else (plain[j + i] + 1) % tiny["cfg"].vocab for i in range(3)]
        gs.set_drafts(d)
        os_.set_drafts(d)
        m, em = gs.spec_round(out[-1])
        mo, emo = os_.spec_round(out[-1])
        assert (m, em) == (mo, emo)
        assert m == n_ok and em == plain[j:j + len(em)]
        out += em
        # the device state equals a plain run to the same position, bit for bit, and the oracle's within 1e-3
        ref = aq.State(tiny["gm"], 0, 160)
        ref.prefill(tiny["prompt"])
        for tok in out[:-1]:
            ref.forward_token(tok)
        a, b = gs.export(), ref.export()
        assert gs.pos == ref.pos == len(tiny["prompt"]) + len(out) - 1
        assert np.array_equal(a[: b.size], b), f"round {r}: spec state differs from the plain state"
        assert np.array_equal(a, os_.export()), f"round {r}: spec state differs from the oracle's"


# ------------------------------------------------------------- the reference's identity gate at every k
STEPS = 200  # spec_identity.rs:20


class PlainTracker:
    """A plain device state advanced token by token to any consumed count (spec_identity.rs:48-72)."""

    def __init__(self, model, prompt, max_pos):
        self.st = aq.State(model, 0, max_pos)
        self.st.prefill(prompt)
        self.consumed = 0

    def at(self, toks, consume):
        assert consume >= self.consumed, "the plain tracker only moves forward"
        for tok in toks[self.consumed:consume]:
            self.st.forward_token(tok)
        self.consumed = consume
        return self.st


@pytest.mark.parametrize("k", [1, 2, 4, 7])
def test_tiny_spec_identity_every_k(ctx, tiny, k):
    """spec_identity.rs:122-205 at k in {1, 2, 4, 7} (7: the largest batch a state takes, 8 verify rows): with the
    MTP's own drafts, 200 greedy ids equal the plain loop's and every round's drafts and accepted count equal the
    oracle's; with forced drafts (the continuation corrupted at position j = round % (k + 1), so every acceptance
    count 0..k occurs), after every round the whole carried state equals a plain state that consumed the same
    tokens bit for bit, and the oracle's."""
    print(f"case tiny spec identity k {k}", flush=True)
    prompt, vocab = tiny["prompt"], tiny["cfg"].vocab
    max_pos = len(prompt) + STEPS + 64
    plain_ids, _ = plain_run(aq.State(tiny["gm"], 0, max_pos), prompt, STEPS + 8)
    # ---- the MTP's own drafts
    gs, os_ = aq.State(tiny["gm"], k, max_pos), O.State(tiny["om"], k, max_pos)
    out, oout = [gs.spec_prefill(prompt)], [os_.spec_prefill(prompt)]
    assert out == oout
    while len(out) < STEPS:
        gd, od = gs.drafts(), os_.drafts()
        m, em = gs.spec_round(out[-1])
        mo, emo = os_.spec_round(oout[-1])
        assert (gd, m, em) == (od, mo, emo), f"k={k} round {gs.stats()['rounds']}: differs from the oracle"
        out += em
        oout += emo
    st = gs.stats()
    print(f"tiny k={k}: {STEPS} ids; rounds {st['rounds']}, accepted {st['accepted']} of {st['drafted']}", flush=True)
    assert out[:STEPS] == plain_ids[:STEPS], f"k={k}: spec ids differ from plain"
    assert np.array_equal(gs.export(), os_.export())
    # ---- forced drafts: every acceptance count, the state checked after every round
    gs, os_ = aq.State(tiny["gm"], k, max_pos), O.State(tiny["om"], k, max_pos)
    tracker = PlainTracker(tiny["gm"], prompt, max_pos)
    out = [gs.spec_prefill(prompt)]
    assert out == [os_.spec_prefill(prompt)]
    rnd, hist = 0, [0] * (k + 1)
    while len(out) < STEPS:
        j, n = rnd % (k + 1), len(out)
        d = list(plain_ids[n:n + k])
        if j < k:
            d[j] = (d[j] + 1) % vocab
        gs.set_drafts(d)
        os_.set_drafts(d)
        m, em = gs.spec_round(out[-1])
        mo, emo = os_.spec_round(out[-1])
        assert (m, em) == (mo, emo), f"k={k} round {rnd}: differs from the oracle"
        assert m == j and em == plain_ids[n:n + len(em)], f"k={k} round {rnd}: accepted {m} for j {j}"
        out += em
        hist[m] += 1
        consumed = gs.pos - len(prompt)
        assert consumed == len(out) - 1
        ref = tracker.at(plain_ids, consumed)
        a, b = gs.export(), ref.export()
        assert gs.pos == ref.pos
        assert np.array_equal(a[: b.size], b), f"k={k} round {rnd}: spec state differs from the plain state"
        assert np.array_equal(a, os_.export()), f"k={k} round {rnd}: spec state differs from the oracle's"
        rnd += 1
    assert gs.stats()["hist"][: k + 1] == hist and all(c > 0 for c in hist), hist
    print(f"tiny k={k} forced: {rnd} rounds, hist {hist}, state equal after every round", flush=True)


@pytest.mark.parametrize("k", [1, 2, 3])
def test_tiny_spec_prefill_on_a_used_state(ctx, tiny, k):
    """spec_identity.rs:211-268: a second prompt fed by spec_prefill to a state that already ran speculative rounds
    (a later chat turn) continues exactly as the plain loop over the same tokens, and as the oracle."""
    print(f"case tiny spec prefill on a used state k {k}", flush=True)
    prompt, vocab = tiny["prompt"], tiny["cfg"].vocab
    second = np.random.default_rng(SEED + 5).integers(0, vocab, 6).astype(np.uint32)
    n1, n2, max_pos = 40, 60, 256
    plain_ids, _ = plain_run(aq.State(tiny["gm"], 0, max_pos), prompt, n1)
    pst = aq.State(tiny["gm"], 0, max_pos)
    pst.prefill(prompt)
    for tok in plain_ids[:n1]:  # the plain loop consumes every emitted token before the new prompt
        pst.forward_token(tok)
    plain2 = [pst.prefill(second)]
    while len(plain2) < n2:
        plain2.append(pst.forward_token(plain2[-1]))
    gs, os_ = aq.State(tiny["gm"], k, max_pos), O.State(tiny["om"], k, max_pos)
    out = [gs.spec_prefill(prompt)]
    assert out == [os_.spec_prefill(prompt)]
    while len(out) < n1:
        m, em = gs.spec_round(out[-1])
        assert (m, em) == os_.spec_round(out[-1])
        out += em
    assert out[:n1] == plain_ids[:n1]
    consumed = gs.pos - len(prompt)
    if consumed > n1:
        pytest.skip(f"k={k}: the spec state consumed {consumed} > {n1} tokens (accepted drafts past the cut)")
    seg2 = np.concatenate([np.asarray(plain_ids[consumed:n1], np.uint32), second])
    out2 = [gs.spec_prefill(seg2)]
    assert out2 == [os_.spec_prefill(seg2)]
    while len(out2) < n2:
        m, em = gs.spec_round(out2[-1])
        assert (m, em) == os_.spec_round(out2[-1])
        out2 += em
    assert out2[:n2] == plain2, f"k={k}: the second segment differs from the plain loop"
    assert np.array_equal(gs.export(), os_.export())


def test_spec_calls_out_of_order_are_refused(ctx, tiny):
    """spec.rs:246 and :337 assert the MTP's row count; here the calls return AQ_ESTATE and change nothing: a
    round after a plain call on a spec state, a spec prefill on a state whose plain calls consumed positions past
    the MTP's rows, a spec prefill after a plain prefill on a fresh spec state."""
    print("case spec calls out of order", flush=True)
    prompt = tiny["prompt"]
    st = aq.State(tiny["gm"], 3, 128)
    x = st.spec_prefill(prompt)
    m, em = st.spec_round(x)
    tok = st.forward_token(em[-1])  # consumes a position; the MTP still holds pos - 1 + k - 1 rows
    with pytest.raises(aq.AqError) as e:
        st.spec_round(tok)
    assert e.value.code == aq.AQ_ESTATE
    pos = st.pos
    st.forward_token(tok)
    st.forward_token(tok)  # now past the MTP's rows (k - 1 = 2 draft rows beyond the consumed positions)
    with pytest.raises(aq.AqError) as e:
        st.spec_prefill(prompt[:4])
    assert e.value.code == aq.AQ_ESTATE and st.pos == pos + 2
    fresh = aq.State(tiny["gm"], 3, 128)
    fresh.prefill(prompt)
    with pytest.raises(aq.AqError) as e:
        fresh.spec_prefill(prompt[:4])
    assert e.value.code == aq.AQ_ESTATE
    # a spec prefill whose positions the MTP still covers is taken (spec.rs:246 asks rows >= pos)
    st2 = aq.State(tiny["gm"], 3, 128)
    x = st2.spec_prefill(prompt)
    st2.spec_round(x)
    st2.forward_token(x)
    st2.spec_prefill(prompt[:4])


# ----------------------------------------------------------------------------------- isolated recurrence
def test_deltanet_recurrence_rollback(ctx):
    nv, nk, dk, dv, t = 32, 16, 128, 128, 4
    rng = np.random.default_rng(5)
    L = O.lib()
    for trial, keep in enumerate([1, 2, 3, 4, 2]):
        print(f"case deltanet trial {trial} keep {keep}", flush=True)
        s0 = (rng.standard_normal((nv, dk, dv)) * 0.1).astype(np.float32)
        q = rng.standard_normal((t, nk * dk)).astype(np.float32)
        k = rng.standard_normal((t, nk * dk)).astype(np.float32)
        for arr in (q, k):
            for i in range(t):
                for h in range(nk):
                    seg = np.ascontiguousarray(arr[i, h * dk:(h + 1) * dk])
                    L.or_l2norm(O.ptr(seg), dk, C.c_float(1e-6))
                    arr[i, h * dk:(h + 1) * dk] = seg
        v = rng.standard_normal((t, nv * dv)).astype(np.float32)
        beta = np.array([[L.or_sigmoid(float(z)) for z in row] for row in rng.standard_normal((t, nv))], np.float32)
        g = np.array([[-L.or_softplus(float(z)) for z in row] for row in rng.standard_normal((t, nv))], np.float32)
        # oracle: sequential steps; the state after `keep` rows
        so = s0.copy()
        out_o = np.zeros((t, nv * dv), np.float32)
        s_keep = None
        for i in range(t):
            for p in range(nv):
                kh = p % nk
                sp = np.ascontiguousarray(so[p])
                o = np.zeros(dv, np.float32)
                L.or_deltanet_step(O.ptr(np.ascontiguousarray(q[i, kh * dk:(kh + 1) * dk])),
                                   O.ptr(np.ascontiguousarray(k[i, kh * dk:(kh + 1) * dk])),
                                   O.ptr(np.ascontiguousarray(v[i, p * dv:(p + 1) * dv])), float(g[i, p]),
                                   float(beta[i, p]), O.ptr(sp), O.ptr(o), dk, dv)
                so[p] = sp
                out_o[i, p * dv:(p + 1) * dv] = o
            if i + 1 == keep:
                s_keep = so.copy()
        st = aq.DeviceBuffer(ctx, s0.nbytes)
        st.upload(s0)
        out_g = aq.deltanet_verify_commit(ctx, nk, nv, dk, dv, keep, q, k, v, g, beta, st)
        s_dev = st.download(np.float32, s0.size).reshape(s0.shape)
        # plain sequential reference on the device: the kept rows only, committed
        st2 = aq.DeviceBuffer(ctx, s0.nbytes)
        st2.upload(s0)
        aq.deltanet_verify_commit(ctx, nk, nv, dk, dv, keep, q[:keep], k[:keep], v[:keep], g[:keep], beta[:keep], st2)
        s_seq = st2.download(np.float32, s0.size).reshape(s0.shape)
        # the device-array form: same bits, no allocation
        bufs = []
        for arr in (q, k, v, g, beta):
            b = aq.DeviceBuffer(ctx, arr.nbytes)
            b.upload(arr)
            bufs.append(b)
        st3, ob = aq.DeviceBuffer(ctx, s0.nbytes), aq.DeviceBuffer(ctx, out_g.nbytes)
        st3.upload(s0)
        before = aq.alloc_counts()
        aq.deltanet_verify_commit_dev(ctx, nk, nv, dk, dv, t, keep, *bufs, st3, ob)
        assert aq.alloc_counts() == before, "the device-array form allocated"
        assert np.array_equal(ob.download(np.float32, out_g.size).reshape(out_g.shape), out_g)
        assert np.array_equal(st3.download(np.float32, s0.size).reshape(s0.shape), s_dev)
        for b in bufs + [st3, ob]:
            b.free()
        r_out, r_state = rel(out_g, out_o), rel(s_dev, s_keep)
        print(f"deltanet keep {keep}: out rel {r_out:.2e}, state rel {r_state:.2e}, "
              f"exact {np.array_equal(out_g, out_o)}/{np.array_equal(s_dev, s_keep)}", flush=True)
        assert np.array_equal(s_dev, s_seq), "rolled-back state differs from the sequential state"
        assert r_out <= 1e-4 and r_state <= 1e-4


# ------------------------------------------------------------------------------------------------- argmax
def ref_argmax(v):
    """model.rs:505-513 literally: best = 0, replaced only when v[i] > v[best]."""
    best = 0
    for i in range(1, len(v)):
        if v[i] > v[best]:
            best = i
    return best


def test_device_argmax_ties_and_nan(ctx):
    print("case argmax ties / NaN", flush=True)
    rng = np.random.default_rng(11)
    n = 248320
    rows = []
    base = rng.standard_normal(n).astype(np.float32)
    r = base.copy(); r[[5, 77777, 200000]] = 9.0; rows.append(r)                  # tie: first wins
    r = base.copy(); r[0] = np.nan; r[1234] = 50.0; rows.append(r)               # NaN at 0: answer 0
    r = base.copy(); r[3] = np.nan; r[100] = np.nan; r[4000] = 7.0; rows.append(r)  # NaN elsewhere skipped
    r = base.copy(); r[::3] = np.nan; rows.append(r)
    r = np.full(n, -np.inf, np.float32); rows.append(r)                           # all -inf: 0
    r = np.full(n, -np.inf, np.float32); r[n - 1] = -1e30; rows.append(r)       # last element
    r = np.full(n, np.nan, np.float32); r[0] = 1.0; rows.append(r)              # only index 0 is a number
    r = base.copy(); r[2048] = r[2047] = r[4095] = 99.0; rows.append(r)           # tie across chunk boundaries
    x = np.stack(rows)
    got = aq.argmax(ctx, x)
    want = [ref_argmax(row.tolist()) for row in x]
    assert got == want, f"device {got} reference rule {want}"
    small = np.float32([[np.nan, 1.0], [1.0, np.nan], [2.0, 2.0], [-0.0, 0.0]])
    assert aq.argmax(ctx, small) == [ref_argmax(v) for v in small.tolist()] == [0, 0, 0, 0]


def test_tiny_prompt_chunks_equal_token_by_token_and_oracle(ctx, tiny):
    """A 150-token prompt runs in chunks of 64, 64 and 22 rows (each layer over a whole chunk: matmuls over all its
    columns, attention per chunk, the DeltaNet recurrence in pieces of 8 rows inside one launch per chunk, the state
    carried in registers and each piece's conv window read from the rows before it):
    the last row's logits and the whole state equal the oracle's prefill and a token-by-token feed, bit for bit
    (model.rs:443-461, the prefill row i is forward_token on row i)."""
    print("case tiny 150-token prompt in chunks", flush=True)
    prompt = np.random.default_rng(SEED + 9).integers(0, tiny["cfg"].vocab, 150).astype(np.uint32)
    g = aq.State(tiny["gm"], 0, 256)
    tg, lg = g.prefill(prompt, want_logits=True)
    o = O.State(tiny["om"], 0, 256)
    to, lo = o.prefill(prompt, want_logits=True)
    assert tg == to and np.array_equal(lg, lo), "prefill logits differ from the oracle"
    assert np.array_equal(g.export(), o.export()), "prefill state differs from the oracle"
    f = aq.State(tiny["gm"], 0, 256)
    f.prefill(prompt[:1])
    for tok in prompt[1:-1]:
        f.forward_token(int(tok))
    tf, lf = f.forward_token(int(prompt[-1]), want_logits=True)
    assert tf == tg and np.array_equal(lf, lg), "prefill differs from the token-by-token feed"
    assert np.array_equal(f.export(), g.export())
    for _ in range(4):  # and decoding continues identically
        tg, tf = g.forward_token(tg), f.forward_token(tf)
        assert tg == tf


def test_tiny_prompt_past_the_attention_lds_equals_token_by_token(ctx, tiny):
    """A 16,400-token prompt on the tiny model, whose attention kernel keeps the scores of at most 16,288 positions
    in LDS (head_dim 64): the chunks before that run attention over the whole chunk, the chunk that crosses it and
    those after run it in 8-row pieces with the score rows in device memory. Logits and the whole state equal a
    token-by-token feed of the same prompt, bit for bit (model.rs:443-461: prefill row i is forward_token on row i)."""
    n = 16400
    print(f"case tiny {n}-token prompt across the attention LDS limit", flush=True)
    prompt = np.random.default_rng(SEED + 11).integers(0, tiny["cfg"].vocab, n).astype(np.uint32)
    g = aq.State(tiny["gm"], 0, n + 16)
    tg, lg = g.prefill(prompt, want_logits=True)
    f = aq.State(tiny["gm"], 0, n + 16)
    f.prefill(prompt[:1])
    for i, tok in enumerate(prompt[1:-1]):
        f.forward_token(int(tok))
        if i % 4096 == 0:
            print(f"token-by-token feed at {i + 1}", flush=True)
    tf, lf = f.forward_token(int(prompt[-1]), want_logits=True)
    assert tf == tg and np.array_equal(lf, lg), "chunked prefill past the LDS limit differs from the token feed"
    assert np.array_equal(f.export(), g.export())
    g.free()
    f.free()
