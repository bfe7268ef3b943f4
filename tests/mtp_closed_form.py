"""Weights under which the speculative loop has a closed form, and that closed form.

Every decoder layer of the tiny hybrid and of its MTP block gets zero output projections (`ssm_out`, `attn_output`,
`ffn_down`): each mixer and MLP then adds an exact +0 to the residual, so a layer is the identity and the main
model's hidden for token x is embed(x) (model.rs:364-368, layers/mod.rs:295-330). `nextn.eh_proj` becomes an F32
selection matrix, so the MTP's input projection is exact:

    "h":   [0 | I]  u = rmsnorm(h, hnorm)                   (the hidden half of the row)
    "e":   [I | 0]  u = rmsnorm(embed(x), enorm)            (the embedding half)
    "sum": [I | I]  u = rmsnorm(embed(x), enorm) + rmsnorm(h, hnorm), one f32 rounding

Then, following docs/mtp.md:57-93 and mtp.rs:95-137 / spec.rs:192-272, 326-433 of the reference:

    f(x)       = argmax(lm_head . Q8_K(rmsnorm(embed(x), output_norm)))     the main model's next token
    row(x, h)  = [rmsnorm(embed(x), enorm) | rmsnorm(h, hnorm)]
    hout(x, h) = rmsnorm(eh_proj . row(x, h), shared_head_norm)             the block is the identity
    draft(v)   = argmax(lm_head . Q8_K(v))

    spec_prefill(ids): x_T = f(ids[-1]); the MTP's last row is (x_T, normed(ids[-1])), d_1 = draft(hout), and each
                       further draft chains on the previous draft's embedding and the previous post-norm hout.
    spec_round(x_p):   batch = [x_p, d_1..d_k]; accept while f(batch[i]) == d_{i+1}; emit f(batch[i]) at each step
                       and f(batch[k]) when all k are accepted; re-feed (emitted[i], normed(batch[i])) for the kept
                       rows, draft from the last kept row, chain.

The expectations below are built only from oracle primitives that the reference's own fixtures pin: the Q4_K
dequantiser (embedding rows, tests/golden/dequant), RMSNorm (tests/golden/kernels/rmsnorm), the Q8_K quantiser and
the K-quant matmul (tests/golden/kernels/{q8k_quantize,dot,matvec}). Nothing here calls the oracle's model code, so a
wrong composition in the oracle's (or the device's) MTP — halves swapped, the pre-norm hidden chained, the wrong
draft's embedding — gives different tokens.
"""
import numpy as np

import oracle_lib as O

ZEROED = ("ssm_out.weight", "attn_output.weight", "ffn_down.weight")


def collapsed_tensors(tensors, cfg, eh_mode, seed, norm_mode="random"):
    """The tensor list with the identity layers and the selection eh_proj. norm_mode "random": enorm, hnorm,
    shared_head_norm and output_norm ~ U(0.5, 1.5); "matched": enorm = output_norm random, hnorm and
    shared_head_norm 1 (the MTP then predicts f almost exactly, so drafts get accepted)."""
    h = cfg.hidden
    rng = np.random.default_rng(seed)
    onorm = rng.uniform(0.5, 1.5, h).astype(np.float32)
    norms = {"output_norm.weight": onorm}
    mi = cfg.n_layer
    pre = f"blk.{mi}.nextn."
    if norm_mode == "random":
        for n in ("enorm", "hnorm", "shared_head_norm"):
            norms[pre + n + ".weight"] = rng.uniform(0.5, 1.5, h).astype(np.float32)
    else:
        norms[pre + "enorm.weight"] = onorm.copy()
        norms[pre + "hnorm.weight"] = np.ones(h, np.float32)
        norms[pre + "shared_head_norm.weight"] = np.ones(h, np.float32)
    eye = np.eye(h, dtype=np.float32)
    zero = np.zeros((h, h), np.float32)
    eh = {"h": np.hstack([zero, eye]), "e": np.hstack([eye, zero]), "sum": np.hstack([eye, eye])}[eh_mode]
    out = []
    for name, t, rows, cols, data in tensors:
        if name.endswith(ZEROED):
            data = np.zeros_like(data)
        elif name in norms:
            data = norms[name]
        elif name == pre + "eh_proj.weight":
            t, data = O.F32, eh
        out.append((name, t, rows, cols, data))
    return out


class ClosedForm:
    """The speculative loop of the collapsed model, from pinned primitives only."""

    MUTANTS = ("swap_halves", "chain_prenorm", "chain_same_token")

    def __init__(self, cfg, tensors, eh_mode, k, mutant=None):
        """mutant: a plausible mistake to compose instead, to show the checks can tell it apart: "swap_halves"
        (the row as [h | e]), "chain_prenorm" (the chain feeds the hidden before shared_head_norm),
        "chain_same_token" (the chain re-embeds the round's token instead of the previous draft)."""
        self.cfg, self.k, self.mode, self.mutant = cfg, k, eh_mode, mutant
        by = {name: (t, rows, cols, data) for name, t, rows, cols, data in tensors}
        self.h, self.vocab, self.eps = cfg.hidden, cfg.vocab, np.float32(cfg.rms_eps)
        t, rows, cols, data = by["token_embd.weight"]
        assert t == O.Q4_K
        self.emb = data.reshape(rows, -1)
        self.lm_t, _, _, lm = by["output.weight"]
        self.lm = lm
        pre = f"blk.{cfg.n_layer}.nextn."
        self.onorm = by["output_norm.weight"][3]
        self.enorm = by[pre + "enorm.weight"][3]
        self.hnorm = by[pre + "hnorm.weight"][3]
        self.shnorm = by[pre + "shared_head_norm.weight"][3]
        self._f = {}

    def embed(self, x):
        return O.dequant(O.Q4_K, self.emb[x], self.h)

    def rms(self, v, w):
        y = np.zeros(self.h, np.float32)
        O.lib().or_rmsnorm(O.ptr(np.ascontiguousarray(v, np.float32)), O.ptr(w), float(self.eps), O.ptr(y), self.h)
        return y

    def logits(self, v):
        return O.matmul(self.lm_t, self.lm, self.vocab, self.h, v)[0]

    def argmax(self, v):
        return int(np.argmax(self.logits(v)))  # first maximum; no NaN here

    def normed(self, x):
        return self.rms(self.embed(x), self.onorm)

    def f(self, x):
        if x not in self._f:
            self._f[x] = self.argmax(self.normed(x))
        return self._f[x]

    def hout(self, x, hvec):
        """(post-norm hidden, the block's output before shared_head_norm) of the MTP row (x, hvec)."""
        if self.mutant == "swap_halves":
            e, hh = self.rms(hvec, self.enorm), self.rms(self.embed(x), self.hnorm)
        else:
            e, hh = self.rms(self.embed(x), self.enorm), self.rms(hvec, self.hnorm)
        u = {"h": hh, "e": e, "sum": (e + hh).astype(np.float32)}[self.mode]
        return self.rms(u, self.shnorm), u

    def chain(self, x_last, hvec):
        """Drafts d_1..d_k from the MTP row (x_last, hvec): d_1 from that row, then chained."""
        ho, u = self.hout(x_last, hvec)
        d = [self.argmax(ho)]
        for _ in range(1, self.k):
            x = x_last if self.mutant == "chain_same_token" else d[-1]
            ho, u = self.hout(x, u if self.mutant == "chain_prenorm" else ho)
            d.append(self.argmax(ho))
        return d

    def spec_prefill(self, ids):
        x_t = self.f(int(ids[-1]))
        return x_t, self.chain(x_t, self.normed(int(ids[-1])))

    def spec_round(self, x_p, drafts):
        batch = [x_p] + list(drafts)
        emitted, m = [], 0
        while m < self.k:
            a = self.f(batch[m])
            emitted.append(a)
            if a != drafts[m]:
                break
            m += 1
        if m == self.k:
            emitted.append(self.f(batch[self.k]))
        keep = m + 1
        new_drafts = self.chain(emitted[keep - 1], self.normed(batch[keep - 1]))
        return m, emitted, new_drafts


def forced_drafts(cf, x_p, c):
    """Drafts for a round at x_p that the main model accepts up to position c exactly (m = c; c >= k: all k): the
    chain of f from x_p, with draft c+1 replaced by another token (the reference's spec_identity.rs:136-170
    cycles the corrupted position the same way)."""
    d, x = [], x_p
    for _ in range(cf.k):
        x = cf.f(x)
        d.append(x)
    if c < cf.k:
        d[c] = (d[c] + 1) % cf.vocab
    return d


def run_trace(state_or_cf, cf, prompt, rounds):
    """The loop's trace — (m, emitted, drafts after the round) per round — on an oracle or device state
    (spec_prefill / spec_round / set_drafts / drafts) or, with state_or_cf = cf, the closed form. Odd rounds run on
    forced drafts whose accepted count cycles 0..k."""
    closed = state_or_cf is cf
    if closed:
        x, d = cf.spec_prefill(prompt)
    else:
        x = state_or_cf.spec_prefill(prompt)
        d = state_or_cf.drafts()
    trace = [("prefill", x, list(d))]
    for r in range(rounds):
        if r % 2 == 1:
            d = forced_drafts(cf, x, (r // 2) % (cf.k + 1))
            if not closed:
                state_or_cf.set_drafts(d)
        if closed:
            m, em, d = cf.spec_round(x, d)
        else:
            m, em = state_or_cf.spec_round(x)
            d = state_or_cf.drafts()
        trace.append((m, list(em), list(d)))
        x = em[-1]
    return trace
