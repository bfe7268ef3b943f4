"""The decode step, the speculative round (greedy, sampled, q8-fine) and the blocked matmul allocate nothing once their
buffers exist: the library's own allocation counters (aq_alloc_counts, which every device and pinned-host allocation
of libaq goes through) do not move across them. The reference asserts the same with a counting allocator
(tests/decode_alloc.rs:80, 185; tests/matmul_t_alloc.rs:76-116)."""
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "qwen-3.8-in-rust_amd"))
import aqueduct as aq  # noqa: E402

pytestmark = pytest.mark.gpu
SEED = 20260905


def test_rounds_steps_and_matmuls_allocate_nothing():
    ctx = aq.Context(0)
    cfg = aq.tiny_config()
    model = aq.Model(ctx, cfg, mix=aq.MIX_TINY, seed=SEED)
    prompt = np.random.default_rng(SEED).integers(0, cfg.vocab, 16).astype(np.uint32)
    spec, plain = aq.State(model, 3, 400), aq.State(model, 0, 400)
    sp = aq.Sampler(ctx, aq.sampler_config(temperature=1.0, top_k=20, top_p=0.95, seed=9), cfg.vocab)
    w = aq.SynthWeight(ctx, aq.synth_spec(aq.Q4_K, 512, 1024, seed=3))
    a = aq.Act(ctx, 1024, 8)
    a.set(np.random.default_rng(1).standard_normal((8, 1024)).astype(np.float32))
    a.quantize(aq.Q4_K, 8)
    y = aq.DeviceBuffer(ctx, 8 * 512 * 4)
    x = spec.spec_prefill(prompt)
    t = plain.prefill(prompt)
    before = aq.alloc_counts()
    print(f"allocations after set-up: {before}", flush=True)
    for r in range(8):
        m, em = spec.spec_round(x)
        x = em[-1]
        t = plain.forward_token(t)
    for r in range(6):
        m, em = spec.spec_round(x, sampler=sp)
        x = em[-1]
        t = plain.forward_token(t, sampler=sp)
    with aq.q8_fine():
        for r in range(4):
            m, em = spec.spec_round(x)
            x = em[-1]
            t = plain.forward_token(t)
    for n in (1, 4, 8):
        aq.lib().aq_matmul(ctx.h, w.h, a.h, n, y.p)
    assert aq.alloc_counts() == before, f"allocations during decode: {before} -> {aq.alloc_counts()}"
