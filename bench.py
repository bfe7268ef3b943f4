#!/usr/bin/env python3
"""bench.py — greedy --spec 3 decode of the random-init 27B-shaped Q4_K_M hybrid on one MI355X.

The workload is the reference's headline path: 64 layers (48 Gated-DeltaNet + 16 gated GQA),
hidden 5120, FFN 17408, vocab 248,320, the MTP block, weights ~N(0, 0.02) quantised to the Q4_K_M type mix and
generated directly in HBM; a 64-token seeded prompt; then speculative rounds with k = 3 drafts. One step = one
speculative round (verify k+1 rows reading every weight once, accept on the device, commit the DeltaNet state,
re-feed the MTP and draft k tokens). `value` = emitted tokens / wall time of the timed rounds.

Printed as one JSON line, with
  roofline      the dominant kernel (the K-quant verify matmul: Q4_K 17408 x 5120 at N = k+1 = 4, the FFN gate/up
                shape that carries 38% of the weight bytes) timed with HIP events on its stream, against 8 TB/s;
  kernels       the matvec (N = 1) and the blocked verify op (N = 2, 4, 6, 8) on the single-op shapes (Q4_K
                17408 x 5120, Q6_K 5120 x 17408) and the lm_head matvec (Q6_K 248320 x 5120), GB/s and fraction of
                8 TB/s per launch;
  cpu_baseline  the CPU oracle (a C restatement of the reference's CPU path) on the box's host cores, on a bounded
                sample of the same workload (a short prompt, then --spec 3 rounds for ~20 s);
and the per-round byte model (weights read once + DeltaNet state + KV + MTP) as round_roofline.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen-3.8-in-rust_amd"))
import aqueduct as aq  # noqa: E402

HBM_PEAK_GBS = 8000.0
SEED = 20260905


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="timed speculative rounds")
    ap.add_argument("--warmup", type=int, default=8, help="untimed speculative rounds")
    ap.add_argument("--spec", type=int, default=3)
    ap.add_argument("--prompt", type=int, default=64)
    ap.add_argument("--plain-tokens", type=int, default=64, help="plain greedy tokens timed for comparison")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-only", action="store_true", help="only the dominant-kernel timing (for counter runs)")
    return ap.parse_args()


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def kernel_roofline(ctx, k):
    """The verify matmul (Q4_K 17408 x 5120, N = k+1 columns) over 8 distinct weights (400 MB, beyond the MALL),
    timed with HIP events on the context stream. Algorithmic bytes per launch: W + N*x + N*y."""
    rows, cols, n = 17408, 5120, k + 1
    ws = [aq.SynthWeight(ctx, aq.synth_spec(aq.Q4_K, rows, cols, seed=SEED + 100 + i)) for i in range(8)]
    x = np.random.default_rng(1).standard_normal((n, cols)).astype(np.float32)
    act = aq.Act(ctx, cols, n)
    act.set(x)
    act.quantize(aq.Q4_K, n)
    y = aq.DeviceBuffer(ctx, n * rows * 4)
    aq.matmul_time(ctx, ws, act, n, y, 32)
    us = aq.matmul_time(ctx, ws, act, n, y, 400)
    wbytes = rows * aq.row_bytes(aq.Q4_K, cols)
    traffic_alg = wbytes + n * (cols // 256) * 292 + n * rows * 4
    achieved = traffic_alg / (us * 1e-6) / 1e9
    for w in ws:
        w.free()
    return {"kernel": f"kq_wave_kernel Q4_K {rows}x{cols} N={n}", "us_per_launch": round(us, 3),
            "bytes_per_launch": traffic_alg, "achieved_GBs": achieved}


def kernel_sweep(ctx):
    """The matvec (N = 1) and the blocked verify op (N = k+1 in {2, 4, 6, 8}) on the single-op shapes: Q4_K
    17408 x 5120 and Q6_K 5120 x 17408 over 8 distinct weights each (beyond the MALL), and the Q6_K lm_head
    248320 x 5120 at N = 1 (the draft chain's matvec). HIP-event time per launch on the context stream; GB/s from
    the algorithmic bytes W + N*x + N*y. Flat GB/s against N means each weight super-block is read once per launch."""
    out = []
    for t, rows, cols, nw, ns in [(aq.Q4_K, 17408, 5120, 8, (1, 2, 4, 6, 8)), (aq.Q6_K, 5120, 17408, 8, (1, 2, 4, 6, 8)),
                                  (aq.Q6_K, 248320, 5120, 1, (1,))]:
        ws = [aq.SynthWeight(ctx, aq.synth_spec(t, rows, cols, seed=SEED + 200 + i)) for i in range(nw)]
        wbytes = rows * aq.row_bytes(t, cols)
        for n in ns:
            x = np.random.default_rng(n).standard_normal((n, cols)).astype(np.float32)
            act = aq.Act(ctx, cols, n)
            act.set(x)
            act.quantize(t, n)
            y = aq.DeviceBuffer(ctx, n * rows * 4)
            reps = 200 if nw > 1 else 20
            aq.matmul_time(ctx, ws, act, n, y, reps // 8)
            us = aq.matmul_time(ctx, ws, act, n, y, reps)
            nbytes = wbytes + n * (cols // 256) * 292 + n * rows * 4
            gbs = nbytes / (us * 1e-6) / 1e9
            name = {aq.Q4_K: "Q4_K", aq.Q6_K: "Q6_K"}[t]
            out.append({"kernel": f"{name} {rows}x{cols}", "n": n, "us_per_launch": round(us, 2),
                        "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)})
            y.free()
            act.free()
        for w in ws:
            w.free()
    return out


def measured_traffic():
    """HBM bytes per launch of the dominant kernel from its committed counter summary (FETCH_SIZE + WRITE_SIZE,
    scaled by a device copy of known size), or None."""
    path = os.path.join(ROOT, "profiles", "kq_wave_q4k_17408x5120_n4.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1])
    return None


def round_bytes(cfg, mb, k, ctx_len):
    """HBM bytes one --spec k round must move at minimum: every weight once (W_main), the DeltaNet state read by the
    verify and read + written by the commit, the conv windows likewise, the KV rows the attention reads, and k MTP
    passes (eh_proj + block + the shared lm_head)."""
    n_dn = sum(1 for i in range(cfg.n_layer) if (i + 1) % cfg.full_attention_interval != 0)
    n_at = cfg.n_layer - n_dn
    rec = n_dn * cfg.dn_n_v_heads * cfg.dn_head_dim_k * cfg.dn_head_dim_v * 4
    kd = cfg.dn_n_k_heads * cfg.dn_head_dim_k
    conv = n_dn * (2 * kd + cfg.dn_n_v_heads * cfg.dn_head_dim_v) * (cfg.dn_conv_kernel - 1) * 4
    kv = n_at * ctx_len * 2 * cfg.n_head_kv * cfg.head_dim * 4
    mtp = k * (mb["mtp_block"] + mb["lm_head"])
    return mb["main"] + 3 * rec + 3 * conv + kv + mtp


def cpu_baseline(cfg, plan, k, seconds, gpu_model):
    """The CPU oracle on the same synthetic 27B model: a 4-token prompt, then --spec k rounds until `seconds` of
    rounds have run. Also checks that the device emits the same ids for the same prompt."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O  # the checker / CPU baseline only

    threads = min(16, os.cpu_count() or 1)
    t0 = time.time()
    tensors = aq.plan_tensors(plan, threads)
    log(f"cpu baseline: host tensors generated in {time.time() - t0:.1f} s")
    ocfg = O.AqModelConfig()
    for name, _ in O.AqModelConfig._fields_:
        setattr(ocfg, name, getattr(cfg, name))
    om = O.Model(ocfg, tensors, threads=threads)
    prompt = np.random.default_rng(SEED + 1).integers(0, cfg.vocab, 4).astype(np.uint32)
    st = O.State(om, k, 64)
    out = [st.spec_prefill(prompt)]
    rounds, emitted, t_rounds = 0, 0, 0.0
    while t_rounds < seconds or rounds < 2:
        t1 = time.time()
        m, em = st.spec_round(out[-1])
        t_rounds += time.time() - t1
        out += em
        rounds += 1
        emitted += len(em)
        if rounds >= 32:
            break
    log(f"cpu baseline: {rounds} rounds, {emitted} tokens in {t_rounds:.1f} s")
    gs = aq.State(gpu_model, k, 64)
    gout = [gs.spec_prefill(prompt)]
    while len(gout) < len(out):
        _, em = gs.spec_round(gout[-1])
        gout += em
    match = gout[: len(out)] == out
    del st, om, tensors
    return {"value": emitted / t_rounds, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"27B-shape Q4_K_M, 4-token prompt, {rounds} greedy --spec {k} rounds ({emitted} tokens) on "
                      f"the C oracle with {threads} threads", "ids_match_device": bool(match)}


def main():
    a = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py runs on one GPU only: this build's path (one MI355X per sequence) has no multi-GPU mode; "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    ctx = aq.Context(0)
    k = a.spec
    kr = kernel_roofline(ctx, k)
    ks = kernel_sweep(ctx) if not a.kernel_only else None
    if a.kernel_only:  # the counter runs: the dominant kernel plus a plain device copy of known size
        nbytes = 512 << 20
        src, dst = aq.DeviceBuffer(ctx, nbytes), aq.DeviceBuffer(ctx, nbytes)
        for _ in range(4):
            dst.copy_from(src, nbytes)
        print(json.dumps({"kernel": kr, "copy_bytes": nbytes}), flush=True)
        return
    cfg = aq.config_27b()
    plan = aq.model_plan(cfg, aq.MIX_Q4_K_M, SEED)
    t0 = time.time()
    model = aq.Model(ctx, cfg, mix=aq.MIX_Q4_K_M, seed=SEED)
    mb = model.bytes()
    log(f"27B model generated in HBM in {time.time() - t0:.1f} s: {mb}")
    prompt = np.random.default_rng(SEED).integers(0, cfg.vocab, a.prompt).astype(np.uint32)
    max_pos = a.prompt + (k + 1) * (a.warmup + a.steps) + a.plain_tokens + 64

    # plain greedy decode (reported beside the speculative number)
    ps = aq.State(model, 0, max_pos)
    plain = [ps.prefill(prompt)]
    for _ in range(4):
        plain.append(ps.forward_token(plain[-1]))
    ctx.sync()
    t1 = time.perf_counter()
    for _ in range(a.plain_tokens):
        plain.append(ps.forward_token(plain[-1]))
    ctx.sync()
    plain_tps = a.plain_tokens / (time.perf_counter() - t1)
    log(f"plain: {plain_tps:.2f} tokens/s")

    # greedy --spec k
    ss = aq.State(model, k, max_pos)
    out = [ss.spec_prefill(prompt)]
    for _ in range(a.warmup):
        _, em = ss.spec_round(out[-1])
        out += em
    st0 = ss.stats()
    ctx.sync()
    t1 = time.perf_counter()
    emitted = 0
    for _ in range(a.steps):
        _, em = ss.spec_round(out[-1])
        out += em
        emitted += len(em)
    ctx.sync()
    dt = time.perf_counter() - t1
    st1 = ss.stats()
    tps = emitted / dt
    ms_round = dt * 1e3 / a.steps
    n_cmp = min(len(out), len(plain))
    ids_equal = out[:n_cmp] == plain[:n_cmp]
    accepted = st1["accepted"] - st0["accepted"]
    verify_ms = (st1["verify_ms"] - st0["verify_ms"]) / a.steps
    stages = {s: round((st1[s] - st0[s]) / a.steps, 3) for s in ("verify_ms", "commit_ms", "refeed_ms", "chain_ms")}
    log(f"spec {k}: {tps:.2f} tokens/s, {ms_round:.2f} ms/round, acceptance {accepted / (k * a.steps):.3f}, "
        f"ids equal plain over {n_cmp}: {ids_equal}, stages {stages}")

    ctx_len = a.prompt + len(out)
    rb = round_bytes(cfg, mb, k, ctx_len)
    result = {
        "metric": "tokens/s, 27B-shape Q4_K_M greedy --spec 3; verify-kernel HBM GB/s vs peak",
        "value": round(tps, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_round, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k_m x q8_k (int8 dot, fp32 accumulate)",
        "data": "synthetic: random-init weights ~N(0,0.02) quantised to the Q4_K_M mix, seeded uniform prompt ids",
        "config": {"workload": "27B-shape hybrid (64 layers: 48 Gated-DeltaNet + 16 gated GQA, hidden 5120, FFN "
                               "17408, vocab 248320, MTP), greedy --spec 3, one step = one speculative round",
                   "prompt": a.prompt, "spec_k": k, "seed": SEED},
        "roofline": {"bound": "hbm", "achieved": round(kr["achieved_GBs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(kr["achieved_GBs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel": kr["kernel"], "us_per_launch": kr["us_per_launch"],
                     "bytes_per_launch": kr["bytes_per_launch"]},
        "kernels": ks,
        "round_roofline": {"bytes_per_round": rb, "ms_per_round": round(ms_round, 3),
                           "achieved_GBs": round(rb / (ms_round * 1e-3) / 1e9, 1),
                           "frac": round(rb / (ms_round * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                           "verify_pass_weight_GBs": round(mb["main"] / (verify_ms * 1e-3) / 1e9, 1)},
        "stages_ms_per_round": stages,
        "acceptance": round(accepted / (k * a.steps), 4),
        "plain_tokens_per_s": round(plain_tps, 3),
        "spec_ids_equal_plain": bool(ids_equal),
        "cpu_baseline": None,
    }
    if not a.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, plan, k, a.cpu_seconds, model)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
