#!/usr/bin/env python3
"""bench.py — greedy --spec 3 decode of the random-init 27B-shaped Q4_K_M hybrid on one MI355X.

The workload is the reference's headline path (the full 27B shape): 64 layers (48 Gated-DeltaNet + 16 gated GQA),
hidden 5120, FFN 17408, vocab 248,320, the MTP block, weights ~N(0, 0.02) quantised to the Q4_K_M type mix and
generated directly in HBM; a 64-token seeded prompt; then speculative rounds with k = 3 drafts. One step = one
speculative round (verify k+1 rows reading every weight once, accept on the device, commit the DeltaNet state,
re-feed the MTP and draft k tokens). `value` = emitted tokens / wall time of the timed rounds.

Printed as one JSON line, with
  roofline      the dominant kernel (the K-quant verify matmul: Q4_K 17408 x 5120 at N = k+1 = 4, the FFN gate/up
                shape that carries 38% of the weight bytes) timed with HIP events on its stream, against 8 TB/s: the
                mean over 1000 back-to-back launches (achieved) and the median of 400 single-launch times; beside
                it the read floor: a plain streaming-read kernel over the same bytes, timed the same way (the least
                time any kernel reads that much on this device: launch, ramp and drain included);
  kernels       the matvec (N = 1) and the blocked verify op (N = 2, 4, 6, 8) on the single-op shapes (Q4_K
                17408 x 5120, Q6_K 5120 x 17408) and the lm_head matvec (Q6_K 248320 x 5120), mean and median
                per-launch time, GB/s, fraction of 8 TB/s and of the read floor of the weights' bytes;
  forced        the same rounds with the drafts set to the greedy continuation (spec_set_drafts, the reference's
                rollback-test hook) so that a chosen number m of them is accepted: tokens/s at full acceptance and
                at the reference's measured mean (about 2 of 3 accepted per round at k = 3 on real weights,
                docs/spec.md:140-142), and the round time by m. Random-init weights make the MTP accept almost
                nothing, so `value` is near one token per round; these show what the round delivers when drafts land;
  prefill       the 64-token prompt's prefill (one pass over the weights per chunk of up to 64 rows) on a fresh state;
  sustained     --spec 3 rounds kept running for --sustain-seconds after the timed ones (the GPU busy long enough to
                be seen by a utilisation sampler), tokens/s over that stretch;
  cpu_baseline  the CPU oracle (a C restatement of the reference's CPU path whose K-quant and Q8_0 / Q4_0 dots
                run in AVX2 forms bit-identical to its scalar ones, as the reference's avx2.rs kernels are) on the
                box's physical cores (at most 16, the box's share): config 4's 64-token prompt, then --spec 3
                rounds for --cpu-seconds, plus its matvec / verify GB/s at the config-2/3 shapes (and the scalar
                dots' GB/s beside them);
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
    ap.add_argument("--sustain-seconds", type=float, default=15.0)
    ap.add_argument("--forced-rounds", type=int, default=48)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-only", action="store_true", help="only the dominant-kernel timing (for counter runs)")
    ap.add_argument("--sweep-only", action="store_true", help="only the matmul sweep (for kernel-trace runs)")
    ap.add_argument("--prefill-only", action="store_true", help="only the prompt prefill timing (for kernel-trace runs)")
    ap.add_argument("--shapes", default="", help="with --sweep-only: comma-separated substrings; only sweep shapes "
                                                  "whose name (e.g. 'Q4_K 5120x6144') contains one of them")
    return ap.parse_args()


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def kernel_roofline(ctx, k):
    """The verify matmul (Q4_K 17408 x 5120, N = k+1 columns) over 8 distinct weights (400 MB, beyond the MALL),
    timed with HIP events on the context stream after a warm-up: the mean of 1000 back-to-back launches, and the
    median of 400 single-launch times. Algorithmic bytes per launch: W + N*x + N*y."""
    rows, cols, n = 17408, 5120, k + 1
    ws = [aq.SynthWeight(ctx, aq.synth_spec(aq.Q4_K, rows, cols, seed=SEED + 100 + i)) for i in range(8)]
    x = np.random.default_rng(1).standard_normal((n, cols)).astype(np.float32)
    act = aq.Act(ctx, cols, n)
    act.set(x)
    act.quantize(aq.Q4_K, n)
    y = aq.DeviceBuffer(ctx, n * rows * 4)
    aq.matmul_time(ctx, ws, act, n, y, 400)
    us = aq.matmul_time(ctx, ws, act, n, y, 1000)
    each = aq.matmul_time_each(ctx, ws, act, n, y, 400)
    wbytes = rows * aq.row_bytes(aq.Q4_K, cols)
    traffic_alg = wbytes + n * (cols // 256) * 292 + n * rows * 4
    achieved = traffic_alg / (us * 1e-6) / 1e9
    for w in ws:
        w.free()
    floor = aq.read_floor_time(ctx, traffic_alg)  # a plain streaming read of the same bytes, timed the same way
    return {"kernel": f"kq_wave_kernel Q4_K {rows}x{cols} N={n}", "us_per_launch": round(us, 3),
            "median_us": round(float(np.median(each)), 3),
            "p10_p90_us": [round(float(np.percentile(each, 10)), 3), round(float(np.percentile(each, 90)), 3)],
            "bytes_per_launch": traffic_alg, "achieved_GBs": achieved, "read_floor_us": round(floor, 3)}


TYPE_NAME = {aq.Q4_K: "Q4_K", aq.Q5_K: "Q5_K", aq.Q6_K: "Q6_K", aq.Q8_0: "Q8_0", aq.Q4_0: "Q4_0"}

# (type, rows, cols, distinct weights, column counts) of the sweep
SWEEP = [(aq.Q4_K, 17408, 5120, 8, (1, 2, 4, 6, 8)), (aq.Q6_K, 5120, 17408, 8, (1, 2, 4, 6, 8)),
         (aq.Q4_K, 5120, 17408, 8, (1, 4)), (aq.Q4_K, 5120, 6144, 8, (1, 4)), (aq.Q5_K, 5120, 6144, 8, (1, 4)),
         (aq.Q6_K, 248320, 5120, 1, (1,)), (aq.Q8_0, 5120, 6144, 8, (1, 4)),
         (aq.Q4_0, 5120, 10240, 8, (1,)), (aq.Q4_K, 17408, 5120, 4, (64,)),
         (aq.Q6_K, 5120, 17408, 4, (64,)), (aq.Q8_0, 5120, 6144, 4, (64,))]


def kernel_sweep(ctx, shapes=""):
    """The matvec (N = 1) and the blocked verify op (N = k+1 in {2, 4, 6, 8}) on the single-op shapes: Q4_K
    17408 x 5120 and Q6_K 5120 x 17408 over 8 distinct weights each (beyond the MALL); the other 5120-row matrices of
    the round at N = 1 and 4 (the Q4_K ffn_down 5120 x 17408, the Q4_K ssm_out and Q5_K attn_output 5120 x 6144); the
    Q6_K lm_head 248320 x 5120 at N = 1 (the draft chain's matvec), the Q8_0 ssm_out (N = 1, 4) and the MTP's Q4_0
    eh_proj (N = 1); then the prompt-chunk product (N = 64, the prefill's matrix-core GEMM) on three of them.
    HIP-event time per launch on the context stream; GB/s from the algorithmic bytes W + N*x + N*y. Flat GB/s against
    N means each weight super-block is read once per launch. `shapes`: comma-separated name filters (all if empty)."""
    out = []
    keys = [k.strip() for k in shapes.split(",") if k.strip()]
    for t, rows, cols, nw, ns in SWEEP:
        name = f"{TYPE_NAME[t]} {rows}x{cols}"
        if keys and not any(k in name for k in keys):
            continue
        ws = [aq.SynthWeight(ctx, aq.synth_spec(t, rows, cols, seed=SEED + 200 + i)) for i in range(nw)]
        wbytes = rows * aq.row_bytes(t, cols)
        floor = aq.read_floor_time(ctx, wbytes, iters=50 if wbytes > (256 << 20) else 500)  # the weights' bytes, plainly read
        for n in ns:
            x = np.random.default_rng(n).standard_normal((n, cols)).astype(np.float32)
            act = aq.Act(ctx, cols, n)
            act.set(x)
            act.quantize(t, n)
            y = aq.DeviceBuffer(ctx, n * rows * 4)
            reps = 200 if nw > 1 else 50
            aq.matmul_time(ctx, ws, act, n, y, reps // 4)
            us = aq.matmul_time(ctx, ws, act, n, y, reps)
            med = float(np.median(aq.matmul_time_each(ctx, ws, act, n, y, max(64, reps // 2))))
            xbytes = (cols // 256) * 292 if t in (aq.Q4_K, aq.Q5_K, aq.Q6_K) else (cols // 32) * 40  # Q8_K / Q8_0 rows
            nbytes = wbytes + n * xbytes + n * rows * 4
            gbs = nbytes / (us * 1e-6) / 1e9
            out.append({"kernel": name, "n": n, "us_per_launch": round(us, 2),
                        "median_us": round(med, 2), "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                        "read_floor_us": round(floor, 2), "of_read_floor": round(floor / us, 3)})
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


def cpu_info():
    """The host's CPU model, the CPUs this process may use, and how many physical cores those are (/proc/cpuinfo)."""
    allowed = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else list(range(os.cpu_count() or 1))
    model, core_of, cur = None, {}, {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" not in line:
                if "processor" in cur:
                    core_of[int(cur["processor"])] = (cur.get("physical id", "0"), cur.get("core id", cur["processor"]))
                cur = {}
                continue
            key, val = (x.strip() for x in line.split(":", 1))
            cur[key] = val
            if key == "model name" and model is None:
                model = val
        if "processor" in cur:
            core_of[int(cur["processor"])] = (cur.get("physical id", "0"), cur.get("core id", cur["processor"]))
    except OSError:
        pass
    phys = len({core_of[c] for c in allowed if c in core_of}) or len(allowed)
    return {"model": model, "logical_cpus": os.cpu_count(), "nproc": len(allowed), "physical_cores": phys}


def cpu_matmul_gbs(O, threads, nmat=8):
    """The oracle's matvec (N = 1, config 2) and verify op (N = 4, config 3 at k = 3) on the two single-op shapes:
    weight GB/s (W bytes / time per call), each timed over >= 1 s. `weight_GBs` rotates through `nmat` distinct
    matrices of the shape (8 x 50-73 MB, beyond the host's last-level cache, as the GPU sweep rotates 8 past the
    MALL), so it is a DRAM rate; `weight_GBs_one_matrix` repeats one matrix, which the cache holds."""
    out = []
    for t, rows, cols in [(aq.Q4_K, 17408, 5120), (aq.Q6_K, 5120, 17408)]:
        hosts = [aq.synth_host(aq.synth_spec(t, rows, cols, seed=SEED + 300 + i), threads).view(np.uint8)
                 for i in range(nmat)]
        wbytes = rows * aq.row_bytes(t, cols)
        x = np.random.default_rng(3).standard_normal((4, cols)).astype(np.float32)
        for n in (1, 4):
            rates = {}
            for label, mats in (("rotate", hosts), ("one", hosts[:1])):
                O.matmul(t, mats[0], rows, cols, x[:n], threads=threads)
                reps, t0 = 0, time.perf_counter()
                while time.perf_counter() - t0 < 1.0 or reps < 2 * len(mats):
                    O.matmul(t, mats[reps % len(mats)], rows, cols, x[:n], threads=threads)
                    reps += 1
                rates[label] = (time.perf_counter() - t0) / reps
            out.append({"kernel": f"{TYPE_NAME[t]} {rows}x{cols}", "n": n, "ms_per_call": round(rates["rotate"] * 1e3, 2),
                        "weight_GBs": round(wbytes / rates["rotate"] / 1e9, 2),
                        "weight_GBs_one_matrix": round(wbytes / rates["one"] / 1e9, 2),
                        "matrices": nmat, "bytes_rotated": nmat * wbytes})
        del hosts
    return out


def cpu_baseline(cfg, plan, k, seconds, gpu_model, prompt):
    """The CPU oracle on the same synthetic 27B model and config 4's prompt: the prefill, then --spec k rounds until
    `seconds` of rounds have run (tokens/s over the rounds). Also checks that the device emits the same ids for the
    same prompt over those rounds, and times the oracle's matvec / verify op alone. The oracle runs with its AVX2
    dots on (oracle_simd.c, bit-identical to its scalar ones), as the reference's CPU path runs its avx2.rs kernels;
    the scalar dots' matvec / verify GB/s are reported beside them."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O  # the checker / CPU baseline only

    with O.simd(True):
        res = cpu_baseline_run(O, cfg, plan, k, seconds, gpu_model, prompt)
    with O.simd(False):
        res["matmul_scalar"] = cpu_matmul_gbs(O, res["cores"], nmat=2)  # the scalar dots are compute-bound
    return res


def cpu_baseline_run(O, cfg, plan, k, seconds, gpu_model, prompt):
    info = cpu_info()
    threads = max(1, min(16, info["physical_cores"]))  # cpu.rs:1-12 uses the physical cores; the box's share is 16
    t0 = time.time()
    tensors = aq.plan_tensors(plan, threads)
    log(f"cpu baseline: {info}; host tensors generated in {time.time() - t0:.1f} s")
    ocfg = O.AqModelConfig()
    for name, _ in O.AqModelConfig._fields_:
        setattr(ocfg, name, getattr(cfg, name))
    om = O.Model(ocfg, tensors, threads=threads)
    st = O.State(om, k, len(prompt) + 256)
    t0 = time.time()
    out = [st.spec_prefill(prompt)]
    prefill_s = time.time() - t0
    log(f"cpu baseline: {len(prompt)}-token spec prefill in {prefill_s:.1f} s")
    rounds, emitted, t_rounds = 0, 0, 0.0
    while (t_rounds < seconds or rounds < 2) and rounds < 200:  # the state holds prompt + 256 positions
        t1 = time.time()
        m, em = st.spec_round(out[-1])
        t_rounds += time.time() - t1
        out += em
        rounds += 1
        emitted += len(em)
    log(f"cpu baseline: {rounds} rounds, {emitted} tokens in {t_rounds:.1f} s")
    gs = aq.State(gpu_model, k, len(prompt) + 256)
    gout = [gs.spec_prefill(prompt)]
    while len(gout) < len(out):
        _, em = gs.spec_round(gout[-1])
        gout += em
    match = gout[: len(out)] == out
    del st, om, tensors
    mm = cpu_matmul_gbs(O, threads)
    return {"value": round(emitted / t_rounds, 4), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"27B-shape Q4_K_M, {len(prompt)}-token prompt (spec prefill {prefill_s:.1f} s, not in the "
                      f"rate), then {rounds} greedy --spec {k} rounds ({emitted} tokens, {t_rounds:.1f} s) on the "
                      f"C restatement of the reference's CPU path with AVX2 forms of its K-quant x Q8_K and "
                      f"Q8_0 / Q4_0 dots (bit-identical to the scalar restatement, as the reference's avx2.rs "
                      f"kernels are to its scalar ones), {threads} threads on physical cores",
            "cpu": info, "prefill_s": round(prefill_s, 2), "matmul": mm, "ids_match_device": bool(match)}


def forced_rounds(model, prompt, plain, k, n_rounds, max_pos):
    """Rounds whose drafts are set to the greedy continuation `plain` with draft m+1 corrupted, so exactly m are
    accepted (the reference's spec_identity.rs:136-170 technique). Every round's emitted ids are checked against
    `plain`. Returns tokens/s at m = k every round and under the schedule 3,2,3,1,2,0,3,2 (mean 2.0 accepted), and
    the mean round time for each m."""
    vocab = model.cfg.vocab
    res, by_m = {}, {m: [] for m in range(k + 1)}
    warm = min(4, n_rounds // 2)  # the first rounds warm up (half of a short run)
    for name, sched in (("full_acceptance", [k]), ("reference_mean", [min(m, k) for m in (3, 2, 3, 1, 2, 0, 3, 2)])):
        st = aq.State(model, k, max_pos)
        out = [st.spec_prefill(prompt)]
        assert out[0] == plain[0]
        emitted, dt, ok = 0, 0.0, True
        for r in range(n_rounds):
            m = sched[r % len(sched)]
            j = len(out)
            d = [plain[j + i] if i != m else (plain[j + i] + 1) % vocab for i in range(k)]
            st.set_drafts(d)
            t1 = time.perf_counter()
            mm, em = st.spec_round(out[-1])
            st.drafts()  # waits for the round's tail (commit, MTP re-feed, next drafts)
            t = time.perf_counter() - t1
            ok = ok and mm == m and em == plain[j:j + len(em)]
            if r >= warm:
                dt += t
                emitted += len(em)
                by_m[m].append(t * 1e3)
            out += em
        res[name] = {"tokens_per_s": round(emitted / dt, 3) if dt > 0 else None,
                     "tokens_per_round": round(emitted / (n_rounds - warm), 3) if n_rounds > warm else None,
                     "ids_equal_plain": bool(ok)}
        st.free()
    res["round_ms_by_m"] = {m: round(float(np.median(v)), 3) for m, v in by_m.items() if v}
    return res


def main():
    a = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py runs on one GPU only: this build's path (one MI355X per sequence) has no multi-GPU mode; "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    ctx = aq.Context(0)
    k = a.spec
    # the sweep also brings the clocks up before the roofline timing
    ks = kernel_sweep(ctx, a.shapes if a.sweep_only else "") if not (a.kernel_only or a.prefill_only) else None
    if a.sweep_only:
        print(json.dumps({"kernel_sweep": ks}), flush=True)
        return
    kr = kernel_roofline(ctx, k) if not a.prefill_only else None
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
    max_pos = (a.prompt + (k + 1) * (a.warmup + a.steps + 2 * a.forced_rounds) + a.plain_tokens + 64 +
               int(400 * a.sustain_seconds))

    # prompt prefill (model.rs:443-461): the 64-token prompt on fresh states, timed after one warm-up run
    pre_ms = []
    for r in range(4):
        st = aq.State(model, 0, a.prompt + 64)
        ctx.sync()
        t1 = time.perf_counter()
        st.prefill(prompt)
        pre_ms.append((time.perf_counter() - t1) * 1e3)
        st.free()
    prefill = {"tokens": a.prompt, "ms": round(float(np.median(pre_ms[1:])), 3),
               "tokens_per_s": round(a.prompt / (float(np.median(pre_ms[1:])) * 1e-3), 1)}
    log(f"prefill: {prefill}")
    if a.prefill_only:
        print(json.dumps({"prefill": prefill}), flush=True)
        return

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
    while len(plain) < (k + 1) * 2 * a.forced_rounds + 8:  # the greedy continuation the forced rounds draft from
        plain.append(ps.forward_token(plain[-1]))

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
    forced = forced_rounds(model, prompt, plain, k, a.forced_rounds, max_pos)
    log(f"forced: {forced}")
    # the GPU kept busy for a while longer (rounds continue from the same state)
    sus_tokens, sus_rounds, t1 = 0, 0, time.perf_counter()
    while time.perf_counter() - t1 < a.sustain_seconds:
        _, em = ss.spec_round(out[-1])
        out += em
        sus_tokens += len(em)
        sus_rounds += 1
    ctx.sync()
    sus_dt = time.perf_counter() - t1
    log(f"sustained: {sus_rounds} rounds, {sus_tokens / max(sus_dt, 1e-9):.2f} tokens/s")
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
                     "kernel": kr["kernel"], "us_per_launch": kr["us_per_launch"], "median_us": kr["median_us"],
                     "p10_p90_us": kr["p10_p90_us"], "bytes_per_launch": kr["bytes_per_launch"],
                     "read_floor_us": kr["read_floor_us"],
                     "of_read_floor": round(kr["read_floor_us"] / kr["us_per_launch"], 3)},
        "kernels": ks,
        "round_roofline": {"bytes_per_round": rb, "ms_per_round": round(ms_round, 3),
                           "achieved_GBs": round(rb / (ms_round * 1e-3) / 1e9, 1),
                           "frac": round(rb / (ms_round * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                           "verify_pass_weight_GBs": round(mb["main"] / (verify_ms * 1e-3) / 1e9, 1)},
        "stages_ms_per_round": stages,
        "acceptance": round(accepted / (k * a.steps), 4),
        "plain_tokens_per_s": round(plain_tps, 3),
        "prefill": prefill,
        "forced": forced,
        "sustained": {"seconds": round(sus_dt, 2), "rounds": sus_rounds,
                      "tokens_per_s": round(sus_tokens / max(sus_dt, 1e-9), 3),
                      "context_end": a.prompt + len(out)},
        "spec_ids_equal_plain": bool(ids_equal),
        "cpu_baseline": None,
    }
    if not a.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, plan, k, a.cpu_seconds, model, prompt)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
