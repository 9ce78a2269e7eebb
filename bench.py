#!/usr/bin/env python3
"""Benchmark of the speculative verify path on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 1|2|3|4|5]

A step is one pass of the hot path over one synthetic batch, with every input
already resident in HBM:
  config 2 (default): one speculative verify step
            of the Qwen3.5-4B-like hybrid decoder — k+1 = 5 rows through 32
            layers (24 Gated DeltaNet + 8 gated attention), LM head over
            151936 tokens, fused greedy acceptance, on-device commit of the
            accepted prefix — as one captured HIP graph; drafts from prompt
            lookup over the history (engine/speculative.go lookupDraft).
  config 3-5 (configs[2..4]): batched verify steps of the batched engine
            (4B-like 16 x k=8 stochastic top-p with a shared prefix; 9B-like
            4 x k=16 greedy at 16K context; MoE-like 8 x k=4 stochastic).
  config 1: activation quantization + one Q4_K
            9216x2560 verify GEMM (M = 5) + fused greedy acceptance over
            5 x 151936 logits.
To defeat the 256 MB Infinity Cache, steps rotate through >= 512 MB of
distinct weight copies.

Prints ONE JSON line. `roofline` covers the dominant kernel (the verify GEMM)
timed live with HIP events on the stream it runs on; `cpu_baseline` times the
oracle (C restatement of tensor/quant.go matmul + engine/speculative.go
accept) on the host cores for a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--config", type=int, default=None,
                    help="one configuration (default: config 2 as the value, configs 1, 3, 4, 5 beside it)")
    ap.add_argument("--drafts", type=int, default=4)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--prompt", type=int, default=None,
                    help="configs 3-5: prompt length override (short traces for profiling)")
    ap.add_argument("--kernel-only", action="store_true",
                    help="time only the dominant kernel, then one 256 MiB copy (profiling calibration)")
    return ap.parse_args()


def ensure_built():
    from yuuka_amd import build as b
    b.ensure_built()


def bench_config1(args):
    """the v10 LM_HEAD op (the verify GEMM as the Go
    engine submits it, backend/hip/hip.go:1187-1235) over one Q4_K 9216x2560
    matrix at M = 5, then the fused greedy acceptance over 5 x 151936 logits,
    as one plan captured in a HIP graph per weight copy."""
    from yuuka_amd import hip, synth

    c = synth.config1(0)
    N, K, M, V, k = c["N"], c["K"], c["M"], c["V"], c["k"]
    wbytes = c["w"].nbytes
    copies = max(1, -(-512 * 2**20 // wbytes))
    dev = hip.Device(0)
    info = dev.info()
    stream = hip.Stream(dev)
    rng = np.random.default_rng(1)
    ws = [dev.upload(c["w"])]
    for _ in range(copies - 1):
        ws.append(dev.upload(synth.quant_matrix(rng, synth.Q4_K, N, K)))
    xb = dev.upload(c["x"])
    out = dev.alloc(M * N * 4)
    lb = dev.upload(c["logits"])
    db = dev.upload(c["drafts"])
    rb = dev.alloc(16)
    rb2 = dev.alloc(16)

    def lm_head_op(plan, w):
        plan.add(hip.OP["LM_HEAD"], [w, xb, out], n=[K, N, M], u=[synth.Q4_K])

    def accept_op(plan, mode, res, temperature=0.0):
        plan.add(hip.OP["ACCEPT"], [lb, db, res], n=[1, k, V, 0, 0, 0], u=[mode, 0, 0, 0], f=[temperature, 1.0])

    plans, graphs = [], []
    for i in range(copies):
        p = hip.Plan(dev)
        lm_head_op(p, ws[i])
        accept_op(p, hip.ACCEPT_GREEDY, rb)
        plans.append(p)
        graphs.append(hip.Graph(p, stream, None))

    def step(i):
        graphs[i % copies].replay(stream)

    for i in range(args.warmup):
        step(i)
    stream.sync()
    e0, e1 = hip.Event(dev, timed=True), hip.Event(dev, timed=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(args.steps):
        step(i)
    e1.record(stream)
    stream.sync()
    wall = time.perf_counter() - t0
    ms_total = e1.elapsed_ms(e0)
    res = rb.read(np.int32)
    tokens_per_step = int(res[0]) + 1
    ms_per_step = ms_total / args.steps

    def timed_graph(build, reps, launches):
        p = hip.Plan(dev)
        for j in range(launches):
            build(p, j)
        g = hip.Graph(p, stream, None)
        g.replay(stream)
        stream.sync()
        e0.record(stream)
        for _ in range(reps):
            g.replay(stream)
        e1.record(stream)
        stream.sync()
        us = e1.elapsed_ms(e0) * 1e3 / (reps * launches)
        g.destroy()
        p.destroy()
        return us

    # Dominant kernel: LM_HEAD launches back to back in one graph, rotating
    # the weight copies (each launch streams its matrix from HBM).
    launches = 4 * copies
    gemm_us = timed_graph(lambda p, j: lm_head_op(p, ws[j % copies]), 20, launches)
    alg_bytes = wbytes + M * K * 4 + M * N * 4  # W + X + Y (fp32 activations in/out)
    achieved = alg_bytes / (gemm_us * 1e-6) / 1e9
    accept_us = timed_graph(lambda p, j: accept_op(p, hip.ACCEPT_GREEDY, rb2), 20, 16)
    accept_t08_us = timed_graph(lambda p, j: accept_op(p, hip.ACCEPT_STOCHASTIC, rb2, 0.8), 20, 16)

    # Correctness of the timed configuration against the oracle.
    from oracle import oracle as O
    hip.lm_head(stream, out, xb, ws[0], K, N, M, synth.Q4_K)
    stream.sync()
    want = O.matmul(O.Q4_K, c["w"], c["x"], N, K)
    got = out.read(np.float32).reshape(M, N)
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    a_ref, nxt_ref, _ = O.accept_greedy(c["logits"], c["drafts"])
    graphs[0].replay(stream)
    stream.sync()
    res0 = rb.read(np.int32)
    parity = bool(res0[0] == a_ref and res0[1] == nxt_ref and np.max(np.abs(got - want)) <= 1e-3 * rms)
    traffic = read_traffic("fgemm_config1_lm_head_pmc.md")

    line = {
        "metric": "accepted tokens/s on 1 MI355X; verify-step HBM GB/s vs peak",
        "value": tokens_per_step / (ms_per_step * 1e-3),
        "unit": "accepted tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights x int16-split activations, int32/fp32 accumulate",
        "data": "synthetic (seeded, BASELINE configs[0]; weights rotated over %d copies = %.0f MB)"
                % (copies, copies * wbytes / 2**20),
        "config": {"workload": "config1: v10 LM_HEAD Q4_K 9216x2560 verify GEMM (M=5) + greedy accept V=151936",
                   "N": N, "K": K, "rows": M, "drafts": k, "vocab": V, "parallelism": "single GPU"},
        "verify_step_us": ms_per_step * 1e3,
        "accepted_tokens_per_step": tokens_per_step,
        "gemm_us": gemm_us,
        "accept_us": accept_us,
        "accept_t0.8_us": accept_t08_us,
        "accept_parity": parity,
        "device": info,
        "wall_s": wall,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "kernel": "fgemm_stream_kernel<12,1,...> (LM_HEAD) Q4_K 9216x2560 M=5",
                     "alg_bytes_per_launch": alg_bytes, "avg_us": gemm_us},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_config1(c, args.cpu_seconds)
    return line


def cpu_baseline_config1(c, budget_s):
    """Oracle verify step on the host: C restatement of tensor/quant.go matmul
    (row chunks over all cores, GOMAXPROCS rule) + greedy accept."""
    from oracle import oracle as O
    N, K = c["N"], c["K"]
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    n = 0
    t0 = time.perf_counter()
    while True:
        O.matmul(O.Q4_K, c["w"], c["x"], N, K, workers=cores)
        a, nxt, _ = O.accept_greedy(c["logits"], c["drafts"])
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 10000:
            break
    step_s = el / n
    return {"value": (a + 1) / step_s, "unit": "accepted tokens/s", "cores": cores, "kind": "port",
            "sample": f"{n} config-1 verify steps (GEMM 9216x2560 Q4_K M=5 + greedy accept) in {el:.1f} s",
            "ms_per_step": step_s * 1e3}


def lookup_draft(history, max_draft, min_match=2):
    """engine/speculative.go:39-66 (prompt-lookup drafts), host side."""
    n = len(history)
    if max_draft <= 0 or n <= min_match:
        return []
    for ln in range(min(8, n - 1), min_match - 1, -1):
        suffix = history[n - ln:]
        for start in range(n - ln - 1, -1, -1):
            if history[start:start + ln] == suffix:
                follow = start + ln
                take = min(max_draft, n - follow)
                if take > 0:
                    return history[follow:follow + take]
    return []


def read_traffic(name):
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE scaled by the copy-kernel
    calibration), or None when the summary is absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", name)
    try:
        with open(path) as f:
            for ln in f:
                if ln.startswith("traffic_bytes_per_launch:"):
                    return float(ln.split(":", 1)[1])
    except OSError:
        pass
    return None


def dominant_kernel(dev, cfg, rows, rng):
    from yuuka_amd import hip, synth
    # Dominant kernel: the fused FFN gate/up verify GEMM (RMSNorm + activation
    # quantization prologue, two Q4_K 9216x2560 weight streams, SwiGLU
    # epilogue), the largest weight stream of every layer, launched exactly as
    # the engine launches it (one GEMM_FUSED op), timed live with HIP events
    # on the stream it runs on. One plan holds `copies` ops over distinct
    # weight buffers (>= 512 MB in all) so that no launch finds its weights
    # in the Infinity Cache.
    N, K = cfg.ffn, cfg.hidden
    wq = synth.quant_matrix(rng, synth.Q4_K, N, K)
    copies = max(1, -(-512 * 2**20 // (2 * wq.nbytes)))
    wg = [dev.upload(wq) for _ in range(copies)]
    wu = [dev.upload(wq) for _ in range(copies)]
    st = hip.Stream(dev)
    xb = dev.upload(rng.normal(0, 1, (rows, K)).astype(np.float32))
    nb = dev.upload((1.0 + 0.1 * rng.normal(0, 1, K)).astype(np.float32))
    ob = dev.alloc(rows * N * 4)
    plan = hip.Plan(dev)
    for i in range(copies):
        hip.gemm_fused_op(plan, xb, K, rows, [(wg[i], synth.Q4_K, N, ob, None), (wu[i], synth.Q4_K, N, None, None)],
                          epilogue=hip.EPI_SWIGLU, norm=nb, eps=cfg.eps)
    for _ in range(2):
        plan.execute(st)
    st.sync()
    e0, e1 = hip.Event(dev, timed=True), hip.Event(dev, timed=True)
    reps = max(1, 200 // copies)
    e0.record(st)
    for _ in range(reps):
        plan.execute(st)
    e1.record(st)
    st.sync()
    gemm_us = e1.elapsed_ms(e0) * 1e3 / (reps * copies)
    gemm_bytes = 2 * wq.nbytes + rows * K * 4 + K * 4 + rows * N * 4
    gemm_ach = gemm_bytes / (gemm_us * 1e-6) / 1e9
    plan.destroy()
    for b in wg + wu:
        b.free()
    if rows <= 8:
        kernel = f"fgemm_stream_kernel<12,2,8,1,true> (GEMM_FUSED SwiGLU) 2x{N}x{K} Q4_K M={rows}"
        traffic = read_traffic("fgemm_ffn_swiglu_pmc.md")
    else:  # many-row GEMM: quantizing prologue + bg_gemm_kernel, timed together
        kernel = f"bg_prologue_kernel + bg_gemm_kernel (GEMM_FUSED SwiGLU, many-row) 2x{N}x{K} Q4_K M={rows}"
        traffic = None
    return {"bound": "hbm", "achieved": gemm_ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": gemm_ach / HBM_PEAK_GBS, "traffic": traffic, "kernel": kernel,
            "alg_bytes_per_launch": gemm_bytes, "avg_us": gemm_us, "launches": reps * copies}


def moe_dominant(dev, cfg, rows, rng):
    """Config 5's dominant kernel: the grouped expert gate/up GEMM (MOE_GATE_UP
    with the SwiGLU epilogue on packed experts, as the engine launches it)
    over rows routed by i.i.d. N(0,1) logits (the configured routing), timed
    with HIP events on its stream; weight copies rotate so that >= 512 MB of
    expert matrices stream per round. Algorithmic bytes: the gate and up
    matrices of the experts the rows selected, the rows, the outputs."""
    from yuuka_amd import hip, synth
    E, used, F, H = cfg.n_experts, cfg.n_experts_used, cfg.expert_ffn, cfg.hidden
    wq = synth.quant_matrix(rng, synth.Q4_K, E * F, H)
    copies = max(1, -(-512 * 2**20 // (2 * wq.nbytes)))
    st = hip.Stream(dev)
    raw = dev.upload(wq)
    packed = []
    for _ in range(2 * copies):
        b = dev.alloc(wq.nbytes)
        hip.moe_pack_q4k(st, b, raw, E * F, H)
        packed.append(b)
    st.sync()
    raw.free()
    lb = dev.upload(rng.normal(0, 1, (rows, E)).astype(np.float32))
    ids, w = dev.alloc(rows * used * 4), dev.alloc(rows * used * 4)
    cnt = dev.alloc(E * 4)
    ar, asl, aw = (dev.alloc(E * rows * used * 4) for _ in range(3))
    xb = dev.upload(rng.normal(0, 1, (rows, H)).astype(np.float32))
    act = dev.alloc(rows * used * F * 4)
    route = hip.Plan(dev)
    route.add(hip.OP["MOE_ROUTE"], [lb, ids, w, cnt, ar, asl, aw], n=[rows, E, used])
    route.execute(st)
    st.sync()
    distinct = int((cnt.read(np.int32, E) > 0).sum())
    plan = hip.Plan(dev)
    for i in range(copies):
        plan.add(hip.OP["MOE_GATE_UP"], [xb, packed[2 * i], packed[2 * i + 1], cnt, ar, asl, act, None],
                 n=[H, F, rows, E, used], u=[synth.Q4_K], flags=hip.FLAG_MOE_SWIGLU | hip.FLAG_MOE_PACKED)
    for _ in range(2):
        plan.execute(st)
    st.sync()
    e0, e1 = hip.Event(dev, timed=True), hip.Event(dev, timed=True)
    reps = max(1, 200 // copies)
    e0.record(st)
    for _ in range(reps):
        plan.execute(st)
    e1.record(st)
    st.sync()
    us = e1.elapsed_ms(e0) * 1e3 / (reps * copies)
    nbytes = distinct * 2 * F * (H // 256) * 144 + rows * H * 4 + rows * used * F * 4
    ach = nbytes / (us * 1e-6) / 1e9
    plan.destroy()
    route.destroy()
    for b in packed + [lb, ids, w, cnt, ar, asl, aw, xb, act]:
        b.free()
    return {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": ach / HBM_PEAK_GBS,
            "traffic": None, "kernel": f"moe_gemm_kernel (MOE_GATE_UP SwiGLU, packed) {E} experts {F}x{H} Q4_K, "
                                       f"{rows} rows x top-{used}, N(0,1) routing: {distinct} experts",
            "alg_bytes_per_launch": nbytes, "avg_us": us, "launches": reps * copies, "distinct_experts": distinct}


def lm_head_only(dev):
    """Config 1's dominant kernel alone: the v10 LM_HEAD op over the Q4_K
    9216x2560 matrix at M = 5, 4 x copies launches per graph replay (weight
    copies rotated, 512 MB in all), 20 replays after one warm-up replay."""
    from yuuka_amd import hip, synth
    c = synth.config1(0)
    N, K, M = c["N"], c["K"], c["M"]
    wbytes = c["w"].nbytes
    copies = max(1, -(-512 * 2**20 // wbytes))
    rng = np.random.default_rng(1)
    ws = [dev.upload(c["w"])] + [dev.upload(synth.quant_matrix(rng, synth.Q4_K, N, K)) for _ in range(copies - 1)]
    xb = dev.upload(c["x"])
    out = dev.alloc(M * N * 4)
    stream = hip.Stream(dev)
    p = hip.Plan(dev)
    launches = 4 * copies
    for j in range(launches):
        p.add(hip.OP["LM_HEAD"], [ws[j % copies], xb, out], n=[K, N, M], u=[synth.Q4_K])
    g = hip.Graph(p, stream, None)
    g.replay(stream)
    stream.sync()
    e0, e1 = hip.Event(dev, timed=True), hip.Event(dev, timed=True)
    reps = 20
    e0.record(stream)
    for _ in range(reps):
        g.replay(stream)
    e1.record(stream)
    stream.sync()
    us = e1.elapsed_ms(e0) * 1e3 / (reps * launches)
    return {"kernel": "LM_HEAD Q4_K 9216x2560 M=5", "avg_us": us, "launches": (reps + 1) * launches}


def kernel_only(args):
    """--kernel-only: the dominant-kernel measurement alone, followed by one
    plain 256 MiB device-to-device copy (the calibration kernel for the
    FETCH_SIZE/WRITE_SIZE counters). Used for the rocprofv3 --pmc passes."""
    from yuuka_amd import hip, model as Mdl
    dev = hip.Device(0)
    rng = np.random.default_rng(2)
    if args.config == 1:
        dk = lm_head_only(dev)
    else:
        dk = dominant_kernel(dev, Mdl.QWEN35_4B_LIKE, args.drafts + 1, rng)
    nbytes = 256 * 2**20
    src, dst = dev.alloc(nbytes), dev.alloc(nbytes)
    st = hip.Stream(dev)
    hip.check(hip.lib().yuuka_buffer_copy(st.ptr, dst.ptr, 0, src.ptr, 0, nbytes, None), "buffer_copy")
    st.sync()
    return {"kernel_only": dk, "copy_calibration_bytes": nbytes}



def bench_config2(args):
    """full verify step on the Qwen3.5-4B-like hybrid
    decoder (random init, Q4_K_M mix), 512-token prompt in paged F16 KV,
    k drafts per step, greedy acceptance."""
    from yuuka_amd import hip, model as Mdl, synth

    k = args.drafts
    steps, warmup = args.steps or 256, args.warmup if args.warmup is not None else 8
    cfg = Mdl.replace(Mdl.QWEN35_4B_LIKE, capacity=512 + (steps + warmup + 2 * 66 + 8) * (k + 1))
    t0 = time.perf_counter()
    w = model_weights("QWEN35_4B_LIKE", cfg)
    gen_s = time.perf_counter() - t0
    wbytes = Mdl.weight_bytes(w)
    dev = hip.Device(0)
    info = dev.info()
    eng = Mdl.Engine(dev, cfg, w)
    rng = np.random.default_rng(2)
    prompt = rng.integers(0, cfg.vocab, 512).astype(np.int32).tolist()
    t0 = time.perf_counter()
    eng.prefill(prompt[:-1], want_logits=False)
    prefill_s = time.perf_counter() - t0
    history = list(prompt)
    pending = prompt[-1]
    acc = Mdl.accept_struct()
    drng = np.random.default_rng(4)

    def geometric_len():
        # leading drafts equal the model's argmax, each with probability 0.7
        # (the draft rule BASELINE configs[3] states); the prescribed accept
        # length is the number of leading hits
        hit = drng.random(k) < 0.7
        return k if hit.all() else int(np.argmin(hit))

    def step_argmax07():
        # k synthetic drafts per step; greedy verify of k+1 rows with the
        # accept length prescribed (the next token is the argmax at the
        # first rejected row)
        nonlocal pending
        toks = np.empty((1, k + 1), np.int32)
        toks[0, 0] = pending
        toks[0, 1:] = drng.integers(0, cfg.vocab, k)
        res = eng.step_batch(toks, 0, acc, np.array([geometric_len()], np.int32))
        history.extend(toks[0, 1:1 + int(res[0, 0])].tolist() + [int(res[0, 1])])
        pending = int(res[0, 1])
        return int(res[0, 0]) + 1, int(res[0, 0]), k, eng.last_step_ms

    lookup_drafts = [0]

    def step_lookup_padded():
        # the headline step: engine/speculative.go:68-261 with prompt-lookup
        # drafts (lookupDraft, :39-66) topped up with uniform ids to the
        # configured k = 4, so every step verifies k + 1 rows; the greedy
        # decision runs on the device's own argmax (nothing prescribed)
        nonlocal pending
        d = lookup_draft(history, k)
        lookup_drafts[0] += len(d)
        d = d + drng.integers(0, cfg.vocab, k - len(d)).tolist()
        res = eng.verify(np.array([pending] + d, np.int32), acc)
        emitted = d[:res[0]] + [int(res[1])]
        history.extend(emitted)
        pending = int(res[1])
        return len(emitted), int(res[0]), k, eng.last_step_ms

    def step_lookup():
        # engine/speculative.go:68-261 with prompt-lookup drafts (lookupDraft,
        # :39-66), unpadded: fewer than k drafts give a shorter verify step,
        # none a one-row step
        nonlocal pending
        d = lookup_draft(history, k)
        res = eng.verify(np.array([pending] + d, np.int32), acc)
        emitted = d[:res[0]] + [int(res[1])]
        history.extend(emitted)
        pending = int(res[1])
        return len(emitted), int(res[0]), len(d), eng.last_step_ms

    def run(step, n_steps, n_warm):
        for _ in range(n_warm):
            step()
        tokens = accepted = drafted = 0
        gpu_ms = []
        t0 = time.perf_counter()
        for _ in range(n_steps):
            n, a, d, ms = step()
            tokens += n
            accepted += a
            drafted += d
            gpu_ms.append(ms)
        return tokens, accepted, drafted, time.perf_counter() - t0, gpu_ms

    # side runs first, so that the headline steps are the last verify steps
    # of the run (the ones a kernel trace summarises)
    f07 = run(step_argmax07, min(steps, 64), 2)
    forced07 = {"accepted_tokens_per_s": f07[0] / f07[3], "accepted_tokens_per_step": f07[0] / min(steps, 64),
                "acceptance_rate": f07[1] / max(1, f07[2]), "steps": min(steps, 64),
                "verify_step_gpu_us_median": float(np.median(f07[4])) * 1e3,
                "rule": "k uniform drafts, accept length prescribed: leading argmax hits with probability 0.7 "
                        "each (the draft rule BASELINE states for configs[3])"}
    lk_steps = min(steps, 64)
    lk = run(step_lookup, lk_steps, 2)
    lookup = {"accepted_tokens_per_s": lk[0] / lk[3], "verify_steps_per_s": lk_steps / lk[3],
              "acceptance_rate": lk[1] / max(1, lk[2]), "drafts_per_step": lk[2] / lk_steps,
              "accepted_tokens_per_step": lk[0] / lk_steps, "steps": lk_steps,
              "verify_step_gpu_us_median": float(np.median(lk[4])) * 1e3}
    tokens, accepted, drafted, wall, gpu_ms = run(step_lookup_padded, steps, warmup)
    ms_per_step = wall * 1e3 / steps
    step_gpu_ms = float(np.median(gpu_ms))
    lookup_share = lookup_drafts[0] / max(1, k * (steps + warmup))
    ctx = eng.position
    rows = k + 1
    kvdim = cfg.kv_heads * cfg.head_dim
    n_attn = sum(1 for i in range(cfg.n_layers) if not cfg.is_recurrent(i))
    n_rec = cfg.n_layers - n_attn
    kv_bytes = n_attn * ctx * kvdim * 2 * 2            # K and V rows read once (F16)
    state_bytes = 2 * n_rec * (cfg.rank * cfg.state_size ** 2 + 3 * cfg.conv_dim) * 4  # read + write once
    logit_bytes = 2 * rows * cfg.vocab * 4              # written by the LM head, read by the acceptance
    step_bytes = wbytes + kv_bytes + state_bytes + logit_bytes
    step_ach = step_bytes / (step_gpu_ms * 1e-3) / 1e9

    dk = dominant_kernel(dev, cfg, rows, rng)

    line = {
        "metric": "accepted tokens/s on 1 MI355X; verify-step HBM GB/s vs peak",
        "value": tokens / wall,
        "unit": "accepted tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k/q6_k weights x int16-split activations (int32 MFMA), fp32 norms/attention/GDN",
        "data": "synthetic: random-init Q4_K_M-mix weights (dequantized std ~0.02), random 512-token prompt; "
                "k = 4 drafts per step from prompt lookup over the history (engine/speculative.go lookupDraft), "
                "topped up with uniform random ids when lookup finds fewer; greedy decisions on the device's "
                "argmax, nothing prescribed",
        "config": {"workload": "config2: Qwen3.5-4B-like hybrid decoder verify step, batch 1",
                   "hidden": cfg.hidden, "ffn": cfg.ffn, "layers": cfg.n_layers, "gdn_heads": cfg.rank,
                   "attn_heads": f"{cfg.heads}q/{cfg.kv_heads}kv x {cfg.head_dim}", "vocab": cfg.vocab,
                   "prompt": 512, "drafts": k, "rows": rows, "acceptance": "greedy", "kv": "paged F16, 16-token blocks",
                   "parallelism": "single GPU"},
        "verify_step_gpu_us": step_gpu_ms * 1e3,
        "verify_steps_per_s": steps / wall,
        "accepted_tokens_per_step": tokens / steps,
        "acceptance_rate": accepted / max(1, drafted),
        "drafts_from_lookup": lookup_share,
        "prompt_lookup_unpadded": lookup,
        "forced_argmax07": forced07,
        "step_roofline": {"bound": "hbm", "achieved": step_ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": step_ach / HBM_PEAK_GBS, "alg_bytes_per_step": step_bytes,
                          "weights": wbytes, "kv": kv_bytes, "gdn_state": state_bytes, "logits": logit_bytes},
        "roofline": dk,
        "context_end": ctx,
        "prefill_s": prefill_s,
        "weight_gen_s": gen_s,
        "device": info,
    }
    eng.close()
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_config2(cfg, w, k, args.cpu_seconds)
    return line


def cpu_baseline_config2(cfg, w, k, budget_s):
    """The oracle decoder (restatement of model/qwen35 forwardOne, every weight
    re-read per token, matmul rows split over all host cores) running the
    same verify steps: k+1 rows of PrefillLogits + greedy accept per step."""
    from oracle import oracle as O
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    orc = O.Q35(cfg, w, kv_format=1, workers=cores)
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, cfg.vocab, 4).astype(np.int32).tolist()
    orc.forward(prompt[:-1])
    pending = prompt[-1]
    drng = np.random.default_rng(4)
    n, tokens = 0, 0
    t0 = time.perf_counter()
    while True:
        # the GPU run's draft rule: k drafts, accept length prescribed
        # (leading hits with probability 0.7 each), next = argmax at that row
        d = drng.integers(0, cfg.vocab, k).tolist()
        hit = drng.random(k) < 0.7
        a = k if hit.all() else int(np.argmin(hit))
        rows = [pending] + d
        snap, pos = orc.snapshot()
        logits = orc.forward(rows, all_logits=True)
        nxt = O.argmax(logits[a])
        if a < k:  # reference rollback: restore and replay the accepted prefix
            orc.restore(snap, pos)
            orc.forward(rows[:a + 1])
        emitted = d[:a] + [nxt]
        pending = nxt
        tokens += len(emitted)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 1000:
            break
    orc.close()
    return {"value": tokens / el, "unit": "accepted tokens/s", "cores": cores, "kind": "port",
            "sample": f"{n} verify steps (k={k}, {k + 1} rows of the full 32-layer model each, the GPU run's "
                      f"draft and acceptance rule, snapshot/replay rollback) in {el:.1f} s",
            "differs_from_gpu_run": "starts after a 4-token prompt instead of the 512-token one (the oracle's "
                                    "512-token prefill alone would take minutes); a CPU verify step re-reads "
                                    "every weight once per row (2.1 GB each), which does not depend on context",
            "ms_per_step": el * 1e3 / n}


BATCHED = {
    # 4B-like, 16 requests x 4096-token prompts
    # sharing a 1024-token prefix, k = 8, stochastic T = 0.7 / top-p 0.9,
    # forced accept length uniform 0..8.
    3: dict(model="QWEN35_4B_LIKE", batch=16, prompt=4096, shared=1024, k=8, accept="stochastic",
            temperature=0.7, top_p=0.9, forced="uniform"),
    # 9B-like, 4 requests x 16384-token context, k = 16, greedy;
    # drafts equal the argmax with probability 0.7 (geometric accept length).
    4: dict(model="QWEN35_9B_LIKE", batch=4, prompt=16384, shared=0, k=16, accept="greedy", forced="geometric"),
    # MoE-like, 8 requests x 2048-token context, k = 4, T = 0.8.
    5: dict(model="QWEN35_MOE_LIKE", batch=8, prompt=2048, shared=0, k=4, accept="stochastic", temperature=0.8,
            top_p=1.0, forced=None, router_normal=True),
}


def bench_batched(args, which):
    """BASELINE configs[2..4]: batched verify steps of the batched engine
    (every request's k+1 rows in one captured graph, acceptance and commit
    per request on the device)."""
    from yuuka_amd import hip, model as Mdl

    spec = BATCHED[which]
    k, B, P = spec["k"], spec["batch"], args.prompt or spec["prompt"]
    steps, warmup = args.steps or 32, args.warmup if args.warmup is not None else 4
    base = getattr(Mdl, spec["model"])
    cap = P + (steps + warmup + 2) * (k + 1) + 16
    cfg = Mdl.replace(base, batch=B, max_rows=max(16, k + 1), capacity=cap,
                      router_normal_seed=7 if spec.get("router_normal") else 0)
    t0 = time.perf_counter()
    w = model_weights(spec["model"], cfg)
    gen_s = time.perf_counter() - t0
    wbytes = Mdl.weight_bytes(w)
    dev = hip.Device(0)
    info = dev.info()
    # config 5's side run with the model's own router goes first, so that the
    # configured run's steps are the last verify steps of the process
    model_routing = moe_model_routing(dev, cfg, w, spec) if spec.get("router_normal") else None
    eng = Mdl.Engine(dev, cfg, w)
    rng = np.random.default_rng(which)
    t0 = time.perf_counter()
    prompts = rng.integers(0, cfg.vocab, (B, P)).astype(np.int32)
    S = min(spec["shared"], P // 4)
    done = 0
    if S:
        prompts[:, :S] = prompts[0, :S]
        eng.prefill_request(0, prompts[0, :S])
        for r in range(1, B):
            eng.fork(0, r)   # shared prefix blocks, reference-counted
        done = S
    rows = 16
    while done < P - 1:
        n = min(rows, P - 1 - done)
        eng.step_batch(prompts[:, done:done + n], mode=1)
        done += n
    prefill_s = time.perf_counter() - t0
    if spec["accept"] == "greedy":
        acc = Mdl.accept_struct()
    else:
        acc = Mdl.accept_struct(mode=1, temperature=spec["temperature"], seed=1234, top_p=spec["top_p"])
    pending = prompts[:, -1].copy()

    def forced_lengths():
        if spec["forced"] == "uniform":
            return rng.integers(0, k + 1, B).astype(np.int32)
        if spec["forced"] == "geometric":
            # leading drafts that equal the argmax, each with probability 0.7
            hit = rng.random((B, k)) < 0.7
            return np.where(hit.all(axis=1), k, np.argmin(hit, axis=1)).astype(np.int32)
        return None

    def step():
        # synthetic drafts (the configurations prescribe them; lookupDraft
        # is replaced, engine/speculative.go:39-66)
        toks = np.empty((B, k + 1), np.int32)
        toks[:, 0] = pending
        toks[:, 1:] = rng.integers(0, cfg.vocab, (B, k))
        forced = forced_lengths()
        res = eng.step_batch(toks, 0, acc, forced)
        pending[:] = res[:, 1]
        return int(res[:, 0].sum()) + B, int(res[:, 0].sum()), eng.last_step_ms

    for _ in range(warmup):
        step()
    routing = None
    if cfg.n_experts:
        # the experts the verify rows actually select, per layer, over a few
        # untimed steps before the timed ones: the expert matrices a step streams
        distinct, top = [], []
        for _ in range(4):
            step()
            for li in range(cfg.n_layers):
                cnt = eng.moe_counts(li)
                distinct.append(int((cnt > 0).sum()))
                top.append(int(cnt.max()))
        routing = {"distinct_experts_per_layer": float(np.mean(distinct)), "max_rows_per_expert": max(top),
                   "sample": f"4 untimed steps before the timed ones, all {cfg.n_layers} layers"}
    tokens, accepted, gpu_ms = 0, 0, []
    t0 = time.perf_counter()
    for _ in range(steps):
        n, a, ms = step()
        tokens += n
        accepted += a
        gpu_ms.append(ms)
    wall = time.perf_counter() - t0
    step_gpu_ms = float(np.median(gpu_ms))
    ctx = [eng.request_position(r) for r in range(B)]
    R1 = k + 1
    kvdim = cfg.kv_heads * cfg.head_dim
    n_attn = sum(1 for i in range(cfg.n_layers) if not cfg.is_recurrent(i))
    n_rec = cfg.n_layers - n_attn
    # unique KV rows read: the shared prefix once, every request's own rows once
    kv_rows = (S + sum(c - S for c in ctx)) if S else sum(ctx)
    kv_bytes = n_attn * kv_rows * kvdim * 2 * 2
    state_bytes = B * 2 * n_rec * (cfg.rank * cfg.state_size ** 2 + 3 * cfg.conv_dim) * 4
    logit_bytes = 2 * B * R1 * cfg.vocab * 4
    step_w = wbytes
    moe_note = None
    if cfg.n_experts:
        # expert bytes actually streamed: the distinct experts the verify rows
        # selected (measured above); uniform routing would touch
        # E (1 - (1 - used / E)^rows) of them
        E, used, ef, H = cfg.n_experts, cfg.n_experts_used, cfg.expert_ffn, cfg.hidden
        distinct = routing["distinct_experts_per_layer"]
        uniform = E * (1 - (1 - used / E) ** (B * R1))
        per_expert = 3 * ef * H // 256 * 144
        step_w = wbytes - cfg.n_layers * E * per_expert + cfg.n_layers * int(distinct * per_expert)
        moe_note = (f"expert bytes for the {distinct:.1f} of {E} experts per layer the rows selected "
                    f"(uniform routing would touch {uniform:.1f})")
    step_bytes = step_w + kv_bytes + state_bytes + logit_bytes
    step_ach = step_bytes / (step_gpu_ms * 1e-3) / 1e9
    line = {
        "metric": "accepted tokens/s on 1 MI355X; verify-step HBM GB/s vs peak",
        "value": tokens / wall,
        "unit": "accepted tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": wall * 1e3 / steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k/q6_k weights x int16-split activations (int32 MFMA), fp32 norms/attention/GDN",
        "data": "synthetic: random-init Q4_K_M-mix weights, random prompts, uniform random drafts" + ("; prescribed accept lengths (" + spec["forced"] + ")" if spec["forced"] else ""),
        "config": {"workload": f"config{which}: {spec['model']} batched verify, {B} requests, k={k}",
                   "requests": B, "prompt": P, "shared_prefix": S, "drafts": k, "rows": B * R1,
                   "acceptance": spec["accept"] + (f" T={spec['temperature']} top-p={spec['top_p']}"
                                                   if spec["accept"] != "greedy" else ""),
                   "hidden": cfg.hidden, "layers": cfg.n_layers, "experts": cfg.n_experts,
                   "parallelism": "single GPU"},
        "verify_step_gpu_us": step_gpu_ms * 1e3,
        "verify_steps_per_s": steps / wall,
        "accepted_tokens_per_step": tokens / steps,
        "acceptance_rate": accepted / (steps * B * k),
        "step_roofline": {"bound": "hbm", "achieved": step_ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": step_ach / HBM_PEAK_GBS, "alg_bytes_per_step": step_bytes, "weights": step_w,
                          "kv": kv_bytes, "gdn_state": state_bytes, "logits": logit_bytes, "note": moe_note},
        "context_end": ctx,
        **({"moe_routing": routing} if routing else {}),
        "prefill_s": prefill_s,
        "weight_gen_s": gen_s,
        "device": info,
    }
    eng.close()
    if cfg.n_experts:
        line["roofline"] = moe_dominant(dev, cfg, B * R1, np.random.default_rng(6))
        if model_routing:
            line["model_routing"] = model_routing
    else:
        line["roofline"] = dominant_kernel(dev, cfg, B * R1, np.random.default_rng(6))
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_batched(cfg, w, spec, args.cpu_seconds)
    return line


def moe_model_routing(dev, cfg, w, spec):
    """Config 5 with the random-init model's own router (no N(0,1)
    replacement): a short run beside the configured one, for the step time
    and the experts the rows select when routing follows the model."""
    from yuuka_amd import model as Mdl
    B, k = spec["batch"], spec["k"]
    c2 = Mdl.replace(cfg, router_normal_seed=0, capacity=512)
    eng = Mdl.Engine(dev, c2, w)
    rng = np.random.default_rng(11)
    prompts = rng.integers(0, c2.vocab, (B, 256)).astype(np.int32)
    for a in range(0, 255, 16):
        eng.step_batch(prompts[:, a:min(a + 16, 255)], mode=1)
    acc = Mdl.accept_struct(mode=1, temperature=spec["temperature"], seed=1234, top_p=spec["top_p"])
    pending = prompts[:, -1].copy()
    ms, distinct = [], []
    for i in range(10):
        toks = np.empty((B, k + 1), np.int32)
        toks[:, 0] = pending
        toks[:, 1:] = rng.integers(0, c2.vocab, (B, k))
        res = eng.step_batch(toks, 0, acc, None)
        pending[:] = res[:, 1]
        if i >= 2:
            ms.append(eng.last_step_ms)
            distinct += [int((eng.moe_counts(li) > 0).sum()) for li in range(c2.n_layers)]
    eng.close()
    return {"verify_step_gpu_us": float(np.median(ms)) * 1e3, "distinct_experts_per_layer": float(np.mean(distinct)),
            "sample": "8 timed steps after 2 warm-up steps, 256-token prompts, the model's router"}


_WEIGHTS = {}


def model_weights(name, cfg):
    """Seeded random-init weights of a BASELINE model, generated once per run
    (configs 2 and 3 share the 4B-like model); MoE experts share one host
    copy across layers."""
    from yuuka_amd import model as Mdl
    if name not in _WEIGHTS:
        _WEIGHTS[name] = Mdl.make_weights(cfg, seed=0, share_experts=True)
    return _WEIGHTS[name]


def cpu_baseline_batched(cfg, w, spec, budget_s):
    """The oracle decoder running verify steps of ONE request of the same
    model (the reference serves requests one after another): k+1 rows of
    PrefillLogits per step, the acceptance rule of the configuration, and the
    reference rollback (snapshot, restore, replay of the accepted rows)."""
    from oracle import oracle as O
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    k = spec["k"]
    cfg1 = Mdl_replace(cfg, batch=1)
    orc = O.Q35(cfg1, w, kv_format=1, workers=cores)
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, cfg.vocab, 4).astype(np.int32).tolist()
    orc.forward(prompt[:-1])
    pending = prompt[-1]
    n, tokens = 0, 0
    t0 = time.perf_counter()
    while True:
        d = list(rng.integers(0, cfg.vocab, k))
        rows = [pending] + d
        snap, pos = orc.snapshot()
        logits = orc.forward(rows, all_logits=True)
        if spec["forced"] == "uniform":
            a = int(rng.integers(0, k + 1))
        elif spec["forced"] == "geometric":
            hit = rng.random(k) < 0.7
            a = k if hit.all() else int(np.argmin(hit))
        elif spec["accept"] == "greedy":
            a = O.accept_greedy(logits, d)[0]
        else:
            a = O.accept_stochastic(logits, d, spec["temperature"], 1234, n, 0, 0, spec["top_p"])[0]
        nxt = O.argmax(logits[a])
        if a < k:
            orc.restore(snap, pos)
            orc.forward(rows[:a + 1])
        pending = nxt
        tokens += a + 1
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 1000:
            break
    orc.close()
    return {"value": tokens / el, "unit": "accepted tokens/s", "cores": cores, "kind": "port",
            "sample": f"{n} verify steps of one request (k={k}, {k + 1} rows of the full model each, "
                      f"same acceptance rule, snapshot/replay rollback) after a 4-token prompt, {el:.1f} s",
            "ms_per_step": el * 1e3 / n}


def Mdl_replace(cfg, **kw):
    from yuuka_amd import model as Mdl
    return Mdl.replace(cfg, **kw)


SUMMARY_KEYS = ("value", "unit", "steps", "warmup", "ms_per_step", "verify_step_us", "verify_step_gpu_us",
                "accepted_tokens_per_step", "acceptance_rate", "config", "data", "step_roofline", "roofline",
                "cpu_baseline", "moe_routing", "model_routing", "accept_parity", "context_end", "prefill_s")


def bench_all(args):
    """The default run: config 2 (the metric's
    configuration) is the line's value; configs 1, 3, 4 and 5 are measured in
    the same process and reported under "configs" with their own step time,
    accepted tokens/s, acceptance, step and kernel rooflines and CPU baseline
    (a 10 s sample each)."""
    import copy
    line = bench_config2(args)
    configs = {}
    for which in (1, 3, 4, 5):
        a = copy.copy(args)
        a.config, a.steps, a.warmup, a.prompt = which, None, None, None
        a.cpu_seconds = min(args.cpu_seconds, 10.0)
        t0 = time.perf_counter()
        if which == 1:
            a.steps, a.warmup = 200, 20
            sub = bench_config1(a)
        else:
            sub = bench_batched(a, which)
        if which == 3:
            _WEIGHTS.pop("QWEN35_4B_LIKE", None)
        rec = {k: sub[k] for k in SUMMARY_KEYS if k in sub}
        rec["wall_s"] = time.perf_counter() - t0
        configs[str(which)] = rec
        print(f"config {which}: {rec['value']:.1f} {rec['unit']} in {rec['wall_s']:.1f} s", file=sys.stderr,
              flush=True)
    line["configs"] = configs
    return line


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not implemented)"}))
        sys.exit(2)
    ensure_built()
    if args.kernel_only:
        line = kernel_only(args)
    elif args.config is None:
        line = bench_all(args)
    elif args.config == 1:
        args.steps = args.steps or 200
        args.warmup = args.warmup if args.warmup is not None else 20
        line = bench_config1(args)
    elif args.config == 2:
        line = bench_config2(args)
    elif args.config in BATCHED:
        line = bench_batched(args, args.config)
    else:
        print(json.dumps({"error": f"config {args.config} not available yet"}))
        sys.exit(2)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
