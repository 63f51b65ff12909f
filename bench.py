#!/usr/bin/env python3
"""Benchmark of the Laya decoder forward path on one MI355X.

Headline (`value`): batched Q8_0 prefill "decide" throughput -- 64 independent requests of
512 prompt tokens + 3 question blocks of 16 tokens (560 tokens each, 35,840 tokens per step),
24-layer d2048 decoder, option scoring over 4 option tokens at each question's answer position.
One step = one full batch: embedding, 24 layers of dequant-fused MFMA GEMMs + paged causal
attention, head rows and option softmax.  Inputs (token ids, page tables) are staged in HBM
before the timed region; the staged batch is rewound and re-executed each step.

Nested under `configs`, each with its own `roofline` and `cpu_baseline` (4 threads, the reference's
default) and `cpu_baseline_all_cores` (16 threads, this job's host share):
  C1  plumbing decide latency (6-layer d512 F16 model, 144-token request);
  C3  batch-1 Q8_0 greedy decode over a 2048-token context, 64 steps (GEMV HBM roofline);
  C4  Q4_K/Q6_K 7B-shape prefill, 32 x 1024 tokens (MFMA roofline);
  C5  F16 7B-shape long context, 16 x 8192 tokens sharing a 6144-token prefix (MFMA roofline of the
      GEMMs and of the attention).
The CPU baselines are the oracle (the reference algorithm restated in C: F32 weights, 4-row x 8-lane
FMA kernel, rows split over threads) timed on bounded samples on this host; each says what it timed
and how it was scaled.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--precision exact|fast] [--configs C1,C3,C4,C5]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "laya-goish_amd"))

import numpy as np  # noqa: E402

import laya_hip as lh  # noqa: E402

METRIC = "prefill tok/s + decide req/s at 1 GPU; Q8_0 GEMV HBM GB/s vs peak"
PEAK_HBM_GBS = 8000.0
PEAK_F16_TFLOPS = 2500.0

PRESET = "q8-2048"
SEED = 20261201
REQUESTS, PROMPT, QBLOCK, QUESTIONS, OPTIONS = 64, 512, 16, 3, 4
DECODE_CTX, DECODE_STEPS = 2048, 64


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_q8-2048_bench.md")
TRAFFIC_FILE_C4 = os.path.join(ROOT, "profiles", "hbm_traffic_q4km-7b_prefill.md")
TRAFFIC_FILE_C5 = os.path.join(ROOT, "profiles", "hbm_traffic_f16-7b_long-context.md")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def measured_traffic(kernel, path=TRAFFIC_FILE):
    """HBM bytes per launch of `kernel` from the committed FETCH_SIZE + WRITE_SIZE counter runs of
    a workload (lines `traffic.<kernel> <bytes>` of its summary), or None when that summary is absent."""
    try:
        for line in open(path):
            parts = line.split()
            if len(parts) == 2 and parts[0] == f"traffic.{kernel}":
                return int(parts[1])
    except OSError:
        pass
    return None


def prefill_workload(vocab):
    rng = np.random.default_rng(SEED)
    n = PROMPT + QUESTIONS * QBLOCK
    reqs = []
    for _ in range(REQUESTS):
        ids = rng.integers(0, vocab, n).astype(np.int32)
        pos = np.array([PROMPT + (q + 1) * QBLOCK - 1 for q in range(QUESTIONS)], np.int32)
        reqs.append((ids, pos))
    option_ids = rng.choice(vocab, OPTIONS, replace=False).astype(np.int32)
    return reqs, option_ids


def bench_prefill(eng, steps, warmup):
    reqs, option_ids = prefill_workload(eng.info["vocab"])
    seqs = [eng.seq_create() for _ in reqs]
    batch = eng.batch([(s, ids, pos) for s, (ids, pos) in zip(seqs, reqs)])
    T = sum(len(ids) for ids, _ in reqs)
    out = None
    for i in range(warmup):
        out = batch.run(option_ids)
        batch.rewind()
    eng.sync()
    t0 = time.perf_counter()
    for i in range(steps):
        out = batch.run(option_ids)  # ends with the results copied to the host
        batch.rewind()
    eng.sync()
    dt = time.perf_counter() - t0
    # one extra step with per-kernel HIP events on the engine stream (not in the timed region)
    eng.profile_reset()
    eng.profile(True)
    batch.run(option_ids)
    batch.rewind()
    eng.profile(False)
    prof = {c: eng.profile_read(c) for c in ("gemm", "attn_prefill", "rope_kv", "rmsnorm", "embed", "head")}
    logits, probs, _ = out
    assert np.isfinite(logits).all() and np.isfinite(probs).all()
    batch.free()
    for s in seqs:
        eng.seq_free(s)
    return T, dt, prof, probs


def roofline(bound, achieved, peak, unit, kernel, launches=None, avg_launch_ms=None, traffic=None, **extra):
    r = {"bound": bound, "achieved": round(achieved, 1), "peak": peak, "unit": unit,
         "frac": round(achieved / peak, 4), "traffic": traffic, "kernel": kernel}
    if launches is not None:
        r["launches"] = launches
    if avg_launch_ms is not None:
        r["avg_launch_ms"] = round(avg_launch_ms, 5)
    r.update(extra)
    return r


def rate(p, what):
    """TFLOP/s (what = "flops") or GB/s ("bytes") of a profiled kernel class."""
    if not p["ms"]:
        return 0.0
    return p[what] / (p["ms"] * 1e-3) / (1e12 if what == "flops" else 1e9)


def cpu_entry(value, unit, cores, sample):
    return {"value": value, "unit": unit, "cores": cores, "kind": "port", "sample": sample}


def oracle_modules():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as po
    return po


def cpu_threads(args):
    """(thread counts to time): the reference's default 4, and the host share this job may use."""
    return [t for t in dict.fromkeys([args.cpu_threads, args.cpu_threads_all]) if t > 0]


def cpu_pair(entries):
    """cpu_baseline (the first thread count) plus, when timed, cpu_baseline_all_cores."""
    out = {}
    if entries:
        out["cpu_baseline"] = entries[0]
    if len(entries) > 1:
        out["cpu_baseline_all_cores"] = entries[1]
    return out


# ---------------------------------------------------------------- C3: batch-1 greedy decode
def c3_decode(eng, args, extras=True):
    """The benchmark's 2048-token context on the Q8_0 d2048 model, then DECODE_STEPS greedy steps
    (one forked sequence per run, so every run decodes the same positions).  extras: also the
    HIP-graph decode and the CPU baseline."""
    steps = args.decode_steps
    rng = np.random.default_rng(SEED + 1)
    ids = rng.integers(0, eng.info["vocab"], DECODE_CTX).astype(np.int32)
    base = eng.seq_create()
    eng.forward(base, ids, [], None)
    first = int(ids[-1])
    runs = []
    for mode in ("warm", "timed", "profiled"):
        s = eng.seq_fork(base, DECODE_CTX)
        if mode == "profiled":
            eng.profile_reset()
            eng.profile(True)
        eng.sync()
        t0 = time.perf_counter()
        toks = eng.decode(s, first, steps)
        eng.sync()
        runs.append((mode, time.perf_counter() - t0, toks))
        if mode == "profiled":
            eng.profile(False)
        eng.seq_free(s)
    prof = {c: eng.profile_read(c) for c in ("gemv", "attn_decode", "argmax", "embed")}
    # the same decode with every kernel of every step captured into one HIP graph and launched once:
    # the GPU time of the launch (through its completion) against the stream-launched run above
    graph = None
    if extras and not args.no_graph:
        s = eng.seq_fork(base, DECODE_CTX)
        gtoks, cap_ms, graph_ms = eng.decode_graph(s, first, steps)
        eng.seq_free(s)
        assert np.array_equal(gtoks, runs[1][2]), "graph decode differs from stream decode"
        graph = {"ms_per_token": round(graph_ms / steps, 4), "capture_instantiate_ms": round(cap_ms, 2),
                 "note": "the same decode with every kernel of every step captured into one HIP graph and "
                         "launched once (lg_decode_graph); tokens equal the stream-launched run"}
    eng.seq_free(base)
    assert np.array_equal(runs[0][2], runs[1][2]), "decode is not deterministic"
    dt = runs[1][1]
    gv, at = prof["gemv"], prof["attn_decode"]
    log(f"C3 decode: {dt / steps * 1e3:.3f} ms/token, gemv {rate(gv, 'bytes'):.0f} GB/s over {gv['launches']} "
        f"launches, attention {rate(at, 'bytes'):.0f} GB/s" +
        (f"; one HIP graph: {graph['ms_per_token']:.3f} ms/token (capture + instantiate "
         f"{graph['capture_instantiate_ms']:.1f} ms)" if graph else ""))
    for c, p in prof.items():
        log(f"  {c:12s} launches {p['launches']:5d}  {p['ms']:8.3f} ms")
    out = {
        "workload": f"Q8_0 batch-1 greedy decode: {DECODE_CTX}-token context, {steps} steps; 24 layers, d_model 2048, "
                    f"16 x 128 heads, FFN 5632, vocab 32000, Q8_0 matrices and head",
        "value": round(steps / dt, 2), "unit": "tok/s", "higher_is_better": True, "steps": steps,
        "ms_per_token": round(dt / steps * 1e3, 4),
        "roofline": roofline("hbm", rate(gv, "bytes"), PEAK_HBM_GBS, "GB/s",
                             "gemv (dequant-fused Q8_0 GEMV, GGUF bytes per launch)", gv["launches"],
                             gv["ms"] / max(1, gv["launches"]), measured_traffic("gemv")),
        "attention": roofline("hbm", rate(at, "bytes"), PEAK_HBM_GBS, "GB/s",
                              "attn_decode (KV bytes read per launch: f16 hi + lo planes in the exact mode, f16 in "
                              "the kv16 and fast modes; incl. the page-combine launch)",
                              at["launches"], at["ms"] / max(1, at["launches"])),
        "kernel_ms_per_token": {c: round(p["ms"] / steps, 4) for c, p in prof.items()},
    }
    if graph:
        out["graph"] = graph
    if extras and not args.no_cpu:
        po = oracle_modules()
        layers = 2
        img = lh.SynthImage(PRESET, seed=SEED, n_layers=layers)
        om = po.Model(po.Gguf(img.array()), threads=args.cpu_threads_all)
        c = om.cache(DECODE_CTX + 8)
        po.set_blocked(True)  # the context is set-up, not timed: same bits, faster
        om.prefill(c, ids, [])
        po.set_blocked(False)
        feed = [first] + [int(t) for t in runs[1][2][:3]]
        t0 = time.perf_counter()
        for t in feed:
            h = om.prefill(c, [t], [0])
            om.head(h)
        t_steps = (time.perf_counter() - t0) / len(feed)
        t0 = time.perf_counter()
        for _ in range(4):
            om.head(h)
        t_head = (time.perf_counter() - t0) / 4
        per_token = (t_steps - t_head) * (24 / layers) + t_head
        out["cpu_baseline"] = cpu_entry(
            round(1 / per_token, 3), "tok/s", 1,
            f"{len(feed)} KV-cached decode steps after the {DECODE_CTX}-token context through {layers} of 24 layers "
            f"({t_steps * 1e3:.0f} ms per step, of which the 32000-row head {t_head * 1e3:.0f} ms), layer part scaled "
            f"x{24 // layers}: {per_token * 1e3:.0f} ms per token. One row per step is one worker in the reference's "
            f"row split (tensor.rs:17-18), whatever the thread count; a KV cache is the oracle's addition (the "
            f"reference recomputes the whole sequence every call)")
        del om
    return out


# ---------------------------------------------------------------- C1: plumbing latency
def c1_plumbing(args, prec):
    """The CPU-runnable plumbing model (6 layers, d512, 8 x 64 heads, F16): one decide request of a
    128-token prompt plus one 16-token yes/no question block, scored at its answer position.
    Latency of the whole request (ids uploaded, forward, option scores read back)."""
    img = lh.SynthImage("plumbing-f16", seed=SEED)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=2048, max_batch_tokens=512, precision=prec)
    ids = np.random.default_rng(SEED + 2).integers(0, 32000, 144).astype(np.int32)
    yes_no = np.array([1939, 4874], np.int32)

    def one():
        s = eng.seq_create()
        logits = eng.forward(s, ids, [143], yes_no)
        probs, _ = lh.option_scores(logits[0])
        eng.seq_free(s)
        return probs
    for _ in range(max(args.warmup, 3)):
        one()
    times = []
    for _ in range(max(args.steps, 20)):
        eng.sync()
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    eng.profile_reset()
    eng.profile(True)
    one()
    eng.profile(False)
    gp = eng.profile_read("gemm")
    eng.close()
    med = float(np.median(times)) * 1e3
    log(f"C1 plumbing: median {med:.3f} ms per decide request (min {min(times) * 1e3:.3f}), gemm "
        f"{rate(gp, 'flops'):.1f} TFLOP/s over {gp['launches']} launches")
    out = {
        "workload": "plumbing decide request: 6 layers, d_model 512, 8 x 64 heads, FFN 1408, vocab 32000, F16 weights "
                    "N(0, 0.02); 128-token prompt + one 16-token noul question block, 2 option tokens",
        "value": round(med, 3), "unit": "ms per request", "higher_is_better": False, "steps": len(times),
        "p50_ms": round(med, 3), "min_ms": round(min(times) * 1e3, 3),
        "roofline": roofline("mfma", rate(gp, "flops"), PEAK_F16_TFLOPS, "TFLOP/s",
                             "gemm (every projection of the 144-token forward; launch-bound at this size)",
                             gp["launches"], gp["ms"] / max(1, gp["launches"])),
    }
    if not args.no_cpu:
        po = oracle_modules()
        om = po.Model(po.Gguf(img.array()), threads=1)
        entries = []
        for t in cpu_threads(args):
            om.set_threads(t)
            ts = []
            for _ in range(3):
                t0 = time.perf_counter()
                w = om.forward(ids, [143], yes_no)
                po.option_scores(w[0])
                ts.append(time.perf_counter() - t0)
            cm = float(np.median(ts)) * 1e3
            entries.append(cpu_entry(round(cm, 2), "ms per request", t,
                                     f"the same request through all 6 layers, median of 3: {cm:.1f} ms"))
        out.update(cpu_pair(entries))
        del om
    return out


# ---------------------------------------------------------------- C4: Q4_K/Q6_K 7B prefill
Q4K_REQS, Q4K_TOKENS = 32, 1024
C5_REQS, C5_PREFIX, C5_OWN, C5_QUESTIONS = 16, 6144, 2048, 8


def q4k_workload():
    """The C4 batch: 32 requests of 1024 random ids, the last position scored over 4 option ids."""
    rng = np.random.default_rng(SEED + 3)
    reqs = [(rng.integers(0, 152064, Q4K_TOKENS).astype(np.int32), np.array([Q4K_TOKENS - 1], np.int32))
            for _ in range(Q4K_REQS)]
    opts = rng.choice(152064, 4, replace=False).astype(np.int32)
    return reqs, opts


def c5_workload():
    """The C5 step's inputs: the shared 6144-id prefix, 16 own 2048-id suffixes, the 8 answer positions
    of each suffix (every 256th token) and 4 option ids."""
    rng = np.random.default_rng(SEED + 4)
    prefix = rng.integers(0, 152064, C5_PREFIX).astype(np.int32)
    own = [rng.integers(0, 152064, C5_OWN).astype(np.int32) for _ in range(C5_REQS)]
    pos = np.arange(C5_OWN // C5_QUESTIONS - 1, C5_OWN, C5_OWN // C5_QUESTIONS).astype(np.int32)
    opts = rng.choice(152064, 4, replace=False).astype(np.int32)
    return prefix, own, pos, opts


def cpu_layer_cost_7b(args, po):
    """The oracle on one layer of the 7B shape (d3584, GQA 28/4 x 128, FFN 18944): seconds for one
    1024-token request through one layer, per thread count (F32 weights after the load-time expansion,
    so the cost is the same for the Q4_K/Q6_K and F16 files)."""
    img = lh.SynthImage("q4km-7b", seed=SEED, n_layers=1)
    om = po.Model(po.Gguf(img.array()), threads=1)
    ids = np.random.default_rng(SEED + 3).integers(0, 152064, Q4K_TOKENS).astype(np.int32)
    cost = {}
    for t in cpu_threads(args):
        om.set_threads(t)
        t0 = time.perf_counter()
        om.forward(ids, [Q4K_TOKENS - 1], [1, 2, 3, 4])
        cost[t] = time.perf_counter() - t0
        log(f"  oracle 7B shape, one layer, {Q4K_TOKENS} tokens, {t} threads: {cost[t]:.2f} s")
    del om
    return cost


def load_entry(eng):
    """Engine load (lg_engine_create: streamed upload, repack, prefill copies, KV pool) of a model."""
    info = eng.info
    sec = info["load_seconds"]
    return {"seconds": round(sec, 3), "gguf_bytes": info["weight_bytes"],
            "GB_per_s": round(info["weight_bytes"] / sec / 1e9, 2) if sec > 0 else None}


def q4k_decode(eng, ids, args, steps=32):
    """Batch-1 greedy decode on the C4 model after one of its 1024-token requests: the dequant-fused Q4_K
    and Q6_K GEMVs (q|k, o, gate|up Q4_K; v, down, head Q6_K) and the GQA-7 decode attention.  Reported
    beside the prefill line (the configuration is a prefill one)."""
    base = eng.seq_create()
    eng.forward(base, ids, [], None)
    first = int(ids[-1])
    times = []
    for mode in ("warm", "timed", "profiled"):
        s = eng.seq_fork(base, len(ids))
        if mode == "profiled":
            eng.profile_reset()
            eng.profile(True)
        eng.sync()
        t0 = time.perf_counter()
        toks = eng.decode(s, first, steps)
        eng.sync()
        times.append(time.perf_counter() - t0)
        if mode == "profiled":
            eng.profile(False)
        eng.seq_free(s)
    eng.seq_free(base)
    assert (toks >= 0).all()
    dt = times[1]
    gv, at = eng.profile_read("gemv"), eng.profile_read("attn_decode")
    log(f"C4 decode: {dt / steps * 1e3:.3f} ms/token, gemv {rate(gv, 'bytes'):.0f} GB/s over {gv['launches']} launches, "
        f"attention {rate(at, 'bytes'):.0f} GB/s")
    return {
        "workload": f"batch-1 greedy decode on the same model: {len(ids)}-token context, {steps} steps",
        "value": round(steps / dt, 2), "unit": "tok/s", "ms_per_token": round(dt / steps * 1e3, 4),
        "roofline": roofline("hbm", rate(gv, "bytes"), PEAK_HBM_GBS, "GB/s",
                             "gemv (dequant-fused Q4_K and Q6_K GEMVs, GGUF bytes per launch)", gv["launches"],
                             gv["ms"] / max(1, gv["launches"])),
        "kernel_ms_per_token": {"gemv": round(gv["ms"] / steps, 4), "attn_decode": round(at["ms"] / steps, 4)},
    }


def c4_q4k(args, prec, layer_cost):
    """Q4_K/Q6_K 7B shape (28 layers, d3584, GQA 28/4 x 128, FFN 18944, vocab 152064, QKV bias):
    a batch of 32 requests x 1024 tokens, 4 option tokens scored at the last position."""
    t0 = time.perf_counter()
    img = lh.SynthImage("q4km-7b", seed=SEED)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=Q4K_REQS * Q4K_TOKENS + 2048, max_batch_tokens=32768,
                    precision=prec)
    load = load_entry(eng)
    log(f"C4 model ready in {time.perf_counter() - t0:.1f}s (engine load {load['seconds']} s, "
        f"{load['GB_per_s']} GB/s of GGUF weights)")
    reqs, opts = q4k_workload()
    seqs = [eng.seq_create() for _ in reqs]
    batch = eng.batch([(s, ids, pos) for s, (ids, pos) in zip(seqs, reqs)])
    warm, steps = 2, args.config_steps
    for _ in range(warm):
        batch.run(opts)
        batch.rewind()
    eng.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = batch.run(opts)
        batch.rewind()
    eng.sync()
    dt = (time.perf_counter() - t0) / steps
    eng.profile_reset()
    eng.profile(True)
    batch.run(opts)
    eng.profile(False)
    prof = {c: eng.profile_read(c) for c in ("gemm", "ksum", "attn_prefill", "rope_kv", "rmsnorm", "head")}
    assert np.isfinite(out[1]).all()
    decode = q4k_decode(eng, reqs[0][0], args)
    eng.close()
    T = Q4K_REQS * Q4K_TOKENS
    gp = prof["gemm"]
    log(f"C4 q4km-7b: {dt * 1e3:.1f} ms/step, {T / dt:.0f} tok/s, gemm {rate(gp, 'flops'):.1f} TFLOP/s")
    for c, p in prof.items():
        log(f"  {c:12s} launches {p['launches']:5d}  {p['ms']:8.3f} ms")
    res = {
        "workload": "Q4_K/Q6_K 7B-shape batched prefill: 28 layers, d_model 3584, GQA 28/4 x 128, FFN 18944, vocab "
                    "152064, QKV bias; Q4_K q/k/o/gate/up, Q6_K v/down/output; 32 requests x 1024 tokens, 4 option "
                    "tokens at the last position",
        "value": round(T / dt, 1), "unit": "tok/s", "higher_is_better": True, "steps": steps, "warmup": warm,
        "ms_per_step": round(dt * 1e3, 2), "req_per_s": round(Q4K_REQS / dt, 2), "load": load,
        "roofline": roofline("mfma", rate(gp, "flops"), PEAK_F16_TFLOPS, "TFLOP/s",
                             "gemm (exact K-quant MFMA GEMM: Q4_K in two f16 passes over exact codes with a depth-K/32 "
                             "correction, Q6_K in three passes over f16 hi/lo weight planes)", gp["launches"],
                             gp["ms"] / max(1, gp["launches"]), measured_traffic("gemm", TRAFFIC_FILE_C4),
                             traffic_source="profiles/hbm_traffic_q4km-7b_prefill.md (FETCH_SIZE + WRITE_SIZE, "
                                            "copy-calibrated)"),
        "kernel_ms_per_step": {c: round(p["ms"], 3) for c, p in prof.items()},
        "decode": decode,
    }
    if layer_cost:
        entries = []
        for t, sec in layer_cost.items():
            per_req = sec * 28
            entries.append(cpu_entry(round(Q4K_TOKENS / per_req, 2), "tok/s", t,
                                     f"one 1024-token request through 1 of 28 layers ({sec:.2f} s; weights "
                                     f"expanded to F32 at load as the reference does), scaled x28: {per_req:.0f} s "
                                     f"per request, requests one after another"))
        res.update(cpu_pair(entries))
    return res


def c5_long_context(args, prec, layer_cost):
    """F16 7B shape with a shared prefix: 16 requests of 8192 tokens sharing their first 6144.
    One step = the prefix computed once, forked into 16 requests, their 2048 own tokens prefilled as
    one batch, 8 answer positions each scored over 4 option tokens."""
    t0 = time.perf_counter()
    img = lh.SynthImage("f16-7b", seed=SEED)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=C5_PREFIX + C5_REQS * C5_OWN + 2048, max_batch_tokens=32768,
                    precision=prec)
    load = load_entry(eng)
    log(f"C5 model ready in {time.perf_counter() - t0:.1f}s (engine load {load['seconds']} s, "
        f"{load['GB_per_s']} GB/s of GGUF weights)")
    prefix, own, pos, opts = c5_workload()

    def step():
        base = eng.seq_create()
        eng.forward(base, prefix, [], opts)
        kids = [eng.seq_fork(base, C5_PREFIX) for _ in own]
        b = eng.batch([(k, ids, pos) for k, ids in zip(kids, own)])
        out = b.run(opts)
        b.free()
        for k in kids:
            eng.seq_free(k)
        eng.seq_free(base)
        return out

    warm, steps = 1, args.config_steps
    for _ in range(warm):
        step()
    eng.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = step()
    eng.sync()
    dt = (time.perf_counter() - t0) / steps
    eng.profile_reset()
    eng.profile(True)
    step()
    eng.profile(False)
    prof = {c: eng.profile_read(c) for c in ("gemm", "ksum", "attn_prefill", "rope_kv", "rmsnorm", "head")}
    assert np.isfinite(out[1]).all()
    eng.close()
    hq, hd, L = 28, 128, 28
    pairs = C5_PREFIX * (C5_PREFIX + 1) // 2 + C5_REQS * (C5_OWN * C5_PREFIX + C5_OWN * (C5_OWN + 1) // 2)
    att_flops = 4.0 * hd * hq * L * pairs
    ap, gp = prof["attn_prefill"], prof["gemm"]
    att_tf = att_flops / (ap["ms"] * 1e-3) / 1e12 if ap["ms"] else 0.0
    computed = C5_PREFIX + C5_REQS * C5_OWN
    log(f"C5 f16-7b long context: {dt * 1e3:.1f} ms/step, {C5_REQS / dt:.2f} req/s, gemm {rate(gp, 'flops'):.1f} "
        f"TFLOP/s, attention {att_tf:.1f} TFLOP/s")
    for c, p in prof.items():
        log(f"  {c:12s} launches {p['launches']:5d}  {p['ms']:8.3f} ms")
    res = {
        "workload": "F16 7B-shape shared-prefix long context: 28 layers, d_model 3584, GQA 28/4 x 128, FFN 18944, "
                    "vocab 152064, F16 weights; 16 requests x 8192 tokens sharing the first 6144 (prefilled once, "
                    "forked), 8 answer positions per request, 4 option tokens each",
        "value": round(C5_REQS / dt, 3), "unit": "req/s", "higher_is_better": True, "steps": steps, "warmup": warm,
        "ms_per_step": round(dt * 1e3, 2), "context_tok_per_s": round(C5_REQS * 8192 / dt, 1),
        "computed_tok_per_s": round(computed / dt, 1), "load": load,
        "roofline": roofline("mfma", rate(gp, "flops"), PEAK_F16_TFLOPS, "TFLOP/s",
                             "gemm (F16 weights, hi/lo split activations: two f16 passes per product)",
                             gp["launches"], gp["ms"] / max(1, gp["launches"]), measured_traffic("gemm", TRAFFIC_FILE_C5),
                             traffic_source="profiles/hbm_traffic_f16-7b_long-context.md (FETCH_SIZE + WRITE_SIZE, "
                                            "copy-calibrated)"),
        "attention": roofline("mfma", att_tf, PEAK_F16_TFLOPS, "TFLOP/s",
                              "attn_prefill (causal GQA over the paged KV cache as f16 hi/lo planes; three f16 passes per product)",
                              ap["launches"], ap["ms"] / max(1, ap["launches"]),
                              algorithmic_flops_per_step=att_flops),
        "kernel_ms_per_step": {c: round(p["ms"], 3) for c, p in prof.items()},
    }
    if layer_cost:
        po = oracle_modules()
        nq, ctx = 64, 8192
        r = np.random.default_rng(5)
        q = r.standard_normal((nq, hq * hd)).astype(np.float32)
        k = r.standard_normal((ctx, 4 * hd)).astype(np.float32)
        v = r.standard_normal((ctx, 4 * hd)).astype(np.float32)
        sample_pairs = sum(ctx - nq + i + 1 for i in range(nq))
        req_pairs = ctx * (ctx + 1) // 2
        entries = []
        for t, sec in layer_cost.items():
            t0 = time.perf_counter()
            po.attention(q, k, v, ctx - nq, hq, 4, threads=t)
            ta = (time.perf_counter() - t0) * req_pairs / sample_pairs
            per_layer = sec / Q4K_TOKENS * ctx + ta
            per_req = per_layer * L
            entries.append(cpu_entry(
                round(1 / per_req, 6), "req/s", t,
                f"one 8192-token request, computed whole as the reference does (no prefix reuse): projections and "
                f"MLP from one 1024-token layer ({sec:.2f} s) scaled x8, causal attention from the last {nq} query "
                f"rows over 8192 keys scaled by the (query, key) pair count x{req_pairs / sample_pairs:.0f} "
                f"({ta:.1f} s per layer); per layer {per_layer:.1f} s, x28 layers = {per_req:.0f} s per request"))
        res.update(cpu_pair(entries))
    return res


def bench_single(args, prec, name):
    """One of the extra configurations as its own JSON line (--workload plumbing|q4k-prefill|long-context)."""
    po = None if args.no_cpu else oracle_modules()
    if name == "plumbing":
        r = c1_plumbing(args, prec)
        metric = "plumbing decide latency (1 request, 144 tokens, yes/no option scoring)"
    elif name == "q4k-prefill":
        r = c4_q4k(args, prec, None if po is None else cpu_layer_cost_7b(args, po))
        metric = "Q4_K/Q6_K 7B batched prefill tok/s (32 x 1024)"
    else:
        r = c5_long_context(args, prec, None if po is None else cpu_layer_cost_7b(args, po))
        metric = "F16 7B shared-prefix long-context decide req/s (16 x 8192, 6144 shared)"
    line = base_line(metric, r.pop("value"), r.pop("unit"), r.pop("higher_is_better"), r.get("steps", args.steps),
                     r.get("warmup", args.warmup), r.get("ms_per_step", r.get("p50_ms", 0.0)), prec,
                     r.pop("workload"))
    line.update(r)
    return line


def base_line(metric, value, unit, higher, steps, warmup, ms, prec, workload, **extra):
    return {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": steps, "warmup": warmup,
            "ms_per_step": round(ms, 3), "higher_is_better": higher, "scaling": "weak", "vs_baseline": None,
            "dtype": "f16" if prec == lh.PREC_FAST else "f32", "data": "synthetic",
            "config": dict(workload=workload, seed=SEED,
                           precision={lh.PREC_EXACT: "exact", lh.PREC_FAST: "fast", lh.PREC_KV16: "kv16"}[prec],
                           **extra)}


def decide_request(vocab, seed):
    """One token-level /v1/decide body: a 480-token state, a 6-option choice question, a 5-level
    score and a yes/no question, 6 option-order passes."""
    rng = np.random.default_rng(seed)

    def toks(n):
        return rng.integers(0, vocab - 300, n).tolist()
    return {"state": toks(480),
            "questions": [{"type": "choice", "instruction": toks(12),
                           "options": [{"name": toks(2), "desc": toks(6)} for _ in range(6)]},
                          {"type": "score", "instruction": toks(10), "options": [{"name": [], "desc": toks(4)}
                                                                                 for _ in range(5)]},
                          {"type": "noul", "instruction": toks(8), "options": [{"name": toks(1)}, {"name": toks(1)}]}],
            "permutations": 6}


def bench_decide_request(args, prec):
    """Request-level decide (lg_decide) on the Q8_0 d2048 model: every option-order pass of one
    request encoded and prefilled as one GPU batch, the 256 slot rows scored at each answer
    position, passes averaged.  Requests run one after another, as the reference serves them."""
    img = lh.SynthImage(PRESET, seed=SEED)
    g = lh.Gguf.from_bytes(img)
    eng = lh.Engine(g, kv_tokens=16384, max_batch_tokens=8192, precision=prec)
    req = decide_request(eng.info["vocab"], SEED + 5)
    out = None
    for _ in range(max(args.warmup, 1)):
        out = eng.decide(req)
    eng.sync()
    steps = max(args.steps, 10)
    t0 = time.perf_counter()
    for _ in range(steps):
        out = eng.decide(req)
    dt = (time.perf_counter() - t0) / steps
    eng.close()
    toks = out["usage"]["input_tokens"] * out["usage"]["permutations"]
    log(f"decide request: {dt * 1e3:.2f} ms per request ({out['usage']['permutations']} passes, {toks} tokens)")
    line = base_line("decide requests/s (Q8_0 d2048, one request of 6 option-order passes)", round(1 / dt, 2),
                     "req/s", True, steps, max(args.warmup, 1), dt * 1e3, prec,
                     "24 layers, d_model 2048, 16 x 128, FFN 5632, vocab 32000, Q8_0; request: 480-token state, "
                     "choice (6 options), score (5 levels), noul; 6 passes prefilled as one batch",
                     tokens_per_request=toks, prefill_tok_per_s=round(toks / dt, 1))
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import pydecide
        import pyoracle as po
        layers = 2
        small = lh.SynthImage(PRESET, seed=SEED, n_layers=layers)
        og = po.Gguf(small.array())
        om = po.Model(og, threads=args.cpu_threads)
        t0 = time.perf_counter()
        pydecide.decide(om, og, req)
        cdt = (time.perf_counter() - t0) * 24 / layers
        line["cpu_baseline"] = {"value": round(1 / cdt, 5), "unit": "req/s", "cores": args.cpu_threads, "kind": "port",
                                "sample": f"the same request through {layers} of 24 layers (passes run one after "
                                          f"another, as the reference does), time scaled x{24 // layers}: "
                                          f"{cdt:.1f} s per request"}
    return line


def decide_batch_body(vocab, seed, states=REQUESTS, state_len=PROMPT):
    """A token-level /v1/decide/batch body (src/server.rs:235-258): `states` states of `state_len`
    ids sharing three 4-option choice questions (the headline workload's shape, through the
    request-level decide path)."""
    rng = np.random.default_rng(seed)

    def toks(n):
        return rng.integers(0, vocab - 300, n).tolist()
    qs = [{"type": "choice", "instruction": toks(4), "options": [{"name": toks(1), "desc": toks(2)} for _ in range(4)]}
          for _ in range(QUESTIONS)]
    return [{"state": toks(state_len), "questions": qs} for _ in range(states)]


def bench_decide_batch(args, prec):
    """lg_decide_batch on the Q8_0 d2048 model: 64 states x 512 ids with three 4-option questions
    (one pass each by the default rule), every state's prompt prefilled in one GPU batch, 256 slot
    rows scored per answer position, one answer per state."""
    img = lh.SynthImage(PRESET, seed=SEED)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=65536, precision=prec)
    reqs = decide_batch_body(eng.info["vocab"], SEED + 9)
    out = None
    for _ in range(max(args.warmup, 1)):
        out = eng.decide_batch(reqs)
    eng.sync()
    steps = max(args.steps, 3)
    t0 = time.perf_counter()
    for _ in range(steps):
        out = eng.decide_batch(reqs)
    dt = (time.perf_counter() - t0) / steps
    eng.close()
    toks = sum(o["usage"]["input_tokens"] * o["usage"]["permutations"] for o in out)
    log(f"decide batch: {dt * 1e3:.1f} ms per body of {len(reqs)} states ({toks} tokens)")
    line = base_line("decide req/s through lg_decide_batch (Q8_0 d2048, /v1/decide/batch of 64 states)",
                     round(len(reqs) / dt, 1), "req/s", True, steps, max(args.warmup, 1), dt * 1e3, prec,
                     f"24 layers, d_model 2048, 16 x 128, FFN 5632, vocab 32000, Q8_0; {len(reqs)} states x {PROMPT} ids, "
                     f"{QUESTIONS} choice questions of {OPTIONS} options, 1 pass each, one lg_decide_batch call",
                     tokens_per_body=toks, prefill_tok_per_s=round(toks / dt, 1))
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import pydecide
        import pyoracle as po
        layers = 2
        small = lh.SynthImage(PRESET, seed=SEED, n_layers=layers)
        og = po.Gguf(small.array())
        om = po.Model(og, threads=args.cpu_threads)
        t0 = time.perf_counter()
        pydecide.decide(om, og, reqs[0])
        cdt = (time.perf_counter() - t0) * 24 / layers
        line["cpu_baseline"] = {"value": round(1 / cdt, 4), "unit": "req/s", "cores": args.cpu_threads, "kind": "port",
                                "sample": f"1 of the {len(reqs)} states through {layers} of 24 layers, time scaled "
                                          f"x{24 // layers}: {cdt:.1f} s per state (the reference runs states one after another)"}
    return line


OT_PRESET = "openthai-0.8b"


def openthai_requests(seed):
    """Token-level counterparts of the reference's timed OpenThai cases
    (validation/openthai.requests.json; timings in validation/openthai-summary.json:11-39):
    case 7, one 255-option choice question in 1 pass, 1437 prompt tokens (57,884 ms on the
    reference's CPU x4); case 8, an 11-option choice question, default 8 passes of 60 tokens
    (13,191 ms)."""
    rng = np.random.default_rng(seed)

    def toks(n):
        return rng.integers(0, 247000, n).tolist()
    # 1437 = state block 7 (marker, 5 ids, newline) + header 6 (marker, kind, 3 ids, newline)
    #        + 255 x (slot marker, name, newline) with 912 name ids + answer block 2
    names = [4] * 147 + [3] * 108
    big = {"state": toks(5), "permutations": 1,
           "questions": [{"type": "choice", "instruction": toks(3), "options": [{"name": toks(n)} for n in names]}]}
    # 60 = 7 + 6 + 11 x 2 + 23 name ids + 2; 11 options -> the default 8 option-order passes
    small = {"state": toks(5),
             "questions": [{"type": "choice", "instruction": toks(3),
                            "options": [{"name": toks(n)} for n in [3] + [2] * 10]}]}
    return big, small


def bench_openthai(args, prec):
    """OpenThai-SystemOne decide on the 0.8B shape (24 layers: 18 gated DeltaNet + 6 gated full
    attention, d 1024, FFN 3584, vocab 248339, F16 weights as the converter writes them): the
    reference's two timed request shapes, each lg_decide call end to end (encode, one GPU batch
    of all passes, slot scoring), requests one after another."""
    img = lh.SynthImage(OT_PRESET, seed=SEED)
    eng = lh.Engine(lh.Gguf.from_bytes(img), precision=prec)
    big, small = openthai_requests(SEED + 7)
    steps = max(args.steps, 5)
    res = {}
    for name, req, want in (("1437x1", big, 1437), ("60x8", small, 60)):
        out = None
        for _ in range(max(args.warmup, 1)):
            out = eng.decide(req)
        eng.sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            out = eng.decide(req)
        dt = (time.perf_counter() - t0) / steps
        assert out["usage"]["input_tokens"] == want, out["usage"]
        res[name] = (dt, out["usage"]["permutations"])
        log(f"openthai {name}: {dt * 1e3:.2f} ms per request ({out['usage']['permutations']} passes)")
    eng.profile_reset()
    eng.profile(True)
    eng.decide(big)
    eng.profile(False)
    classes = ("gemm", "ot_attn", "ot_attn_prep", "ot_delta_prep", "ot_delta_scan", "ot_delta_out", "rmsnorm",
               "embed")
    prof = {c: eng.profile_read(c) for c in classes}
    for c in classes:
        p = prof[c]
        log(f"  {c:14s} {p['launches']:4d} launches {p['ms']:8.3f} ms")
    eng.close()
    g = prof["gemm"]
    gemm_tflops = g["flops"] / (g["ms"] * 1e-3) / 1e12 if g["ms"] > 0 else 0.0
    dt_big, _ = res["1437x1"]
    dt_small, np_small = res["60x8"]
    line = base_line("OpenThai decide req/s (0.8B shape, 1437-token request)", round(1 / dt_big, 3), "req/s", True,
                     steps, max(args.warmup, 1), dt_big * 1e3, prec,
                     "OpenThai-SystemOne 0.8B shape (24 layers: 18 gated DeltaNet + 6 gated full attention, "
                     "d 1024, FFN 3584, 8/2 x 256 heads, 16 linear heads x 128, vocab 248339, F16); request: "
                     "1 choice question of 255 options, 1437 tokens, 1 pass",
                     ms_per_request=round(dt_big * 1e3, 2),
                     ms_per_request_60x8=round(dt_small * 1e3, 2), passes_60x8=np_small,
                     reference_cpu_ms={"1437x1": 57884, "60x8": 13191},
                     kernel_ms={c: round(prof[c]["ms"], 3) for c in classes})
    line["roofline"] = {"bound": "mfma", "achieved": round(gemm_tflops, 1), "peak": PEAK_F16_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(gemm_tflops / PEAK_F16_TFLOPS, 4), "traffic": None,
                        "kernel": "gemm (every projection and MLP matrix of the 1437-token forward)"}
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import pydecide
        import pyoracle as po
        layers = 4
        smallimg = lh.SynthImage(OT_PRESET, seed=SEED, n_layers=layers)
        og = po.Gguf(smallimg.array())
        om = po.OpenThai(og, threads=args.cpu_threads)
        t0 = time.perf_counter()
        pydecide.decide(om, og, big)
        cdt = (time.perf_counter() - t0) * 24 / layers
        line["cpu_baseline"] = {"value": round(1 / cdt, 5), "unit": "req/s", "cores": args.cpu_threads, "kind": "port",
                                "sample": f"the 1437-token request through {layers} of 24 layers (3 DeltaNet + 1 "
                                          f"full attention, the model's own 3:1 mix), time scaled x{24 // layers}: "
                                          f"{cdt:.1f} s per request"}
    return line


def c2_cpu_baseline(args):
    """The oracle on a bounded sample of the headline workload: one 560-token request through all 24
    layers (the reference's loop order), per thread count."""
    po = oracle_modules()
    img = lh.SynthImage(PRESET, seed=SEED)
    om = po.Model(po.Gguf(img.array()), threads=1)
    reqs, option_ids = prefill_workload(om.V)
    ids, pos = reqs[0]
    entries = []
    for t in cpu_threads(args):
        om.set_threads(t)
        t0 = time.perf_counter()
        om.forward(ids, pos, option_ids)
        dt = time.perf_counter() - t0
        log(f"  oracle C2 request, 24 layers, {t} threads: {dt:.2f} s")
        entries.append(cpu_entry(
            round(len(ids) / dt, 2), "tok/s", t,
            f"1 of the {REQUESTS} requests ({len(ids)} tokens, {QUESTIONS} answer positions, {OPTIONS} options) "
            f"through all 24 layers: {dt:.2f} s; C restatement of the reference CPU algorithm (F32 weights "
            f"expanded at load, 4-row x 8-lane FMA kernel, rows split over {t} threads)"))
    del om
    return entries


LAYA_PRESET = "laya-english"
LAYA_CPU_MS = {"refund": 1232, "types": 4967, "unicode": 2035, "truncation": 23884}


def laya_requests(seed):
    """Token-level counterparts of the reference's four timed Laya English cases
    (validation/check.py:14-21, latencies in validation/laya_english_f16.report.json): refund (1 noul
    question, 45 tokens), types (a 3-option choice, a 3-level score and a noul question, 183
    tokens over the three forwards), unicode (1 noul question, 68 tokens) and truncation (1 noul
    question whose state is cut to the 512-token context).  Instruction and option token counts
    follow the English texts ("noul question: Does the customer ask for money back?" is 12
    tokens, the two default noul options 9 and 7)."""
    rng = np.random.default_rng(seed)

    def toks(n):
        return rng.integers(0, 50000, n).tolist()

    def noul():
        return {"type": "noul", "instruction": toks(12), "options": [{"name": toks(9)}, {"name": toks(7)}]}
    # per question: [cls] ins [sep] ([mask] option)... [sep] state [sep]
    refund = {"state": toks(11), "questions": [noul()]}  # 1 + 12 + 1 + 18 + 1 + 11 + 1 = 45
    types = {"state": toks(23), "questions": [  # 66 + 60 + 57 = 183 with a 23-token state
        {"type": "choice", "instruction": toks(12), "options": [{"name": toks(n)} for n in (9, 8, 7)]},
        {"type": "score", "instruction": toks(9), "options": [{"name": toks(n)} for n in (6, 7, 8)]},
        noul()]}
    unicode = {"state": toks(34), "questions": [noul()]}  # 34 + 34 = 68
    truncation = {"state": toks(1100), "questions": [noul()]}
    return {"refund": (refund, 45), "types": (types, 183), "unicode": (unicode, 68), "truncation": (truncation, 512)}


def bench_laya(args, prec):
    """Laya English decide on the ModernBERT-base shape (22 layers, d 768, 12 x 64 heads, GeGLU
    1152, window-64 local / global RoPE attention every third layer, vocab 50368, F16 weights): the
    reference's four timed request shapes through lg_decide one after another, then 64 states of
    the 512-token case through lg_decide_batch."""
    img = lh.SynthImage(LAYA_PRESET, seed=SEED)
    eng = lh.Engine(lh.Gguf.from_bytes(img), precision=prec)
    cases = laya_requests(SEED + 9)
    steps = max(args.steps, 5)
    res = {}
    for name, (req, want) in cases.items():
        out = None
        for _ in range(max(args.warmup, 1)):
            out = eng.decide(req)
        eng.sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            out = eng.decide(req)
        dt = (time.perf_counter() - t0) / steps
        assert out["usage"]["input_tokens"] == want, (name, out["usage"])
        res[name] = dt
        log(f"laya {name}: {dt * 1e3:.2f} ms per request ({want} tokens; reference CPU x4 {LAYA_CPU_MS[name]} ms)")
    big = cases["truncation"][0]
    states = [big] * 64
    eng.decide_batch(states)
    eng.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        eng.decide_batch(states)
    dtb = (time.perf_counter() - t0) / steps
    log(f"laya batch: 64 x 512-token states in {dtb * 1e3:.2f} ms ({64 / dtb:.1f} req/s)")
    eng.profile_reset()
    eng.profile(True)
    eng.decide_batch(states)
    eng.profile(False)
    classes = ("gemm", "laya_attn", "layer_norm", "laya_tail", "embed")
    prof = {c: eng.profile_read(c) for c in classes}
    for c in classes:
        p = prof[c]
        log(f"  {c:12s} {p['launches']:4d} launches {p['ms']:8.3f} ms")
    eng.close()
    g = prof["gemm"]
    gemm_tflops = g["flops"] / (g["ms"] * 1e-3) / 1e12 if g["ms"] > 0 else 0.0
    dt = res["truncation"]
    line = base_line("Laya decide req/s (512-token request)", round(1 / dt, 3), "req/s", True, steps,
                     max(args.warmup, 1), dt * 1e3, prec,
                     "Laya English ModernBERT-base shape (22 layers, d 768, 12 x 64 heads, GeGLU 1152, "
                     "local window 64 / global every 3rd layer, 2 head layers, vocab 50368, F16); request: 1 noul "
                     "question, state cut to the 512-token context",
                     ms_per_request={k: round(v * 1e3, 3) for k, v in res.items()},
                     reference_cpu_ms=LAYA_CPU_MS,
                     batch64_req_s=round(64 / dtb, 1), batch64_ms=round(dtb * 1e3, 2),
                     kernel_ms_batch64={c: round(prof[c]["ms"], 3) for c in classes})
    line["roofline"] = {"bound": "mfma", "achieved": round(gemm_tflops, 1), "peak": PEAK_F16_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(gemm_tflops / PEAK_F16_TFLOPS, 4), "traffic": None,
                        "kernel": "gemm (every projection and MLP matrix of the 64 x 512-token batch)"}
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import pydecide
        import pyoracle as po
        og = po.Gguf(img.array())
        om = po.Laya(og, threads=args.cpu_threads)
        t0 = time.perf_counter()
        pydecide.laya_decide(om, og, big)
        cdt = time.perf_counter() - t0
        line["cpu_baseline"] = {"value": round(1 / cdt, 5), "unit": "req/s", "cores": args.cpu_threads, "kind": "port",
                                "sample": f"the 512-token request through all 22 layers: {cdt:.1f} s per request"}
    return line


VENDOR_SHAPES = {
    "C2 q|k|v": (35840, 6144, 2048), "C2 o": (35840, 2048, 2048), "C2 gate|up": (35840, 11264, 2048),
    "C2 down": (35840, 2048, 5632), "7B q|k|v": (32768, 4608, 3584), "7B o": (32768, 3584, 3584),
    "7B gate|up": (32768, 37888, 3584), "7B down": (32768, 3584, 18944),
}


def bench_vendor_gemm(args, prec):
    """The practical f16 MFMA rate at the prefill projection shapes: torch.matmul (x[M][K] . W[N][K]^T in
    f16 with f32 accumulation, ROCm's vendor GEMM libraries) on the same GPU.  One f16 pass per product,
    so half this rate bounds a two-pass (hi/lo split) GEMM of the same shape built on the same libraries.
    Not a path of the library: a measured anchor for the roofline fractions."""
    import torch

    dev = torch.device("cuda:0")
    libs = [("hipblaslt", "cublaslt"), ("rocblas", "cublas")]
    rows = {}
    for label, (M, N, K) in VENDOR_SHAPES.items():
        g = torch.Generator(device=dev).manual_seed(1)
        a = torch.randn(M, K, device=dev, dtype=torch.float16, generator=g)
        w = torch.randn(N, K, device=dev, dtype=torch.float16, generator=g)
        row = {"M": M, "N": N, "K": K}
        for name, key in libs:
            try:
                torch.backends.cuda.preferred_blas_library(key)
                for _ in range(3):
                    torch.matmul(a, w.t())
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                reps = 10
                e0.record()
                for _ in range(reps):
                    torch.matmul(a, w.t())
                e1.record()
                torch.cuda.synchronize()
                ms = e0.elapsed_time(e1) / reps
                tf = 2.0 * M * N * K / (ms * 1e-3) / 1e12
                row[name] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1), "frac": round(tf / PEAK_F16_TFLOPS, 4)}
                log(f"vendor f16 GEMM {label:12s} {M} x {N} x {K} ({name}): {ms:.3f} ms, {tf:.1f} TFLOP/s")
            except RuntimeError as e:  # a library that refuses the shape or is absent
                row[name] = {"error": str(e)[:200]}
        rows[label] = row
        del a, w
    torch.backends.cuda.preferred_blas_library("cublaslt")
    return {"workload": "vendor f16 GEMM at the prefill projection shapes (torch.matmul, f16 operands, f32 "
                        "accumulation): a measured practical MFMA rate, not part of the library's path",
            "peak_TFLOP/s": PEAK_F16_TFLOPS, "shapes": rows}


DECODE_MATRIX_BYTES = {"o": 4456448, "down": 12255232, "q|k|v": 13369344, "gate|up": 24510464, "head": 69632000}


def bench_launch_floor(args, prec):
    """The GPU-side cost of one dependent launch at the decode matrix sizes: chains of 200 back-to-back
    launches of the library's plain read kernel (lg_probe_read: 16-byte loads, nothing written), each over
    its own slice of each matrix's GGUF byte count (about 2 GiB of slices, so the bytes come from HBM as
    the decode's distinct matrices do), timed with events on one stream, and one 16-byte read for the
    launch alone.  A line through the sizes gives the fixed cost per launch and the streaming rate
    that the decode GEMV's launches are measured against."""
    chain = 200
    rows = {}
    sizes = dict(DECODE_MATRIX_BYTES)
    sizes["empty"] = 16
    for label, nbytes in sizes.items():
        us = lh.probe_read(nbytes, chain)
        rows[label] = {"bytes": nbytes, "us_per_launch": round(us, 3),
                       "GB_per_s": round(nbytes / (us * 1e-6) / 1e9, 1) if label != "empty" else None}
        log(f"launch floor {label:8s} {nbytes:10d} B: {us:7.3f} us per launch")
    xs = np.array([v["bytes"] for k, v in rows.items() if k != "empty"], np.float64)
    ys = np.array([v["us_per_launch"] for k, v in rows.items() if k != "empty"], np.float64)
    slope, icpt = np.polyfit(xs, ys, 1)
    return {"workload": "launch floor at the decode matrix sizes: chains of 200 dependent launches of a plain "
                        "read kernel (lg_probe_read), each over its own slice of each matrix's GGUF bytes (about 2 GiB of slices: "
                        "HBM reads), on one stream",
            "sizes": rows, "fit": {"fixed_us": round(float(icpt), 3), "streaming_TB_per_s": round(1e-6 / float(slope), 2)}}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--precision", choices=["exact", "fast", "kv16"], default="exact")
    ap.add_argument("--workload", choices=["decide", "plumbing", "q4k-prefill", "long-context", "decide-request",
                                           "decide-batch", "openthai-decide", "laya-decide", "vendor-gemm", "launch-floor"],
                    default="decide",
                    help="decide (default): the Q8_0 d2048 batched decide headline with the other four workload "
                         "configurations (C1 plumbing, C3 decode, C4 Q4_K 7B prefill, C5 long context) nested in "
                         "`configs`; the others run one configuration as its own JSON line")
    ap.add_argument("--configs", default="C1,C3,C4,C5",
                    help="nested configurations of the default run (comma list; empty for the headline only)")
    ap.add_argument("--config-steps", type=int, default=3, help="timed steps of C4 and C5 (about 1.5 s each)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="skip the HIP-graph decode measurement (rocprofv3 kernel tracing crashes on graph launches)")
    ap.add_argument("--decode-steps", type=int, default=DECODE_STEPS,
                    help="greedy steps per decode run (fewer keeps counter-collection runs short)")
    ap.add_argument("--cpu-threads", type=int, default=4, help="threads of the CPU baseline (the reference's default)")
    ap.add_argument("--cpu-threads-all", type=int, default=16,
                    help="threads of the second CPU baseline: the host cores this job may use (0 to skip)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="first run the F32 dequant kernel over MIB MiB: a plain copy (4 B read, 4 B written "
                         "per element), so a counter profile of this command also holds the kernel that "
                         "scales FETCH_SIZE / WRITE_SIZE to bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the library has no multi-GPU path (asked for {args.gpus}); "
              "the workload's requests are independent, so N GPUs would each run their own batch.",
              file=sys.stderr)
        sys.exit(2)
    prec = {"exact": lh.PREC_EXACT, "fast": lh.PREC_FAST, "kv16": lh.PREC_KV16}[args.precision]
    if args.copy_calibration > 0:
        n = args.copy_calibration * (1 << 20) // 4
        src = np.arange(n, dtype=np.float32)
        for _ in range(2):
            assert np.array_equal(lh.dequant(lh.F32, src.view(np.uint8)), src)
        log(f"copy calibration: 2 launches of the F32 dequant kernel, {n * 4} B read + {n * 4} B written each")
    if args.workload in ("plumbing", "q4k-prefill", "long-context"):
        print(json.dumps(bench_single(args, prec, args.workload)), flush=True)
        return
    if args.workload != "decide":
        fn = {"decide-request": bench_decide_request, "decide-batch": bench_decide_batch,
              "openthai-decide": bench_openthai, "laya-decide": bench_laya, "vendor-gemm": bench_vendor_gemm, "launch-floor": bench_launch_floor}
        print(json.dumps(fn[args.workload](args, prec)), flush=True)
        return
    wanted = [c.strip().upper() for c in args.configs.split(",") if c.strip()]
    log(f"generating {PRESET} (seed {SEED})")
    t0 = time.perf_counter()
    img = lh.SynthImage(PRESET, seed=SEED)
    g = lh.Gguf.from_bytes(img)
    eng = lh.Engine(g, device=0, kv_tokens=REQUESTS * 640 + DECODE_CTX * 3 + 512, max_batch_tokens=40000,
                    precision=prec)
    log(f"model ready in {time.perf_counter() - t0:.1f}s: {eng.info}")

    T, dt, prof, probs = bench_prefill(eng, args.steps, args.warmup)
    ms = dt / args.steps * 1e3
    tok_s = T * args.steps / dt
    gp = prof["gemm"]
    gemm_tflops = rate(gp, "flops")
    log(f"C2 prefill: {ms:.2f} ms/step, {tok_s:.0f} tok/s, gemm {gemm_tflops:.1f} TFLOP/s over "
        f"{gp['launches']} launches ({gp['ms']:.2f} ms)")
    for c, p in prof.items():
        log(f"  {c:12s} launches {p['launches']:5d}  {p['ms']:8.3f} ms")
    line = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if prec == lh.PREC_FAST else "f32",
        "data": "synthetic",
        "config": {
            "workload": f"Q8_0 batched prefill decide: {REQUESTS} requests x {PROMPT + QUESTIONS * QBLOCK} tokens "
                        f"({PROMPT} prompt + {QUESTIONS} question blocks of {QBLOCK}), {OPTIONS} option tokens "
                        f"scored at each answer position; 24 layers, d_model 2048, 16 heads x 128, FFN 5632, "
                        f"vocab 32000, Q8_0 matrices, F16 embeddings",
            "requests": REQUESTS,
            "tokens_per_step": T,
            "seed": SEED,
            "precision": args.precision,
            "arithmetic": {lh.PREC_EXACT: "f16 hi/lo split MFMA with f32 accumulation, exact Q8_0 block scaling, KV "
                                          "cache as f16 hi/lo planes",
                           lh.PREC_KV16: "f16 hi/lo split MFMA with f32 accumulation, exact Q8_0 block scaling, f16 KV "
                                         "cache",
                           lh.PREC_FAST: "f16 MFMA, f32 accumulation, f16 KV cache"}[prec],
        },
        "decide_req_per_s": round(REQUESTS * args.steps / dt, 2),
        "roofline": roofline("mfma", gemm_tflops, PEAK_F16_TFLOPS, "TFLOP/s",
                             "gemm (exact Q8_0 MFMA GEMM: f16 codes and block scales, two f16 passes per product)",
                             gp["launches"], gp["ms"] / max(1, gp["launches"]), measured_traffic("gemm"),
                             traffic_source="profiles/hbm_traffic_q8-2048_bench.md (FETCH_SIZE + WRITE_SIZE, "
                                            "copy-calibrated)",
                             algorithmic_flops_per_step=gp["flops"]),
        "kernel_ms_per_step": {c: round(p["ms"], 3) for c, p in prof.items()},
    }
    configs = {}
    if "C3" in wanted:
        configs["C3"] = c3_decode(eng, args)
    eng.close()
    if "C3" in wanted and prec == lh.PREC_EXACT:
        # the same decode over an f16 paged KV cache (the kv16 mode).  Reported beside the measured line
        # only: at 24 layers of this model its logits miss the 2e-2 bar
        eng = lh.Engine(g, device=0, kv_tokens=DECODE_CTX * 3 + 512, precision=lh.PREC_KV16)
        kv = c3_decode(eng, args, extras=False)
        eng.close()
        configs["C3"]["kv16"] = {
            "ms_per_token": kv["ms_per_token"], "value": kv["value"], "unit": "tok/s",
            "kernel_ms_per_token": kv["kernel_ms_per_token"], "attention": kv["attention"],
            "parity": "outside the parity bars: decode logits up to 9.2e-2 of the largest |logit| against "
                      "2e-2, and the greedy argmax differs from the oracle at 5 of 64 steps outside the near-tie "
                      "window (tests/test_gpu_fulldepth.py, strict xfail); not the measured value",
        }
    del g, img
    if "C1" in wanted:
        configs["C1"] = c1_plumbing(args, prec)
    layer_cost = None
    if ("C4" in wanted or "C5" in wanted) and not args.no_cpu:
        layer_cost = cpu_layer_cost_7b(args, oracle_modules())
    if "C4" in wanted:
        configs["C4"] = c4_q4k(args, prec, layer_cost)
    if "C5" in wanted:
        configs["C5"] = c5_long_context(args, prec, layer_cost)
    if not args.no_cpu:
        log("C2 CPU baseline")
        line.update(cpu_pair(c2_cpu_baseline(args)))
        if "C3" in configs and "cpu_baseline" in line:
            # the reference has no cache: every step recomputes the whole 2049-token sequence
            per_tok = line["cpu_baseline"]["value"]
            configs["C3"]["cpu_baseline"]["reference_without_cache_s_per_token"] = round((DECODE_CTX + 1) / per_tok, 1)
    line["configs"] = configs
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
