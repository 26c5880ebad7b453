#!/usr/bin/env python3
"""Benchmark of the MI355X fused Q4 decode step.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Headline (value): decode tok/s of the 135M Q4 model at batch 1 -- BASELINE
config 1: SmolLM2-135M shape, weights N(0, 0.02) from seed 0 quantised by the
converter's quant_q4, a 32-token prompt uniform over the vocab (seed 1),
greedy decode.  A step is one decode token; K chained steps are timed after
the prompt has been prefilled, with the weights and KV cache resident in HBM.

One JSON line on stdout carries, besides the driver's fields:
  roofline      the kernel that runs the timed decode: in exec mode 3 (default)
                the persistent k_flow, one launch per chain, whose algorithmic
                bytes are the per-token Q4 weights + norms + KV reads summed
                over the chain's steps, divided by the chain's duration from
                HIP events on the model's stream; in modes 1/2 the dominant
                phase kernel (mode 4: k_flow through an ordinary launch, for
                profilers)
  precision     what the arithmetic is: 24-bit activations per 32-element
                group, exact int32 group dots, f32 across groups
  gemv_roofline the lm_head-shaped Q4 GEMV (49152 x 960, config 2) read cold
  cpu_baseline  the oracle (C restatement of engine/infer.js, fp64 accumulate,
                1 thread) on a bounded sample of the same decode, with the
                host CPU model; configs 2-5 carry their own CPU figures
  gemv_sweep    config 2: Q4 / Q8 group-32 GEMV GB/s on the 360M shapes
                (warm = MALL-resident, cold = rotating >= 1 GiB of copies,
                stacked = 32 matrices per launch)
  configs       config 3 (prompt-lookup speculation, k = 4 / 8), config 4
                (GPT-2 124M), config 5 (362M, fp16 KV: the 1536-token prompt
                through the batched path, and through the 16-token passes of
                the decode phases for comparison; then 511 decode steps)

    python bench.py --prefill-only   config 5's prompt through the batched
                                     path three times (for profilers)
    python bench.py --decode-360m    config 5's decode alone: the prompt, then
                                     the 511-step chain as one dispatch (for
                                     profilers; --exec-mode 4 keeps it an
                                     ordinary launch)
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "microllm-lab_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import numpy as np  # noqa: E402

METRIC = "decode tok/s (135M Q4, bs1) + Q4 GEMV GB/s as % of 8 TB/s HBM peak"
HBM_PEAK_GBS = 8000.0
LAYER_PHASES = ("QKV", "ATTN", "MLP")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------- bytes
def q4_bytes(rows, cols):
    return rows * cols // 2 + rows * (cols // 32) * 4


def phase_bytes(cfg, seq, kv_bytes=4):
    """Algorithmic bytes per launch of each decode phase at one token with `seq`
    positions in the cache: the weights it reads once plus one read of its input
    vector and one write of its output (the split-K partials the engine passes
    between phases are implementation traffic and are not counted)."""
    D, FF, V = cfg.d_model, cfg.d_ff, cfg.vocab_size
    hd = D // cfg.n_heads
    kvd = cfg.n_kv_heads * hd
    qkv_rows = D + 2 * kvd
    mlp_in = 1 if cfg.arch == "gpt2" else 2
    return {
        "QKV": q4_bytes(qkv_rows, D) + 4 * D * 2 + 4 * qkv_rows,
        "ATTN": 2 * cfg.n_kv_heads * seq * hd * kv_bytes + 4 * D + q4_bytes(D, D) + 4 * D,
        "MLP": mlp_in * q4_bytes(FF, D) + q4_bytes(D, FF) + 4 * D * 2 + 4 * D,
        "FINAL": 4 * D * 3,
        "LM": q4_bytes(V, D) + 4 * D + 4 * V,
        "ARGMAX": 0,
    }


def token_bytes(cfg, seq, kv_bytes=4):
    """Algorithmic bytes of one decode token: the Q4 weights, the norm gains
    and the KV rows read at context mean_seq."""
    D, FF = cfg.d_model, cfg.d_ff
    hd = D // cfg.n_heads
    kvd = cfg.n_kv_heads * hd
    mats = q4_bytes(D + 2 * kvd, D) + q4_bytes(D, D) + (1 if cfg.arch == "gpt2" else 2) * q4_bytes(FF, D) + q4_bytes(D, FF)
    weights = cfg.n_layers * mats + q4_bytes(cfg.vocab_size, D)
    norms = (2 * cfg.n_layers + 1) * D * 4
    kv = 2 * cfg.n_kv_heads * hd * kv_bytes * cfg.n_layers * seq
    return weights + norms + kv


def kind_bytes(rows, cols, kind):
    """Bytes of one matrix in its storage (data + scales)."""
    return {"q4": q4_bytes(rows, cols), "q8": rows * cols + 4 * rows, "q8g32": rows * cols + rows * (cols // 32) * 4,
            "f16": 2 * rows * cols, "bf16": 2 * rows * cols, "f32": 4 * rows * cols}[kind]


def kind_token_bytes(cfg, seq, kind, kv_bytes=4):
    """token_bytes for a model whose matrices are stored as `kind`."""
    D, FF = cfg.d_model, cfg.d_ff
    hd = D // cfg.n_heads
    kvd = cfg.n_kv_heads * hd
    mats = (kind_bytes(D + 2 * kvd, D, kind) + kind_bytes(D, D, kind) +
            (1 if cfg.arch == "gpt2" else 2) * kind_bytes(FF, D, kind) + kind_bytes(D, FF, kind))
    weights = cfg.n_layers * mats + kind_bytes(cfg.vocab_size, D, kind)
    norms = (2 * cfg.n_layers + 1) * D * 4
    kv = 2 * cfg.n_kv_heads * hd * kv_bytes * cfg.n_layers * seq
    return weights + norms + kv


def bench_kinds(mllm, pgw, steps=127):
    """Config 1's workload (135M shape, 32-token prompt, greedy chain) with
    the matrices stored per-row Q8, f16, bf16 and f32 -- the kinds the
    reference times on its GPU engine (WRITEUP.md:31-35) -- through the
    kind-generic step."""
    cfg = pgw.CONFIGS["smollm2-135m"]
    prompt = [int(v) for v in np.random.default_rng(1).integers(0, cfg.vocab_size, 32)]
    res = {}
    for kind in ("q8", "f16", "bf16", "f32"):
        g = mllm.PetitGPT(pgw.parse_pgw(pgw.make_llama(cfg, seed=0, kind=kind)))
        for _ in range(2):
            g.resetCache()
            g.forwardPrompt(prompt)
            g.decodeChain(g.last_argmax, steps)
        ms, n = g.last_timing()
        algo = sum(kind_token_bytes(cfg, 33 + i, kind) for i in range(n)) / n
        us = ms * 1e3 / n
        res[kind] = {"kernel": g.decodeKernel, "us_per_token": round(us, 2), "tok_s": round(n / (ms * 1e-3), 1),
                     "algorithmic_bytes_per_token": int(algo), "gbs": round(algo / us / 1e3, 1)}
        log(f"[bench] kinds {kind}: {res[kind]}")
        g.destroy()
    res["workload"] = (f"smollm2-135m shape, matrices stored as each kind (N(0,0.02), seed 0), 32-token prompt, "
                       f"{steps} chained greedy decode steps (config 1's workload)")
    return res


def traffic_record(kernel):
    """The rocprofv3 FETCH_SIZE / WRITE_SIZE record of `kernel` in
    profiles/decode_traffic.json (counters scaled by what they read on a plain
    copy of known size), or None when no record matches."""
    path = os.path.join(ROOT, "profiles", "decode_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(kernel)
    except (OSError, ValueError):
        return None


def measured_traffic(kernel):
    """HBM bytes per launch of a phase kernel, or None."""
    rec = traffic_record(kernel)
    return None if rec is None else rec.get("hbm_bytes_per_launch")


def copy_calibration(torch):
    """A plain device copy of known size, for scaling FETCH_SIZE / WRITE_SIZE."""
    n = 256 << 20
    src = torch.ones(n // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "launches": 5}), flush=True)


# ---------------------------------------------------------------- decode
def bench_decode(mllm, pgw, torch, args):
    cfg = pgw.CONFIGS["smollm2-135m"]
    t = time.time()
    bundle = pgw.parse_pgw(pgw.make_llama(cfg, seed=0))
    log(f"[bench] 135M model generated in {time.time() - t:.1f}s")
    prompt = [int(v) for v in np.random.default_rng(1).integers(0, cfg.vocab_size, 32)]
    g = mllm.PetitGPT(bundle, exec_mode=args.exec_mode)
    mode = g.execMode  # the mode the engine really uses (a refused cooperative launch falls back to 1)
    kname = g.decodeKernel  # the kernel the engine really runs the decode step with
    # warmup: W chained steps after a prefill
    g.resetCache()
    g.forwardPrompt(prompt)
    if args.warmup > 0:
        g.decodeChain(g.last_argmax, args.warmup)
    # timed region: K chained decode steps after an (untimed) prefill
    g.resetCache()
    g.forwardPrompt(prompt)
    first = g.last_argmax
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ids = g.decodeChain(first, args.steps)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    gpu_ms, n = g.last_timing()
    assert n == args.steps == len(ids)
    wall = t1 - t0
    mode = g.execMode
    # reference-style rate (worker.js:166,176): n / totalMs of a whole
    # generate call, prompt included -- 128 tokens after the 32-token prompt
    r = g.generate(prompt, maxNewTokens=128, mode="chain", chainChunk=128)
    r = g.generate(prompt, maxNewTokens=128, mode="chain", chainChunk=128)
    ref_style = len(r["generatedIds"]) / (r["totalMs"] / 1e3)
    # per-phase kernel times (events around each launch, same stream)
    g.resetCache()
    g.forwardPrompt(prompt)
    prof = g.profile_decode(first, 32)
    seq_mean = len(prompt) + 16
    pb = phase_bytes(cfg, seq_mean)
    per_token_us = {ph: us * (cfg.n_layers if ph in LAYER_PHASES else 1) for ph, us in prof.items()}
    dom = max(per_token_us, key=per_token_us.get)
    if mode >= 3:
        # one k_flow launch ran the whole timed chain: step i attends over
        # len(prompt) + 1 + i cached positions
        chain_bytes = sum(token_bytes(cfg, len(prompt) + 1 + i) for i in range(args.steps))
        achieved = chain_bytes / (gpu_ms * 1e-3) / 1e9
        rec = traffic_record(kname)
        traffic = None if rec is None else int(rec["hbm_bytes_per_step"] * args.steps)
        roof = {
            "bound": "hbm",
            "kernel": f"{kname} (persistent decode kernel, one launch = the {args.steps}-step chain, 135M)",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 5),
            "traffic": traffic,
            "bytes_per_launch": chain_bytes,
            "us_per_launch": round(gpu_ms * 1e3, 1),
        }
    else:
        achieved = pb[dom] / (prof[dom] * 1e-6) / 1e9
        roof = {
            "bound": "hbm",
            "kernel": f"k_phase<{dom}> (decode phase {dom}, 135M, seq ~{seq_mean})",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 5),
            "traffic": measured_traffic(f"k_phase<{dom}>"),
            "bytes_per_launch": pb[dom],
            "us_per_launch": round(prof[dom], 3),
        }
    # host loop: forwardDecode per token with the logits copied back (PCIe-inclusive; not `value`)
    g.resetCache()
    g.forwardPrompt(prompt)
    nxt = g.last_argmax
    n_host = 32
    t0 = time.perf_counter()
    for _ in range(n_host):
        g.forwardDecode(nxt)
        nxt = g.last_argmax
    host_tok_s = n_host / (time.perf_counter() - t0)
    g.destroy()
    mean_seq = len(prompt) + (args.steps + 1) / 2
    step_bytes = token_bytes(cfg, mean_seq)
    return {
        "value": args.steps / wall,
        "exec_mode": mode,
        "ref_style_tok_s": round(ref_style, 1),
        "ttft_ms": round(r["ttftMs"], 3),
        "ms_per_step": wall / args.steps * 1e3,
        "kernel_ms_per_step": gpu_ms / args.steps,
        "first_ids": ids[:8],
        "roofline": roof,
        "phase_us": {k: round(v, 3) for k, v in prof.items()},
        "decode_step_gbs": round(step_bytes / (wall / args.steps) / 1e9, 2),
        "decode_step_bytes": step_bytes,
        "host_loop_tok_s": round(host_tok_s, 1),
    }


def host_cpu():
    """The host CPU's model name (/proc/cpuinfo) and logical CPU count."""
    name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return name, os.cpu_count()


def cpu_decode_rate(oracle, bundle, budget_s, prompt=None, context=None, gpt2=False, max_steps=256):
    """Greedy decode steps of the oracle (one thread) timed for ~budget_s: after
    a real prompt, or with the cache length set to `context` directly (the
    cached values are then not computed: a step's cost does not depend on
    them).  Returns (tok/s, steps, prompt seconds or None)."""
    m = oracle.OracleModel(bundle)
    pre = None
    if prompt is not None:
        t0 = time.perf_counter()
        lg = m.forward_prompt(prompt)
        pre = time.perf_counter() - t0
        hist = []
        tok = oracle.argmax_gpt2(lg, hist) if gpt2 else oracle.argmax(lg)
    else:
        m.cache_len = context
        tok, hist = 1, []
    n = 0
    t0 = time.perf_counter()
    while True:
        lg = m.forward_decode(tok)
        hist.append(tok)
        tok = oracle.argmax_gpt2(lg, hist) if gpt2 else oracle.argmax(lg)
        n += 1
        if time.perf_counter() - t0 > budget_s or n >= max_steps:
            break
    dt = time.perf_counter() - t0
    m.close()
    return n / dt, n, pre


def bench_cpu(pgw, oracle, budget_s):
    """The oracle (infer.js arithmetic in C, one thread) on the same model:
    prefill 32 tokens (timed for the reference-style n / totalMs), then time
    greedy decode steps for ~budget_s."""
    cfg = pgw.CONFIGS["smollm2-135m"]
    bundle = pgw.parse_pgw(pgw.make_llama(cfg, seed=0))
    prompt = [int(v) for v in np.random.default_rng(1).integers(0, cfg.vocab_size, 32)]
    rate, n, pre = cpu_decode_rate(oracle, bundle, budget_s, prompt=prompt)
    cpu, nproc = host_cpu()
    return {
        "value": round(rate, 3),
        "unit": "tok/s",
        "cores": 1,
        "kind": "port",
        "host_cpu": cpu,
        "host_nproc": nproc,
        # 128 tokens: the prompt's token, then 127 steps at the measured rate
        "ref_style_tok_s": round(128 / (pre + 127 / rate), 3),
        "prompt_ms": round(pre * 1e3, 1),
        "sample": f"135M Q4 greedy decode, {n} steps after a 32-token prompt, oracle/mllm_oracle.c "
                  f"(engine/infer.js fp64 arithmetic), 1 thread",
    }


# ---------------------------------------------------------------- GEMV sweep
def cpu_gemv_q4(oracle, pgw, m, n, budget_s=1.0):
    """The CPU baseline of config 2: the C restatement of kernels.rs gemv_q4
    (f32 accumulation in the reference's order, scalar, one thread) on a
    matrix of the shape; GB/s of the same algorithmic bytes."""
    rng = np.random.default_rng(m + n)
    packed, sc = pgw.quant_q4((rng.standard_normal((m, n)) * 0.02).astype(np.float32))
    x = rng.standard_normal(n).astype(np.float32)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.gemv_q4(packed, sc, x, mode="wasm")
        reps += 1
        if time.perf_counter() - t0 > budget_s:
            break
    us = (time.perf_counter() - t0) / reps * 1e6
    return {"us": round(us, 1), "gbs": round((m * n // 2 + m * n // 8 + 4 * n + 4 * m) / us / 1e3, 2), "reps": reps}


def graph_us(torch, enqueue, n_launch, replays=5):
    """Microseconds per launch of n_launch launches captured in one graph
    (enqueue(stream_handle) issues them), replayed `replays` times; the
    launches allocate nothing and clear nothing, so they capture as is."""
    cs = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        enqueue(C.c_void_p(cs.cuda_stream))
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (replays * n_launch)
    del g
    return round(us, 3)


def bench_gemv(torch, abi, pgw, oracle=None, quick=False):
    """Config 2's sweep.  quick: 20 warm launches, 40 cold ones over 40
    copies, 10 stacked ones and no graph replays -- for counter runs, where
    every launch is serialised and sampled (the per-launch counters do not
    depend on the repetition count)."""
    shapes = [(960, 960), (320, 960), (2560, 960), (960, 2560), (49152, 960)]
    stream = torch.cuda.current_stream()
    sp = C.c_void_p(stream.cuda_stream)
    rng = np.random.default_rng(2)
    out = []
    for fmt in ("q4", "q8g32"):
        for (m, n) in shapes:
            wbytes = m * n // 2 if fmt == "q4" else m * n
            sbytes = m * (n // 32) * 4
            algo = wbytes + sbytes + 4 * n + 4 * m
            copies = max(4, math.ceil((1 << 30) / (wbytes + sbytes)))
            if quick:
                copies = min(copies, 40)
            W = torch.randint(0, 256, (copies, wbytes), dtype=torch.uint8, device="cuda")
            S = torch.empty((copies, sbytes // 4), dtype=torch.float32, device="cuda").uniform_(1e-3, 1e-2)
            x = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda()
            y = torch.empty(m, dtype=torch.float32, device="cuda")

            def launch(i, s=sp):
                if fmt == "q4":
                    rc = abi.lib().mllm_gemv_q4(m, n, W[i].data_ptr(), S[i].data_ptr(), 32, x.data_ptr(),
                                                y.data_ptr(), s)
                else:
                    rc = abi.lib().mllm_gemv_q8_g32(m, n, W[i].data_ptr(), S[i].data_ptr(), x.data_ptr(),
                                                    y.data_ptr(), s)
                abi.check("gemv", rc)

            res = {"fmt": fmt, "shape": [m, n], "bytes": algo}
            for mode in ("warm", "cold"):
                reps = 200 if mode == "warm" else max(200, copies)  # cold: every copy once, >= 1 GiB
                if quick:
                    reps = 20 if mode == "warm" else copies
                for i in range(10):
                    launch(0 if mode == "warm" else i % copies)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for i in range(reps):
                    launch(0 if mode == "warm" else i % copies)
                e1.record(stream)
                e1.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / reps
                res[f"{mode}_us"] = round(us, 3)
                res[f"{mode}_gbs"] = round(algo / us / 1e3, 1)
            # the cold launches again, replayed from a captured graph: kernel
            # time without the host's per-call cost (ctypes, launch)
            if not quick:
                res["cold_graph_us"] = graph_us(torch, lambda s: [launch(i % copies, s) for i in range(reps)], reps)
                res["cold_graph_gbs"] = round(algo / res["cold_graph_us"] / 1e3, 1)
            batched = abi.lib().mllm_gemv_q4_batched if fmt == "q4" else abi.lib().mllm_gemv_q8_g32_batched
            # layer-stacked: 32 distinct matrices per launch
            cnt = 32
            groups = max(1, copies // cnt)
            tabs = []
            for gi in range(min(groups, 64)):
                idx = [(gi * cnt + j) % copies for j in range(cnt)]
                tp = torch.tensor([W[i].data_ptr() for i in idx], dtype=torch.int64, device="cuda")
                ts = torch.tensor([S[i].data_ptr() for i in idx], dtype=torch.int64, device="cuda")
                tx = torch.tensor([x.data_ptr()] * cnt, dtype=torch.int64, device="cuda")
                ys = torch.empty((cnt, m), dtype=torch.float32, device="cuda")
                ty = torch.tensor([ys[j].data_ptr() for j in range(cnt)], dtype=torch.int64, device="cuda")
                tabs.append((tp, ts, tx, ty, ys))
            reps = 10 if quick else 100
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            for i in range(3):
                tp, ts, tx, ty, _ = tabs[i % len(tabs)]
                abi.check("batched", batched(cnt, m, n, tp.data_ptr(), ts.data_ptr(), tx.data_ptr(),
                                             ty.data_ptr(), sp))
            e0.record(stream)
            for i in range(reps):
                tp, ts, tx, ty, _ = tabs[i % len(tabs)]
                abi.check("batched", batched(cnt, m, n, tp.data_ptr(), ts.data_ptr(), tx.data_ptr(),
                                             ty.data_ptr(), sp))
            e1.record(stream)
            e1.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / reps
            res["stacked32_us"] = round(us, 3)
            res["stacked32_gbs"] = round(cnt * algo / us / 1e3, 1)

            def stacked(s):
                for i in range(reps):
                    tp, ts, tx, ty, _ = tabs[i % len(tabs)]
                    abi.check("batched", batched(cnt, m, n, tp.data_ptr(), ts.data_ptr(), tx.data_ptr(),
                                                 ty.data_ptr(), s))
            if not quick:
                res["stacked32_graph_us"] = graph_us(torch, stacked, reps)
                res["stacked32_graph_gbs"] = round(cnt * algo / res["stacked32_graph_us"] / 1e3, 1)
            del tabs
            res["cold_frac_hbm"] = round(res["cold_gbs"] / HBM_PEAK_GBS, 4)
            if fmt == "q4" and oracle is not None:
                res["cpu_kernels_rs"] = cpu_gemv_q4(oracle, pgw, m, n)
            out.append(res)
            del W, S
            torch.cuda.empty_cache()
            log(f"[bench] gemv {fmt} {m}x{n}: {res}")
    return out


# ---------------------------------------------------------------- configs 3-5
def spans_prompt(rng, vocab, length, copy_frac=0.4):
    out = []
    while len(out) < length:
        n = int(rng.integers(8, 33))
        if out and rng.random() < copy_frac and len(out) > n:
            s = int(rng.integers(0, len(out) - n))
            out += out[s:s + n]
        else:
            out += [int(v) for v in rng.integers(0, vocab, n)]
    return out[:length]


def verify_pass_us(g, prompt, m, reps=20):
    """GPU time of one (k+1)-row verify pass of m tokens at the end of the
    prompt: the rows are a copy span of the prompt (forced drafts, so the pass
    is the full k+1 rows whatever the model would accept), rolled back after
    each pass."""
    g.forwardPrompt(prompt)
    base = g.cacheLen
    span = prompt[100:100 + m]
    times = []
    for _ in range(reps):
        g.forwardVerify(span)
        times.append(g.last_timing()[0])
        g.cacheLen = base
    return round(float(np.median(times)) * 1e3, 1)


def batched_pass_us(g, prompt, m, reps=20):
    """GPU time of the batched prompt path (matrix-core GEMMs) over the
    same m rows, as a prompt at position 0 (its lm_head forms the last row
    only): the matrix-core alternative to a verify pass of m rows.  Prompts
    of two tokens or more take that path by default."""
    times = []
    for _ in range(reps):
        g.forwardPrompt(prompt[100:100 + m])
        times.append(g.last_timing()[0])
    return round(float(np.median(times)) * 1e3, 1)


def bench_verify(mllm, pgw, args):
    """Config 3's verify passes alone (for kernel traces): M = 1, 5, 9 rows with
    forced drafts after a 512-token prompt, and the batched matrix-core path
    over the same rows."""
    cfg = pgw.CONFIGS["smollm2-135m"]
    g = mllm.PetitGPT(pgw.parse_pgw(pgw.make_llama(cfg, seed=0)), exec_mode=args.exec_mode)
    prompt = spans_prompt(np.random.default_rng(3), cfg.vocab_size, 512)
    out = {"workload": "smollm2-135m q4: verify passes of M rows after a 512-token prompt (forced drafts)",
           "exec_mode": g.execMode, "flow_verify_tokens": g.flowVerifyTokens}
    out["verify_pass_us"] = {}
    for m in (1, 2, 3, 4, 5, 9):
        out["verify_pass_us"][f"m{m}"] = verify_pass_us(g, prompt, m)
        log(f"[bench] verify M = {m}: {out['verify_pass_us'][f'm{m}']} us")
    out["batched_prompt_us"] = {f"m{m}": batched_pass_us(g, prompt, m) for m in (5, 9)}
    log(f"[bench] batched path: {out['batched_prompt_us']}")
    g.destroy()
    return out


def bench_configs(mllm, pgw, args, oracle=None):
    res = {}
    cpu_s = 0.0 if oracle is None else max(3.0, args.cpu_seconds / 3)
    # config 3: prompt-lookup speculation on the 135M shape
    cfg = pgw.CONFIGS["smollm2-135m"]
    bundle = pgw.parse_pgw(pgw.make_llama(cfg, seed=0))
    g = mllm.PetitGPT(bundle, exec_mode=args.exec_mode)
    prompt = spans_prompt(np.random.default_rng(3), cfg.vocab_size, 512)
    base = g.generate(prompt, maxNewTokens=256, mode="chain")
    base = g.generate(prompt, maxNewTokens=256, mode="chain")
    spec3 = {"prompt": 512, "new": 256, "chain_tok_s": round(255 / ((base["totalMs"] - base["ttftMs"]) / 1e3), 1)}
    for k in (4, 8):
        r = g.generate(prompt, maxNewTokens=256, mode="spec", specK=k)
        r = g.generate(prompt, maxNewTokens=256, mode="spec", specK=k)
        spec3[f"k{k}"] = {
            "tok_s": round(255 / ((r["totalMs"] - r["ttftMs"]) / 1e3), 1),
            "specHits": r["specHits"],
            "specTries": r["specTries"],
            "same_as_greedy": r["generatedIds"] == base["generatedIds"],
        }
    # the synthetic model's greedy output repeats one token, so lookupDraft
    # only finds 1-token drafts (the most recent match of the last 3 tokens
    # overlaps them); the verify pass itself at M = k + 1 rows, forced drafts:
    spec3["verify_pass_us"] = {f"m{m}": verify_pass_us(g, prompt, m) for m in (1, 5, 9)}
    spec3["note"] = ("greedy output of the synthetic model repeats one token: every draft is 1 token long; "
                     "verify_pass_us times M-row passes with forced drafts; full_drafts shows k at work")
    g.destroy()
    # beside the BASELINE workload: the same shape with a 12-token greedy cycle
    # (pgw.make_cycle_llama), the prompt holding the cycle once, so that
    # prompt-lookup drafts are full length and accepted: what k changes
    rng = np.random.default_rng(7)
    cycle = [int(v) for v in rng.choice(cfg.vocab_size, 12, replace=False)]
    gc = mllm.PetitGPT(pgw.parse_pgw(pgw.make_cycle_llama(cfg, cycle, seed=0)), exec_mode=args.exec_mode)
    cprompt = spans_prompt(np.random.default_rng(3), cfg.vocab_size, 512 - 14) + cycle + cycle[:2]
    cbase = gc.generate(cprompt, maxNewTokens=256, mode="chain")
    cbase = gc.generate(cprompt, maxNewTokens=256, mode="chain")
    full = {"model": "smollm2-135m shape, greedy output a 12-token cycle (pgw.make_cycle_llama)", "prompt": 512,
            "new": 256, "chain_tok_s": round(255 / ((cbase["totalMs"] - cbase["ttftMs"]) / 1e3), 1)}
    for k in (4, 8):
        r = gc.generate(cprompt, maxNewTokens=256, mode="spec", specK=k)
        r = gc.generate(cprompt, maxNewTokens=256, mode="spec", specK=k)
        full[f"k{k}"] = {"tok_s": round(255 / ((r["totalMs"] - r["ttftMs"]) / 1e3), 1),
                         "specHits": r["specHits"], "specTries": r["specTries"],
                         "accepted_per_pass": round(r["specHits"] / max(1, r["specTries"]), 2),
                         "same_as_greedy": r["generatedIds"] == cbase["generatedIds"]}
        log(f"[bench] spec full drafts k={k}: {full[f'k{k}']}")
    spec3["full_drafts"] = full
    gc.destroy()
    if oracle is not None:
        # the reference's CPU path has no speculation (it is in the GPU engine
        # only, webgpu.js:1239-1270): greedy decode at the prompt's context
        rate, n, _ = cpu_decode_rate(oracle, bundle, cpu_s, context=512)
        spec3["cpu"] = {"value": round(rate, 3), "unit": "tok/s", "cores": 1, "kind": "port",
                        "sample": f"{n} greedy decode steps from context 512 (cache length set directly; "
                                  "the reference CPU path has no speculation)"}
    res["spec_135m"] = spec3
    # config 4: GPT-2 124M, 16-token prompt, 256 tokens with argmaxGpt2
    cfg = pgw.CONFIGS["gpt2-124m"]
    g = mllm.PetitGPT(pgw.parse_pgw(pgw.make_gpt2(cfg, seed=0)), exec_mode=args.exec_mode)
    prompt = [int(v) for v in np.random.default_rng(4).integers(0, cfg.vocab_size, 16)]
    r = g.generate(prompt, maxNewTokens=256, mode="chain")
    r = g.generate(prompt, maxNewTokens=256, mode="chain")
    res["gpt2_124m"] = {"decode_tok_s": round(255 / ((r["totalMs"] - r["ttftMs"]) / 1e3), 1),
                        "ttft_ms": round(r["ttftMs"], 2), "distinct_ids": len(set(r["generatedIds"])),
                        "ref_style_tok_s": round(len(r["generatedIds"]) / (r["totalMs"] / 1e3), 1)}
    if oracle is not None:
        rate, n, pre = cpu_decode_rate(oracle, g.bundle, cpu_s, prompt=prompt, gpt2=True)
        res["gpt2_124m"]["cpu"] = {"value": round(rate, 3), "unit": "tok/s", "cores": 1, "kind": "port",
                                   "ref_style_tok_s": round(256 / (pre + 255 / rate), 3),
                                   "sample": f"{n} decode steps (argmaxGpt2) after the 16-token prompt"}
    g.destroy()
    # config 5: 362M, fp16 KV, 1536-token prefill then 512 decode steps to 2048
    cfg = pgw.CONFIGS["smollm2-360m"]
    g = mllm.PetitGPT(pgw.parse_pgw(pgw.make_llama(cfg, seed=0)), kv_fp16=True, exec_mode=args.exec_mode)
    prompt = [int(v) for v in np.random.default_rng(5).integers(0, cfg.vocab_size, 1536)]
    # the prompt through the 16-token passes of the decode phases (the path
    # shorter prompts take), then the batched path twice (the second is timed)
    g.set_prefill(0)
    t0 = time.perf_counter()
    g.forwardPrompt(prompt)
    pass_s = time.perf_counter() - t0
    g.set_prefill(64)
    g.forwardPrompt(prompt)
    t0 = time.perf_counter()
    g.forwardPrompt(prompt)
    ttft = time.perf_counter() - t0
    prefill_gpu_ms, _ = g.last_timing()
    first = g.last_argmax
    # the same prompt four times more (a server taking prompts back to back):
    # GPU times of the five batched runs, the first being the one above
    runs = [prefill_gpu_ms]
    for _ in range(4):
        g.forwardPrompt(prompt)
        runs.append(g.last_timing()[0])
    first = g.last_argmax  # the chain below starts from the last run's cache and token
    t0 = time.perf_counter()
    ids = g.decodeChain(first, 511)
    dt = time.perf_counter() - t0
    chain_ms, n = g.last_timing()
    # step i of the chain attends over 1537 + i cached positions
    chain_bytes = sum(token_bytes(cfg, 1537 + i, 2) for i in range(n))
    rec = traffic_record("k_flow3_360m_fp16kv")
    achieved = chain_bytes / (chain_ms * 1e-3) / 1e9
    res["smollm2_360m_fp16kv"] = {"prefill_ms": round(ttft * 1e3, 2), "prefill_gpu_ms": round(prefill_gpu_ms, 2),
                                  "prefill_gpu_ms_runs": [round(v, 3) for v in runs],
                                  "prefill_gpu_ms_median": round(float(np.median(runs)), 2),
                                  "prefill_tok_s": round(1536 / ttft, 1),
                                  "prefill_pass_path_ms": round(pass_s * 1e3, 1),
                                  "decode_tok_s": round(len(ids) / dt, 1),
                                  "decode_roofline": {
                                      "bound": "hbm", "kernel": f"{g.decodeKernel} (one launch = the 511-step chain)",
                                      "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                      "frac": round(achieved / HBM_PEAK_GBS, 5),
                                      "traffic": None if rec is None else int(rec["hbm_bytes_per_step"] * n),
                                      "bytes_per_launch": int(chain_bytes), "us_per_launch": round(chain_ms * 1e3, 1)}}
    if oracle is not None:
        # the oracle keeps an f32 cache (the reference's); 1536 prompt tokens
        # would take minutes, so the cache length is set to 1792 directly
        rate, n, _ = cpu_decode_rate(oracle, g.bundle, cpu_s, context=1792, max_steps=64)
        res["smollm2_360m_fp16kv"]["cpu"] = {"value": round(rate, 3), "unit": "tok/s", "cores": 1, "kind": "port",
                                             "sample": f"{n} decode steps from context 1792 (f32 cache, length set "
                                                       "directly; the 1536-token prompt is not run on the CPU)"}
    g.destroy()
    return res


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=127, help="decode steps timed (tokens 2..K+1)")
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--exec-mode", type=int, default=3, choices=(1, 2, 3, 4),
                    help="3 persistent kernel (default), 1 graph replay, 2 direct launches, "
                         "4 persistent kernel through an ordinary launch (for profilers)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-configs", action="store_true")
    ap.add_argument("--prefill-only", action="store_true", help="config 5's prompt, batched, three times")
    ap.add_argument("--sweep-only", action="store_true",
                    help="only the Q4 / Q8 GEMV sweep (config 2), no decode and no cooperative launch")
    ap.add_argument("--sweep-quick", action="store_true",
                    help="the sweep with few launches per shape and no graph replays (counter runs)")
    ap.add_argument("--verify-only", action="store_true",
                    help="only config 3's verify passes at M = 1, 5, 9 (and the batched path at M = 5, 9)")
    ap.add_argument("--decode-360m", action="store_true",
                    help="only config 5's decode: the 1536-token prompt (batched), then one chained decode of 511 "
                         "steps to 2048 context (one persistent-kernel dispatch; the traffic record behind it)")
    ap.add_argument("--kinds-only", action="store_true",
                    help="only config 1's workload with Q8 / f16 / bf16 / f32 matrices (the kind-generic step)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device copy (counter calibration for the traffic figure)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the decode step is batch-1 on one device; data-parallel sequences would each run their own", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.steps + args.warmup + 40 > 2048:
        print("--steps/--warmup out of range for a 2048 context", file=sys.stderr)
        sys.exit(2)

    import torch

    import mllm
    from mllm import abi, pgw

    abi.lib()
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if args.copy_calibration:
        copy_calibration(torch)
        return
    if args.sweep_only or args.sweep_quick:
        print(json.dumps({"gemv_sweep": bench_gemv(torch, abi, pgw, quick=args.sweep_quick)}))
        return
    if args.verify_only:
        print(json.dumps(bench_verify(mllm, pgw, args)))
        return
    if args.kinds_only:
        print(json.dumps({"kinds_135m": bench_kinds(mllm, pgw)}))
        return
    if args.prefill_only:
        cfg = pgw.CONFIGS["smollm2-360m"]
        g = mllm.PetitGPT(pgw.parse_pgw(pgw.make_llama(cfg, seed=0)), kv_fp16=True, exec_mode=args.exec_mode)
        prompt = [int(v) for v in np.random.default_rng(5).integers(0, cfg.vocab_size, 1536)]
        runs = []
        for _ in range(3):
            g.forwardPrompt(prompt)
            runs.append(round(g.last_timing()[0], 3))
            log(f"[bench] prefill 1536 tokens: {runs[-1]} ms (GPU)")
        g.destroy()
        print(json.dumps({"prefill_gpu_ms": runs, "tokens": 1536, "workload": "smollm2-360m fp16 KV (config 5)"}))
        return
    if args.decode_360m:
        cfg = pgw.CONFIGS["smollm2-360m"]
        g = mllm.PetitGPT(pgw.parse_pgw(pgw.make_llama(cfg, seed=0)), kv_fp16=True, exec_mode=args.exec_mode)
        prompt = [int(v) for v in np.random.default_rng(5).integers(0, cfg.vocab_size, 1536)]
        g.forwardPrompt(prompt)
        kname = g.decodeKernel
        ids = g.decodeChain(g.last_argmax, 511)
        ms, n = g.last_timing()
        chain_bytes = sum(token_bytes(cfg, 1537 + i, 2) for i in range(n))
        g.destroy()
        print(json.dumps({"workload": "smollm2-360m q4, fp16 KV: 511 chained decode steps after a 1536-token prompt "
                                      "(config 5)", "kernel": kname, "exec_mode": args.exec_mode, "steps": n,
                          "gpu_ms": round(ms, 3), "us_per_step": round(ms * 1e3 / n, 2),
                          "tok_s": round(n / (ms * 1e-3), 1), "algorithmic_bytes_per_step": int(chain_bytes / n),
                          "first_ids": ids[:6]}))
        return
    dec = bench_decode(mllm, pgw, torch, args)
    log(f"[bench] decode {dec['value']:.1f} tok/s, phases {dec['phase_us']}")
    line = {
        "metric": METRIC,
        "value": round(dec["value"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "precision": {"weights": "q4 group-32 nibbles, f32 scales (PGW1)",
                      "activations": "24-bit integers per 32-element group, rounding <= 6.4e-8 x the group's "
                                     "max |x| (one f32 rounding of its largest element)",
                      "accumulation": "exact int32 per group, f32 across groups",
                      "measured": "decode logits within 2e-6 x max|logit| of the fp64 oracle (tests)"},
        "data": "synthetic: N(0,0.02) weights (seed 0) quantised by quant_q4; 32 prompt ids uniform (seed 1)",
        "config": {"workload": "smollm2-135m-q4 greedy decode, 32-token prompt, batch 1 (BASELINE config 1)",
                   "weights": "q4 group-32 (PGW1)", "exec_mode": dec["exec_mode"], "kv_cache": "f32",
                   "norm_eps": 1e-6,
                   "norm_eps_note": "the reference's constant (infer.js:8); BASELINE config 1 states 1e-5"},
        "roofline": dec["roofline"],
        "kernel_ms_per_step": round(dec["kernel_ms_per_step"], 4),
        "phase_us": dec["phase_us"],
        "decode_step_gbs": dec["decode_step_gbs"],
        "decode_step_bytes": dec["decode_step_bytes"],
        "host_loop_tok_s": dec["host_loop_tok_s"],
        "ref_style_tok_s": dec["ref_style_tok_s"],
        "ttft_ms": dec["ttft_ms"],
    }
    oracle = None if args.no_cpu else __import__("oracle")
    if oracle is not None:
        line["cpu_baseline"] = bench_cpu(pgw, oracle, args.cpu_seconds)
        line["speedup_vs_cpu"] = round(line["value"] / line["cpu_baseline"]["value"], 1)
    if not args.no_sweep:
        sweep = bench_gemv(torch, abi, pgw, oracle)
        line["gemv_sweep"] = sweep
        best = max(r["cold_gbs"] for r in sweep if r["fmt"] == "q4")
        line["gemv_q4_best_cold_frac_hbm"] = round(best / HBM_PEAK_GBS, 4)
        lm = next(r for r in sweep if r["fmt"] == "q4" and r["shape"] == [49152, 960])
        line["gemv_roofline"] = {"bound": "hbm", "kernel": "k_gemv_q4 (49152 x 960, cold)",
                                 "achieved": lm["cold_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                 "frac": lm["cold_frac_hbm"], "bytes_per_launch": lm["bytes"],
                                 "us_per_launch": lm["cold_us"]}
    if not args.no_configs:
        line["configs"] = bench_configs(mllm, pgw, args, oracle)
        line["configs"]["kinds_135m"] = bench_kinds(mllm, pgw)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
