#!/usr/bin/env python3
"""Benchmark of the GPU forward pass on one MI355X.

Workload: a seeded random-init Qwen2.5-0.5B-shaped qwen2
model (24 layers, hidden 896, 14/2 heads, FFN 4864, vocab 151936, Q4_0 layers
and embedding, Q8_0 output matrix), a 128-token prompt in 64-token prefill
chunks, 128 greedy tokens at 8 tokens per submit, context 512, f32 KV cache.
One step is one `bench` round of the reference (examples/generate/main.go:183-207):
Generate(prompt, 128) with eos -1; `value` is decode tok/s over the K timed
rounds (prefill tok/s reported beside it).  Inputs are resident in HBM before
the timed region (the model is loaded once).

Also measured: the device time of each launch of a decode step (the fused
pass that runs every layer, the head, the sampling kernel: HIP events on the
model's stream around eager steps) for the roofline of the dominant kernel,
whose duration comes from the committed kernel trace of these sources when
there is one; the one-launch-per-phase kernels (prefill, the fallback,
config 4's decode) back to back; the isolated GEMV sweep
with weights read from HBM (rotated copies > 512 MB) and warm; and the CPU
oracle (a C restatement of the reference's cpu.go) timed on this host's
cores.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_MFMA_F16_TFLOPS = 2500.0  # dense f16/bf16
METRIC = "decode & prefill tok/s at Qwen2.5-0.5B shape; Q4_0 GEMV HBM GB/s vs peak"
SWEEP = [(576, 576), (1536, 576), (576, 1536), (896, 896), (4864, 896), (896, 4864), (151936, 896)]
# HBM bytes per launch measured by rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
# runs of this script, scaled by the same counters on a copy of known size
PMC_SUMMARY = os.path.join(ROOT, "profiles", "pmc_decode_qwen25.txt")


def kernel_symbols(attn_full):
    """Device symbol of each decode kernel class of the config-3 model (Q4_0
    layers, Q8_0 head): the fused pass pass_kernel<head size, binary16 cache,
    Q8_0 matrices, long form>, the sampling kernel, and for one launch per phase
    gemv_kernel<type, tokens, prologue, epilogue, units
    per staging batch> (K1 after layer 0 adds the previous down projection's
    two k-halves, prologue 65; K5 before the last layer stores those halves,
    epilogue 0, three block groups per wave: four per staging batch), the
    one-chunk or split attention, the streaming head <type,
    prologue, epilogue, groups per tile>."""
    return {"pass": "pass_kernel<64u, false, false, false>", "argmax": "argmax_kernel<2u>",
            "k1": "gemv_kernel<2u, 1, 65, 2, 2>",
            "k2": "attn_kernel<64u, 8u, false, false, false>" if attn_full else
                  "attn_kernel<64u, 8u, true, false, false>",
            "k3": "gemv_kernel<2u, 1, 0, 1, 2>", "k4": "gemv_kernel<2u, 1, 1, 3, 2>", "k5": "gemv_kernel<2u, 1, 0, 0, 4>",
            "head": "gemv_stream_kernel<8u, 1, 4, 7>"}


def pmc_value(kind, cls):
    """A figure of a decode kernel class from the committed rocprofv3 summary
    (lines `traffic_bytes <class> <bytes>`: HBM bytes per launch from the
    FETCH_SIZE / WRITE_SIZE runs; `duration_us <class> <us>`: the kernel
    trace's median duration), if that summary measured the kernel sources of
    this tree (its `sources_hash` line against llm_amd.profsum.sources_hash()).
    A stale figure is not reported: (None, reason)."""
    from llm_amd import profsum
    want, got, value = profsum.sources_hash(), None, None
    try:
        with open(PMC_SUMMARY) as f:
            for line in f:
                p = line.split()
                if len(p) == 2 and p[0] == "sources_hash":
                    got = p[1]
                if len(p) == 3 and p[0] == kind and p[1] == cls:
                    value = float(p[2]) if kind == "duration_us" else int(p[2])
    except OSError:
        return None, "no counter summary"
    if got != want:
        return None, f"{os.path.relpath(PMC_SUMMARY, ROOT)} measured sources {got}, this tree is {want}"
    return value, f"{os.path.relpath(PMC_SUMMARY, ROOT)} (sources {got})"


def copy_calibration():
    """A plain 256 MiB device-to-device copy (the runtime's copy kernel,
    __amd_rocclr_copyBuffer): the known-size reference for the FETCH_SIZE /
    WRITE_SIZE counters."""
    from llm_amd import kernels
    kernels.copy_calibration(256 << 20)
    log(f"copy calibration: {256 << 20} bytes read, {256 << 20} bytes written")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def generation(args):
    from llm_amd import kernels, llm, synth
    spec = synth.qwen25(seed=0)
    t0 = time.time()
    path = synth.cached(spec)
    log(f"model file {path} ready in {time.time() - t0:.1f}s")
    t0 = time.time()
    g = llm.NewGPU(0, None, path, args.ctx)
    log(f"load: {time.time() - t0:.2f}s, GPU memory {g.MemoryUsed()} bytes")
    prompt = list(synth.prompt(0, args.prompt, spec.vocab))
    for i in range(args.warmup):
        tm = g.Generate(prompt, args.gen, -1)
        log(f"warmup {i}: prefill {tm.PromptTokens / tm.Prefill:.1f} tok/s, decode {tm.Generated / tm.Decode:.1f} tok/s")
    kernels.synchronize()
    rounds = []
    t0 = time.perf_counter()
    for i in range(args.steps):
        tm = g.Generate(prompt, args.gen, -1)
        rounds.append(tm)
        log(f"round {i}: prefill {tm.PromptTokens / tm.Prefill:.1f} tok/s, decode {tm.Generated / tm.Decode:.1f} "
            f"tok/s ({tm.Dispatches} dispatches)")
    kernels.synchronize()
    wall = time.perf_counter() - t0
    dec = sum(r.Generated for r in rounds) / sum(r.Decode for r in rounds)
    pre = sum(r.PromptTokens for r in rounds) / sum(r.Prefill for r in rounds)
    per_round = {
        "prefill_tok_s": {"median": statistics.median(r.PromptTokens / r.Prefill for r in rounds),
                          "min": min(r.PromptTokens / r.Prefill for r in rounds),
                          "max": max(r.PromptTokens / r.Prefill for r in rounds)},
        "decode_tok_s": {"median": statistics.median(r.Generated / r.Decode for r in rounds),
                         "min": min(r.Generated / r.Decode for r in rounds),
                         "max": max(r.Generated / r.Decode for r in rounds)},
    }
    # device times of a decode step's launches (the fused pass, the head, the
    # sampling kernel): HIP events on the model's stream around each launch of
    # eager decode steps at the positions after the timed rounds
    g.Generate(prompt, 1, -1)
    agg = {}
    for _ in range(args.profile_steps):
        per = {}
        for c, _layer, b, us in g.profile(2):
            per.setdefault(c, []).append((b, us))
        for c, v in per.items():
            a = agg.setdefault(c, {"n": len(v), "us": [], "bytes": []})
            a["us"].append(sum(u for _, u in v) / len(v))
            a["bytes"].append(sum(b for b, _ in v) / len(v))
    syms = kernel_symbols(args.prompt + 1 < 256)
    classes = {}
    for c, a in agg.items():
        us, nbytes = statistics.mean(a["us"]), int(statistics.mean(a["bytes"]))
        classes[c] = {"launches_per_token": a["n"], "avg_us": round(us, 3), "bytes": nbytes,
                      "us_per_token": round(us * a["n"], 2), "gbps": round(nbytes / us * 1e-3, 1) if nbytes else None,
                      "symbol": syms.get(c)}
    step_kernel_us = sum(c["us_per_token"] for c in classes.values())
    # the dominant kernel: the class with the most device time per decode token;
    # frac from the profiler's duration of that kernel (the committed kernel
    # trace of this tree's sources), the HIP-event figure beside it
    dom = max(classes, key=lambda k: classes[k]["us_per_token"])
    d = classes[dom]
    traced_us, tsource = pmc_value("duration_us", dom)
    traffic, source = pmc_value("traffic_bytes", dom)
    dur = traced_us if traced_us else d["avg_us"]
    achieved = d["bytes"] / dur * 1e-3
    roofline = {"bound": "hbm", "kernel": dom, "symbol": syms.get(dom), "achieved": round(achieved, 1),
                "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                "traffic": traffic, "traffic_source": source, "bytes_per_launch": d["bytes"],
                "duration_us": dur, "duration_source": tsource if traced_us else "HIP events (no current trace)",
                "event_us": d["avg_us"], "event_achieved": round(d["bytes"] / d["avg_us"] * 1e-3, 1)}
    if dom == "pass":
        roofline["note"] = ("one launch runs every layer of the step: its phases hand their results to each other "
                            "through flag-carrying words, five dependent hand-offs per layer, so the launch is "
                            "bound by that chain's latency, not by HBM (algorithmic bytes: every layer matrix once "
                            "and the KV rows attended)")
    # the kernels of one launch per phase (prefill, the decode fallback, and
    # the long-context decode, which the fused pass does not take): each class
    # launched back to back across the 24 layers between HIP events
    unfused = {}
    per_tok = {"k1": spec.layers, "k2": spec.layers, "k3": spec.layers, "k4": spec.layers, "k5": spec.layers}
    for cls, n in per_tok.items():
        us, nbytes = g.bench_kernel(cls, 240)
        unfused[cls] = {"launches_per_token": n, "avg_us": round(us, 3), "bytes": nbytes,
                        "us_per_token": round(us * n, 2), "gbps": round(nbytes / us * 1e-3, 1) if nbytes else None,
                        "symbol": syms[cls]}
    dispatches = round(sum(r.Dispatches for r in rounds) / max(1, sum(r.Generated for r in rounds)), 1)
    return g, {
        "value": dec, "prefill": pre, "wall": wall, "rounds": per_round, "ms_per_step": wall / args.steps * 1e3,
        "classes": classes, "unfused": unfused, "step_kernel_us": step_kernel_us, "roofline": roofline,
        "dispatches_per_token": dispatches,
    }


MFMA_SUMMARY = os.path.join(ROOT, "profiles", "mfma_util_qwen25.md")


def prefill_counter():
    """The prefill products' MFMA busy fraction from the committed rocprofv3
    counter summary (rocprofv3's MfmaUtil over every gemm_kernel dispatch),
    if it measured this tree's sources: (percent or None, source)."""
    from llm_amd import profsum
    want, got, value = profsum.sources_hash(), None, None
    try:
        with open(MFMA_SUMMARY) as f:
            for line in f:
                p = line.split()
                if len(p) == 2 and p[0] == "sources_hash":
                    got = p[1]
                if len(p) == 2 and p[0] == "prefill_gemm_mfma_util":
                    value = float(p[1])
    except OSError:
        return None, "no counter summary"
    if got != want:
        return None, f"{os.path.relpath(MFMA_SUMMARY, ROOT)} measured sources {got}, this tree is {want}"
    return value, f"{os.path.relpath(MFMA_SUMMARY, ROOT)} (sources {got})"


def prefill_roofline(tok_s):
    """MFMA utilisation of the prefill chunks: the layers'
    matrix FLOPs (2 per weight per token) at the measured prefill rate, against
    MI355X's dense f16 MFMA peak, and beside it the counter figure: the MFMA
    busy fraction of the products while they run."""
    from llm_amd import synth
    s = synth.qwen25(seed=0)
    kvd = s.kv_heads * (s.embd // s.heads)
    per_token = 2 * s.layers * (s.embd * (s.embd + 2 * kvd) + s.embd * s.embd + 3 * s.ff * s.embd)
    achieved = per_token * tok_s * 1e-12
    busy, source = prefill_counter()
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_MFMA_F16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_MFMA_F16_TFLOPS, 5), "flops_per_token": per_token,
            "gemm_mfma_busy_pct": busy, "gemm_mfma_busy_source": source,
            "note": "layer matrix FLOPs over the whole prefill time (prep, attention and the head included); the "
                    "products run on v_mfma_f32_16x16x32_f16 with each activation split into two f16 rows, so the "
                    "MFMA units execute twice these FLOPs"}


def loader(args):
    """The loader's fast path (llm_new_gpu: runs of consecutive tensors read by
    parallel pread straight into pinned staging, one DMA per run on its own
    stream, the repack on the device) for the config-3 file from the page
    cache, against the pinned host-to-device copy rate measured here."""
    from llm_amd import kernels, llm, synth
    path = synth.cached(synth.qwen25(seed=0))
    f = llm.Parse(path)
    tensor_bytes = sum(t.Size for t in f.Tensors)
    f.close()
    ts = []
    for i in range(6):
        t0 = time.perf_counter()
        g = llm.NewGPU(0, None, path, args.ctx)
        ts.append(time.perf_counter() - t0)
        g.close()
    ts = sorted(ts[1:])
    h2d = kernels.bench_h2d(64 << 20, 10)
    med = ts[len(ts) // 2]
    res = {"seconds": round(med, 5), "min_seconds": round(ts[0], 5), "tensor_bytes": tensor_bytes,
           "gb_s": round(tensor_bytes / med * 1e-9, 2), "h2d_pinned_gb_s": round(h2d, 2),
           "frac_of_h2d": round(tensor_bytes / med * 1e-9 / h2d, 3),
           "note": "NewGPU of the config-3 GGUF, file in the page cache, median of 5 after one untimed load; "
                   "the bound is the pinned host-to-device rate (64 MiB copies)"}
    log(f"loader: {med * 1e3:.1f} ms for {tensor_bytes} tensor bytes = {res['gb_s']} GB/s "
        f"(pinned H2D {res['h2d_pinned_gb_s']} GB/s)")
    return res


def long_context(args):
    """2048-token prompt (32 chunks), 512 greedy tokens, ctx 4096, mixed types."""
    from llm_amd import llm, synth
    spec = synth.qwen25_mixed(seed=0)
    g = llm.NewGPU(0, None, synth.cached(spec), 4096)
    prompt = list(synth.prompt(0, 2048, spec.vocab))
    g.Generate(prompt, 512, -1)  # round 0, dropped (as the reference's bench drops it): graphs built
    tm = g.Generate(prompt, 512, -1)
    # the decode step's launches at the last positions (the fused pass's long form)
    fused = {}
    for _ in range(4):
        for c, _layer, b, u in g.profile(2):
            f = fused.setdefault(c, {"us": [], "bytes": b})
            f["us"].append(u)
    fused = {c: {"avg_us": round(statistics.mean(f["us"]), 3), "bytes": f["bytes"],
                 "gbps": round(f["bytes"] / statistics.mean(f["us"]) * 1e-3, 1) if f["bytes"] else None}
             for c, f in fused.items()}
    us, nbytes = g.bench_kernel("k2", 96)
    classes = {}
    for cls in ("k1", "k3", "k4", "k5", "head"):
        cu, cb = g.bench_kernel(cls, 96 if cls != "head" else 20)
        classes[cls] = {"avg_us": round(cu, 3), "bytes": cb, "gbps": round(cb / cu * 1e-3, 1)}
    g.close()
    res = {"workload": "BASELINE config 4: qwen2.5-0.5b shape, Q4_1 ffn_down on odd layers, Q8_0 head, 2048-token "
                       "prompt, 512 greedy tokens, ctx 4096",
           "prefill_tok_s": round(tm.PromptTokens / tm.Prefill, 1), "decode_tok_s": round(tm.Generated / tm.Decode, 1),
           "decode_step_at_end": fused,
           "attention_at_end": {"avg_us": round(us, 2), "kv_bytes": nbytes, "gbps": round(nbytes / us * 1e-3, 1),
                                "note": "one launch per phase (the fallback): the split attention kernel (chunks of "
                                        "256 rows); their merge runs in the output projection's prologue, so "
                                        "classes_at_end.k3 carries it (k3 merges nothing at config 3: "
                                        "decode_step.unfused_classes.k3)"},
           "classes_at_end": classes}
    log(f"long context: prefill {res['prefill_tok_s']} tok/s, decode {res['decode_tok_s']} tok/s, "
        f"attention {us:.1f} us for {nbytes} KV bytes")
    return res


def sweep(args):
    """Config 1: each shape's launches back to back in a hipGraph (captured
    once, replayed), over rotated copies > 640 MB for HBM and one copy for the
    warm figure; with LLMHIP_EAGER=1 (kernel tracing) as stream launches."""
    import numpy as np
    from llm_amd import kernels, synth
    graph = os.environ.get("LLMHIP_EAGER", "") not in ("1", "true")
    out = []
    for qtype, tname in ((kernels.Q4_0, "q4_0"), (kernels.Q8_0, "q8_0")):
        for rows, k in SWEEP:
            rng = np.random.default_rng([1, rows, k, qtype])
            m = kernels.QMat(qtype, rows, k, synth.quant_blocks(qtype, rows, k, rng, q8_div=8.0))
            x = kernels.DeviceBuffer.from_numpy(np.random.default_rng([2, rows, k]).standard_normal((1, k), np.float32))
            y = kernels.DeviceBuffer(rows * 4)
            nbytes = m.gguf_bytes
            warm = kernels.bench([m], x, y, 1, iters=200, warmup=20, graph=graph)
            copies = [m] + [m.clone() for _ in range(min(4095, max(0, -(-args.hbm_bytes // nbytes) - 1)))]
            iters = max(len(copies), 200)
            hbm = kernels.bench(copies, x, y, 1, iters=iters, warmup=len(copies), graph=graph)
            stream = kernels.bench(copies, x, y, 1, iters=iters, warmup=len(copies))
            out.append({"type": tname, "rows": rows, "k": k, "n": 1, "bytes": nbytes,
                        "hbm_us": round(hbm, 3), "hbm_gbps": round(nbytes / hbm * 1e-3, 1),
                        "hbm_frac": round(nbytes / hbm * 1e-3 / PEAK_HBM_GBS, 4), "copies": len(copies),
                        "warm_us": round(warm, 3), "warm_gbps": round(nbytes / warm * 1e-3, 1),
                        "launch": "graph" if graph else "stream", "stream_hbm_us": round(stream, 3)})
            log(f"gemv {tname} {rows}x{k}: HBM {out[-1]['hbm_gbps']} GB/s ({out[-1]['hbm_frac']:.1%}) over "
                f"{len(copies)} copies, warm {out[-1]['warm_gbps']} GB/s")
            # prefill-chunk token counts: the activation prep and the product
            # (one launch pair) over the same rotated copies
            for n in (8, 64):
                xn = kernels.DeviceBuffer.from_numpy(
                    np.random.default_rng([3, n, k]).standard_normal((n, k), np.float32))
                yn = kernels.DeviceBuffer(n * rows * 4)
                us = kernels.bench(copies, xn, yn, n, iters=iters, warmup=len(copies), graph=graph)
                tf = 2.0 * rows * k * n / us * 1e-6
                out.append({"type": tname, "rows": rows, "k": k, "n": n, "bytes": nbytes, "hbm_us": round(us, 3),
                            "hbm_gbps": round(nbytes / us * 1e-3, 1),
                            "hbm_frac": round(nbytes / us * 1e-3 / PEAK_HBM_GBS, 4), "copies": len(copies),
                            "tflops": round(tf, 2), "mfma_frac": round(tf / PEAK_MFMA_F16_TFLOPS, 5)})
                log(f"gemm {tname} {rows}x{k} n={n}: {us:.2f} us (prep + product), {tf:.1f} TFLOP/s, "
                    f"weights {out[-1]['hbm_gbps']} GB/s")
                xn.close()
                yn.close()
            for c in copies:
                c.close()
            x.close()
            y.close()
            kernels.synchronize()
    return out


def one_gemv(spec, hbm_bytes):
    """One sweep shape alone (the --gemv option), TYPE:ROWSxK[:N]: the same
    rotated copies and stream launches as the sweep's stream figure, so that a
    profiler's kernel trace and counters cover exactly these launches."""
    import numpy as np
    from llm_amd import kernels, synth
    spec = spec.split(":")
    types = {"q4_0": kernels.Q4_0, "q8_0": kernels.Q8_0, "q4_1": kernels.Q4_1}
    qtype = types[spec[0]]
    rows, k = (int(v) for v in spec[1].split("x"))
    n = int(spec[2]) if len(spec) > 2 else 1
    rng = np.random.default_rng([1, rows, k, qtype])
    m = kernels.QMat(qtype, rows, k, synth.quant_blocks(qtype, rows, k, rng, q8_div=8.0))
    x = kernels.DeviceBuffer.from_numpy(np.random.default_rng([2, rows, k]).standard_normal((n, k), np.float32))
    y = kernels.DeviceBuffer(n * rows * 4)
    nbytes = m.gguf_bytes
    copies = [m] + [m.clone() for _ in range(min(4095, max(0, -(-hbm_bytes // nbytes) - 1)))]
    iters = max(len(copies), 100)
    us = kernels.bench(copies, x, y, n, iters=iters, warmup=len(copies))
    log(f"gemv {spec[0]} {rows}x{k} n={n}: {us:.2f} us over {len(copies)} copies")
    out = {"type": spec[0], "rows": rows, "k": k, "n": n, "bytes": nbytes, "copies": len(copies),
           "launches": iters + len(copies), "stream_us": round(us, 3), "gbps": round(nbytes / us * 1e-3, 1)}
    for c in copies:
        c.close()
    x.close()
    y.close()
    return out


def _cpu_model():
    """The host CPU's model name (lscpu's "Model name", from /proc/cpuinfo)."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _oracle_decode(cpu, prompt, seconds, ctx):
    """(prefill tok/s over the prompt, decode tok/s, decode tokens) of the
    oracle, decoding greedily for about `seconds` after the prompt."""
    from oracle import cpuref
    t0 = time.perf_counter()
    for t in prompt:
        logits = cpu.forward(t)
    pre = len(prompt) / (time.perf_counter() - t0)
    n = 0
    t0 = time.perf_counter()
    while (time.perf_counter() - t0 < seconds or n < 4) and len(prompt) + n < ctx:
        logits = cpu.forward(cpuref.argmax(logits))
        n += 1
    return pre, n / (time.perf_counter() - t0), n


def cpu_baseline(args):
    """The CPU oracle (the C restatement of cpu.go, -O2 -ffp-contract=off) on
    a bounded sample of the same workload: single-threaded, as cpu.go's
    Forward runs on one goroutine (cpu.go:225) -- the `value` -- and
    row-parallel over the host's cores (bit-identical results) beside it."""
    from llm_amd import synth
    from oracle import cpuref
    spec = synth.qwen25(seed=0)
    path = synth.cached(spec)
    prompt = list(synth.prompt(0, 8, spec.vocab))
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = min(affinity or 1, int(os.environ.get("OMP_NUM_THREADS", "16")), 16)
    cpu = cpuref.CPU(path, args.ctx, threads=1)
    pre1, dec1, n1 = _oracle_decode(cpu, prompt, args.cpu_seconds, args.ctx)
    cpu.close()
    cpu = cpuref.CPU(path, args.ctx, threads=threads)
    pre, dec, n = _oracle_decode(cpu, prompt, args.cpu_seconds, args.ctx)
    cpu.close()
    log(f"cpu oracle: 1 thread decode {dec1:.2f} tok/s ({n1} tokens); {threads} threads decode {dec:.2f} tok/s "
        f"({n} tokens); host {_cpu_model()}, {os.cpu_count()} CPUs, {affinity} in this process's affinity")
    return {"value": round(dec1, 3), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"qwen2.5-0.5b shape (the same seeded model), 8 prompt tokens then {n1} greedy decode tokens "
                      f"(~{args.cpu_seconds:.0f}s) on one thread, decode tok/s",
            "prefill_tok_s": round(pre1, 3),
            "row_parallel": {"value": round(dec, 3), "unit": "tok/s", "cores": threads, "prefill_tok_s": round(pre, 3),
                             "sample": f"the same, {n} decode tokens, matvec rows and attention heads over "
                                       f"{threads} threads"},
            "host": {"cpu_model": _cpu_model(), "nproc": os.cpu_count(), "affinity": affinity}}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--gen", type=int, default=128)
    ap.add_argument("--ctx", type=int, default=512)
    ap.add_argument("--hbm-bytes", type=int, default=640 << 20, help="rotated copies per sweep shape")
    ap.add_argument("--profile-steps", type=int, default=12, help="eager decode steps timed per launch")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-long", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--copy-calibration", action="store_true", help="only run the counter calibration copy")
    ap.add_argument("--gemv", metavar="TYPE:ROWSxK[:N][,...]",
                    help="only these sweep shapes (q4_0 / q8_0 / q4_1), in order, each over rotated copies with "
                         "stream launches, for a profiler: e.g. q4_0:151936x896,q8_0:896x896:64")
    args = ap.parse_args()
    if args.gpus != 1:
        log("bench.py: this build measures one GPU; the path shards by independent sequences, one "
            "process per GPU, and no multi-GPU figure is taken")
        sys.exit(2)
    from llm_amd import _lib
    if _lib.device_count() < 1:
        log("bench.py: no GPU")
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gemv:
        print(json.dumps([one_gemv(spec, args.hbm_bytes) for spec in args.gemv.split(",")]), flush=True)
        return
    g, r = generation(args)
    g.close()
    res = {
        "metric": METRIC, "value": round(r["value"], 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(r["ms_per_step"], 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: seeded random-init Qwen2.5-0.5B-shaped GGUF (Q4_0 layers/embedding, Q8_0 output)",
        "config": {"workload": "BASELINE config 3: qwen2 24L/896/14:2 heads/FFN 4864/vocab 151936, 128-token "
                               "prompt (64-token chunks), 128 greedy tokens (8 per submit), ctx 512, f32 KV",
                   "prompt": args.prompt, "generate": args.gen, "ctx": args.ctx, "prefill_chunk": 64,
                   "decode_batch": 8},
        "prefill_tok_s": round(r["prefill"], 2),
        "rounds": r["rounds"],
        "roofline": r["roofline"],
        "prefill_roofline": prefill_roofline(r["prefill"]),
        "decode_step": {"kernel_us": round(r["step_kernel_us"], 2), "wall_us": round(1e6 / r["value"], 2),
                        "dispatches_per_token": r["dispatches_per_token"], "classes": r["classes"],
                        "unfused_classes": r["unfused"]},
    }
    res["load"] = loader(args)
    if not args.no_long:
        res["long_context"] = long_context(args)
    if not args.no_sweep:
        res["gemv_sweep"] = sweep(args)
        # the GEMVs `metric` names (one token, the vocabulary shape), at a glance
        res["gemv_roofline"] = {
            f"{e['type']}_{e['rows']}x{e['k']}": {"us": e["hbm_us"], "achieved": e["hbm_gbps"], "peak": PEAK_HBM_GBS,
                                                  "unit": "GB/s", "frac": e["hbm_frac"]}
            for e in res["gemv_sweep"] if e["n"] == 1 and e["rows"] == 151936}
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
