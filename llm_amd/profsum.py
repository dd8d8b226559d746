"""The rocprofv3 runs behind profiles/ and their summaries.

    python3 -m llm_amd.profsum run OUT        # on a GPU machine: every pass, raw output under OUT
    python3 -m llm_amd.profsum summarize OUT  # the text summaries from OUT into profiles/

`run` starts each pass as a child process (rocprofv3 first, the program
right after its `--`), from /tmp with TMPDIR=/tmp, under a time limit of its
own, and stops at the first pass that fails.  Kernel-trace passes set
LLMHIP_EAGER=1: decode and prefill passes then go to the stream as direct
launches instead of hipGraph replays (the same kernels, arguments and order)
and the sweep uses stream launches, because rocprofv3's kernel trace of graph
replays ended in a host fault.  Counter passes take one counter block each
(FETCH_SIZE, WRITE_SIZE, then the SQ instruction counters), as rocprofv3
collects a pass per run.

Every summary records the fingerprint of the kernel sources it measured
(`sources_hash`), so that bench.py can tell a stale traffic figure from a
current one.
"""
import collections
import csv
import hashlib
import json
import os
import re
import statistics
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PROFILES = os.path.join(ROOT, "profiles")
BENCH = os.path.join(ROOT, "bench.py")
CLASSES = ["pass", "head", "argmax"]  # a decode step's launches
UNFUSED = ["k1", "k2", "k3", "k4", "k5"]  # one launch per phase (prefill, fallback, config-4 decode)
SWEEP = [(576, 576), (1536, 576), (576, 1536), (896, 896), (4864, 896), (896, 4864), (151936, 896)]
VOCAB = "q4_0:151936x896"
# MFMA utilisation (rocprofv3's MfmaUtil: SQ_VALU_MFMA_BUSY_CYCLES summed over the SIMDs, over GRBM_GUI_ACTIVE
# times the SIMDs) and the instruction mix, per dispatch
MFMA = ["MfmaUtil", "SQ_INSTS_MFMA", "SQ_INSTS_VALU", "SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE"]
SQ = ["SQ_WAVES", "SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_VMEM_RD", "SQ_INSTS_LDS", "SQ_INSTS_SALU",
      "SQ_BUSY_CYCLES", "SQ_WAVE_CYCLES"]


def sources_hash():
    """First 12 hex digits of the SHA-256 over the kernel and host sources
    (llm_amd/csrc, sorted by name)."""
    h = hashlib.sha256()
    csrc = os.path.join(HERE, "csrc")
    for name in sorted(os.listdir(csrc)):
        p = os.path.join(csrc, name)
        if os.path.isfile(p):
            h.update(name.encode())
            with open(p, "rb") as f:
                h.update(f.read())
    return h.hexdigest()[:12]


def sweep_specs():
    specs = [f"{t}:{r}x{k}" for t in ("q4_0", "q8_0") for r, k in SWEEP]
    specs += [f"q4_0:{r}x{k}:64" for r, k in SWEEP]
    return specs


def passes(out):
    """(name, timeout s, environment additions, rocprofv3 options, program arguments)."""
    py = [sys.executable or "python3", BENCH]
    eager = {"LLMHIP_EAGER": "1"}
    decode = py + ["--no-sweep", "--no-long", "--no-cpu", "--steps", "1", "--warmup", "0"]
    trace = ["--kernel-trace", "--stats"]
    return [
        ("kt", 600, eager, trace, py + ["--no-sweep", "--no-cpu", "--steps", "2"]),
        ("ktsweep", 600, eager, trace, py + ["--gemv", ",".join(sweep_specs())]),
        ("psq", 300, eager, ["--pmc"] + MFMA, decode),
        ("pf", 300, eager, ["--pmc", "FETCH_SIZE"], decode),
        ("pw", 300, eager, ["--pmc", "WRITE_SIZE"], decode),
        ("cf", 120, {}, ["--pmc", "FETCH_SIZE"], py + ["--copy-calibration"]),
        ("cw", 120, {}, ["--pmc", "WRITE_SIZE"], py + ["--copy-calibration"]),
        ("vf", 120, {}, ["--pmc", "FETCH_SIZE"], py + ["--gemv", VOCAB]),
        ("vw", 120, {}, ["--pmc", "WRITE_SIZE"], py + ["--gemv", VOCAB]),
        ("vsq", 120, {}, ["--pmc"] + SQ, py + ["--gemv", VOCAB]),
    ]


def command_text(name, env, opts, prog):
    e = "".join(f"export {k}={v} && " for k, v in env.items())
    args = " ".join(os.path.relpath(a, ROOT) if a.startswith(ROOT) else a for a in prog[1:])
    return (f"cd /tmp && export TMPDIR=/tmp && {e}rocprofv3 {' '.join(opts)} --output-format csv "
            f"-d <out>/{name} -o run -- python3 /root/repo/{args}")


def run(out):
    out = os.path.abspath(out)  # (the passes run from /tmp)
    os.makedirs(out, exist_ok=True)
    with open(os.path.join(out, "sources_hash"), "w") as f:
        f.write(sources_hash() + "\n")
    # the unprofiled figures first: bench.py as the driver runs it
    print("pass live", flush=True)
    with open(os.path.join(out, "live.log"), "w") as f:
        rc = subprocess.run([sys.executable, BENCH, "--no-cpu"], stdout=f, stderr=subprocess.STDOUT,
                            timeout=900).returncode
    if rc:
        return rc
    for name, limit, env, opts, prog in passes(out):
        print(f"pass {name}: {command_text(name, env, opts, prog)}", flush=True)
        e = dict(os.environ, TMPDIR="/tmp", **env)
        cmd = ["rocprofv3"] + opts + ["--output-format", "csv", "-d", os.path.join(out, name), "-o", "run", "--"] + prog
        with open(os.path.join(out, name + ".log"), "w") as f:
            try:
                rc = subprocess.run(cmd, cwd="/tmp", env=e, stdout=f, stderr=subprocess.STDOUT,
                                    timeout=limit).returncode
            except subprocess.TimeoutExpired:
                rc = 124
        if rc:
            print(f"pass {name} failed: {rc}", flush=True)
            return rc
    return 0


# ------------------------------------------------------------------ summaries

def jlines(path):
    out = []
    with open(path) as f:
        for line in f:
            if line.startswith("{") or line.startswith("["):
                out.append(json.loads(line))
    return out


def short(name):
    return name.split("(")[0].replace("void ", "").replace("llmhip::", "")


def trace_rows(path):
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            gx, gy = int(r["Grid_Size_X"]), int(r["Grid_Size_Y"])
            rows.append((int(r["Start_Timestamp"]), short(r["Kernel_Name"]), gx, gy,
                         (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0))
    rows.sort()
    return rows


def stats(v):
    v = sorted(v)
    return {"n": len(v), "median": v[len(v) // 2], "mean": statistics.mean(v), "min": v[0], "max": v[-1]}


def counters(path):
    """{(kernel, grid): {counter: [values per dispatch]}}"""
    agg = collections.defaultdict(lambda: collections.defaultdict(list))
    with open(path) as f:
        for r in csv.DictReader(f):
            agg[(short(r["Kernel_Name"]), int(r["Grid_Size"]))][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return agg


def calibration(out):
    """FETCH_SIZE and WRITE_SIZE of the 256 MiB calibration copy: bytes per KiB read."""
    def biggest(d, counter):
        vals = [max(v[counter]) for (k, _), v in counters(os.path.join(out, d, "run_counter_collection.csv")).items()
                if "copyBuffer" in k and counter in v]
        return max(vals)
    f_kib, w_kib = biggest("cf", "FETCH_SIZE"), biggest("cw", "WRITE_SIZE")
    return f_kib, w_kib, 262144 / f_kib * 1024, 262144 / w_kib * 1024


def class_grids(rows, symbols):
    """The (symbol, grid x, grid y) of each decode class in a kernel trace: the
    most launched grid of the class's symbol (k3 and k5 share a symbol in some
    builds and differ in grid: k3 the smaller)."""
    by = collections.Counter((n, gx, gy) for _, n, gx, gy, _ in rows if gy <= 2)
    out = {}
    for c, sym in symbols.items():
        sym = sym.split(" + ")[0]
        cands = sorted(((gx, gy) for (n, gx, gy) in by if n == sym), key=lambda g: -by[(sym,) + g])
        if not cands:
            continue
        if c in ("k3", "k5") and symbols["k3"] == symbols["k5"] and len(cands) > 1:
            two = sorted(cands[:2])
            out[c] = (sym,) + (two[0] if c == "k3" else two[1])
        else:
            out[c] = (sym,) + cands[0]
    return out


def summarize(out):
    h = open(os.path.join(out, "sources_hash")).read().strip()
    live = jlines(os.path.join(out, "live.log"))[-1]
    traced = jlines(os.path.join(out, "kt.log"))[-1]
    rows = trace_rows(os.path.join(out, "kt", "run_kernel_trace.csv"))
    by = collections.defaultdict(list)
    for _, n, gx, gy, d in rows:
        by[(n, gx, gy)].append(d)
    cls = dict(live["decode_step"]["classes"])
    cls.update(live["decode_step"].get("unfused_classes", {}))
    syms = {c: cls[c]["symbol"] for c in CLASSES + UNFUSED if c in cls and cls[c].get("symbol")}
    grids = class_grids(rows, syms)

    md = ["# Decode and prefill kernels, Qwen2.5-0.5B shape (BASELINE config 3), one MI355X", "",
          f"Sources `{h}` (`llm_amd.profsum.sources_hash()`). Commands (GPU box, repository root at /root/repo; "
          "`python3 -m llm_amd.profsum run <out>` runs them all, `summarize <out>` wrote this file):", "", "```",
          "python3 /root/repo/bench.py --no-cpu                       # live figures, no profiler",
          command_text("kt", {"LLMHIP_EAGER": "1"}, ["--kernel-trace", "--stats"],
                       ["python3", BENCH, "--no-sweep", "--no-cpu", "--steps", "2"]),
          "```", "",
          "`LLMHIP_EAGER=1`: passes go to the stream as direct launches instead of hipGraph replays (same kernels, "
          "arguments and order); rocprofv3's kernel trace of graph replays ended in a host fault. Traced durations "
          "are per dispatch from the profiler's start and end stamps. Live figures (no profiler): a decode step's "
          "launches between HIP events on the model's stream (`llmhip_model_profile`, eager steps after the timed "
          "rounds), and for the one-launch-per-phase classes back-to-back launches of one class over the 24 layers "
          "(`llmhip_model_bench_kernel`).", "",
          "A decode step (the fused pass: every layer in one launch):", "",
          "| class | symbol | grid (threads x rows) | traced launches | traced median us | mean | min | live us (unprofiled) | "
          "bytes | GB/s (live) | GB/s (traced median) |",
          "|---|---|---|---|---|---|---|---|---|---|---|"]
    machine_d = []

    def row(c):
        sym, g, gy = grids[c]
        st = stats(by[(sym, g, gy)])
        b = cls[c]["bytes"]
        gl = f"{b / cls[c]['avg_us'] * 1e-3:.1f}" if b else "-"
        gt = f"{b / st['median'] * 1e-3:.1f}" if b else "-"
        machine_d.append(f"duration_us {c} {st['median']:.3f}")
        return (f"| {c} | `{sym}` | {g}x{gy} | {st['n']} | {st['median']:.2f} | {st['mean']:.2f} | {st['min']:.2f} | "
                f"{cls[c]['avg_us']:.3f} | {b} | {gl} | {gt} |")
    for c in CLASSES:
        if c in grids:
            md.append(row(c))
    md += ["", "One launch per phase (prefill's kernels, the decode fallback, and config 4's decode, which takes the "
           "split attention):", "",
           "| class | symbol | grid (threads x rows) | traced launches | traced median us | mean | min | live us (unprofiled) | "
           "bytes | GB/s (live) | GB/s (traced median) |",
           "|---|---|---|---|---|---|---|---|---|---|---|"]
    for c in UNFUSED:
        if c in grids:
            md.append(row(c))
    md += ["", f"Live: decode {live['value']} tok/s, prefill {live['prefill_tok_s']} tok/s, decode step kernel sum "
           f"{live['decode_step']['kernel_us']} us of {live['decode_step']['wall_us']} us per token; traced run: "
           f"decode {traced['value']} tok/s.", "",
           "Prefill kernels of the traced run (64-token chunks of configs 3 and 4; grid = threads x workgroups "
           "along y), by total time. Prompts of two or more chunks run as a two-lane wavefront, two chunks' kernels "
           "at once, so a duration here includes the other lane's load:", "",
           "| symbol | grid | launches | median us | mean |", "|---|---|---|---|---|"]
    for (n, gx, gy), v in sorted(by.items(), key=lambda kv: -sum(kv[1])):
        if any(k in n for k in ("gemm", "prep", "attn_mma", "attn_multi")) or (n.startswith("attn_kernel") and "true>" in n):
            st = stats(v)
            md.append(f"| `{n}` | {gx // gy}x{gy} | {st['n']} | {st['median']:.2f} | {st['mean']:.2f} |")
    lc = live.get("long_context")
    if lc:
        k3e, k3 = lc["classes_at_end"]["k3"]["avg_us"], live["decode_step"]["unfused_classes"]["k3"]["avg_us"]
        md += ["", f"Config 4 (2048-token prompt, 512 tokens, ctx 4096), live: prefill {lc['prefill_tok_s']} tok/s, "
               f"decode {lc['decode_tok_s']} tok/s (the fused pass's long form: "
               f"{lc.get('decode_step_at_end', {}).get('pass', {}).get('avg_us', '-')} us per launch at the last "
               f"positions); one launch per phase (the fallback) at the last position: the split attention kernel "
               f"{lc['attention_at_end']['avg_us']} us for {lc['attention_at_end']['kv_bytes']} KV bytes "
               f"({lc['attention_at_end']['gbps']} GB/s); its chunks are merged in the output projection's prologue, "
               f"K3 {k3e} us there against {k3} us at config 3. Traced decode attention kernels and the merging "
               "K3 (prologue argument 4 + 8 (chunks / 2 - 1)), and the fused pass's long form, of the run:", "",
               "| symbol | grid | launches | median us | mean |", "|---|---|---|---|---|"]
        for (n, gx, gy), v in sorted(by.items(), key=lambda kv: -sum(kv[1])):
            mk3 = re.match(r"gemv_kernel<\w+, 1, (\d+), 1, 2>", n)
            if (n.startswith("attn_kernel") and "true, false, false" in n) or (mk3 and int(mk3.group(1)) >= 4) or \
                    (n.startswith("pass_kernel") and n.endswith("true>")):
                st = stats(v)
                md.append(f"| `{n}` | {gx // gy}x{gy} | {st['n']} | {st['median']:.2f} | {st['mean']:.2f} |")
    write(os.path.join(PROFILES, "decode_kernels_qwen25.md"), md)

    # HBM traffic of the decode classes
    f_kib, w_kib, fs, ws = calibration(out)
    pf = counters(os.path.join(out, "pf", "run_counter_collection.csv"))
    pw = counters(os.path.join(out, "pw", "run_counter_collection.csv"))
    t = ["HBM traffic per launch of the decode kernels, Qwen2.5-0.5B shape (BASELINE config 3), one MI355X.",
         f"sources {h}", "",
         "Commands (one counter per pass; then the same two on the calibration copy):"]
    for name, limit, env, opts, prog in passes(out):
        if name in ("pf", "pw", "cf", "cw"):
            t.append("  " + command_text(name, env, opts, prog))
    t += ["", f"Calibration: a 256 MiB device copy (__amd_rocclr_copyBuffer) reads FETCH_SIZE {f_kib:.1f} KiB and "
          f"WRITE_SIZE {w_kib:.1f} KiB per dispatch for 262144 KiB moved each way: bytes = FETCH_SIZE x {fs:.1f}, "
          f"WRITE_SIZE x {ws:.1f}.", "",
          "class  symbol  grid  FETCH_SIZE_KiB  WRITE_SIZE_KiB  traffic_bytes  algorithmic_bytes  traffic/algorithmic"]
    machine = []
    for c in CLASSES + UNFUSED:
        if c not in grids:
            continue
        sym, gx, gy = grids[c]
        g = gx * gy
        if (sym, g) not in pf or "FETCH_SIZE" not in pf[(sym, g)]:
            continue
        fv = statistics.median(pf[(sym, g)]["FETCH_SIZE"])
        wv = statistics.median(pw[(sym, g)]["WRITE_SIZE"])
        tb = int(round(fv * fs + wv * ws))
        ab = cls[c]["bytes"]
        t.append(f"{c}  {sym}  {gx}x{gy}  {fv:.1f}  {wv:.1f}  {tb}  {ab}  " + (f"{tb / ab:.3f}" if ab else "-"))
        machine.append(f"traffic_bytes {c} {tb}")
    t += ["", "The fused pass polls flag-carrying words with coherent loads, which are served beyond the L2: its",
          "FETCH_SIZE counts those polls beside the weights and KV rows (the algorithmic bytes).", "",

          "k2 algorithmic bytes are the KV rows of the positions attended at the profiled position; the one-chunk",
          "kernel reads the rows up to the next multiple of 64 (a graph variant), and each XCD that serves a KV head",
          "reads its rows once.", "", "Machine-readable (bench.py reads these lines for roofline.traffic when",
          "sources_hash matches the tree it runs from; duration_us: the kernel trace's median, above):",
          f"sources_hash {h}"] + machine + machine_d
    write(os.path.join(PROFILES, "pmc_decode_qwen25.txt"), t)

    # MFMA utilisation of the prefill kernels (and the decode launches)
    ms = counters(os.path.join(out, "psq", "run_counter_collection.csv"))
    mu = ["# MFMA utilisation per kernel, Qwen2.5-0.5B shape (BASELINE config 3), one MI355X", "",
          f"Sources `{h}`. Command (direct launches, one counter pass):", "", "```"]
    for name, limit, env, opts, prog in passes(out):
        if name == "psq":
            mu.append(command_text(name, env, opts, prog))
    mu += ["```", "",
           "`MfmaUtil` is rocprofv3's derived counter: SQ_VALU_MFMA_BUSY_CYCLES summed over the SIMDs over "
           "(GRBM_GUI_ACTIVE x the SIMDs) x 100, for the dispatch alone (counter collection runs one dispatch at a "
           "time). Medians per dispatch of each kernel and grid (grid = threads); the prefill pair of a 64-token "
           "chunk is prep_kernel (activation staging) + gemm_kernel; attn_mma_kernel is the chunk's attention.", "",
           "| kernel | grid | dispatches | MfmaUtil % | SQ_INSTS_MFMA | SQ_INSTS_VALU | MFMA / VALU |",
           "|---|---|---|---|---|---|---|"]
    machine_m = []
    rows_m = []
    for (k, g), v in ms.items():
        if not any(x in k for x in ("gemm_kernel", "prep_kernel", "attn_mma", "attn_multi", "pass_kernel",
                                    "gemv_stream_kernel")):
            continue
        if "MfmaUtil" not in v:
            continue
        n = len(v["MfmaUtil"])
        util = statistics.median(v["MfmaUtil"])
        im = statistics.median(v.get("SQ_INSTS_MFMA", [0]))
        iv = statistics.median(v.get("SQ_INSTS_VALU", [0]))
        rows_m.append((k, g, n, util, im, iv))
    for k, g, n, util, im, iv in sorted(rows_m, key=lambda r: (-r[2], r[0])):
        mu.append(f"| `{k}` | {g} | {n} | {util:.2f} | {im:.0f} | {iv:.0f} | {im / iv if iv else 0:.3f} |")
        machine_m.append(f"mfma_util {k.replace(' ', '')}@{g} {util:.3f}")
    gm = [r for r in rows_m if r[0].startswith("gemm_kernel")]
    if gm:
        wsum = sum(r[3] * r[2] for r in gm) / sum(r[2] for r in gm)
        mu += ["", f"Prefill products (every gemm_kernel dispatch, dispatch-weighted mean): {wsum:.2f}% MFMA busy."]
        machine_m.append(f"prefill_gemm_mfma_util {wsum:.3f}")
    mu += ["", "Machine-readable (bench.py reads prefill_gemm_mfma_util when sources_hash matches):",
           f"sources_hash {h}"] + machine_m
    write(os.path.join(PROFILES, "mfma_util_qwen25.md"), mu)

    # config-1 sweep: live graph replays beside the traced durations
    srows = trace_rows(os.path.join(out, "ktsweep", "run_kernel_trace.csv"))
    specs = jlines(os.path.join(out, "ktsweep.log"))[-1]
    blocks = gemv_blocks(srows, specs)
    sw = ["# GEMV sweep (BASELINE config 1), one MI355X", "", f"Sources `{h}`. Commands:", "", "```",
          "python3 /root/repo/bench.py --no-cpu        # live: gemv_sweep, hipGraph replays",
          command_text("ktsweep", {"LLMHIP_EAGER": "1"}, ["--kernel-trace", "--stats"],
                       ["python3", BENCH, "--gemv", "<every shape below>"]), "```", "",
          "Live: each shape's launches captured once in a hipGraph over rotated copies above 640 MB (HBM) and "
          "replayed (`llmhip_qmat_bench_graph`), HIP events around the replays; `stream` the same launches "
          "without the graph. Traced: rocprofv3 kernel durations of the same shape's launches over the same "
          "rotated copies (`bench.py --gemv`, stream launches; N = 64 is the prep kernel plus the product).", "",
          "| type | rows x k | N | bytes | live graph us | GB/s | frac of 8 TB/s | live stream us | traced kernels | "
          "traced median us | traced GB/s |", "|---|---|---|---|---|---|---|---|---|---|---|"]
    sweep = {(e["type"], e["rows"], e["k"], e["n"]): e for e in live.get("gemv_sweep", [])}
    for spec, blk in zip(specs, blocks):
        e = sweep.get((spec["type"], spec["rows"], spec["k"], spec["n"]))
        if not e:
            continue
        names = " + ".join(f"`{n}`" for n in blk["names"])
        sw.append(f"| {spec['type']} | {spec['rows']}x{spec['k']} | {spec['n']} | {spec['bytes']} | "
                  f"{e['hbm_us']:.2f} | {e['hbm_gbps']} | {e['hbm_frac']:.3f} | "
                  f"{fmt(e.get('stream_hbm_us'))} | {names} | "
                  f"{blk['median']:.2f} | {spec['bytes'] / blk['median'] * 1e-3:.1f} |")
    write(os.path.join(PROFILES, "gemv_sweep_config1.md"), sw)

    # the Q4_0 vocabulary-shape product: traffic and instruction mix
    vf = counters(os.path.join(out, "vf", "run_counter_collection.csv"))
    vw = counters(os.path.join(out, "vw", "run_counter_collection.csv"))
    vs = counters(os.path.join(out, "vsq", "run_counter_collection.csv"))
    key = next(k for k in vs if k[0].startswith("gemv_stream_kernel"))
    fv, wv = statistics.median(vf[key]["FETCH_SIZE"]), statistics.median(vw[key]["WRITE_SIZE"])
    sq = {c: statistics.median(vs[key][c]) for c in SQ if c in vs[key]}
    vspec = jlines(os.path.join(out, "vf.log"))[-1][0]
    rows_, k_ = vspec["rows"], vspec["k"]
    blocks_ = rows_ * k_ // 32
    wblk = blocks_ / 16  # a wave's block: one 32-element block of a 16-row tile
    vt = [f"# Q4_0 151936x896 product (config 1, N = 1): HBM traffic and instruction mix", "",
          f"Sources `{h}`. Commands:", "", "```"]
    for name, limit, env, opts, prog in passes(out):
        if name in ("vf", "vw", "vsq"):
            vt.append(command_text(name, env, opts, prog))
    vsweep = sweep.get(("q4_0", rows_, k_, 1), {})
    vblk = next((b for s_, b in zip(specs, blocks) if (s_["type"], s_["rows"], s_["k"], s_["n"]) ==
                 ("q4_0", rows_, k_, 1)), None)
    vt += ["```", "", f"Kernel `{key[0]}`, grid {key[1]} threads; {vspec['bytes']} algorithmic bytes per launch "
           f"({blocks_} blocks of 18 bytes).", "",
           f"* duration: live graph replay {vsweep.get('hbm_us', float('nan')):.2f} us "
           f"({vsweep.get('hbm_gbps', float('nan'))} GB/s, {vsweep.get('hbm_frac', float('nan'))} of 8 TB/s); "
           + (f"traced median {vblk['median']:.2f} us ({vspec['bytes'] / vblk['median'] * 1e-3:.0f} GB/s)"
              if vblk else ""),
           f"* HBM traffic: FETCH_SIZE {fv:.1f} KiB, WRITE_SIZE {wv:.1f} KiB per dispatch -> "
           f"{int(fv * fs + wv * ws)} bytes ({(fv * fs + wv * ws) / vspec['bytes']:.3f} of the algorithmic bytes)",
           "* SQ counters per dispatch (medians), and per 16-row x 32-element block (one MFMA's worth):", ""]
    vt += ["| counter | per dispatch | per block |", "|---|---|---|"]
    for c, v in sq.items():
        vt.append(f"| {c} | {v:.0f} | {v / wblk:.2f} |")
    write(os.path.join(PROFILES, "gemv_q40_vocab.md"), vt)
    return 0


def fmt(v):
    return "-" if v is None else f"{v:.2f}"


def gemv_blocks(rows, specs):
    """For each --gemv shape in order: the kernels of its timed launches (the
    run of identical (kernel, grid) dispatches of product kernels after its
    matrix was created), median duration per launch (prep + product summed
    for N > 1)."""
    prod = [r for r in rows if r[1].startswith(("gemv_kernel", "gemv_stream_kernel", "gemm_kernel", "prep_kernel"))]
    # consecutive runs of the same kernel set
    out, i = [], 0
    for spec in specs:
        per = 2 if spec["n"] >= 5 else 1
        want = spec["launches"] * per
        seg = prod[i:i + want]
        i += want
        names = sorted({r[1] for r in seg})
        durs = [r[4] for r in seg]
        if per == 2:
            durs = [durs[j] + durs[j + 1] for j in range(0, len(durs) - 1, 2)]
        out.append({"names": names, "median": statistics.median(durs) if durs else float("nan")})
    return out


def write(path, lines):
    with open(path, "w") as f:
        f.write("\n".join(lines).rstrip() + "\n")
    print(f"wrote {path}", file=sys.stderr)


def main():
    if len(sys.argv) != 3 or sys.argv[1] not in ("run", "summarize"):
        print(__doc__, file=sys.stderr)
        return 2
    return run(sys.argv[2]) if sys.argv[1] == "run" else summarize(sys.argv[2])


if __name__ == "__main__":
    sys.exit(main())
