"""llm-generate on the GPU: each mode of examples/generate/main.go run as a
separate process over the C-ABI and checked against the library through
ctypes and against the CPU oracle's reference files (check :141-181, trace
:212-240, bench :183-207, run :109-117), plus dump, which writes the GPU's
own results in the reference format."""
import os
import re
import subprocess

import numpy as np
import pytest

from llm_amd import reffile, synth
from tests.parity import cpu_greedy

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "llm_amd", "llm-generate")


def run(*args):
    cmd = [CLI, *map(str, args)]
    print("$", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    return r.returncode, r.stdout, r.stderr


def _oracle_ref(spec, prompt, n, path, layers=(), exact=False):
    """The CPU oracle's records for check / trace (what a CPU run of cpu.go writes)."""
    from oracle import cpuref
    model = synth.cached(spec)
    cpu = cpuref.CPU(model, 512, threads=16, exact_ggml=exact)
    toks, lgs = cpu_greedy(cpu, prompt, n)
    recs = {"prompt": np.asarray(prompt, np.int32), "logits": lgs[0], "tokens": np.asarray(toks, np.int32)}
    for k in layers:
        cpu.set_max_layers(k)
        cpu.reset()
        cpu.forward(prompt[0])
        recs[f"x.{k}"] = cpu.last_x()
    reffile.write(path, recs)
    return recs


def test_run_and_dump(gpu, tmp_path):
    from llm_amd import llm
    spec = synth.tiny_qwen()
    model = synth.cached(spec)
    prompt = list(synth.prompt(3, 40, spec.vocab))
    ids = ",".join(map(str, prompt))
    rc, out, err = run("run", "-model", model, "-ctx", 256, "-n", 20, "-ids", ids)
    assert rc == 0
    g = llm.NewGPU(0, None, model, 256)
    want = []
    g.Generate(prompt, 20, -1, lambda t: want.append(t) or True)
    m = re.search(r"^tokens: \[([\d ]*)\]$", out, re.M)
    assert m and [int(t) for t in m.group(1).split()] == want
    assert re.search(r"^prefill: 40 tokens in [\d.]+ ms = [\d.]+ tok/s$", out, re.M)
    assert re.search(r"^decode: 20 tokens in [\d.]+ ms = [\d.]+ tok/s \(\d+ submits, \d+ dispatches in all\)$", out, re.M)
    assert re.search(r"^load: \d+ ms, GPU memory \d+ bytes, \d+ submits$", out, re.M)
    # dump: the same logits bit for bit, the same tokens, and the residual stream of the trace mode
    ref = tmp_path / "gpu.llmref"
    rc, out, err = run("dump", "-model", model, "-ctx", 256, "-n", 20, "-ids", ids, "-layers", "-1,1,2", "-out", ref)
    assert rc == 0
    r = reffile.read(ref)
    assert list(r["prompt"]) == prompt and list(r["tokens"]) == want
    assert np.array_equal(r["logits"].view(np.uint32), g.PrefillLogits(prompt).view(np.uint32))
    assert set(k for k in r if k.startswith("x.")) == {"x.-1", "x.1", "x.2"}
    # the tool's own dump passes its check exactly
    rc, out, err = run("check", "-model", model, "-ctx", 256, "-n", 20, "-ref", ref)
    assert rc == 0 and "relative 0.000e+00" in out and "equal prefix: 20 of 20" in out


def test_check_against_oracle(gpu, tmp_path):
    spec = synth.tiny_llama(seed=4, layers=3)
    prompt = list(synth.prompt(8, 70, spec.vocab))
    ref = tmp_path / "cpu.llmref"
    _oracle_ref(spec, prompt, 30, ref)
    rc, out, err = run("check", "-model", synth.cached(spec), "-n", 30, "-ref", ref)
    assert rc == 0, out
    m = re.search(r"relative ([\d.e+-]+), argmax gpu (\d+) cpu (\d+)", out)
    assert m and float(m.group(1)) <= 1e-4 and m.group(2) == m.group(3)
    assert "equal prefix: 30 of 30" in out
    # a reference that disagrees: exit 3
    r = reffile.read(ref)
    r["tokens"] = r["tokens"].copy()
    r["tokens"][5] = (r["tokens"][5] + 1) % spec.vocab
    bad = tmp_path / "bad.llmref"
    reffile.write(bad, r)
    rc, out, err = run("check", "-model", synth.cached(spec), "-n", 30, "-ref", bad)
    assert rc == 3 and "equal prefix: 5 of 30" in out and "outside tolerance" in out


def test_trace_against_oracle(gpu, tmp_path):
    spec = synth.tiny_llama(layers=3)
    prompt = list(synth.prompt(3, 5, spec.vocab))
    ref = tmp_path / "cpu.llmref"
    _oracle_ref(spec, prompt, 2, ref, layers=(-1, 1, 2, 3))
    rc, out, err = run("trace", "-model", synth.cached(spec), "-ctx", 128, "-ref", ref)
    assert rc == 0
    rows = re.findall(r"^layers (-?\d+): x max \|gpu-cpu\| = ([\d.e+-]+) \(max \|x\| ([\d.]+)\)", out, re.M)
    assert [int(r[0]) for r in rows] == [-1, 1, 2, 3]
    for k, d, mx in rows:
        assert float(d) == 0.0 if k == "-1" else float(d) <= 1e-5 * float(mx), (k, d, mx)
    assert len(re.findall(r"^state bits ", out, re.M)) == 4


def test_bench(gpu):
    spec = synth.tiny_qwen()
    rc, out, err = run("bench", "-model", synth.cached(spec), "-rounds", 2, "-p", 64, "-n", 16, "-ctx", 256)
    assert rc == 0
    assert len(re.findall(r"^round \d: prefill [\d.]+ tok/s, decode [\d.]+ tok/s$", out, re.M)) == 2
    assert re.search(r"^bench p=64 n=16 rounds=2: prefill median [\d.]+ \(min [\d.]+ max [\d.]+\) tok/s, "
                     r"decode median [\d.]+ \(min [\d.]+ max [\d.]+\) tok/s$", out, re.M)


def test_check_exact_ggml(gpu, tmp_path):
    """-exactggml against the oracle's ExactGGML records (a short prompt: no code on a rounding boundary)."""
    spec = synth.tiny_qwen()
    prompt = list(synth.prompt(21, 4, spec.vocab))
    ref = tmp_path / "cpu_exact.llmref"
    _oracle_ref(spec, prompt, 8, ref, exact=True)
    rc, out, err = run("check", "-exactggml", "-model", synth.cached(spec), "-n", 8, "-ref", ref)
    assert rc == 0 and "equal prefix: 8 of 8" in out
    rc, out, err = run("check", "-model", synth.cached(spec), "-n", 8, "-ref", ref, "-tol", "1e-4")
    assert rc == 3, "the f32 numerics must not pass the ExactGGML reference at 1e-4"
