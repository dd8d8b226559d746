"""BASELINE config 4 on the GPU: the Qwen2.5-0.5B shape at long context (a
2048-token prompt in 32 prefill chunks, 512 greedy tokens, context 4096, f32 KV
cache ~100 MB) with the baseline type mix (Q4_1 ffn_down on odd layers, Q8_0
head), against golden CPU-oracle results written by tests/golden/make_config4.py:
every step-1 logit (tests/golden/config4_logits.npz, the check of
examples/generate/main.go:159-165: max|gpu - cpu| / max|cpu| <= 1e-4) and the
512 greedy tokens (tests/golden/config4.json); and the extended mix (Q8_0 and
Q4_1 on every kind of matrix) at the same shape against the oracle run here.
"""
import hashlib
import json
import os

import numpy as np
import pytest

from llm_amd import synth
from tests.parity import LOGIT_TOL, cpu_greedy, greedy_parity, gpu_generate, rel_err

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config4.json")
LOGITS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config4_logits.npz")


def test_config4_long_context(gpu):
    from llm_amd import llm
    gold = json.load(open(GOLDEN))
    spec = synth.qwen25_mixed(seed=0)
    path = synth.cached(spec)
    print(f"config 4: {path}, prompt {gold['prompt']}, generate {gold['generate']}, ctx {gold['ctx']}", flush=True)
    g = llm.NewGPU(0, None, path, gold["ctx"])
    prompt = [int(t) for t in synth.prompt(gold["prompt_seed"], gold["prompt"], spec.vocab)]
    # step-1 logits: all of them, within the tolerance of max|logits|
    cpu = np.load(LOGITS)["logits"]
    assert hashlib.sha256(cpu.astype("<f4").tobytes()).hexdigest() == gold["logits_sha256"]
    assert cpu.shape == (spec.vocab,) and float(np.max(np.abs(cpu))) == gold["steps"][0]["maxabs"]
    logits = g.PrefillLogits(prompt)
    rel = rel_err(logits, cpu)
    print(f"config 4: step-1 logits relative error {rel:.3e} over {cpu.size}", flush=True)
    assert rel <= LOGIT_TOL
    for i, v in gold["first_top16"]:
        assert float(cpu[i]) == v
    want = [s["tok"] for s in gold["steps"]]
    done, ties = 0, 0
    while done < len(want):
        got = gpu_generate(g, prompt + want[:done], len(want) - done)
        j = next((k for k in range(len(got)) if got[k] != want[done + k]), None)
        if j is None:
            break
        s = gold["steps"][done + j]
        assert got[j] == s["second"] and s["gap"] <= LOGIT_TOL * s["maxabs"], \
            f"token {done + j}: gpu {got[j]} cpu {s['tok']} (runner-up {s['second']}, gap {s['gap']:.3e})"
        ties += 1
        done += j + 1
    print(f"{len(want)} greedy tokens equal ({ties} accepted near-ties)", flush=True)


def test_extended_mix_qwen_shape(gpu):
    from llm_amd import llm
    from oracle import cpuref
    spec = synth.qwen25_mixed_ext(seed=1)
    path = synth.cached(spec)
    g = llm.NewGPU(0, None, path, 512)
    cpu = cpuref.CPU(path, 512, threads=16)
    prompt = synth.prompt(5, 200, spec.vocab)
    logits = g.PrefillLogits(prompt)
    toks, lgs = cpu_greedy(cpu, prompt, 48)
    rel = rel_err(logits, lgs[0])
    print(f"extended mix: step-1 logits relative error {rel:.3e}", flush=True)
    assert rel <= LOGIT_TOL
    ties = greedy_parity(g, prompt, toks, lgs)
    print(f"48 greedy tokens equal ({ties} accepted near-ties)", flush=True)
