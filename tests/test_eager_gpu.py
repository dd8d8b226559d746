"""LLMHIP_EAGER=1 (each pass sent to the stream as direct launches instead of a
graph replay, for kernel tracers) computes what the graph replays compute: a
child process runs the same prompt and decode in eager mode and its logits and
tokens must equal this process's bit for bit (same kernels, same arguments,
same order).  The mode is read once per process, hence the child."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

from llm_amd import synth

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r"""
import json, sys
sys.path.insert(0, sys.argv[1])
from llm_amd import llm
g = llm.NewGPU(0, None, sys.argv[2], 512)
prompt = json.loads(sys.argv[3])
logits = g.PrefillLogits(prompt)
out = []
g.Generate(prompt, 40, -1, lambda t: out.append(int(t)) or True)
print(json.dumps({"logits": logits.astype(float).tolist(), "tokens": out}))
g.close()
"""


def test_eager_matches_graph(gpu):
    from llm_amd import llm
    spec = synth.tiny_qwen(seed=21)
    path = synth.cached(spec)
    prompt = [int(t) for t in synth.prompt(5, 300, spec.vocab)]  # prefill chunks on both attention forms
    g = llm.NewGPU(0, None, path, 512)
    logits = g.PrefillLogits(prompt)
    toks = []
    g.Generate(prompt, 40, -1, lambda t: toks.append(int(t)) or True)
    g.close()
    env = dict(os.environ, LLMHIP_EAGER="1")
    print("child: eager pass", flush=True)
    r = subprocess.run([sys.executable, "-c", CHILD, ROOT, path, json.dumps(prompt)], env=env,
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-2000:]
    child = json.loads(r.stdout.strip().splitlines()[-1])
    assert np.array_equal(np.asarray(child["logits"], np.float32), logits)
    assert child["tokens"] == toks
