"""Golden greedy tokens of BASELINE config 4 (Qwen2.5-0.5B shape, baseline
mixed types: Q4_1 ffn_down on odd layers, Q8_0 head; 2048-token prompt, 512
greedy tokens, context 4096), computed with the CPU oracle (oracle/cpuref.c,
the C restatement of cpu.go; row- and head-parallel runs are bit-identical
to single-threaded ones).  Writes tests/golden/config4.json: the prompt seed,
every CPU token, and at each step the runner-up token and the CPU logit gap
to it, so a GPU divergence can be judged by the near-tie rule without
re-running the CPU; and tests/golden/config4_logits.npz: all vocab step-1
logits of the CPU (f32, compressed), whose sha256 the JSON records.
Run:  python tests/golden/make_config4.py [threads]
"""
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from llm_amd import synth  # noqa: E402
from oracle import cpuref  # noqa: E402

PROMPT, GEN, CTX, SEED = 2048, 512, 4096, 0


def main():
    threads = int(sys.argv[1]) if len(sys.argv) > 1 else os.cpu_count()
    spec = synth.qwen25_mixed(seed=0)
    path = synth.cached(spec)
    cpu = cpuref.CPU(path, CTX, threads=threads)
    prompt = [int(t) for t in synth.prompt(SEED, PROMPT, spec.vocab)]
    t0 = time.time()
    for i, t in enumerate(prompt):
        logits = cpu.forward(t)
        if i % 256 == 0:
            print(f"prompt {i}/{PROMPT} {time.time() - t0:.0f}s", flush=True)
    here = os.path.dirname(os.path.abspath(__file__))
    npz = os.path.join(here, "config4_logits.npz")
    np.savez_compressed(npz, logits=logits.astype(np.float32))
    digest = hashlib.sha256(logits.astype("<f4").tobytes()).hexdigest()
    steps = []
    first_top = None
    while len(steps) < GEN:
        order = np.argsort(-logits.astype(np.float64), kind="stable")
        top = cpuref.argmax(logits)
        second = int(order[1]) if int(order[0]) == top else int(order[0])
        steps.append({"tok": top, "second": second, "gap": float(logits[top]) - float(logits[second]),
                      "maxabs": float(np.max(np.abs(logits)))})
        if first_top is None:
            first_top = [[int(i), float(logits[i])] for i in order[:16]]
        if len(steps) < GEN:
            logits = cpu.forward(top)
        if len(steps) % 64 == 0:
            print(f"gen {len(steps)}/{GEN} {time.time() - t0:.0f}s", flush=True)
    out = {"spec": "synth.qwen25_mixed(seed=0)", "prompt_seed": SEED, "prompt": PROMPT, "generate": GEN, "ctx": CTX,
           "first_top16": first_top, "logits_sha256": digest, "logits_file": os.path.basename(npz), "steps": steps}
    dst = os.path.join(here, "config4.json")
    json.dump(out, open(dst, "w"), separators=(",", ":"))
    print(f"wrote {dst} in {time.time() - t0:.0f}s")


if __name__ == "__main__":
    main()
