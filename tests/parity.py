"""Shared parity helpers: the `check` mode of examples/generate/main.go:141-181
(logits max-abs / max-ref, equal greedy prefix), with the near-tie rule for
free-running greedy decoding: a GPU token may differ from the CPU's only where
the CPU's logits of the two tokens are within 1e-4 * max|logits|; the
comparison then continues with the CPU's token fed to both (teacher forcing).
"""
import numpy as np

LOGIT_TOL = 1e-4


def rel_err(gpu, cpu):
    gpu = np.asarray(gpu, np.float64)
    cpu = np.asarray(cpu, np.float64)
    return float(np.max(np.abs(gpu - cpu)) / max(np.max(np.abs(cpu)), 1e-30))


def cpu_greedy(cpu, prompt, n):
    """CPU tokens and the logits each was sampled from (examples/generate/main.go:155-175)."""
    from oracle import cpuref
    cpu.reset()
    logits = None
    for t in prompt:
        logits = cpu.forward(int(t))
    toks, lgs = [], []
    while len(toks) < n:
        nxt = cpuref.argmax(logits)
        toks.append(nxt)
        lgs.append(logits)
        if len(toks) < n:
            logits = cpu.forward(nxt)
    return toks, lgs


def gpu_generate(g, prompt, n):
    out = []
    g.Generate(list(prompt), n, -1, lambda t: out.append(t) or True)
    return out


def greedy_parity(g, prompt, cpu_toks, cpu_logits, tol=LOGIT_TOL):
    """Compare free-running GPU tokens with the CPU's; returns the number of
    accepted near-tie divergences.  Raises AssertionError on a real one."""
    prompt = list(prompt)
    n = len(cpu_toks)
    done, ties = 0, 0
    while done < n:
        got = gpu_generate(g, prompt + cpu_toks[:done], n - done)
        assert len(got) == n - done
        i = next((j for j in range(len(got)) if got[j] != cpu_toks[done + j]), None)
        if i is None:
            return ties
        k = done + i
        l = cpu_logits[k]
        gap = float(l[cpu_toks[k]]) - float(l[got[i]])
        assert gap <= tol * float(np.max(np.abs(l))), \
            f"token {k}: gpu {got[i]} cpu {cpu_toks[k]}, logit gap {gap:.3e} above {tol} relative"
        ties += 1
        done = k + 1
    return ties
