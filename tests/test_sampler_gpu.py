"""Greedy sampling on the GPU against the oracle's Argmax (cpu.go:389-397; the
reference's GPU sampler kernels.go:354-394): the lowest index wins a tie, a NaN
logit never wins, a NaN logit 0 keeps token 0, and all-equal logits give
token 0.

Each case is a tiny model whose head matrix is edited in the file so that the
logits hold the case exactly, on the GPU and in the oracle alike:
  tie    the rows of the oracle's maximum copied to one lower row (in another
         workgroup, and for the streaming kernel in the same wave) and one
         higher row: three bitwise-equal maxima, the lowest must win;
  nan    an f16 NaN block scale on a row below the maximum (same workgroup)
         and on one far from it (another workgroup): NaN logits there, which
         must not win;
  nan0   an f16 NaN scale on row 0: token 0, whatever the maximum;
  equal  every row equal: token 0.
Every case runs through both head kernels: the tile kernel (vocabularies
under 65,536 rows) and the streaming kernel (65,536 rows and more), with a
tied Q4_0 head and a Q8_0 output matrix.  The GPU's sampled tokens (the
first from the prefill, the rest from decode steps), its `tokens` and `outb`
buffers and its logits (NaN where the oracle's are) are compared with the
oracle's.
"""
import os

import numpy as np
import pytest

from llm_amd import synth
from tests.parity import rel_err

pytestmark = pytest.mark.gpu

F16_NAN = 0x7E00
GEN = 4

HEADS = {
    # vocab 4096: 256 tiles, the tile kernel (64 rows per workgroup)
    "tile-q4_0-tied": lambda: synth.tiny_llama(seed=21, vocab=4096),
    "tile-q8_0": lambda: synth.tiny_qwen(seed=22, vocab=4096),
    # vocab 70000: 4375 tiles, the streaming kernel (4096 waves, wave w walks tiles w, w + 4096)
    "stream-q8_0": lambda: synth.tiny_qwen(seed=23, vocab=70000),
    "stream-q4_0-tied": lambda: synth.tiny_llama(seed=24, vocab=70000),
}


def _head(spec):
    return ("token_embd.weight", spec.embd_type) if spec.tied else ("output.weight", spec.out_type)


def _row_span(path, spec):
    """(file offset of the head matrix, bytes per row)."""
    from llm_amd import llm
    name, qtype = _head(spec)
    f = llm.Parse(path)
    t, ok = f.Tensor(name)
    assert ok and t.Type == qtype
    off = f.DataOffset + t.Offset
    f.close()
    be, bb = synth.BLOCK[qtype]
    return off, spec.embd // be * bb


def _edit(src, dst, spec, edits):
    """Copy the model file, applying edits: ("copy", from_row, to_row),
    ("nan", row) (the row's first block scale set to an f16 NaN), ("fill",)
    (every row equal to row 0)."""
    data = bytearray(open(src, "rb").read())
    off, rb = _row_span(src, spec)
    for e in edits:
        if e[0] == "copy":
            a, b = e[1], e[2]
            data[off + b * rb:off + (b + 1) * rb] = data[off + a * rb:off + (a + 1) * rb]
        elif e[0] == "nan":
            r = e[1]
            data[off + r * rb:off + r * rb + 2] = F16_NAN.to_bytes(2, "little")
        elif e[0] == "fill":
            row0 = bytes(data[off:off + rb])
            data[off:off + spec.vocab * rb] = row0 * spec.vocab
    with open(dst, "wb") as f:
        f.write(bytes(data))
    return dst


PROMPT = [11, 17, 23, 29, 31, 37, 41, 43, 47]  # nine ids clear of every edited row


def _case_edits(case, spec, top):
    """The edits of a case given the unedited model's top token, and the rows
    the case is about."""
    V = spec.vocab
    far = 65541 if V > 65541 else V - 7  # streaming: tile 4096 (the same wave as row 5)
    if case == "tie":
        lo = 5 if top > 5 else None
        rows = [r for r in (lo, 3001, far) if r is not None and r != top]
        return [("copy", top, r) for r in rows], rows
    if case == "nan":
        near = top - 1 if top > 0 else top + 1  # the same 16-row tile or its neighbour
        other = (top + V // 2) % V
        if other == 0:
            other = 1
        return [("nan", near), ("nan", other)], [near, other]
    if case == "nan0":
        return [("nan", 0)], [0]
    return [("fill",)], []


@pytest.mark.parametrize("case", ["tie", "nan", "nan0", "equal"])
@pytest.mark.parametrize("head", list(HEADS))
def test_sampler_rules(gpu, head, case):
    from llm_amd import llm
    from oracle import cpuref
    from tests.parity import cpu_greedy
    spec = HEADS[head]()
    base = synth.cached(spec)
    cpu = cpuref.CPU(base, 256, threads=8)
    toks0, _ = cpu_greedy(cpu, PROMPT, 1)
    edits, rows = _case_edits(case, spec, toks0[0])
    path = _edit(base, os.path.join(os.path.dirname(base), f"sampler_{head}_{case}.gguf"), spec, edits)
    print(f"{head} {case}: top {toks0[0]}, edits {edits[:3]} -> {path}", flush=True)

    cpu = cpuref.CPU(path, 256, threads=8)
    want, lgs = cpu_greedy(cpu, PROMPT, GEN)
    l0 = lgs[0]
    # the case holds in the oracle's logits
    if case == "tie":
        m = np.nanmax(l0)
        assert all(l0[r] == m for r in rows) and l0[toks0[0]] == m
        assert want[0] == min(rows + [toks0[0]])
    elif case == "nan":
        assert all(np.isnan(l0[r]) for r in rows) and want[0] == toks0[0]
    elif case == "nan0":
        assert np.isnan(l0[0]) and want[0] == 0
    else:
        assert np.all(l0 == l0[0]) and want[0] == 0
    # the maximum stands clear of the runner-up (no near-tie can decide the case)
    finite = np.where(np.isnan(l0), -np.inf, l0.astype(np.float64))
    top_v = finite[want[0]] if not np.isnan(l0[want[0]]) else -np.inf
    others = np.delete(finite, [want[0]] + [r for r in rows if case == "tie"] + ([toks0[0]] if case == "tie" else []))
    if case in ("tie", "nan"):
        assert top_v - np.max(others) > 1e-4 * np.max(np.abs(finite[np.isfinite(finite)]))

    g = llm.NewGPU(0, None, path, 256)
    logits = g.PrefillLogits(PROMPT)
    nan_gpu, nan_cpu = np.isnan(logits), np.isnan(l0)
    assert np.array_equal(nan_gpu, nan_cpu), (np.flatnonzero(nan_gpu)[:8], np.flatnonzero(nan_cpu)[:8])
    if not np.all(nan_cpu):
        assert rel_err(logits[~nan_cpu], l0[~nan_cpu]) <= 1e-4
    if case == "tie":  # the GPU's maxima are bitwise equal too
        assert len({float(logits[r]) for r in rows + [toks0[0]]}) == 1
    got = []
    g.Generate(PROMPT, GEN, -1, lambda t: got.append(t) or True)
    print(f"gpu {got} cpu {want}", flush=True)
    assert got == want
    toks = g.Peek("tokens", len(PROMPT) + GEN).view(np.int32)
    assert list(toks[:len(PROMPT)]) == PROMPT and list(toks[len(PROMPT):]) == want
    assert int(g.Peek("outb", 1).view(np.int32)[0]) == want[-1]
    g.close()
