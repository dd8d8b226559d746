"""GPU forward pass against the CPU oracle, through the C-ABI (llm_* / llmhip_*).

Tiny random-init llama and qwen2 models exercise every path (tied Q4_0 head,
Q8_0 head, NEOX, biases, mixed Q4_0/Q4_1/Q8_0 types, multi-chunk prompts,
decode batches, the Layers trace, refusals); the BASELINE shapes (SmolLM2 and
Qwen2.5-0.5B) are checked end to end: step-1 logits within 1e-4 relative and
greedy tokens identical except at a top-2 logit gap below that tolerance.
"""
import numpy as np
import pytest

from llm_amd import synth
from tests.parity import LOGIT_TOL, cpu_greedy, gpu_generate, greedy_parity, rel_err

pytestmark = pytest.mark.gpu


def _open(spec, ctx, f16kv=False, exact=False):
    from llm_amd import llm
    from oracle import cpuref
    path = synth.cached(spec)
    print(f"model {spec.arch} L{spec.layers} E{spec.embd} V{spec.vocab} ctx {ctx} f16kv {f16kv} exact {exact} at "
          f"{path}", flush=True)
    old = llm.F16KV, llm.ExactGGML
    llm.F16KV, llm.ExactGGML = f16kv, exact
    try:
        g = llm.NewGPU(0, None, path, ctx)
    finally:
        llm.F16KV, llm.ExactGGML = old
    cpu = cpuref.CPU(path, ctx, threads=16, f16kv=f16kv, exact_ggml=exact)
    return g, cpu


def _check(g, cpu, prompt, n):
    logits = g.PrefillLogits(prompt)
    toks, lgs = cpu_greedy(cpu, prompt, n)
    rel = rel_err(logits, lgs[0])
    print(f"step-1 logits relative error {rel:.3e}", flush=True)
    assert rel <= LOGIT_TOL
    ties = greedy_parity(g, prompt, toks, lgs)
    print(f"{n} greedy tokens equal ({ties} accepted near-ties)", flush=True)
    return rel, ties


TINY = {
    "llama": lambda: synth.tiny_llama(),
    "qwen2": lambda: synth.tiny_qwen(),
    "qwen2-mixed": lambda: synth.tiny_qwen(seed=3, types={
        "attn_q": synth.Q8_0, "attn_k": synth.Q4_1, "attn_v": synth.Q4_0, "attn_output": synth.Q4_1,
        "ffn_gate": synth.Q8_0, "ffn_up": synth.Q4_0, "ffn_down": lambda l: synth.Q4_1 if l % 2 else synth.Q8_0}),
    "llama-q8embd": lambda: synth.tiny_llama(seed=4, embd_type=synth.Q8_0,
                                             types={"ffn_down": synth.Q4_1, "attn_output": synth.Q8_0}),
    "llama-untied-q41": lambda: synth.tiny_llama(seed=5, tied=False, out_type=synth.Q4_1, layers=3),
}


@pytest.mark.parametrize("name", list(TINY))
def test_tiny_parity(gpu, name):
    spec = TINY[name]()
    g, cpu = _open(spec, 512)
    prompt = synth.prompt(1, 150, spec.vocab)  # three prefill chunks of 64, 64, 22
    _check(g, cpu, prompt, 40)


@pytest.mark.parametrize("prompt_len,batch", [(65, 64), (129, 64), (21, 1), (30, 4)])
def test_prefill_chunk_edges(gpu, prompt_len, batch):
    """Prompts whose last prefill chunk is one token (65, 129: a 64-token
    chunk and a one-token chunk on two lanes of the wavefront), and small
    PrefillBatch values (every chunk one token on three lanes; chunks of
    four), on a six-layer model, so that graph segments of three and six
    layers end between a layer's K1 and its K3: logits and greedy tokens
    against the oracle's.  A one-token pass of a prefill runs its down
    projection whole (the two-part form's buffer belongs to decode)."""
    from llm_amd import llm
    spec = synth.tiny_qwen(seed=30, layers=6)
    old = llm.PrefillBatch
    llm.PrefillBatch = batch
    try:
        g, cpu = _open(spec, 256)
    finally:
        llm.PrefillBatch = old
    _check(g, cpu, synth.prompt(31, prompt_len, spec.vocab), 12)


_TWO_LANES = r"""
import sys
sys.path.insert(0, sys.argv[1])
from llm_amd import synth
from tests.test_model_gpu import _open, _check
spec = synth.tiny_qwen(seed=30, layers=8)
g, cpu = _open(spec, 512)
_check(g, cpu, synth.prompt(32, int(sys.argv[2]), spec.vocab), 8)
print("two-lane wavefront ok", flush=True)
"""


@pytest.mark.parametrize("prompt_len", [150, 300])
def test_prefill_two_lanes_staggered(gpu, prompt_len):
    """The wavefront on two lanes for prompts of three and five chunks
    (LLMHIP_PREFILL_LANES=2, read once per process, so in a child process):
    each chunk's segments start c % 6 slots later than the first's, and a
    segment waits for the previous chunk's segment that holds the slot before
    its own last (seg_start / seg_of); logits and greedy tokens against the
    oracle's on an eight-layer model."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, LLMHIP_PREFILL_LANES="2")
    r = subprocess.run([sys.executable, "-c", _TWO_LANES, root, str(prompt_len)], env=env, cwd=root,
                       capture_output=True, text=True, timeout=240)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "two-lane wavefront ok" in r.stdout


@pytest.mark.parametrize("prompt_len,heads,kv_heads,hd", [
    (230, 4, 4, 64), (300, 4, 2, 64), (250, 8, 2, 64), (200, 16, 2, 64), (100, 2, 1, 128), (140, 4, 2, 128)])
def test_attention_paths(gpu, prompt_len, heads, kv_heads, hd):
    """Both attention forms and the switch between them: passes whose
    positions are all below 256 (head size 64) or 128 (head size 128) run one
    chunk per query head, later ones chunks (prefill: 128 rows, merged by a
    second kernel; decode: 256 rows, merged in the output projection's
    prologue); prefill chunks and decode steps on both sides, for 1, 2, 4 and
    8 query heads per KV head and head sizes 64 and 128."""
    spec = synth.tiny_llama(seed=6 + heads + kv_heads + hd, embd=hd * heads, heads=heads, kv_heads=kv_heads)
    g, cpu = _open(spec, 512)
    prompt = synth.prompt(7, prompt_len, spec.vocab)
    _check(g, cpu, prompt, (320 if hd == 64 else 200) - prompt_len)


@pytest.mark.parametrize("hd,ctx,prompt_len", [(64, 512, 300), (128, 512, 150), (64, 4096, 2100)])
def test_att_merged_in_projection(gpu, hd, ctx, prompt_len):
    """One-token passes past the one-chunk bound run the split attention and
    merge its chunk partials in the output projection's prologue (no merge
    kernel): 2, 2 and 10 chunks of 256 rows here.  Peek("att") -- the last
    layer's merged attention output, which the projection's first tile also
    stores -- against the oracle's after the last of four decode steps, and
    the tokens against the oracle's."""
    spec = synth.tiny_qwen(seed=11 + hd, embd=4 * hd, ctx=max(ctx, 1024))
    g, cpu = _open(spec, ctx)
    prompt = [int(t) for t in synth.prompt(9, prompt_len, spec.vocab)]
    out = gpu_generate(g, prompt, 4)
    cpu.reset()
    for t in prompt + out[:3]:
        cpu.forward(t)
    rel = rel_err(g.Peek("att", spec.embd), cpu.last_att())
    print(f"att after decode at position {prompt_len + 2}: {rel:.2e}", flush=True)
    assert rel <= 1e-5
    toks, lgs = cpu_greedy(cpu, prompt, 4)
    greedy_parity(g, prompt, toks, lgs)


@pytest.mark.parametrize("prompt_len,heads,kv_heads", [(520, 14, 2), (330, 8, 8), (460, 9, 3)])
def test_prefill_attention_mma(gpu, prompt_len, heads, kv_heads):
    """The matrix-core form of prefill attention past 256 positions: query
    groups of 64 that cut across tokens (7, 1 and 3 query heads per KV head),
    a last prefill chunk of 8 tokens (520 = 8 x 64 + 8), chunks whose rows
    reach past some queries' causal bound, then decode steps over the cache
    it wrote."""
    spec = synth.tiny_llama(seed=40 + heads + kv_heads, embd=64 * heads, heads=heads, kv_heads=kv_heads, ctx=1024)
    g, cpu = _open(spec, 640)
    prompt = synth.prompt(8, prompt_len, spec.vocab)
    _check(g, cpu, prompt, 16)


@pytest.mark.parametrize("name,prompt_len,n", [("llama", 150, 40), ("qwen2", 150, 40), ("qwen2-split", 300, 24),
                                               ("llama-hd128", 140, 40)])
def test_f16_kv_cache(gpu, name, prompt_len, n):
    """The binary16 KV cache (F16KV, cpu.go:22-24, 298-299) against the oracle
    in the same mode: one-chunk and split attention, head sizes 64 and 128;
    the cache holds the oracle's rounded values exactly."""
    spec = {"llama": lambda: synth.tiny_llama(), "qwen2": lambda: synth.tiny_qwen(),
            "qwen2-split": lambda: synth.tiny_qwen(seed=8), "llama-hd128": lambda: synth.tiny_llama(
                seed=9, embd=256, heads=2, kv_heads=1)}[name]()
    g, cpu = _open(spec, 512, f16kv=True)
    prompt = synth.prompt(12, prompt_len, spec.vocab)
    _check(g, cpu, prompt, n)
    kvd = spec.kv_heads * (spec.embd // spec.heads)
    kv = g.Peek("kvblk.0", 2 * 512 * kvd).reshape(2, 512, kvd)[:, :prompt_len]
    assert np.array_equal(kv, kv.astype(np.float16).astype(np.float32)), "cache values are not binary16"
    assert np.all(np.abs(kv[:, 1:]).max(axis=-1) > 0)


def test_qwen25_f16_kv_cache(gpu):
    """BASELINE config 3's shape with the binary16 cache, against the oracle's F16KV mode."""
    spec = synth.qwen25()
    g, cpu = _open(spec, 512, f16kv=True)
    _check(g, cpu, synth.prompt(0, 128, spec.vocab), 64)


# ExactGGML end to end.  Every activation code is a discontinuous function
# of an f32 value: two correct implementations whose f32 sums round in a
# different order disagree on the codes that sit within that difference of a
# rounding boundary, and each such flip moves the logits by ~1e-3 (the
# independent float64 restatement of tests/test_oracle.py shows the same
# 2.7e-3 / 3.6e-3 steps against the oracle on the same tiny-model inputs).
# The products themselves are pinned on identical inputs at the summation
# bound (tests/test_gemv_gpu.py::test_exact_ggml_gemv).  End to end every
# run is held to the flip level -- EXACT_TOL on the tiny models, where one
# flip moves the logits by 2.7e-3 to 6.6e-3 (measured, GPU and float64
# restatement alike), and 5e-3 and closer to the oracle's ExactGGML than to
# its f32 mode at the Qwen shape -- with greedy tokens equal up to near-ties
# at that level.  A flip can happen at any prompt length: a 3-token prompt of
# the mixed-type model was measured with its first layer's output within
# 7.5e-9 of the oracle's and one flip in the second layer (225 of 256 rows of
# its output 1e-4..4e-4 off, logits 4.1e-3), while the same prompts in f32
# mode stay below 1e-6 (test_short_prompts).
EXACT_TOL = 1e-2
EXACT_TINY = dict(TINY, **{"qwen2-split": lambda: synth.tiny_qwen(seed=8)})


def _short_prompts(g, cpu, spec):
    out = []
    for plen in (1, 2, 3, 4):
        prompt = list(synth.prompt(20 + plen, plen, spec.vocab))
        cpu.reset()
        for t in prompt:
            want = cpu.forward(t)
        out.append(rel_err(g.PrefillLogits(prompt), want))
        print(f"prompt {plen}: logits relative error {out[-1]:.3e}", flush=True)
    return out


@pytest.mark.parametrize("name", list(TINY))
def test_short_prompts(gpu, name):
    """Prompts of 1 to 4 tokens run the decode tile kernel with 1, 2 and 4
    token slots (one pass each): logits within 1e-4 of the oracle's."""
    spec = TINY[name]()
    g, cpu = _open(spec, 128)
    assert max(_short_prompts(g, cpu, spec)) <= LOGIT_TOL


@pytest.mark.parametrize("name", list(TINY))
def test_exact_ggml_short(gpu, name):
    """ExactGGML (cpu.go:15-21, 117-140, 166-214) through the decode kernels
    with 1, 2 and 4 token slots: prompts of 1 to 4 tokens, logits within the
    flip level of the oracle's."""
    spec = TINY[name]()
    g, cpu = _open(spec, 128, exact=True)
    assert max(_short_prompts(g, cpu, spec)) <= EXACT_TOL


@pytest.mark.parametrize("name,prompt_len,n", [("llama", 150, 40), ("qwen2", 150, 40), ("qwen2-mixed", 150, 40),
                                               ("llama-untied-q41", 100, 30), ("qwen2-split", 300, 24)])
def test_exact_ggml(gpu, name, prompt_len, n):
    """ExactGGML through the prefill pair, both attention forms and decode:
    Q8_0 / Q8_1 activation blocks for Q4_0, Q4_1 and Q8_0 weights, the
    binary16 cache; logits and greedy tokens at the flip level."""
    spec = EXACT_TINY[name]()
    g, cpu = _open(spec, 512, exact=True)
    prompt = synth.prompt(13, prompt_len, spec.vocab)
    logits = g.PrefillLogits(prompt)
    toks, lgs = cpu_greedy(cpu, prompt, n)
    rel = rel_err(logits, lgs[0])
    print(f"step-1 logits relative error {rel:.3e}", flush=True)
    assert rel <= EXACT_TOL
    ties = greedy_parity(g, prompt, toks, lgs, tol=EXACT_TOL)
    print(f"{n} greedy tokens equal ({ties} accepted near-ties)", flush=True)
    kvd = spec.kv_heads * (spec.embd // spec.heads)
    kv = g.Peek("kvblk.0", 2 * 512 * kvd).reshape(2, 512, kvd)[:, :prompt_len]
    assert np.array_equal(kv, kv.astype(np.float16).astype(np.float32)), "cache values are not binary16"


def test_qwen25_exact_ggml(gpu):
    """BASELINE config 3's shape in the ExactGGML mode: ~180k activation codes
    per token, so flips are certain; measured 0.7e-3 to 1.2e-3 from the
    oracle's ExactGGML against 2.3e-3 to 3.2e-3 between the oracle's own f32
    and ExactGGML modes."""
    from oracle import cpuref
    spec = synth.qwen25()
    g, cpu = _open(spec, 512, exact=True)
    cpu32 = cpuref.CPU(synth.cached(spec), 512, threads=16)
    prompt = synth.prompt(0, 128, spec.vocab)
    logits = g.PrefillLogits(prompt)
    toks, lgs = cpu_greedy(cpu, prompt, 48)
    for t in prompt:
        l32 = cpu32.forward(t)
    rel, rel32 = rel_err(logits, lgs[0]), rel_err(logits, l32)
    print(f"step-1 logits: {rel:.3e} from the oracle's ExactGGML, {rel32:.3e} from its f32 mode", flush=True)
    assert rel <= 5e-3 and rel <= 0.6 * rel32
    ties = greedy_parity(g, prompt, toks, lgs, tol=5e-3)
    print(f"48 greedy tokens equal ({ties} accepted near-ties)", flush=True)


def test_decode_batches_and_stops(gpu):
    from llm_amd import llm
    spec = synth.tiny_qwen()
    g, cpu = _open(spec, 512)
    prompt = synth.prompt(2, 37, spec.vocab)
    ref = gpu_generate(g, prompt, 30)
    old = llm.DecodeBatch
    try:
        for b in (1, 3, 8, 16, 40):
            llm.DecodeBatch = b
            assert gpu_generate(g, prompt, 30) == ref, f"decode batch {b}"
    finally:
        llm.DecodeBatch = old
    # eos is not emitted and ends the generation (gpu.go:971-976)
    out = []
    tm = g.Generate(list(prompt), 30, ref[5], lambda t: out.append(t) or True)
    assert out == ref[:ref.index(ref[5])] and tm.Generated == len(out)
    # emit returning false stops after that token (gpu.go:979-982)
    out = []
    g.Generate(list(prompt), 30, -1, lambda t: out.append(t) or len(out) < 4)
    assert out == ref[:4]
    # n = 0 generates nothing; n = 1 is the prefill's token
    assert gpu_generate(g, prompt, 0) == []
    assert gpu_generate(g, prompt, 1) == ref[:1]


def test_trace_layers(gpu):
    """The residual stream after k layers (trace mode, examples/generate/main.go:212-240)."""
    spec = synth.tiny_llama(layers=3)
    g, cpu = _open(spec, 128)
    prompt = synth.prompt(3, 5, spec.vocab)
    for k in (-1, 1, 2, 3):
        g.Layers = k
        cpu.set_max_layers(k)
        cpu.reset()
        for t in prompt:
            cpu.forward(t)
        want = cpu.last_x()
        g.PrefillLogits(prompt)
        pm = 64
        got = g.Peek("x", spec.embd * len(prompt)).reshape(len(prompt), spec.embd)[-1]
        rel = rel_err(got, want)
        print(f"layers {k}: x relative error {rel:.3e}", flush=True)
        assert rel <= 1e-5 if k != -1 else np.array_equal(got.view(np.uint32), want.view(np.uint32))
    g.Layers = 0
    st = g.Peek("state", 2).view(np.uint32)
    assert list(st) == [len(prompt), len(prompt)]


def test_state_and_tokens(gpu):
    spec = synth.tiny_llama()
    g, cpu = _open(spec, 256)
    prompt = synth.prompt(4, 70, spec.vocab)
    out = gpu_generate(g, prompt, 12)
    toks = g.Peek("tokens", 70 + 12).view(np.int32)
    assert list(toks[:70]) == list(prompt) and list(toks[70:]) == out
    st = g.Peek("state", 2).view(np.uint32)
    assert list(st) == [70 + 11, 70 + 11]
    assert g.Peek("outb", 1).view(np.int32)[0] == out[-1]
    s = g.Stats
    assert s.dispatches > 0 and s.submits > 0


@pytest.mark.parametrize("name", ["qwen2", "qwen2-mixed"])
def test_peek_buffers(gpu, name):
    """Peek's trace buffers (gpu.go:513-516, 1015-1043) against the oracle's
    values of the same pass, after a two-chunk prefill and after decode steps:
    h (the head's input: RMSNorm of the last residual row with output_norm),
    up (the last layer's up product, through the fused gate/up epilogue and,
    for gate and up of different types, the SwiGLU one), k and v (the cache
    rows the pass appended last, in the last layer)."""
    spec = TINY[name]()
    g, cpu = _open(spec, 256)
    L, E, F, kvd = spec.layers, spec.embd, spec.ff, spec.kvd
    prompt = [int(t) for t in synth.prompt(8, 70, spec.vocab)]

    def check(fed, last_row):
        cpu.reset()
        for t in fed:
            cpu.forward(t)
        h = g.Peek("h", E)
        up = g.Peek("up", (last_row + 1) * F)[last_row * F:]
        k, v = g.Peek("k", kvd), g.Peek("v", kvd)
        errs = [rel_err(h, cpu.last_h()), rel_err(up, cpu.last_up()),
                rel_err(k, cpu.kv_row(L - 1, len(fed) - 1)), rel_err(v, cpu.kv_row(L - 1, len(fed) - 1, v=True))]
        print(f"{len(fed)} tokens fed: h {errs[0]:.2e} up {errs[1]:.2e} k {errs[2]:.2e} v {errs[3]:.2e}", flush=True)
        assert max(errs) <= 1e-5
        kv = g.Peek(f"kvblk.{L - 1}.", 2 * 256 * kvd).reshape(2, 256, kvd)
        assert np.array_equal(k, kv[0, len(fed) - 1]) and np.array_equal(v, kv[1, len(fed) - 1])

    g.PrefillLogits(prompt)  # chunks of 64 and 6 tokens: the last pass's last token is row 5
    check(prompt, 5)
    out = gpu_generate(g, prompt, 5)  # the prefill, then 4 decode steps of one token
    check(prompt + out[:4], 0)
    with pytest.raises(Exception):
        g.Peek("h", E + 1)


def test_refusals(gpu):
    from llm_amd import llm
    from llm_amd._lib import LLMError
    spec = synth.tiny_llama()
    path = synth.cached(spec)
    g = llm.NewGPU(0, None, path, 64)
    with pytest.raises(LLMError) as e:
        g.Generate([1] * 60, 10)  # gpu.go:948-950
    assert e.value.kind == "CONTEXT"
    with pytest.raises(LLMError) as e:
        g.PrefillLogits([1] * 64)  # gpu.go:905-907
    assert e.value.kind == "CONTEXT"
    with pytest.raises(LLMError) as e:
        g.Generate([], 3)  # gpu.go:854-856
    assert "empty prompt" in str(e.value)
    with pytest.raises(LLMError) as e:
        g.Generate([spec.vocab], 3)
    assert e.value.kind == "ARG"
    with pytest.raises(LLMError) as e:
        g.Peek("nothing", 1)
    lim = llm.DefaultLimits()
    lim.memory_budget = 4096
    with pytest.raises(LLMError) as e:
        llm.NewGPU(0, lim, path, 64)  # gpu.go:175-177
    assert e.value.kind == "BUDGET"
    # the budget is what MemoryUsed reports
    lim.memory_budget = g.MemoryUsed()
    g2 = llm.NewGPU(0, lim, path, 64)
    assert g2.MemoryUsed() <= lim.memory_budget
    # head sizes without an attention kernel are refused at load
    with pytest.raises(LLMError) as e:
        llm.NewGPU(0, None, synth.cached(synth.tiny_llama(seed=9, embd=192, heads=2)), 64)
    assert e.value.kind == "FORMAT" and "head size 96" in str(e.value)


@pytest.mark.parametrize("config", ["smollm2", "qwen25"])
def test_baseline_shapes(gpu, config):
    """BASELINE configs 2 and 3: 128-token prompt in 64-token chunks, 128 greedy tokens, ctx 512."""
    spec = synth.smollm2() if config == "smollm2" else synth.qwen25()
    g, cpu = _open(spec, 512)
    prompt = synth.prompt(0, 128, spec.vocab)
    _check(g, cpu, prompt, 128)


