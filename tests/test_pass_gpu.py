"""The fused decode pass (llm_amd/csrc/pass.hip): every layer of a decode step
in one persistent launch whose phases hand their results to each other through
flag-carrying words.  Against the CPU oracle (logits and greedy tokens, as the
other parity tests) and against the same model's steps taken one launch per
kernel, on tiny models of every matrix type, both head sizes, NORM and NEOX
RoPE and the binary16 cache, and at the BASELINE configs' shapes; plus the
bounded wait: a host-forced poll limit of one makes the decode call fail and
later steps fall back to one launch per kernel."""
import pytest

from llm_amd import synth
from tests.parity import cpu_greedy, gpu_generate, greedy_parity
from tests.test_model_gpu import TINY, _check, _open

pytestmark = pytest.mark.gpu

CASES = {
    "llama": lambda: TINY["llama"](),
    "qwen2": lambda: TINY["qwen2"](),
    "llama-q8embd": lambda: TINY["llama-q8embd"](),          # Q4_1 down, Q8_0 output projection
    "llama-untied-q41": lambda: TINY["llama-untied-q41"](),  # 3 layers, Q4_1 head
    "qwen2-q8": lambda: synth.tiny_qwen(seed=21, types={"attn_q": synth.Q8_0, "attn_k": synth.Q8_0,
                                                        "attn_v": synth.Q8_0, "ffn_gate": synth.Q8_0,
                                                        "ffn_up": synth.Q8_0}),
    "llama-hd128": lambda: synth.tiny_llama(seed=9, embd=256, heads=2, kv_heads=1),
    "llama-gqa4-6layers": lambda: synth.tiny_llama(seed=22, embd=512, heads=8, kv_heads=2, layers=6, ff=640),
}


def _fused(g):
    taken, why = g.set_fused(True)
    assert taken, why
    return taken


@pytest.mark.parametrize("name", list(CASES))
def test_pass_parity(gpu, name):
    """Decode steps through the fused launch against the oracle, and the
    logits of a decode step against those of the same step taken one launch
    per kernel (the same arithmetic, summed in another order)."""
    spec = CASES[name]()
    g, cpu = _open(spec, 256)
    _fused(g)
    prompt = synth.prompt(41, 70, spec.vocab)
    _check(g, cpu, prompt, 60)
    _fused_vs_plain(g, spec, prompt)


def _fused_vs_plain(g, spec, prompt):
    """The logits after 1 and 8 decode steps through the fused launch against
    those of the same steps taken one launch per kernel (the same arithmetic,
    summed in another order), where the tokens agree."""
    import numpy as np
    from tests.parity import rel_err
    for steps in (2, 9):
        fused = gpu_generate(g, prompt, steps)
        lf = g.Peek("logits", spec.vocab)
        g.set_fused(False)
        plain = gpu_generate(g, prompt, steps)
        lp = g.Peek("logits", spec.vocab)
        _fused(g)
        print(f"{steps - 1} decode steps: tokens equal {fused == plain}, logits {rel_err(lf, lp):.2e}", flush=True)
        if fused == plain:
            assert rel_err(lf, lp) <= 1e-5 and np.all(np.isfinite(lf))


@pytest.mark.parametrize("start,kv16", [(250, False), (300, False), (505, False), (1500, False), (1500, True)])
def test_pass_long_context(gpu, start, kv16):
    """Decode steps past attn_full_max through the long form of the fused
    launch (256-row chunks, one workgroup per query head and chunk, the last
    chunk's workgroup merging the others): against the oracle, and against
    the same steps taken one launch per kernel (the split attention).  From
    250 the steps cross 256: a submit whose last position is past it runs all
    its steps in the long form, those below 256 as one chunk; from 505 a
    submit crosses 512, where the graph variant's rows grow; at 1500 also
    with the binary16 cache."""
    spec = synth.tiny_qwen(seed=24, ctx=2048)
    g, cpu = _open(spec, 2048, f16kv=kv16)
    _fused(g)
    prompt = synth.prompt(43, start, spec.vocab)
    _check(g, cpu, prompt, 24)
    _fused_vs_plain(g, spec, prompt)


def test_pass_long_form_all_chunks(gpu):
    """The long form at its most chunks (16 of 256 rows: positions past 3584
    at ctx 4096) with 14 query heads on 2 KV heads, as at the Qwen shape: the
    query heads of a (chunk, KV head) pair, grouped on one XCD, then take
    224 workgroups and reach down into those of the [q; k; v] tiles, which run
    both phases in turn.  Against the oracle and against the same steps one
    launch per kernel; the dispatch counts show the fused launch ran."""
    spec = synth.tiny_qwen(seed=25, embd=896, heads=14, kv_heads=2, ff=512, ctx=4096)
    g, cpu = _open(spec, 4096)
    _fused(g)
    prompt = synth.prompt(44, 3900, spec.vocab)
    fused = g.Generate(list(prompt), 9, -1)
    g.set_fused(False)
    plain = g.Generate(list(prompt), 9, -1)
    _fused(g)
    print(f"dispatches: fused {fused.Dispatches}, one launch per kernel {plain.Dispatches}", flush=True)
    assert fused.Dispatches + 8 * 2 * 4 <= plain.Dispatches
    _check(g, cpu, prompt, 8)
    _fused_vs_plain(g, spec, prompt)


@pytest.mark.parametrize("kv16", [False, True])
def test_pass_f16_kv(gpu, kv16):
    spec = synth.tiny_qwen(seed=23)
    g, cpu = _open(spec, 256, f16kv=kv16)
    _fused(g)
    _check(g, cpu, synth.prompt(42, 90, spec.vocab), 40)


@pytest.mark.parametrize("config", ["smollm2", "qwen25"])
def test_pass_baseline_shapes(gpu, config):
    """BASELINE configs 2 and 3 with the fused launch (their default): 128
    greedy tokens after a 128-token prompt, positions up to 255."""
    spec = synth.smollm2() if config == "smollm2" else synth.qwen25()
    g, cpu = _open(spec, 512)
    _fused(g)
    _check(g, cpu, synth.prompt(0, 128, spec.vocab), 128)


def test_pass_refusals(gpu):
    """Models the fused launch does not take say why, and decode one launch per kernel."""
    from llm_amd import llm
    spec = TINY["qwen2-mixed"]()  # q, k, v of different types: no fused [q; k; v] matrix
    g = llm.NewGPU(0, None, synth.cached(spec), 256)
    taken, why = g.set_fused(True)
    assert not taken and "different types" in why
    spec = synth.tiny_llama(seed=24, embd=1536, heads=12, kv_heads=4)
    g = llm.NewGPU(0, None, synth.cached(spec), 256)
    taken, why = g.set_fused(True)
    assert not taken and "embedding" in why


def test_pass_wait_limit(gpu):
    """A poll limit of one (set from the host): some hand-off of the first
    decode call cannot be met in one poll, the call reports the timed-out
    waits as a device error, and the model's later decode steps run one launch
    per kernel, correct against the oracle."""
    from llm_amd._lib import LLMError
    spec = TINY["llama"]()
    g, cpu = _open(spec, 256)
    taken, _ = g.set_fused(True, poll_limit=1)
    assert taken
    prompt = synth.prompt(43, 20, spec.vocab)
    with pytest.raises(LLMError) as e:
        gpu_generate(g, prompt, 8)
    print(e.value, flush=True)
    assert e.value.kind == "DEVICE" and "timed out" in str(e.value)
    taken, why = g.set_fused(True, poll_limit=0)
    assert not taken and "timed out" in why
    toks, lgs = cpu_greedy(cpu, prompt, 24)
    greedy_parity(g, prompt, toks, lgs)
