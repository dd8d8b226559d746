"""The loader's paths build bit-identical models.

The C++ host loader (llm_new_gpu: runs of consecutive tensors read from the
file straight into pinned staging, llmhip_model_upload_file_tensors) against
the device layer driven the way the Go binding drives it (every tensor
declared, then PieceSize pieces of whole blocks from host memory through
llmhip_model_upload, as streamMat reads them, gpu.go:356-389), against ragged
whole-block file pieces in shuffled order (llmhip_model_upload_file), and
against one batched call over the tensors in a shuffled order.  Equal models give equal
bits: the step-1 logits and every layer's KV cache after a prefill are
compared bit for bit.  Also the loader's refusals (bad descriptor, a read past
the end of the file, pieces that are not whole blocks).
"""
import ctypes
import os

import numpy as np
import pytest

from llm_amd import synth

pytestmark = pytest.mark.gpu

BLOCK = {0: (1, 4), 2: (32, 18), 3: (32, 20), 8: (32, 34)}  # ggml type -> (elements, bytes) per block
PIECE = 4 << 20


def _create(path, ctx):
    from llm_amd import _lib, llm
    L = _lib.lib()
    f = llm.Parse(path)
    cfg = llm.ConfigFrom(f)
    m = ctypes.c_void_p()
    llm.check(L.llmhip_model_create(0, None, ctypes.byref(cfg), ctx, 64, ctypes.byref(m)))
    for t in f.Tensors:
        dims = (ctypes.c_uint64 * len(t.Dims))(*t.Dims)
        llm.check(L.llmhip_model_tensor(m, t.Name.encode(), t.Type, dims, len(t.Dims)))
    return L, f, cfg, m


def _pieces(t, rng):
    """Ragged whole-block pieces of a tensor, shuffled: [(byte offset, bytes)]."""
    bb = BLOCK[t.Type][1]
    nblk = t.Size // bb
    cuts = sorted(set(rng.integers(1, max(nblk, 2), size=min(6, max(nblk - 1, 0))).tolist()))
    edges = [0] + [c for c in cuts if 0 < c < nblk] + [nblk]
    out = [(a * bb, (b - a) * bb) for a, b in zip(edges, edges[1:])]
    rng.shuffle(out)
    return out


def _device_layer_load(path, ctx, mode, seed=0):
    from llm_amd import llm
    L, f, cfg, m = _create(path, ctx)
    rng = np.random.default_rng(seed)
    fd = os.open(path, os.O_RDONLY)
    try:
        for t in f.Tensors:
            base = f.DataOffset + t.Offset
            if mode == "pieces":  # the Go binding's protocol: PieceSize pieces from host memory, in order
                per = PIECE // BLOCK[t.Type][1] * BLOCK[t.Type][1]
                for a in range(0, t.Size, per):
                    n = min(per, t.Size - a)
                    buf = ctypes.create_string_buffer(os.pread(fd, n, base + a), n)
                    llm.check(L.llmhip_model_upload(m, t.Name.encode(), buf, n, a))
            elif mode == "ragged-file":  # ragged whole-block pieces read from the file, shuffled
                for a, n in _pieces(t, rng):
                    llm.check(L.llmhip_model_upload_file(m, t.Name.encode(), fd, base + a, n, a))
        if mode == "batch-shuffled":  # one batched call over the tensors in a shuffled order
            ts = list(f.Tensors)
            rng.shuffle(ts)
            names = (ctypes.c_char_p * len(ts))(*[t.Name.encode() for t in ts])
            offs = (ctypes.c_uint64 * len(ts))(*[f.DataOffset + t.Offset for t in ts])
            llm.check(L.llmhip_model_upload_file_tensors(m, fd, len(ts), names, offs))
        llm.check(L.llmhip_model_finalize(m))
    finally:
        os.close(fd)
    return L, cfg, m


def _prefill(L, m, vocab, prompt):
    from llm_amd import llm
    p = np.ascontiguousarray(prompt, np.int32)
    out = np.empty(vocab, np.float32)
    first = np.zeros(16, np.int32)
    llm.check(L.llmhip_model_prefill(m, p.ctypes.data_as(ctypes.c_void_p), p.size,
                                     out.ctypes.data_as(ctypes.c_void_p), first.ctypes.data_as(ctypes.c_void_p)))
    return out


def _kv(L, m, layer, n):
    from llm_amd import llm
    out = np.empty(n, np.float32)
    llm.check(L.llmhip_model_peek(m, f"kvblk.{layer}".encode(), out.ctypes.data_as(ctypes.c_void_p), n))
    return out


SPECS = {
    "qwen2-mixed": lambda: synth.tiny_qwen(seed=3, types={
        "attn_q": synth.Q8_0, "attn_k": synth.Q4_1, "attn_v": synth.Q4_0, "attn_output": synth.Q4_1,
        "ffn_gate": synth.Q8_0, "ffn_up": synth.Q4_0, "ffn_down": lambda l: synth.Q4_1 if l % 2 else synth.Q8_0}),
    "llama-tied": lambda: synth.tiny_llama(seed=4, layers=3),
    "qwen25": lambda: synth.qwen25(),
}


@pytest.mark.parametrize("name", list(SPECS))
@pytest.mark.parametrize("mode", ["pieces", "ragged-file", "batch-shuffled"])
def test_loaders_agree(gpu, name, mode):
    from llm_amd import _lib, llm
    spec = SPECS[name]()
    path = synth.cached(spec)
    ctx = 256
    print(f"model {name} at {path}, device-layer load mode {mode}", flush=True)
    g = llm.NewGPU(0, None, path, ctx)
    L = _lib.lib()
    m_fast = g._m
    L2, cfg, m = _device_layer_load(path, ctx, mode, seed=len(name))
    try:
        prompt = synth.prompt(5, 70, spec.vocab)
        want = _prefill(L, m_fast, spec.vocab, prompt)
        got = _prefill(L2, m, spec.vocab, prompt)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "step-1 logits differ"
        kvn = 2 * ctx * cfg.kv_heads * cfg.head_dim
        for layer in range(cfg.layers):
            assert np.array_equal(_kv(L2, m, layer, kvn).view(np.uint32), _kv(L, m_fast, layer, kvn).view(np.uint32)), layer
        assert L2.llmhip_model_memory_used(m) == g.MemoryUsed()
    finally:
        L2.llmhip_model_free(m)


def test_loader_refusals(gpu, tmp_path):
    from llm_amd import _lib, llm
    from llm_amd._lib import LLMError
    spec = synth.tiny_llama(seed=4, layers=3)
    path = synth.cached(spec)
    L, f, cfg, m = _create(path, 64)
    try:
        t = next(t for t in f.Tensors if t.Type == 2)
        bb = BLOCK[2][1]
        size = os.path.getsize(path)
        fd = os.open(path, os.O_RDONLY)
        try:
            with pytest.raises(LLMError) as e:
                llm.check(L.llmhip_model_upload_file(m, t.Name.encode(), -1, 0, bb, 0))
            assert e.value.kind == "ARG"
            with pytest.raises(LLMError) as e:  # past the end of the file: a short read, nothing staged
                llm.check(L.llmhip_model_upload_file(m, t.Name.encode(), fd, size - bb // 2, 2 * bb, 0))
            assert e.value.kind == "IO" and "short read" in str(e.value)
            with pytest.raises(LLMError) as e:  # not whole blocks
                llm.check(L.llmhip_model_upload_file(m, t.Name.encode(), fd, f.DataOffset + t.Offset, bb + 1, 0))
            assert e.value.kind == "ARG"
            with pytest.raises(LLMError) as e:  # a tensor never declared
                names = (ctypes.c_char_p * 1)(b"blk.0.nothing.weight")
                offs = (ctypes.c_uint64 * 1)(f.DataOffset)
                llm.check(L.llmhip_model_upload_file_tensors(m, fd, 1, names, offs))
            assert e.value.kind == "ARG"
            with pytest.raises(LLMError) as e:  # a batch that runs past the end of the file
                names = (ctypes.c_char_p * 1)(t.Name.encode())
                offs = (ctypes.c_uint64 * 1)(size - bb)
                llm.check(L.llmhip_model_upload_file_tensors(m, fd, 1, names, offs))
            assert e.value.kind == "IO"
            with pytest.raises(LLMError) as e:  # past the tensor
                llm.check(L.llmhip_model_upload_file(m, t.Name.encode(), fd, f.DataOffset + t.Offset, t.Size, bb))
            assert e.value.kind == "ARG"
        finally:
            os.close(fd)
        with pytest.raises(LLMError) as e:  # nothing complete yet
            llm.check(L.llmhip_model_finalize(m))
        assert e.value.kind == "FORMAT"
    finally:
        L.llmhip_model_free(m)
    # a truncated file is refused by the header parser before any upload
    data = open(path, "rb").read()
    bad = tmp_path / "truncated.gguf"
    bad.write_bytes(data[: len(data) - 100])
    with pytest.raises(LLMError):
        llm.NewGPU(0, None, str(bad), 64)


def test_upload_coverage(gpu):
    """Upload completeness counts covered bytes, not received bytes: a range
    that overlaps one uploaded before is refused (so a tensor half of which
    came twice is never taken as complete), a tensor listed twice in one
    batched call is refused, and finalize accepts the model once every byte
    arrived exactly once (its logits then equal the fast loader's)."""
    from llm_amd import _lib, llm
    from llm_amd._lib import LLMError
    spec = synth.tiny_llama(seed=4, layers=3)
    path = synth.cached(spec)
    L, f, cfg, m = _create(path, 64)
    fd = os.open(path, os.O_RDONLY)
    try:
        t = next(t for t in f.Tensors if t.Type == 2 and t.Name.startswith("blk.1."))
        bb = BLOCK[2][1]
        half = t.Size // bb // 2 * bb
        base = f.DataOffset + t.Offset

        def up(a, n):
            llm.check(L.llmhip_model_upload_file(m, t.Name.encode(), fd, base + a, n, a))

        up(0, half)
        for a, n in ((0, half), (bb, bb), (half - bb, 2 * bb), (0, t.Size)):
            with pytest.raises(LLMError) as e:
                up(a, n)
            assert e.value.kind == "ARG" and "overlaps" in str(e.value), (a, n)
        with pytest.raises(LLMError) as e:  # the same tensor twice in one batch
            names = (ctypes.c_char_p * 2)(b"output_norm.weight", b"output_norm.weight")
            o = f.DataOffset + f.Tensor("output_norm.weight")[0].Offset
            offs = (ctypes.c_uint64 * 2)(o, o)
            llm.check(L.llmhip_model_upload_file_tensors(m, fd, 2, names, offs))
        assert e.value.kind == "ARG" and "twice" in str(e.value)
        # everything else, then t's second half in two pieces (adjacent ranges merge)
        rest = [x for x in f.Tensors if x.Name != t.Name]
        names = (ctypes.c_char_p * len(rest))(*[x.Name.encode() for x in rest])
        offs = (ctypes.c_uint64 * len(rest))(*[f.DataOffset + x.Offset for x in rest])
        llm.check(L.llmhip_model_upload_file_tensors(m, fd, len(rest), names, offs))
        with pytest.raises(LLMError) as e:  # half of t still missing
            llm.check(L.llmhip_model_finalize(m))
        assert e.value.kind == "FORMAT" and t.Name in str(e.value)
        mid = half + (t.Size - half) // bb // 2 * bb
        up(mid, t.Size - mid)
        up(half, mid - half)
        llm.check(L.llmhip_model_finalize(m))
        g = llm.NewGPU(0, None, path, 64)
        prompt = synth.prompt(5, 9, spec.vocab)
        want = _prefill(_lib.lib(), g._m, spec.vocab, prompt)
        got = _prefill(L, m, spec.vocab, prompt)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        g.close()
    finally:
        os.close(fd)
        L.llmhip_model_free(m)
