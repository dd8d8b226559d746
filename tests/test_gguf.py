"""The C++ GGUF header parser and ConfigFrom (host layer, llm_gguf_* /
llm_config_from), on the CPU: the reference's gguf_test.go cases restated, its
fuzz corpus (tests/golden/gguf_fuzz, copied from gguf/testdata/fuzz/FuzzParse),
random mutations of a valid header, the refusals of config.go:29-73, and a
cross-check against the oracle's independent reader on the synthetic models.
"""
import glob
import os
import struct

import numpy as np
import pytest

from llm_amd import llm, synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
U32, F32_, STR = 4, 6, 8


def build(mut=None):
    """gguf_test.go:13-40: one metadata string, one U32, one F32 tensor of 4."""
    b = bytearray(b"GGUF")
    w = lambda fmt, *v: b.extend(struct.pack("<" + fmt, *v))

    def s(x):
        w("Q", len(x))
        b.extend(x.encode())

    w("I", 3)
    w("Q", 1)
    w("Q", 2)
    s("general.architecture")
    w("I", STR)
    s("llama")
    s("x.count")
    w("I", U32)
    w("I", 7)
    s("w")
    w("I", 1)
    w("Q", 4)
    w("I", 0)
    w("Q", 0)
    while len(b) % 32:
        b.append(0)
    b.extend(bytes(16))
    if mut:
        mut(b)
    return bytes(b)


def test_parse():
    """TestParse, gguf_test.go:42-58."""
    f = llm.Parse(build())
    assert f.Str("general.architecture") == ("llama", True)
    assert f.Uint("x.count") == (7, True)
    t, ok = f.Tensor("w")
    assert ok and t.Size == 16 and f.DataOffset % 32 == 0 and t.Dims == [4] and t.Type == 0


def test_refusals():
    """TestRefusals, gguf_test.go:60-78."""
    d = build()
    cases = {
        "magic": (b"GGUX" + d[4:], "magic"),
        "version": (d[:4] + b"\x02" + d[5:], "version"),
        "tensors": (d[:15] + b"\x7f" + d[16:], "bound"),
        "truncated": (d[:40], None),
        "past end": (d[:-4], "bound"),
    }
    for name, (data, kind) in cases.items():
        with pytest.raises(llm.GGUFError) as e:
            llm.Parse(data)
        if kind:
            assert e.value.gguf_kind == kind, name


def _go_bytes(text):
    """The []byte("...") literal of a `go test fuzz v1` corpus file."""
    body = text.split("\n", 1)[1].strip()
    assert body.startswith('[]byte("') and body.endswith('")')
    s = body[len('[]byte("'):-2]
    out = bytearray()
    i = 0
    simple = {"n": 10, "t": 9, "r": 13, "a": 7, "b": 8, "f": 12, "v": 11, "\\": 92, '"': 34, "'": 39}
    while i < len(s):
        ch = s[i]
        if ch != "\\":
            out.extend(ch.encode())
            i += 1
            continue
        e = s[i + 1]
        if e == "x":
            out.append(int(s[i + 2:i + 4], 16))
            i += 4
        elif e in "uU":
            n = 4 if e == "u" else 8
            out.extend(chr(int(s[i + 2:i + 2 + n], 16)).encode())
            i += 2 + n
        elif e in simple:
            out.append(simple[e])
            i += 2
        else:
            out.append(int(s[i + 1:i + 4], 8))
            i += 4
    return bytes(out)


def test_fuzz_corpus():
    """FuzzParse (gguf_test.go:80-85) over the reference's committed corpus:
    every input either parses or is refused with a typed error; none crashes
    and none reads past the bytes it was given."""
    files = sorted(glob.glob(os.path.join(GOLDEN, "gguf_fuzz", "*")))
    assert len(files) == 216
    kinds = {}
    for p in files:
        data = _go_bytes(open(p, encoding="utf-8").read())
        try:
            f = llm.Parse(data)
            assert f.DataOffset <= len(data) or not f.Tensors
            for t in f.Tensors:
                assert f.DataOffset + t.Offset + t.Size <= len(data)
            kinds["ok"] = kinds.get("ok", 0) + 1
        except llm.GGUFError as e:
            assert e.gguf_kind in ("magic", "version", "bound", "format", "io")
            kinds[e.gguf_kind] = kinds.get(e.gguf_kind, 0) + 1
    assert sum(kinds.values()) == 216


def test_random_mutations():
    """Byte flips, truncations and extensions of a valid header never crash."""
    rng = np.random.default_rng(0)
    base = bytearray(build())
    for _ in range(3000):
        d = bytearray(base)
        for _ in range(rng.integers(1, 6)):
            d[rng.integers(0, len(d))] = rng.integers(0, 256)
        if rng.random() < 0.3:
            d = d[:rng.integers(0, len(d))]
        try:
            llm.Parse(bytes(d))
        except llm.GGUFError:
            pass


def test_alignment():
    """general.alignment must be a positive multiple of 8 (gguf/gguf.go:335-342)."""
    tens = [("w", [4], 0)]
    for al, ok in ((64, True), (8, True), (12, False), (0, False)):
        meta = [("general.alignment", U32, al)]
        if ok:
            f = llm.Parse(_header(meta, tens, align=al))
            assert f.Alignment == al and f.DataOffset % al == 0
        else:
            with pytest.raises(llm.GGUFError) as e:
                llm.Parse(_header(meta, tens))
            assert e.value.gguf_kind == "format"


def test_config_from_synthetic(tmp_path):
    for spec in (synth.tiny_llama(), synth.tiny_qwen(), synth.smollm2(), synth.qwen25()):
        path = synth.cached(spec)
        c = llm.ConfigFrom(llm.Parse(path))
        assert (c.layers, c.embd, c.ff, c.heads, c.kv_heads, c.vocab) == \
               (spec.layers, spec.embd, spec.ff, spec.heads, spec.kv_heads, spec.vocab)
        assert c.head_dim == spec.embd // spec.heads and c.ctx == spec.ctx
        assert c.rope_base == np.float32(spec.rope_base) and c.eps == np.float32(spec.eps)
        assert c.arch == (spec.arch == "qwen2") and c.rope_neox == (spec.arch == "qwen2")
        assert c.bias == (spec.arch == "qwen2") and c.tied_output == spec.tied


def _header(meta, tensors, align=32):
    """A GGUF header with the given metadata [(key, type, value)] and tensors
    [(name, dims, type)], data section zero-filled."""
    b = bytearray(b"GGUF")
    b += struct.pack("<IQQ", 3, len(tensors), len(meta))

    def s(x):
        b.extend(struct.pack("<Q", len(x)) + x.encode())

    for k, t, v in meta:
        s(k)
        b.extend(struct.pack("<I", t))
        if t == STR:
            s(v)
        elif t == U32:
            b.extend(struct.pack("<I", v))
        else:
            b.extend(struct.pack("<f", v))
    off = 0
    sizes = []
    for name, dims, ty in tensors:
        be, bb = synth.BLOCK[ty]
        size = int(np.prod(dims)) // be * bb
        s(name)
        b.extend(struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims))
        b.extend(struct.pack("<IQ", ty, off))
        sizes.append(size)
        off += (size + align - 1) // align * align
    while len(b) % align:
        b.append(0)
    b.extend(bytes(off))
    return bytes(b)


def _cfg_meta(arch="llama", **over):
    m = {"general.architecture": (STR, arch), f"{arch}.block_count": (U32, 1), f"{arch}.embedding_length": (U32, 64),
         f"{arch}.feed_forward_length": (U32, 128), f"{arch}.attention.head_count": (U32, 2),
         f"{arch}.attention.head_count_kv": (U32, 1), f"{arch}.context_length": (U32, 256),
         f"{arch}.rope.freq_base": (F32_, 1e4), f"{arch}.attention.layer_norm_rms_epsilon": (F32_, 1e-5)}
    for k, v in over.items():
        k = k.replace("__", ".")
        if v is None:
            m.pop(k, None)
        else:
            m[k] = v
    return [(k, t, v) for k, (t, v) in m.items()]


def test_config_from_refusals():
    """config.go:29-73."""
    tens = [("token_embd.weight", [64, 100], synth.Q4_0)]
    ok = llm.ConfigFrom(llm.Parse(_header(_cfg_meta(), tens)))
    assert ok.vocab == 100 and ok.tied_output and not ok.bias and ok.head_dim == 32
    # no head_count_kv: KVHeads = Heads; no freq_base: 10000
    c = llm.ConfigFrom(llm.Parse(_header(_cfg_meta(**{"llama.attention.head_count_kv": None,
                                                      "llama.rope.freq_base": None}), tens)))
    assert c.kv_heads == c.heads and c.rope_base == 10000
    bad = {
        "arch": (_cfg_meta("gpt2"), tens),
        "heads": (_cfg_meta(**{"llama.attention.head_count": (U32, 3)}), tens),
        "kvheads": (_cfg_meta(**{"llama.attention.head_count_kv": (U32, 3)}), tens),
        "layers": (_cfg_meta(**{"llama.block_count": None}), tens),
        "rope_dim": (_cfg_meta() + [("llama.rope.dimension_count", U32, 16)], tens),
        "scaling": (_cfg_meta() + [("llama.rope.scaling.type", STR, "linear")], tens),
        "no_embd": (_cfg_meta(), [("output.weight", [64, 100], synth.Q8_0)]),
        "llama_bias": (_cfg_meta(), tens + [("blk.0.attn_q.bias", [64], 0)]),
        "qwen_no_bias": (_cfg_meta("qwen2"), tens),
    }
    for name, (meta, t) in bad.items():
        with pytest.raises(llm.LLMError) as e:
            llm.ConfigFrom(llm.Parse(_header(meta, t)))
        assert e.value.kind == "FORMAT", name
        assert str(e.value).startswith("llm: "), name
    c = llm.ConfigFrom(llm.Parse(_header(_cfg_meta("qwen2"), tens + [("blk.0.attn_q.bias", [64], 0)])))
    assert c.rope_neox and c.bias


def test_parser_agrees_with_oracle_reader():
    """Tensor table of the product parser vs the oracle's independent reader."""
    from oracle import cpuref
    for spec in (synth.tiny_qwen(), synth.tiny_llama(embd_type=synth.Q8_0)):
        path = synth.cached(spec)
        f = llm.Parse(path)
        cpu = cpuref.CPU(path, 8)
        raw = open(path, "rb").read()
        for t in f.Tensors:
            data, ty, dims = cpu.tensor(t.Name)
            assert ty == t.Type and dims[:len(t.Dims)] == t.Dims and len(data) == t.Size
            assert data == raw[f.DataOffset + t.Offset:f.DataOffset + t.Offset + t.Size]
