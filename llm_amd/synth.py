"""Seeded synthetic GGUF v3 models of the benchmark shapes.

There are no model files on the build or GPU machines, so every parity test
and benchmark runs on random-init weights written here, in the exact on-disk
format the reference's loader reads (gguf/gguf.go:292-407 layout; block
formats of cpu.go:164-215).  Distributions:

* Q4_0 block: d = f16(|N(0, 0.02)| / 8), 32 nibbles uniform in 0..15.
* Q4_1 block: d as Q4_0, m = f16(-8 d), nibbles uniform in 0..15.
* Q8_0 block: d = f16(|N(0, 0.02)| / div), int8 uniform in [-127, 127];
  div = 8 for the output matrix, 128 inside the layers (keeps the layer
  outputs at the scale of the Q4_0 layers).
* Norm weights f32 1 + N(0, 0.01); QKV biases f32 N(0, 0.02).
* Prompts: token ids uniform in [0, vocab).

Each tensor draws from its own generator seeded by (model seed, crc32(name)),
so a tensor's bytes do not depend on which other tensors the file holds.
"""
import atexit
import dataclasses
import os
import shutil
import struct
import tempfile
import zlib

import numpy as np

# ggml types (gguf/gguf.go:60-69) and (elements, bytes) per block (:72-92).
F32, F16, Q4_0, Q4_1, Q8_0 = 0, 1, 2, 3, 8
BLOCK = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q8_0: (32, 34)}
TYPE_NAMES = {"f32": F32, "q4_0": Q4_0, "q4_1": Q4_1, "q8_0": Q8_0}

# metadata value types (gguf/gguf.go:40-54)
_U32, _F32, _STR = 4, 6, 8


@dataclasses.dataclass
class Spec:
    """A model shape and its tensor types."""
    arch: str = "llama"
    layers: int = 30
    embd: int = 576
    heads: int = 9
    kv_heads: int = 3
    ff: int = 1536
    vocab: int = 49152
    ctx: int = 8192
    rope_base: float = 1e5
    eps: float = 1e-5
    tied: bool = True
    embd_type: int = Q4_0
    out_type: int = Q8_0
    seed: int = 0
    # per-layer matrix types: name -> type, or a callable (layer) -> type
    types: dict = dataclasses.field(default_factory=dict)
    q8_div_layers: float = 128.0
    q8_div_out: float = 8.0

    @property
    def head_dim(self):
        return self.embd // self.heads

    @property
    def kvd(self):
        return self.kv_heads * self.head_dim

    def mat_type(self, name, layer):
        t = self.types.get(name, Q4_0)
        return t(layer) if callable(t) else t


def smollm2(seed=0):
    """Config 0/2: SmolLM2-135M shape, llama, tied Q4_0 embedding."""
    return Spec(seed=seed)


def qwen25(seed=0):
    """Config 3: Qwen2.5-0.5B shape, qwen2 (NEOX, QKV biases), Q4_0 embedding, Q8_0 output."""
    return Spec(arch="qwen2", layers=24, embd=896, heads=14, kv_heads=2, ff=4864, vocab=151936, ctx=32768,
                rope_base=1e6, eps=1e-6, tied=False, embd_type=Q4_0, out_type=Q8_0, seed=seed)


def qwen25_mixed(seed=0):
    """Config 4's baseline mix: Q4_1 ffn_down on odd layers, Q8_0 head."""
    s = qwen25(seed)
    s.types = {"ffn_down": lambda l: Q4_1 if l % 2 == 1 else Q4_0}
    return s


def qwen25_mixed_ext(seed=0):
    """Config 4's extended mix: Q8_0 and Q4_1 on every kind of matrix."""
    s = qwen25(seed)
    kinds = ["attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"]
    cyc = [Q4_0, Q4_1, Q8_0]
    s.types = {k: (lambda l, i=i: cyc[(l + i) % 3]) for i, k in enumerate(kinds)}
    return s


def tiny_llama(seed=1, **kw):
    d = dict(arch="llama", layers=2, embd=128, heads=2, kv_heads=1, ff=256, vocab=512, ctx=512,
             rope_base=1e4, eps=1e-5, tied=True, seed=seed)
    d.update(kw)
    return Spec(**d)


def tiny_qwen(seed=2, **kw):
    d = dict(arch="qwen2", layers=2, embd=256, heads=4, kv_heads=2, ff=384, vocab=640, ctx=1024,
             rope_base=1e6, eps=1e-6, tied=False, out_type=Q8_0, seed=seed)
    d.update(kw)
    return Spec(**d)


def _rng(seed, name):
    return np.random.default_rng([seed, zlib.crc32(name.encode())])


def quant_blocks(qtype, rows, k, rng, q8_div=8.0):
    """Raw GGUF bytes of a [rows][k] matrix of the given type."""
    nb = k // 32
    n = rows * nb
    d = (np.abs(rng.standard_normal(n, dtype=np.float32)) * np.float32(0.02 / (q8_div if qtype == Q8_0 else 8.0))
         ).astype(np.float16)
    if qtype == Q4_0:
        blk = np.empty(n, dtype=[("d", "<f2"), ("qs", "u1", 16)])
        blk["d"] = d
        blk["qs"] = rng.integers(0, 256, size=(n, 16), dtype=np.uint8)
    elif qtype == Q4_1:
        blk = np.empty(n, dtype=[("d", "<f2"), ("m", "<f2"), ("qs", "u1", 16)])
        blk["d"] = d
        blk["m"] = (d.astype(np.float32) * np.float32(-8)).astype(np.float16)
        blk["qs"] = rng.integers(0, 256, size=(n, 16), dtype=np.uint8)
    elif qtype == Q8_0:
        blk = np.empty(n, dtype=[("d", "<f2"), ("qs", "i1", 32)])
        blk["d"] = d
        blk["qs"] = rng.integers(-127, 128, size=(n, 32), dtype=np.int8)
    else:
        raise ValueError(f"unsupported type {qtype}")
    return blk.tobytes()


def tensors(spec):
    """(name, dims, type, generator of bytes) of every tensor, in file order."""
    s = spec
    out = []

    def mat(name, k, rows, qtype, div):
        out.append((name, [k, rows], qtype, lambda: quant_blocks(qtype, rows, k, _rng(s.seed, name), div)))

    def vec(name, n, kind):
        def gen():
            r = _rng(s.seed, name).standard_normal(n, dtype=np.float32)
            v = np.float32(1) + r * np.float32(0.01) if kind == "norm" else r * np.float32(0.02)
            return v.astype("<f4").tobytes()
        out.append((name, [n], F32, gen))

    mat("token_embd.weight", s.embd, s.vocab, s.embd_type, s.q8_div_out)
    vec("output_norm.weight", s.embd, "norm")
    if not s.tied:
        mat("output.weight", s.embd, s.vocab, s.out_type, s.q8_div_out)
    for l in range(s.layers):
        p = f"blk.{l}."
        vec(p + "attn_norm.weight", s.embd, "norm")
        mat(p + "attn_q.weight", s.embd, s.embd, s.mat_type("attn_q", l), s.q8_div_layers)
        mat(p + "attn_k.weight", s.embd, s.kvd, s.mat_type("attn_k", l), s.q8_div_layers)
        mat(p + "attn_v.weight", s.embd, s.kvd, s.mat_type("attn_v", l), s.q8_div_layers)
        if s.arch == "qwen2":
            vec(p + "attn_q.bias", s.embd, "bias")
            vec(p + "attn_k.bias", s.kvd, "bias")
            vec(p + "attn_v.bias", s.kvd, "bias")
        mat(p + "attn_output.weight", s.embd, s.embd, s.mat_type("attn_output", l), s.q8_div_layers)
        vec(p + "ffn_norm.weight", s.embd, "norm")
        mat(p + "ffn_gate.weight", s.embd, s.ff, s.mat_type("ffn_gate", l), s.q8_div_layers)
        mat(p + "ffn_up.weight", s.embd, s.ff, s.mat_type("ffn_up", l), s.q8_div_layers)
        mat(p + "ffn_down.weight", s.ff, s.embd, s.mat_type("ffn_down", l), s.q8_div_layers)
    return out


def _str(b, s):
    e = s.encode()
    b += struct.pack("<Q", len(e)) + e


def write(path, spec, alignment=32):
    """Write the model as a GGUF v3 file; returns the path."""
    s = spec
    a = s.arch
    meta = [("general.architecture", _STR, a), ("general.alignment", _U32, alignment),
            (a + ".block_count", _U32, s.layers), (a + ".context_length", _U32, s.ctx),
            (a + ".embedding_length", _U32, s.embd), (a + ".feed_forward_length", _U32, s.ff),
            (a + ".attention.head_count", _U32, s.heads), (a + ".attention.head_count_kv", _U32, s.kv_heads),
            (a + ".rope.dimension_count", _U32, s.head_dim), (a + ".rope.freq_base", _F32, s.rope_base),
            (a + ".attention.layer_norm_rms_epsilon", _F32, s.eps)]
    ts = tensors(s)
    hdr = bytearray(b"GGUF")
    hdr += struct.pack("<IQQ", 3, len(ts), len(meta))
    for k, t, v in meta:
        _str(hdr, k)
        hdr += struct.pack("<I", t)
        if t == _STR:
            _str(hdr, v)
        elif t == _U32:
            hdr += struct.pack("<I", v)
        else:
            hdr += struct.pack("<f", v)
    off = 0
    offsets = []
    for name, dims, qt, _ in ts:
        be, bb = BLOCK[qt]
        n = int(np.prod(dims))
        size = n // be * bb
        offsets.append((off, size))
        _str(hdr, name)
        hdr += struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        hdr += struct.pack("<IQ", qt, off)
        off = (off + size + alignment - 1) // alignment * alignment
    pad = (-len(hdr)) % alignment
    tmp = f"{path}.{os.getpid()}.tmp"  # a writer of its own, then one atomic rename
    with open(tmp, "wb") as f:
        f.write(hdr)
        f.write(b"\0" * pad)
        pos = 0
        for (name, dims, qt, gen), (o, size) in zip(ts, offsets):
            f.write(b"\0" * (o - pos))
            data = gen()
            assert len(data) == size, name
            f.write(data)
            pos = o + size
    os.replace(tmp, path)
    return path


_PRIVATE = None


def _private_dir():
    """A directory of this process, created on first use and removed at exit.
    Files under a shared temporary directory with deterministic names can be
    rewritten by another process (another test run or job on the same host)
    between the GPU loading a model and the oracle loading it."""
    global _PRIVATE
    if _PRIVATE is None:
        _PRIVATE = tempfile.mkdtemp(prefix="llm_synth_")
        atexit.register(shutil.rmtree, _PRIVATE, True)
    return _PRIVATE


def cached(spec, directory=None):
    """Write the model once into `directory` (default $LLM_SYNTH_DIR, else a
    directory of this process) and reuse it."""
    directory = directory or os.environ.get("LLM_SYNTH_DIR") or _private_dir()
    os.makedirs(directory, exist_ok=True)
    key = zlib.crc32(repr(dataclasses.asdict(dataclasses.replace(spec, types={}))).encode()
                     + repr(sorted((k, [spec.mat_type(k, l) for l in range(spec.layers)])
                                   for k in spec.types)).encode())
    path = os.path.join(directory, f"llm_synth_{spec.arch}_{spec.layers}x{spec.embd}_{key:08x}.gguf")
    if not os.path.exists(path):
        write(path, spec)
    return path


def prompt(seed, n, vocab):
    """n token ids uniform in [0, vocab)."""
    return np.random.default_rng([seed, 0x70726F6D]).integers(0, vocab, size=n).astype(np.int32)
