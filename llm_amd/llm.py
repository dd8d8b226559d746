"""Python mirror of the reference's Go API (package llm), over libllmhip.so.

Names follow the Go package so that code and tests read like the reference's:
gguf.Parse -> Parse, ConfigFrom, NewGPU, GPU.Generate / PrefillLogits / Peek /
MemoryUsed, Limits, DefaultLimits, Stats, Timing and the DecodeBatch /
PrefillBatch tunables.  Every method is a thin call into the C-ABI (the C++
host layer llm_* and the device layer llmhip_*); nothing here computes.
"""
import ctypes
import dataclasses
import os

import numpy as np

from . import _lib
from ._lib import Config, LLMError, Limits, check, lib

# package tunables (gpu.go:20-23, 165, 1046-1054)
ChunkSize = 16 << 20
PieceSize = 4 << 20
MaxBatch = 16
PrefillBatch = 64
DecodeBatch = 8
# binary16 KV cache for the next NewGPU (the F16KV mode of cpu.go:22-24)
F16KV = False
# ggml's CPU-backend products for the next NewGPU: Q8 activation blocks, binary16 cache (cpu.go:15-21)
ExactGGML = False


def DefaultLimits(ordinal=0):
    """The device's limits (Limits of gpu.go:28-36 filled from hipDeviceProp_t)."""
    return _lib.device_limits(ordinal)


class File:
    """A parsed GGUF header (gguf.File, gguf/gguf.go:114-122)."""

    def __init__(self, handle):
        self._h = handle
        nt, nkv, off, al = (ctypes.c_uint64() for _ in range(4))
        ver = ctypes.c_uint32()
        check(lib().llm_gguf_info(handle, ctypes.byref(nt), ctypes.byref(nkv), ctypes.byref(off), ctypes.byref(al),
                                  ctypes.byref(ver)))
        self.Version, self.DataOffset, self.Alignment, self.NumMeta = ver.value, off.value, al.value, nkv.value
        self.Tensors = []
        name = ctypes.create_string_buffer(1024)
        for i in range(nt.value):
            t, nd = ctypes.c_uint32(), ctypes.c_uint32()
            dims = (ctypes.c_uint64 * 4)()
            o, sz = ctypes.c_uint64(), ctypes.c_uint64()
            check(lib().llm_gguf_tensor_info(handle, i, name, 1024, ctypes.byref(t), ctypes.byref(nd), dims,
                                             ctypes.byref(o), ctypes.byref(sz)))
            self.Tensors.append(Tensor(name.value.decode(errors="surrogateescape"), list(dims[:nd.value]), t.value,
                                       o.value, sz.value))
        self._by_name = {t.Name: t for t in self.Tensors}

    def Tensor(self, name):
        t = self._by_name.get(name)
        return t, t is not None

    def Uint(self, key):
        v = ctypes.c_uint64()
        ok = lib().llm_gguf_meta_uint(self._h, key.encode(), ctypes.byref(v))
        return v.value, bool(ok)

    def Float(self, key):
        v = ctypes.c_double()
        ok = lib().llm_gguf_meta_float(self._h, key.encode(), ctypes.byref(v))
        return v.value, bool(ok)

    def Str(self, key):
        buf = ctypes.create_string_buffer(1 << 16)
        ok = lib().llm_gguf_meta_str(self._h, key.encode(), buf, len(buf))
        return buf.value.decode(errors="replace"), bool(ok)

    def close(self):
        if self._h:
            lib().llm_gguf_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclasses.dataclass
class Tensor:
    """gguf.Tensor, gguf/gguf.go:96-102."""
    Name: str
    Dims: list
    Type: int
    Offset: int
    Size: int


class GGUFError(LLMError):
    """A refused header; kind is "magic", "version", "bound", "format" or "io"."""

    KINDS = {1: "magic", 2: "version", 3: "bound", 4: "format", 5: "io"}

    def __init__(self, code, msg, kind):
        super().__init__(code, msg)
        self.gguf_kind = self.KINDS.get(kind, "?")


def Parse(src):
    """gguf.Parse of a path or of bytes."""
    h, kind = ctypes.c_void_p(), ctypes.c_int()
    if isinstance(src, (bytes, bytearray, memoryview)):
        buf = ctypes.create_string_buffer(bytes(src), len(src)) if len(src) else ctypes.create_string_buffer(1)
        rc = lib().llm_gguf_parse_bytes(buf, len(src), ctypes.byref(h), ctypes.byref(kind))
    else:
        rc = lib().llm_gguf_parse_file(os.fsencode(src), ctypes.byref(h), ctypes.byref(kind))
    if rc != 0:
        raise GGUFError(rc, lib().llmhip_last_error().decode(errors="replace"), kind.value)
    return File(h)


def ConfigFrom(f):
    """ConfigFrom, config.go:29-73."""
    c = Config()
    check(lib().llm_config_from(f._h, ctypes.byref(c)))
    return c


@dataclasses.dataclass
class Timing:
    """Timing of a generation (gpu.go:930-939), seconds."""
    Prefill: float
    Decode: float
    PromptTokens: int
    Generated: int
    Submits: int
    Dispatches: int
    Record: float
    Submit: float


class GPU:
    """The forward pass on one MI355X (the reference's *GPU, gpu.go:116-159)."""

    def __init__(self, handle):
        self._h = handle
        self._m = ctypes.c_void_p(lib().llm_gpu_model(handle))
        c, ctx = Config(), ctypes.c_int()
        check(lib().llm_gpu_config(handle, ctypes.byref(c), ctypes.byref(ctx)))
        self.Cfg, self.ctx = c, ctx.value
        self._layers = 0
        self._skip = {}

    # --- fields of the Go struct
    @property
    def Stats(self):
        s = _lib.Stats()
        check(lib().llmhip_model_stats(self._m, ctypes.byref(s)))
        return s

    @property
    def Layers(self):
        return self._layers

    @Layers.setter
    def Layers(self, n):
        check(lib().llmhip_model_set_layers(self._m, int(n)))
        self._layers = int(n)

    @property
    def Skip(self):
        return dict(self._skip)

    @Skip.setter
    def Skip(self, classes):
        classes = classes or {}
        names = [k for k, v in classes.items() if v] if isinstance(classes, dict) else list(classes)
        check(lib().llmhip_model_set_skip(self._m, ",".join(names).encode()))
        self._skip = {k: True for k in names}

    # --- methods
    def MemoryUsed(self):
        return lib().llmhip_model_memory_used(self._m)

    def Generate(self, prompt, n, eos=-1, emit=None):
        """Greedy generation; emit(tok) -> bool is called with each new token."""
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        errors = []

        def cb(tok, _user):
            if emit is None:
                return 1
            try:
                return 1 if emit(int(tok)) else 0
            except BaseException as e:  # stop generation, re-raise after
                errors.append(e)
                return 0

        fn = _lib.EMIT(cb)
        tm = _lib.Timing()
        lib().llm_set_decode_batch(int(DecodeBatch))
        check(lib().llm_gpu_generate(self._h, p.ctypes.data_as(ctypes.c_void_p), p.size, int(n), int(eos), fn, None,
                                     ctypes.byref(tm)))
        if errors:
            raise errors[0]
        return Timing(tm.prefill_ns * 1e-9, tm.decode_ns * 1e-9, tm.prompt_tokens, tm.generated, tm.submits,
                      tm.dispatches, tm.record_ns * 1e-9, tm.submit_ns * 1e-9)

    def PrefillLogits(self, prompt):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(self.Cfg.vocab, np.float32)
        check(lib().llm_gpu_prefill_logits(self._h, p.ctypes.data_as(ctypes.c_void_p), p.size,
                                           out.ctypes.data_as(ctypes.c_void_p)))
        return out

    def Peek(self, name, n):
        out = np.empty(n, np.float32)
        check(lib().llm_gpu_peek(self._h, name.encode(), out.ctypes.data_as(ctypes.c_void_p), n))
        return out

    def set_fused(self, on=True, poll_limit=0):
        """Decode steps as the fused launch (llmhip_model_set_fused): returns
        (taken, reason it is not)."""
        why = ctypes.create_string_buffer(256)
        rc = lib().llmhip_model_set_fused(self._m, int(bool(on)), int(poll_limit), why, 256)
        if rc < 0:
            check(rc)
        return rc == 1, why.value.decode()

    def bench_kernel(self, kernel, iters):
        """(avg microseconds, algorithmic bytes) of one launch of a decode-step kernel."""
        us, b = ctypes.c_float(), ctypes.c_uint64()
        check(lib().llmhip_model_bench_kernel(self._m, kernel.encode(), iters, ctypes.byref(us), ctypes.byref(b)))
        return us.value, b.value

    def profile(self, tokens=3, cap=4096):
        """Per-launch device times of one decode step, taken with HIP events on
        the model's stream after `tokens - 1` warm steps: [(cls, layer, bytes, us)].
        Advances the generation like `tokens` decode steps."""
        arr = (_lib.KernelTime * cap)()
        n = ctypes.c_int()
        check(lib().llmhip_model_profile(self._m, tokens, arr, cap, ctypes.byref(n)))
        return [(r.cls.decode(), r.layer, r.bytes, r.us) for r in arr[:n.value]]

    def close(self):
        if getattr(self, "_h", None):
            lib().llm_gpu_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def NewGPU(dev, lim, path, ctx):
    """NewGPU (gpu.go:465-764): dev is the HIP device ordinal, lim a Limits or
    None for the device's own, path the GGUF file, ctx the KV cache length."""
    lib().llm_set_prefill_batch(int(PrefillBatch))
    lib().llm_set_f16kv(int(F16KV))
    lib().llm_set_exact_ggml(int(ExactGGML))
    h = ctypes.c_void_p()
    check(lib().llm_new_gpu(int(dev), ctypes.byref(lim) if lim is not None else None, os.fsencode(path), int(ctx),
                            ctypes.byref(h)))
    return GPU(h)


def Argmax(logits):
    """The first index of the largest logit (cpu.go:389-397), on the host."""
    l = np.asarray(logits, np.float32)
    if l.size == 0 or np.isnan(l[0]):
        return 0
    m = np.nanmax(l)
    return int(np.flatnonzero(l == m)[0])
