"""ctypes binding of the CPU oracle (libcpuref.so, built from cpuref.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package (llm_amd).
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "libcpuref.so")


def build():
    """Compile libcpuref.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


class Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in
                ("layers", "embd", "ff", "heads", "kv_heads", "head_dim", "vocab", "ctx")] + \
               [("rope_base", ctypes.c_float), ("eps", ctypes.c_float)] + \
               [(n, ctypes.c_int) for n in ("arch_qwen2", "rope_neox", "bias", "tied_output")]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        P, F, I, U32 = ctypes.c_void_p, ctypes.c_float, ctypes.c_int, ctypes.c_uint32
        L.cpuref_error.restype = ctypes.c_char_p
        L.cpuref_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.cpuref_f16_to_f32.restype = F
        L.cpuref_f32_to_f16.argtypes = [F]
        L.cpuref_f32_to_f16.restype = ctypes.c_uint16
        L.cpuref_round_f16.argtypes = [F]
        L.cpuref_round_f16.restype = F
        L.cpuref_f16_to_f32_n.argtypes = [P, P, ctypes.c_size_t]
        L.cpuref_f32_to_f16_n.argtypes = [P, P, ctypes.c_size_t]
        L.cpuref_rmsnorm.argtypes = [P, P, P, I, F]
        L.cpuref_matvec.argtypes = [P, P, U32, P, I, I, I]
        L.cpuref_matvec_q8.argtypes = [P, P, U32, P, I, I, I]
        L.cpuref_dequant.argtypes = [P, U32, P, ctypes.c_uint64]
        L.cpuref_rope.argtypes = [P, I, I, I, F, I]
        L.cpuref_rope_table.argtypes = [P, I, I, F]
        L.cpuref_argmax.argtypes = [P, I]
        L.cpuref_argmax.restype = ctypes.c_int32
        L.cpuref_quantize_q8.argtypes = [P, I, P, P, P]
        L.cpuref_load.argtypes = [ctypes.c_char_p, I, ctypes.POINTER(P)]
        L.cpuref_free.argtypes = [P]
        L.cpuref_get_config.argtypes = [P, ctypes.POINTER(Config)]
        L.cpuref_set_mode.argtypes = [P, I, I]
        L.cpuref_set_threads.argtypes = [P, I]
        L.cpuref_set_max_layers.argtypes = [P, I]
        L.cpuref_reset.argtypes = [P]
        L.cpuref_pos.argtypes = [P]
        L.cpuref_last_x.argtypes = [P, P]
        L.cpuref_last_h.argtypes = [P, P]
        L.cpuref_last_up.argtypes = [P, P]
        L.cpuref_last_att.argtypes = [P, P]
        L.cpuref_kv_row.argtypes = [P, I, I, I, P]
        L.cpuref_forward.argtypes = [P, ctypes.c_int32, P]
        L.cpuref_tensor.argtypes = [P, ctypes.c_char_p, ctypes.POINTER(P), ctypes.POINTER(ctypes.c_uint64),
                                    ctypes.POINTER(ctypes.c_uint32), P]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def f16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().cpuref_f16_to_f32_n(_p(h), _p(out), h.size)
    return out


def f32_to_f16(f):
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().cpuref_f32_to_f16_n(_p(f), _p(out), f.size)
    return out


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().cpuref_rmsnorm(_p(out), _p(x), _p(w), x.size, eps)
    return out


def matvec(qtype, raw, rows, k, x, threads=1, q8=False):
    """y = W x for `rows` rows of `k` weights given as raw GGUF blocks; q8:
    the ExactGGML form (x quantised to Q8 blocks, integer block products)."""
    raw = np.ascontiguousarray(np.frombuffer(raw, np.uint8) if isinstance(raw, (bytes, bytearray)) else raw,
                               np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    fn = lib().cpuref_matvec_q8 if q8 else lib().cpuref_matvec
    if fn(_p(y), _p(x), qtype, _p(raw), k, rows, threads) != 0:
        raise RuntimeError(lib().cpuref_error().decode())
    return y


def dequant(qtype, raw, nblocks):
    raw = np.ascontiguousarray(np.frombuffer(raw, np.uint8) if isinstance(raw, (bytes, bytearray)) else raw,
                               np.uint8)
    out = np.empty(nblocks * 32, np.float32)
    if lib().cpuref_dequant(_p(out), qtype, _p(raw), nblocks) != 0:
        raise RuntimeError(lib().cpuref_error().decode())
    return out


def rope(x, pos, heads, dim, base, neox):
    x = np.array(x, np.float32, copy=True)
    lib().cpuref_rope(_p(x), pos, heads, dim, base, int(neox))
    return x


def rope_table(ctx, hd, base):
    cs = np.empty(ctx * hd, np.float32)
    lib().cpuref_rope_table(_p(cs), ctx, hd, base)
    return cs


def argmax(l):
    l = np.ascontiguousarray(l, np.float32)
    return int(lib().cpuref_argmax(_p(l), l.size))


def quantize_q8(x):
    x = np.ascontiguousarray(x, np.float32)
    nb = x.size // 32
    d, s, qs = np.empty(nb, np.float32), np.empty(nb, np.float32), np.empty(x.size, np.int8)
    lib().cpuref_quantize_q8(_p(x), x.size, _p(d), _p(s), _p(qs))
    return d, s, qs


class CPU:
    """The oracle model: LoadCPU / Forward / Reset / Pos / Argmax of cpu.go."""

    def __init__(self, path, max_ctx, threads=1, exact_ggml=False, f16kv=False):
        h = ctypes.c_void_p()
        if lib().cpuref_load(os.fsencode(path), max_ctx, ctypes.byref(h)) != 0:
            raise RuntimeError(lib().cpuref_error().decode())
        self._h = h
        c = Config()
        lib().cpuref_get_config(h, ctypes.byref(c))
        self.cfg = c
        lib().cpuref_set_threads(h, threads)
        lib().cpuref_set_mode(h, int(exact_ggml), int(f16kv))

    def close(self):
        if self._h:
            lib().cpuref_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_threads(self, n):
        lib().cpuref_set_threads(self._h, n)

    def set_max_layers(self, n):
        lib().cpuref_set_max_layers(self._h, n)

    def reset(self):
        lib().cpuref_reset(self._h)

    def pos(self):
        return lib().cpuref_pos(self._h)

    def forward(self, tok):
        out = np.empty(self.cfg.vocab, np.float32)
        rc = lib().cpuref_forward(self._h, int(tok), _p(out))
        if rc < 0:
            raise RuntimeError(lib().cpuref_error().decode())
        return out if rc == 1 else None

    def last_x(self):
        out = np.empty(self.cfg.embd, np.float32)
        lib().cpuref_last_x(self._h, _p(out))
        return out

    def last_h(self):
        """The head's input row of the last forward (rmsNorm with output_norm)."""
        out = np.empty(self.cfg.embd, np.float32)
        lib().cpuref_last_h(self._h, _p(out))
        return out

    def last_up(self):
        """The up product of the last layer the last forward ran."""
        out = np.empty(self.cfg.ff, np.float32)
        lib().cpuref_last_up(self._h, _p(out))
        return out

    def last_att(self):
        """The attention output of the last layer the last forward ran (cpu.go:300-334)."""
        out = np.empty(self.cfg.heads * self.cfg.head_dim, np.float32)
        lib().cpuref_last_att(self._h, _p(out))
        return out

    def kv_row(self, layer, pos, v=False):
        """The cached K (v False) or V row of a layer at a position."""
        out = np.empty(self.cfg.kv_heads * self.cfg.head_dim, np.float32)
        if lib().cpuref_kv_row(self._h, layer, pos, int(v), _p(out)) != 0:
            raise RuntimeError(lib().cpuref_error().decode())
        return out

    def tensor(self, name):
        d, n, t = ctypes.c_void_p(), ctypes.c_uint64(), ctypes.c_uint32()
        dims = (ctypes.c_uint64 * 4)()
        if lib().cpuref_tensor(self._h, name.encode(), ctypes.byref(d), ctypes.byref(n), ctypes.byref(t), dims) != 0:
            raise RuntimeError(lib().cpuref_error().decode())
        buf = (ctypes.c_uint8 * n.value).from_address(d.value)
        return bytes(buf), int(t.value), [int(v) for v in dims]

    def greedy(self, prompt, n):
        """The CPU half of generate `check` (examples/generate/main.go:155-175):
        forward the prompt, then n greedy tokens. Returns (first logits, tokens)."""
        self.reset()
        logits = None
        for t in prompt:
            logits = self.forward(t)
        first = logits.copy()
        toks = []
        nxt = argmax(logits)
        while len(toks) < n:
            toks.append(nxt)
            if len(toks) == n:
                break
            nxt = argmax(self.forward(nxt))
        return first, toks
