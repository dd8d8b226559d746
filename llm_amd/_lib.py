"""ctypes binding of libllmhip.so (the C-ABI declared in include/llmhip.h).

The library is built in-tree by llm_amd/build.py.  There is no fallback: if
the shared library is missing, importing the binding raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libllmhip.so")

ERRORS = {-1: "ARG", -2: "DEVICE", -3: "BUDGET", -4: "TYPE", -5: "CONTEXT", -6: "FORMAT", -7: "STATE", -8: "IO"}

Q4_0, Q4_1, Q8_0, F32 = 2, 3, 8, 0


class LLMError(RuntimeError):
    """A negative status of the C-ABI, with llmhip_last_error()'s message."""

    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code
        self.kind = ERRORS.get(code, str(code))


class Limits(ctypes.Structure):
    _fields_ = [("max_invocations_per_workgroup", ctypes.c_uint32), ("max_workgroup_storage", ctypes.c_uint32),
                ("max_workgroups_per_dimension", ctypes.c_uint32), ("max_storage_buffers", ctypes.c_uint32),
                ("max_binding_size", ctypes.c_uint64), ("max_buffer_size", ctypes.c_uint64),
                ("memory_budget", ctypes.c_uint64)]


_lib = None

P, I, U32, U64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float

# (name, restype, argtypes) of every exported function
SIGNATURES = [
    ("llmhip_last_error", ctypes.c_char_p, []),
    ("llmhip_device_count", I, [ctypes.POINTER(I)]),
    ("llmhip_device_limits", I, [I, ctypes.POINTER(Limits)]),
    ("llmhip_qmat_create", I, [I, U32, U64, U64, ctypes.POINTER(P)]),
    ("llmhip_qmat_upload", I, [P, P, U64, U64]),
    ("llmhip_qmat_dequant", I, [P, P, P]),
    ("llmhip_qmat_gemv", I, [P, P, P, I, I, P]),
    ("llmhip_qmat_bytes", U64, [P]),
    ("llmhip_qmat_gguf_bytes", U64, [P]),
    ("llmhip_qmat_bench", I, [ctypes.POINTER(P), I, P, P, I, I, I, P, ctypes.POINTER(F)]),
    ("llmhip_qmat_free", None, [P]),
]


def lib():
    """The loaded library (raises if it was never built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m llm_amd.build` "
                              "(there is no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc != 0:
        raise LLMError(rc, lib().llmhip_last_error().decode(errors="replace"))
    return rc


def device_count():
    n = ctypes.c_int()
    check(lib().llmhip_device_count(ctypes.byref(n)))
    return n.value


def device_limits(ordinal=0):
    l = Limits()
    check(lib().llmhip_device_limits(ordinal, ctypes.byref(l)))
    return l
