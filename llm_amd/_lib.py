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


class Config(ctypes.Structure):
    """Config, config.go:11-23."""
    _fields_ = [(n, ctypes.c_int32) for n in
                ("layers", "embd", "ff", "heads", "kv_heads", "head_dim", "vocab", "ctx")] + \
               [("rope_base", ctypes.c_float), ("eps", ctypes.c_float)] + \
               [(n, ctypes.c_int32) for n in ("arch", "rope_neox", "bias", "tied_output")]


class Stats(ctypes.Structure):
    """Stats, gpu.go:56-60."""
    _fields_ = [("submits", ctypes.c_int64), ("dispatches", ctypes.c_int64), ("tokens", ctypes.c_int64)]


class Timing(ctypes.Structure):
    """Timing, gpu.go:930-939, in nanoseconds."""
    _fields_ = [(n, ctypes.c_int64) for n in ("prefill_ns", "decode_ns", "prompt_tokens", "generated", "submits",
                                                "dispatches", "record_ns", "submit_ns")]


class KernelTime(ctypes.Structure):
    """llmhip_kernel_time: one profiled launch."""
    _fields_ = [("cls", ctypes.c_char * 8), ("layer", ctypes.c_int32), ("bytes", ctypes.c_uint64),
                ("us", ctypes.c_float)]


EMIT = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_int32, ctypes.c_void_p)

_lib = None

P, I, U32, U64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float
PU64 = ctypes.POINTER(ctypes.c_uint64)

# (name, restype, argtypes) of every exported function
SIGNATURES = [
    ("llmhip_last_error", ctypes.c_char_p, []),
    ("llmhip_device_count", I, [ctypes.POINTER(I)]),
    ("llmhip_device_limits", I, [I, ctypes.POINTER(Limits)]),
    ("llmhip_buffer_alloc", I, [I, U64, ctypes.POINTER(P)]),
    ("llmhip_buffer_free", None, [P]),
    ("llmhip_buffer_write", I, [P, P, U64]),
    ("llmhip_buffer_read", I, [P, P, U64]),
    ("llmhip_device_synchronize", I, [I]),
    ("llmhip_bench_h2d", I, [I, U64, I, ctypes.POINTER(F)]),
    ("llmhip_copy_calibration", I, [I, U64]),
    ("llmhip_qmat_create", I, [I, U32, U64, U64, ctypes.POINTER(P)]),
    ("llmhip_qmat_upload", I, [P, P, U64, U64]),
    ("llmhip_qmat_dequant", I, [P, P, P]),
    ("llmhip_qmat_gemv", I, [P, P, P, I, I, P]),
    ("llmhip_qmat_gemv_noalloc", I, [P, P, P, I, I, P]),
    ("llmhip_qmat_gemv_q8", I, [P, P, P, I, P]),
    ("llmhip_qmat_bytes", U64, [P]),
    ("llmhip_qmat_gguf_bytes", U64, [P]),
    ("llmhip_qmat_bench", I, [ctypes.POINTER(P), I, P, P, I, I, I, P, ctypes.POINTER(F)]),
    ("llmhip_qmat_bench_graph", I, [ctypes.POINTER(P), I, P, P, I, I, I, P, ctypes.POINTER(F)]),
    ("llmhip_qmat_clone", I, [P, ctypes.POINTER(P)]),
    ("llmhip_qmat_free", None, [P]),
    ("llmhip_model_create", I, [I, ctypes.POINTER(Limits), ctypes.POINTER(Config), I, I, ctypes.POINTER(P)]),
    ("llmhip_model_tensor", I, [P, ctypes.c_char_p, U32, PU64, U32]),
    ("llmhip_model_upload", I, [P, ctypes.c_char_p, P, U64, U64]),
    ("llmhip_model_upload_file", I, [P, ctypes.c_char_p, I, U64, U64, U64]),
    ("llmhip_model_upload_file_tensors", I, [P, I, U32, ctypes.POINTER(ctypes.c_char_p), PU64]),
    ("llmhip_model_finalize", I, [P]),
    ("llmhip_model_prefill", I, [P, P, I, P, P]),
    ("llmhip_model_decode", I, [P, I, P]),
    ("llmhip_model_peek", I, [P, ctypes.c_char_p, P, U64]),
    ("llmhip_model_memory_used", U64, [P]),
    ("llmhip_model_stats", I, [P, ctypes.POINTER(Stats)]),
    ("llmhip_model_config", I, [P, ctypes.POINTER(Config), ctypes.POINTER(I)]),
    ("llmhip_model_set_fused", I, [P, I, U32, ctypes.c_char_p, U64]),
    ("llmhip_model_set_layers", I, [P, I]),
    ("llmhip_model_set_kv_f16", I, [P, I]),
    ("llmhip_model_set_exact_ggml", I, [P, I]),
    ("llmhip_model_set_skip", I, [P, ctypes.c_char_p]),
    ("llmhip_model_bench_kernel", I, [P, ctypes.c_char_p, I, ctypes.POINTER(F), PU64]),
    ("llmhip_model_profile", I, [P, I, P, I, ctypes.POINTER(I)]),
    ("llmhip_model_free", None, [P]),
    ("llm_gguf_parse_file", I, [ctypes.c_char_p, ctypes.POINTER(P), ctypes.POINTER(I)]),
    ("llm_gguf_parse_bytes", I, [P, U64, ctypes.POINTER(P), ctypes.POINTER(I)]),
    ("llm_gguf_free", None, [P]),
    ("llm_gguf_info", I, [P, PU64, PU64, PU64, PU64, ctypes.POINTER(U32)]),
    ("llm_gguf_tensor_info", I, [P, U64, ctypes.c_char_p, U64, ctypes.POINTER(U32), ctypes.POINTER(U32), PU64, PU64,
                                 PU64]),
    ("llm_gguf_find_tensor", I, [P, ctypes.c_char_p, PU64]),
    ("llm_gguf_meta_uint", I, [P, ctypes.c_char_p, PU64]),
    ("llm_gguf_meta_float", I, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
    ("llm_gguf_meta_str", I, [P, ctypes.c_char_p, ctypes.c_char_p, U64]),
    ("llm_config_from", I, [P, ctypes.POINTER(Config)]),
    ("llm_set_decode_batch", I, [I]),
    ("llm_set_prefill_batch", I, [I]),
    ("llm_set_f16kv", I, [I]),
    ("llm_set_exact_ggml", I, [I]),
    ("llm_new_gpu", I, [I, ctypes.POINTER(Limits), ctypes.c_char_p, I, ctypes.POINTER(P)]),
    ("llm_gpu_generate", I, [P, P, I, I, ctypes.c_int32, EMIT, P, ctypes.POINTER(Timing)]),
    ("llm_gpu_prefill_logits", I, [P, P, I, P]),
    ("llm_gpu_peek", I, [P, ctypes.c_char_p, P, U64]),
    ("llm_gpu_config", I, [P, ctypes.POINTER(Config), ctypes.POINTER(I)]),
    ("llm_gpu_model", P, [P]),
    ("llm_gpu_free", None, [P]),
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
