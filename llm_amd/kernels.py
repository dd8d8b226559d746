"""Kernel-level surface: a quantised matrix on the GPU (llmhip_qmat_*).

Device memory and streams come from torch (plumbing only); every computation
runs in libllmhip.so.
"""
import ctypes

import numpy as np

from . import _lib
from ._lib import check, lib


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


class QMat:
    """A [rows][k] Q4_0 / Q4_1 / Q8_0 matrix repacked on the device from raw GGUF blocks."""

    def __init__(self, qtype, rows, k, raw=None, device=0):
        self.qtype, self.rows, self.k, self.device = qtype, rows, k, device
        h = ctypes.c_void_p()
        check(lib().llmhip_qmat_create(device, qtype, rows, k, ctypes.byref(h)))
        self._h = h
        if raw is not None:
            self.upload(raw)

    def upload(self, raw, byte_offset=0):
        buf = np.ascontiguousarray(np.frombuffer(raw, np.uint8) if isinstance(raw, (bytes, bytearray)) else raw,
                                   np.uint8)
        check(lib().llmhip_qmat_upload(self._h, buf.ctypes.data_as(ctypes.c_void_p), buf.size, byte_offset))

    def dequant(self):
        import torch
        out = torch.empty((self.rows, self.k), dtype=torch.float32, device=f"cuda:{self.device}")
        check(lib().llmhip_qmat_dequant(self._h, ctypes.c_void_p(out.data_ptr()), _stream()))
        return out

    def gemv(self, x, y=None, accumulate=False, stream=None):
        """y[n][rows] (+)= W x[n][k] for x a float32 CUDA tensor of n <= 64 rows."""
        import torch
        x = x.contiguous()
        n = 1 if x.dim() == 1 else x.shape[0]
        if x.dtype != torch.float32 or x.numel() != n * self.k or not x.is_cuda:
            raise ValueError("x must be a float32 CUDA tensor of n rows of k")
        if y is None:
            y = torch.empty((n, self.rows), dtype=torch.float32, device=x.device)
        if y.dtype != torch.float32 or y.numel() != n * self.rows or not y.is_contiguous():
            raise ValueError("y must be a contiguous float32 tensor of n rows of `rows`")
        check(lib().llmhip_qmat_gemv(self._h, ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr()), n,
                                     int(accumulate), _stream(stream)))
        return y

    def gemv_q8(self, x, stream=None):
        """The ExactGGML product: each row of x quantised to Q8 blocks, integer block dots."""
        import torch
        x = x.contiguous()
        n = 1 if x.dim() == 1 else x.shape[0]
        if x.dtype != torch.float32 or x.numel() != n * self.k or not x.is_cuda:
            raise ValueError("x must be a float32 CUDA tensor of n rows of k")
        y = torch.empty((n, self.rows), dtype=torch.float32, device=x.device)
        check(lib().llmhip_qmat_gemv_q8(self._h, ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr()), n,
                                        _stream(stream)))
        return y

    def clone(self):
        """A device-to-device copy (for rotating benchmark copies)."""
        c = QMat.__new__(QMat)
        c.qtype, c.rows, c.k, c.device = self.qtype, self.rows, self.k, self.device
        h = ctypes.c_void_p()
        check(lib().llmhip_qmat_clone(self._h, ctypes.byref(h)))
        c._h = h
        return c

    @property
    def nbytes(self):
        return lib().llmhip_qmat_bytes(self._h)

    @property
    def gguf_bytes(self):
        return lib().llmhip_qmat_gguf_bytes(self._h)

    def close(self):
        if getattr(self, "_h", None):
            lib().llmhip_qmat_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def bench(mats, x, y, iters, warmup=10, stream=None):
    """Average microseconds of one gemv, cycling back-to-back through `mats`."""
    arr = (ctypes.c_void_p * len(mats))(*[m._h.value for m in mats])
    n = 1 if x.dim() == 1 else x.shape[0]
    us = ctypes.c_float()
    check(lib().llmhip_qmat_bench(arr, len(mats), ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr()), n,
                                  iters, warmup, _stream(stream), ctypes.byref(us)))
    return us.value


Q4_0, Q4_1, Q8_0 = _lib.Q4_0, _lib.Q4_1, _lib.Q8_0
