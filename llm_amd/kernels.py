"""Kernel-level surface: a quantised matrix on the GPU (llmhip_qmat_*) and the
device buffers its products read and write (llmhip_buffer_*).

Everything runs in libllmhip.so, on the HIP runtime it links (no second
runtime in the process): host arrays go in and out through the library's
pinned staging.
"""
import ctypes

import numpy as np

from . import _lib
from ._lib import check, lib


class DeviceBuffer:
    """Zeroed device memory of `nbytes` on one device (llmhip_buffer_alloc)."""

    def __init__(self, nbytes, device=0):
        p = ctypes.c_void_p()
        check(lib().llmhip_buffer_alloc(device, int(nbytes), ctypes.byref(p)))
        self._p, self.nbytes, self.device = p, int(nbytes), device

    @classmethod
    def from_numpy(cls, a, device=0):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes, device)
        b.write(a)
        return b

    @property
    def ptr(self):
        return ctypes.c_void_p(self._p.value)

    def write(self, a):
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError(f"{a.nbytes} bytes into a buffer of {self.nbytes}")
        check(lib().llmhip_buffer_write(self._p, a.ctypes.data_as(ctypes.c_void_p), a.nbytes))

    def numpy(self, dtype, shape):
        out = np.empty(shape, dtype)
        if out.nbytes > self.nbytes:
            raise ValueError(f"{out.nbytes} bytes from a buffer of {self.nbytes}")
        check(lib().llmhip_buffer_read(out.ctypes.data_as(ctypes.c_void_p), self._p, out.nbytes))
        return out

    def close(self):
        if getattr(self, "_p", None) is not None and self._p.value:
            lib().llmhip_buffer_free(self._p)
        self._p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def synchronize(device=0):
    check(lib().llmhip_device_synchronize(device))


def _f32(x, k):
    x = np.ascontiguousarray(x, np.float32)
    n = 1 if x.ndim == 1 else x.shape[0]
    if x.size != n * k:
        raise ValueError(f"x must hold n rows of {k} float32 values")
    return x.reshape(n, k), n


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
        """The f32 weights [rows][k] (exact dequantisation), as a numpy array."""
        out = DeviceBuffer(self.rows * self.k * 4, self.device)
        check(lib().llmhip_qmat_dequant(self._h, out.ptr, None))
        synchronize(self.device)
        return out.numpy(np.float32, (self.rows, self.k))

    def gemv_dev(self, x, y, n, accumulate=False):
        """y[n][rows] (+)= W x[n][k] on device buffers (n <= 64)."""
        check(lib().llmhip_qmat_gemv(self._h, x.ptr, y.ptr, int(n), int(accumulate), None))

    def gemv(self, x, y=None, accumulate=False):
        """y[n][rows] (+)= W x[n][k] for host float32 arrays; returns y."""
        x, n = _f32(x, self.k)
        xd = DeviceBuffer.from_numpy(x, self.device)
        if y is None:
            y = np.zeros((n, self.rows), np.float32)
        y = np.ascontiguousarray(y, np.float32).reshape(n, self.rows)
        yd = DeviceBuffer.from_numpy(y, self.device)
        self.gemv_dev(xd, yd, n, accumulate)
        synchronize(self.device)
        return yd.numpy(np.float32, (n, self.rows))

    def gemv_q8(self, x):
        """The ExactGGML product: each row of x quantised to Q8 blocks, integer block dots."""
        x, n = _f32(x, self.k)
        xd = DeviceBuffer.from_numpy(x, self.device)
        yd = DeviceBuffer(n * self.rows * 4, self.device)
        check(lib().llmhip_qmat_gemv_q8(self._h, xd.ptr, yd.ptr, n, None))
        synchronize(self.device)
        return yd.numpy(np.float32, (n, self.rows))

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


def bench(mats, x, y, n, iters, warmup=10, graph=False):
    """Average microseconds of one gemv of n tokens, cycling back-to-back
    through `mats`, on device buffers x and y: stream launches, or (graph)
    replays of a hipGraph of the launches."""
    arr = (ctypes.c_void_p * len(mats))(*[m._h.value for m in mats])
    us = ctypes.c_float()
    fn = lib().llmhip_qmat_bench_graph if graph else lib().llmhip_qmat_bench
    check(fn(arr, len(mats), x.ptr, y.ptr, int(n), iters, warmup, None, ctypes.byref(us)))
    return us.value


def bench_h2d(nbytes, iters, device=0):
    """The pinned host-to-device copy rate in GB/s."""
    g = ctypes.c_float()
    check(lib().llmhip_bench_h2d(device, int(nbytes), iters, ctypes.byref(g)))
    return g.value


def copy_calibration(nbytes, device=0):
    """One device-to-device copy of nbytes."""
    check(lib().llmhip_copy_calibration(device, int(nbytes)))


Q4_0, Q4_1, Q8_0 = _lib.Q4_0, _lib.Q4_1, _lib.Q8_0
