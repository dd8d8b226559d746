"""llmhip_qmat_gemv_noalloc, the allocation-free form of llmhip_qmat_gemv
(for callers that cannot allocate), against llmhip_qmat_gemv through the
C-ABI: the same kernels, so the same bits.  Two calls in a row on the
process's one scratch array, the second with a smaller input (fewer tokens,
a shorter k, a different matrix), then the decode form (no scratch), the
accumulate epilogue, and the refusals (k above the array's maximum, n above
64).  Run alone in a fresh process and after the rest of the suite."""
import ctypes

import numpy as np
import pytest

from llm_amd import synth

pytestmark = pytest.mark.gpu


def _pair(m, x, n, accumulate=False, y0=None):
    from llm_amd import _lib, kernels
    L = _lib.lib()
    xd = kernels.DeviceBuffer.from_numpy(x)
    init = np.zeros((n, m.rows), np.float32) if y0 is None else y0
    ya, yb = kernels.DeviceBuffer.from_numpy(init), kernels.DeviceBuffer.from_numpy(init)
    _lib.check(L.llmhip_qmat_gemv(m._h, xd.ptr, ya.ptr, n, int(accumulate), None))
    _lib.check(L.llmhip_qmat_gemv_noalloc(m._h, xd.ptr, yb.ptr, n, int(accumulate), None))
    kernels.synchronize()
    a, b = ya.numpy(np.float32, (n, m.rows)), yb.numpy(np.float32, (n, m.rows))
    for d in (xd, ya, yb):
        d.close()
    return a, b


def test_noalloc_matches_gemv(gpu):
    from llm_amd import _lib, kernels
    from llm_amd._lib import LLMError
    from oracle import cpuref
    L = _lib.lib()
    rng = np.random.default_rng(11)
    cases = [(synth.Q4_0, 4864, 896, 64), (synth.Q8_0, 896, 4864, 64),  # gate/up and down shapes, 64 tokens
             (synth.Q4_1, 576, 576, 9), (synth.Q4_0, 100, 96, 5)]       # then smaller inputs
    for qt, rows, k, n in cases:
        print(f"type {qt} {rows}x{k}, {n} tokens", flush=True)
        raw = synth.quant_blocks(qt, rows, k, rng, q8_div=8.0)
        m = kernels.QMat(qt, rows, k, raw)
        x = rng.standard_normal((n, k), dtype=np.float32)
        a, b = _pair(m, x, n)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        want = np.stack([cpuref.matvec(qt, raw, rows, k, x[t]) for t in range(n)])
        assert float(np.max(np.abs(b - want)) / np.max(np.abs(want))) <= 1e-5
        m.close()
    # the decode form (no scratch) and the accumulate epilogue
    raw = synth.quant_blocks(synth.Q4_0, 896, 896, rng)
    m = kernels.QMat(synth.Q4_0, 896, 896, raw)
    for n in (1, 4, 12):
        x = rng.standard_normal((n, 896), dtype=np.float32)
        y0 = rng.standard_normal((n, 896), dtype=np.float32)
        a, b = _pair(m, x, n, accumulate=True, y0=y0)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), n
    # refusals: n outside 1..64, k above the scratch's maximum
    xd, yd = kernels.DeviceBuffer(65 * 896 * 4), kernels.DeviceBuffer(65 * 896 * 4)
    for n in (0, 65):
        with pytest.raises(LLMError):
            _lib.check(L.llmhip_qmat_gemv_noalloc(m._h, xd.ptr, yd.ptr, n, 0, None))
    big = kernels.QMat(synth.Q4_0, 16, 8192 + 32, synth.quant_blocks(synth.Q4_0, 16, 8192 + 32, rng))
    with pytest.raises(LLMError) as e:
        _lib.check(L.llmhip_qmat_gemv_noalloc(big._h, xd.ptr, yd.ptr, 8, 0, None))
    assert e.value.kind == "ARG" and "8192" in str(e.value)
    for o in (xd, yd, big, m):
        o.close()


def _hip():
    """The HIP runtime libllmhip.so links (already mapped: the same instance)."""
    from llm_amd import _lib
    _lib.lib()
    hip = ctypes.CDLL("libamdhip64.so.7")
    vp = ctypes.c_void_p
    for name, args in (("hipStreamCreateWithFlags", [ctypes.POINTER(vp), ctypes.c_uint]),
                       ("hipStreamBeginCapture", [vp, ctypes.c_int]), ("hipStreamEndCapture", [vp, ctypes.POINTER(vp)]),
                       ("hipGraphInstantiate", [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t]),
                       ("hipGraphLaunch", [vp, vp]), ("hipStreamSynchronize", [vp]), ("hipGraphExecDestroy", [vp]),
                       ("hipGraphDestroy", [vp]), ("hipStreamDestroy", [vp]), ("hipSetDevice", [ctypes.c_int])):
        getattr(hip, name).argtypes = args
        getattr(hip, name).restype = ctypes.c_int
    return hip


def test_noalloc_under_graph_capture(gpu):
    """The allocation-free product captured into a HIP graph (64 tokens: the
    prep and product pair on the scratch array) on a non-blocking stream,
    captured from a fresh matrix whose first product is the captured one
    (nothing is left to allocate or look up at call time), then replayed five
    times with eager products of another matrix on the same scratch in
    between; every replay is bit-equal to llmhip_qmat_gemv's result."""
    from llm_amd import _lib, kernels
    L, hip = _lib.lib(), _hip()
    rng = np.random.default_rng(23)
    rows, k, n = 4864, 896, 64
    raw = synth.quant_blocks(synth.Q4_0, rows, k, rng)
    m = kernels.QMat(synth.Q4_0, rows, k, raw)
    other = kernels.QMat(synth.Q8_0, 896, 4864, synth.quant_blocks(synth.Q8_0, 896, 4864, rng, q8_div=8.0))
    x = rng.standard_normal((n, k), dtype=np.float32)
    xd = kernels.DeviceBuffer.from_numpy(x)
    yd = kernels.DeviceBuffer(n * rows * 4)
    x2 = kernels.DeviceBuffer.from_numpy(rng.standard_normal((n, 4864), dtype=np.float32))
    y2 = kernels.DeviceBuffer(n * 896 * 4)
    s, g, ex = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipSetDevice(0) == 0
    assert hip.hipStreamCreateWithFlags(ctypes.byref(s), 1) == 0  # hipStreamNonBlocking
    try:
        assert hip.hipStreamBeginCapture(s, 1) == 0  # hipStreamCaptureModeThreadLocal
        rc = L.llmhip_qmat_gemv_noalloc(m._h, xd.ptr, yd.ptr, n, 0, s)
        assert hip.hipStreamEndCapture(s, ctypes.byref(g)) == 0
        _lib.check(rc)
        assert hip.hipGraphInstantiate(ctypes.byref(ex), g, None, None, 0) == 0
        ref = kernels.DeviceBuffer(n * rows * 4)
        _lib.check(L.llmhip_qmat_gemv(m._h, xd.ptr, ref.ptr, n, 0, None))
        kernels.synchronize()
        want = ref.numpy(np.float32, (n, rows))
        for rep in range(5):
            yd.write(np.full((n, rows), np.nan, np.float32))
            _lib.check(L.llmhip_qmat_gemv_noalloc(other._h, x2.ptr, y2.ptr, n, 0, None))  # the scratch, reused
            kernels.synchronize()
            assert hip.hipGraphLaunch(ex, s) == 0 and hip.hipStreamSynchronize(s) == 0
            got = yd.numpy(np.float32, (n, rows))
            print(f"replay {rep}: bit-equal {np.array_equal(got.view(np.uint32), want.view(np.uint32))}", flush=True)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rep
        ref.close()
    finally:
        if ex.value:
            hip.hipGraphExecDestroy(ex)
        if g.value:
            hip.hipGraphDestroy(g)
        hip.hipStreamDestroy(s)
        for o in (xd, yd, x2, y2, m, other):
            o.close()
