"""The C-ABI library on a machine without a GPU: it loads, it exports every
function include/llmhip.h declares, the ctypes binding covers exactly those,
and the calls that need no device behave (no compute calls are made here)."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "llmhip.h")).read()
    return set(re.findall(r"LLMHIP_API\s+[\w\s\*]+?\b(llm\w+)\s*\(", src))


def test_header_symbols_exported():
    from llm_amd import _lib
    names = declared()
    assert len(names) >= 40
    so = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in sorted(names) if not hasattr(so, n)]
    assert not missing, missing


def test_binding_matches_header():
    from llm_amd import _lib
    bound = {n for n, _, _ in _lib.SIGNATURES}
    assert bound == declared()
    _lib.lib()  # every signature resolves


def test_oracle_library_loads():
    from oracle import cpuref
    L = cpuref.lib()
    for n in ("cpuref_forward", "cpuref_matvec", "cpuref_f16_to_f32", "cpuref_load", "cpuref_argmax"):
        assert hasattr(L, n)


def test_no_device_calls_fail_cleanly():
    from llm_amd import _lib
    n = ctypes.c_int(-1)
    rc = _lib.lib().llmhip_device_count(ctypes.byref(n))
    assert rc in (0, -2) and n.value >= 0
    assert isinstance(_lib.lib().llmhip_last_error(), bytes)


def test_host_argmax_and_tunables():
    from llm_amd import llm
    assert llm.Argmax([1, 5, 5, 2]) == 1
    assert llm.Argmax([np.nan, 3]) == 0
    assert llm.Argmax([1, np.nan, 4]) == 2
    assert llm.MaxBatch == 16 and llm.DecodeBatch == 8 and llm.PrefillBatch == 64
    assert llm.PieceSize == 4 << 20 and llm.ChunkSize == 16 << 20


def test_synth_writer_layout(tmp_path):
    """The synthetic files hold the block formats and distributions they claim."""
    from llm_amd import synth
    spec = synth.tiny_qwen(types={"ffn_down": synth.Q4_1, "attn_v": synth.Q8_0})
    path = synth.write(str(tmp_path / "m.gguf"), spec)
    from llm_amd import llm
    f = llm.Parse(path)
    raw = open(path, "rb").read()
    t, ok = f.Tensor("blk.1.ffn_down.weight")
    assert ok and t.Type == synth.Q4_1 and t.Dims == [spec.ff, spec.embd]
    blk = np.frombuffer(raw[f.DataOffset + t.Offset:f.DataOffset + t.Offset + t.Size], np.uint8).reshape(-1, 20)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32)
    m = blk[:, 2:4].copy().view(np.float16).astype(np.float32)
    assert np.all(d >= 0) and np.array_equal(m, (d * -8).astype(np.float16).astype(np.float32))
    t, _ = f.Tensor("blk.0.attn_v.weight")
    blk = np.frombuffer(raw[f.DataOffset + t.Offset:f.DataOffset + t.Offset + t.Size], np.uint8).reshape(-1, 34)
    q = blk[:, 2:].view(np.int8)
    assert q.min() >= -127 and q.max() <= 127
    n, _ = f.Tensor("blk.0.attn_norm.weight")
    w = np.frombuffer(raw[f.DataOffset + n.Offset:f.DataOffset + n.Offset + n.Size], np.float32)
    assert abs(w.mean() - 1) < 0.01 and 0.003 < w.std() < 0.03
    # the same seed gives the same bytes
    path2 = synth.write(str(tmp_path / "m2.gguf"), spec)
    assert open(path2, "rb").read() == raw
    p = synth.prompt(3, 100, 640)
    assert p.min() >= 0 and p.max() < 640 and np.array_equal(p, synth.prompt(3, 100, 640))
