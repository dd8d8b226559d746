"""Pins of the CPU oracle (oracle/cpuref.c), on the CPU.

Each oracle function is checked against something that would catch a plausible
mistake in it: the reference's own known values and invariants
(tokenizer_test.go:42-52, kernels_test.go:24-58), exhaustive comparisons with
numpy's IEEE conversions, and independent float64 formulations (vectorised
numpy, written from the mathematics rather than from cpu.go's loop order).
"""
import os
import struct

import numpy as np
import pytest

from llm_amd import synth
from tests import npblocks
from oracle import cpuref

F16_INF = 0x7C00


def f32(x):
    return np.float32(x)


# ---------------------------------------------------------------- f16.go

def test_f16_to_f32_exhaustive():
    """F16ToF32 (f16.go:6-28) of all 65536 patterns against numpy; NaN by class."""
    pat = np.arange(65536, dtype=np.uint16)
    got = cpuref.f16_to_f32(pat)
    want = pat.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # the Go function keeps the NaN payload: mantissa << 13, sign kept
    g = got[nan].view(np.uint32)
    p = pat[nan].astype(np.uint32)
    assert np.array_equal(g, ((p >> 15) << 31) | (0xFF << 23) | ((p & 0x3FF) << 13))


def test_f16_known_values():
    """tokenizer_test.go:42-52."""
    L = cpuref.lib()
    assert L.cpuref_f32_to_f16(1.0) == 0x3C00
    assert L.cpuref_f16_to_f32(0x3C00) == 1.0
    assert L.cpuref_f32_to_f16(65520.0) == 0x7C00
    for v in [0, 1, -2, 0.5, 65504, 6.1e-5, 5.96e-8, 3.14159]:
        h = L.cpuref_f32_to_f16(v)
        assert L.cpuref_f32_to_f16(L.cpuref_f16_to_f32(h)) == h


def test_f32_to_f16_matches_ieee_rne():
    """F32ToF16 (f16.go:30-66) is IEEE round-to-nearest-even: numpy on every
    finite f16 (exact round trip), on 2^20 random f32 patterns and on the
    halfway cases between adjacent f16 values."""
    pat = np.arange(65536, dtype=np.uint16)
    fin = pat[(pat & 0x7C00) != 0x7C00]
    assert np.array_equal(cpuref.f32_to_f16(fin.view(np.float16).astype(np.float32)), fin)
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    # bias toward the f16 range: exponents 100..143 cover subnormals, normals and overflow
    e = rng.integers(100, 144, size=bits.size).astype(np.uint32)
    bits = (bits & 0x807FFFFF) | (e << 23)
    x = bits.view(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(cpuref.f32_to_f16(x), want)
    # halfway points: midpoints of consecutive positive finite f16 values
    lo = fin[(fin < 0x7BFF)].view(np.float16).astype(np.float64)
    hi = (fin[(fin < 0x7BFF)] + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    ok = mid.astype(np.float64) == (lo + hi) / 2  # exactly representable midpoints
    assert np.array_equal(cpuref.f32_to_f16(mid[ok]), mid[ok].astype(np.float16).view(np.uint16))
    # NaN keeps its sign and becomes the quiet 0x7e00 (f16.go:35-37)
    nan_bits = np.array([0x7FC00000, 0xFFC00001, 0x7F800001], np.uint32)
    assert list(cpuref.f32_to_f16(nan_bits.view(np.float32))) == [0x7E00, 0xFE00, 0x7E00]


# ---------------------------------------------------------------- cpu.go

def test_rmsnorm_against_float64():
    rng = np.random.default_rng(1)
    for n in (32, 576, 896, 4864):
        x = rng.standard_normal(n).astype(np.float32) * 3
        w = (1 + 0.01 * rng.standard_normal(n)).astype(np.float32)
        got = cpuref.rmsnorm(x, w, 1e-5)
        xd = x.astype(np.float64)
        want = xd / np.sqrt(np.mean(xd * xd) + 1e-5) * w
        assert np.max(np.abs(got - want)) <= 2e-6 * np.max(np.abs(want))
    # closed form: a constant vector
    x = np.full(64, 2.0, np.float32)
    got = cpuref.rmsnorm(x, np.ones(64, np.float32), 0.0)
    assert np.allclose(got, 1.0, rtol=0, atol=1e-7)


@pytest.mark.parametrize("qtype", [synth.Q4_0, synth.Q4_1, synth.Q8_0])
def test_dequant_closed_form(qtype):
    rng = np.random.default_rng([2, qtype])
    raw = synth.quant_blocks(qtype, 7, 96, rng)
    got = cpuref.dequant(qtype, raw, 21)
    want = npblocks.dequant(qtype, raw, 21)
    # Q4_0 / Q8_0 products are exact in f32; Q4_1 has one rounding (d*q) and one (+m)
    if qtype == synth.Q4_1:
        assert np.max(np.abs(got - want)) <= 2 * np.finfo(np.float32).eps * np.max(np.abs(want))
    else:
        assert np.array_equal(got.astype(np.float64), want)


@pytest.mark.parametrize("qtype", [synth.Q4_0, synth.Q4_1, synth.Q8_0])
@pytest.mark.parametrize("rows,k", [(1, 32), (9, 64), (40, 576), (16, 1536)])
def test_matvec_against_float64(qtype, rows, k):
    rng = np.random.default_rng([3, qtype, rows, k])
    raw = synth.quant_blocks(qtype, rows, k, rng)
    x = rng.standard_normal(k).astype(np.float32)
    got = cpuref.matvec(qtype, raw, rows, k, x)
    W = npblocks.dequant(qtype, raw, rows * k // 32).reshape(rows, k)
    want = W @ x.astype(np.float64)
    scale = np.abs(W) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(got - want) <= 1e-6 * scale + 1e-30)
    # threads change nothing (rows keep their order)
    assert np.array_equal(cpuref.matvec(qtype, raw, rows, k, x, threads=4), got)


def test_matvec_single_block_closed_forms():
    # Q4_0 with every nibble 8 is zero; nibble 9 with d=1 gives sum(x)
    x = np.arange(32, dtype=np.float32) - 10
    blk = bytes(struct.pack("<e", 1.0)) + bytes([0x88] * 16)
    assert cpuref.matvec(synth.Q4_0, blk, 1, 32, x)[0] == 0
    blk = bytes(struct.pack("<e", 1.0)) + bytes([0x99] * 16)
    assert cpuref.matvec(synth.Q4_0, blk, 1, 32, x)[0] == np.sum(x)
    # Q4_1 with q=0 is m * sum(x); Q8_0 picks one element
    blk = bytes(struct.pack("<ee", 2.0, 0.5)) + bytes(16)
    assert cpuref.matvec(synth.Q4_1, blk, 1, 32, x)[0] == 0.5 * np.sum(x)
    q = np.zeros(32, np.int8)
    q[5] = -3
    blk = bytes(struct.pack("<e", 0.25)) + q.tobytes()
    assert cpuref.matvec(synth.Q8_0, blk, 1, 32, x)[0] == 0.25 * -3 * x[5]
    # F32 weights: a plain dot product
    w = np.random.default_rng(4).standard_normal((3, 32)).astype(np.float32)
    y = np.empty(3, np.float32)
    L = cpuref.lib()
    assert L.cpuref_matvec(y.ctypes.data, x.ctypes.data, 0, w.ctypes.data, 32, 3, 1) == 0
    assert np.allclose(y, w.astype(np.float64) @ x, rtol=1e-6)


def _neox_map(nr, hd):
    """fused.go:331-334."""
    h, k = divmod(nr, hd)
    return h * hd + k // 2 + (k % 2) * (hd // 2)


def test_rope_neox_invariant_exact():
    """kernels_test.go:24-58: adjacent-pair RoPE on neoxMap-permuted rows equals
    the permuted NEOX RoPE, exactly (hd 64, 3 heads, pos 37, base 1e6)."""
    hd, heads = 64, 3
    x = np.array([np.float32((i * 7919) % 101) / np.float32(17) - np.float32(3) for i in range(hd * heads)],
                 np.float32)
    perm = np.array([_neox_map(nr, hd) for nr in range(hd * heads)])
    assert len(set(perm)) == hd * heads
    want = cpuref.rope(x, 37, heads, hd, 1e6, True)[perm]
    got = cpuref.rope(x[perm], 37, heads, hd, 1e6, False)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    b = bytes(range(8))  # neoxRows byte case: rows 0,2,1,3 of 2 bytes
    rows = [b[2 * _neox_map(nr, 4):2 * _neox_map(nr, 4) + 2] for nr in range(4)]
    r = b"".join(rows)
    assert r[2] == 4 and r[4] == 2


def test_rope_against_float64_rotation():
    rng = np.random.default_rng(5)
    hd, heads = 64, 4
    x = rng.standard_normal(hd * heads).astype(np.float32)
    assert np.array_equal(cpuref.rope(x, 0, heads, hd, 1e4, False), x)  # pos 0 is the identity
    for neox in (False, True):
        for pos in (1, 37, 511, 4095):
            got = cpuref.rope(x, pos, heads, hd, 1e6 if neox else 1e4, neox).astype(np.float64)
            base = 1e6 if neox else 1e4
            want = x.astype(np.float64).copy()
            for h in range(heads):
                for i in range(hd // 2):
                    th = pos * base ** (-2 * i / hd)
                    a, bb = (h * hd + i, h * hd + i + hd // 2) if neox else (h * hd + 2 * i, h * hd + 2 * i + 1)
                    xa, xb = x[a], x[bb]
                    want[a] = xa * np.cos(th) - xb * np.sin(th)
                    want[bb] = xa * np.sin(th) + xb * np.cos(th)
            assert np.max(np.abs(got - want)) <= 1e-6


def test_rope_table():
    """The GPU's host table (gpu.go:524-534) holds the f32 cos and sin of cpu.go's theta."""
    cs = cpuref.rope_table(16, 64, 1e4).reshape(16, 32, 2)
    for pos in (0, 3, 15):
        for i in (0, 7, 31):
            th = pos * (1e4 ** (-2 * i / 64))
            assert abs(cs[pos, i, 0] - np.cos(th)) <= 6e-8 and abs(cs[pos, i, 1] - np.sin(th)) <= 6e-8


def test_argmax_special_cases():
    """cpu.go:389-397: first index of the maximum; NaN never wins; a NaN at 0 stays."""
    a = cpuref.argmax
    assert a([1, 3, 3, 2]) == 1
    assert a([5, 5, 5]) == 0
    assert a([1, np.nan, 2, 2]) == 2
    assert a([np.nan, 9, 10]) == 0
    assert a([-np.inf, -np.inf]) == 0
    assert a([-np.inf, -1e30]) == 1
    assert a([0.0, -0.0, 1e-45]) == 2


def test_quantize_q8_closed_form():
    """quantizeQ8 (cpu.go:117-140, ExactGGML mode; not on the graded path)."""
    x = np.linspace(-2, 2, 64).astype(np.float32)
    d, s, qs = cpuref.quantize_q8(x)
    for b in range(2):
        amax = np.max(np.abs(x[b * 32:(b + 1) * 32]))
        dd = np.float32(amax) / np.float32(127)
        assert d[b] == np.float16(dd).astype(np.float32)
        q = np.round(x[b * 32:(b + 1) * 32].astype(np.float64) * (np.float32(1) / dd)).astype(np.int8)
        assert np.array_equal(qs[b * 32:(b + 1) * 32], q)
    assert np.all(cpuref.quantize_q8(np.zeros(32, np.float32))[2] == 0)


def test_quantize_q8_invariants():
    """quantizeQ8's rounding and scales pinned by cases the mathematics fixes:
    with amax = 127 the scale is 1 and halfway values round away from zero
    (Go's math.Round; half-to-even would give 0, 2, -2); the element of
    largest magnitude maps to +-127; the Q8_1 sum s uses the unrounded scale;
    and every element dequantises to within half a step of its value."""
    x = np.zeros(64, np.float32)
    x[:8] = [127, 0.5, -0.5, 2.5, -2.5, 1.5, -126.5, 3.4999998]
    x[32:] = np.float32(1.0) / np.arange(1, 33, dtype=np.float32)  # amax 1: d = 1/127 is not a binary16 value
    d, s, qs = cpuref.quantize_q8(x)
    assert d[0] == 1 and list(qs[:8]) == [127, 1, -1, 3, -3, 2, -127, 3]
    assert s[0] == np.float16(np.sum(qs[:32].astype(np.int64))).astype(np.float32)
    d1 = np.float32(1) / np.float32(127)
    assert d[1] == np.float16(d1).astype(np.float32) and d[1] != d1 and qs[32] == 127
    assert s[1] == np.float16(d1 * np.float32(np.sum(qs[32:].astype(np.int64)))).astype(np.float32)
    rng = np.random.default_rng(3)
    y = (rng.standard_normal(32 * 50) * np.exp(rng.uniform(-8, 8, 1600))).astype(np.float32)
    d, s, qs = cpuref.quantize_q8(y)
    yb = y.reshape(50, 32).astype(np.float64)
    step = np.max(np.abs(yb), axis=1) / 127
    err = np.abs(qs.reshape(50, 32).astype(np.float64) * step[:, None] - yb)
    assert np.all(err <= step[:, None] * (0.5 + 1e-5))
    assert np.all(np.abs(qs.reshape(50, 32)).max(axis=1) == 127)


# ----------------------------------------------- the forward pass, float64

def _forward64(path, tokens, f16kv=False, exact=False):
    """An independent float64 forward pass of the model (cpu.go:225-366 as
    mathematics: dequantised matrices, vectorised attention with the global
    max), returning the logits of the last token.  f16kv: K and V rounded
    through binary16 before they enter the cache (numpy's float16 cast,
    round to nearest even).  exact: the products of ggml's CPU backend --
    each input vector (cast to f32) quantised to Q8 blocks, the integer block
    dot products exact, sum_b d_w d_x (w . x_q) (+ m_w s_x) in float64 -- and
    the binary16 cache."""
    from llm_amd import llm
    f = llm.Parse(path)
    c = llm.ConfigFrom(f)
    raw = open(path, "rb").read()
    f16kv = f16kv or exact

    def T(name):
        t, ok = f.Tensor(name)
        assert ok, name
        data = raw[f.DataOffset + t.Offset:f.DataOffset + t.Offset + t.Size]
        if t.Type == synth.F32:
            return np.frombuffer(data, np.float32).astype(np.float64)
        rows, k = t.Dims[1], t.Dims[0]
        wd = npblocks.dequant(t.Type, data, rows * k // 32).reshape(rows, k)
        if not exact:
            return wd
        d, m, q = npblocks.blocks(t.Type, data, rows * k // 32)
        return _QMat(wd, d.reshape(rows, -1), m.reshape(rows, -1), q.reshape(rows, k // 32, 32))

    E, H, KVH, HD, FF = c.embd, c.heads, c.kv_heads, c.head_dim, c.ff
    emb = T("token_embd.weight")
    out = emb if c.tied_output else T("output.weight")
    emb = emb.wd if exact else emb

    def rms(v, w):
        return v / np.sqrt(np.mean(v * v) + c.eps) * w

    def rope(v, pos, nh):
        v = v.reshape(nh, HD).copy()
        i = np.arange(HD // 2)
        th = pos * np.power(float(c.rope_base), -2.0 * i / HD)
        cs, sn = np.cos(th), np.sin(th)
        if c.rope_neox:
            a, b = v[:, :HD // 2].copy(), v[:, HD // 2:].copy()
            v[:, :HD // 2], v[:, HD // 2:] = a * cs - b * sn, a * sn + b * cs
        else:
            a, b = v[:, 0::2].copy(), v[:, 1::2].copy()
            v[:, 0::2], v[:, 1::2] = a * cs - b * sn, a * sn + b * cs
        return v.reshape(-1)

    L = [{n: T(f"blk.{l}.{n}") for n in ["attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight",
                                          "attn_output.weight", "ffn_norm.weight", "ffn_gate.weight",
                                          "ffn_up.weight", "ffn_down.weight"] +
          (["attn_q.bias", "attn_k.bias", "attn_v.bias"] if c.bias else [])} for l in range(c.layers)]
    K = [[] for _ in range(c.layers)]
    V = [[] for _ in range(c.layers)]
    for pos, tok in enumerate(tokens):
        x = emb[tok].copy()
        for l, w in enumerate(L):
            h = rms(x, w["attn_norm.weight"])
            q, k, v = w["attn_q.weight"] @ h, w["attn_k.weight"] @ h, w["attn_v.weight"] @ h
            if c.bias:
                q, k, v = q + w["attn_q.bias"], k + w["attn_k.bias"], v + w["attn_v.bias"]
            q, k = rope(q, pos, H), rope(k, pos, KVH)
            if f16kv:
                k, v = (z.astype(np.float32).astype(np.float16).astype(np.float64) for z in (k, v))
            K[l].append(k)
            V[l].append(v)
            Km, Vm = np.array(K[l]).reshape(pos + 1, KVH, HD), np.array(V[l]).reshape(pos + 1, KVH, HD)
            att = np.empty(H * HD)
            for hh in range(H):
                g = hh // (H // KVH)
                s = Km[:, g, :] @ q[hh * HD:(hh + 1) * HD] / np.sqrt(HD)
                p = np.exp(s - s.max())
                p /= p.sum()
                att[hh * HD:(hh + 1) * HD] = p @ Vm[:, g, :]
            x = x + w["attn_output.weight"] @ att
            h = rms(x, w["ffn_norm.weight"])
            gg, uu = w["ffn_gate.weight"] @ h, w["ffn_up.weight"] @ h
            x = x + w["ffn_down.weight"] @ (gg / (1 + np.exp(-gg)) * uu)
    return out @ rms(x, T("output_norm.weight"))


class _QMat:
    """A quantised matrix whose product with a vector is ggml's: x quantised by
    npblocks.quantize_q8, integer block dots, scales applied in float64."""

    def __init__(self, wd, d, m, q):
        self.wd, self.d, self.m, self.q = wd, d, m, q

    def __matmul__(self, x):
        dx, sx, qx = npblocks.quantize_q8(x)
        si = np.einsum("obj,bj->ob", self.q, qx).astype(np.float64)
        return (self.d * dx[None, :] * si).sum(axis=1) + (self.m * sx[None, :]).sum(axis=1)


@pytest.mark.parametrize("spec", [synth.tiny_llama(), synth.tiny_qwen(),
                                  synth.tiny_qwen(seed=7, types={"ffn_down": synth.Q4_1, "attn_v": synth.Q8_0})],
                         ids=["llama", "qwen2", "qwen2-mixed"])
def test_forward_against_float64(spec):
    path = synth.cached(spec)
    toks = list(synth.prompt(6, 9, spec.vocab))
    cpu = cpuref.CPU(path, 64)
    for t in toks:
        got = cpu.forward(t)
    want = _forward64(path, toks)
    rel = np.max(np.abs(got - want)) / np.max(np.abs(want))
    assert rel <= 1e-5, rel
    assert cpu.pos() == len(toks)


@pytest.mark.parametrize("spec", [synth.tiny_llama(), synth.tiny_qwen(),
                                  synth.tiny_qwen(seed=7, types={"ffn_down": synth.Q4_1, "attn_v": synth.Q8_0})],
                         ids=["llama", "qwen2", "qwen2-mixed"])
def test_forward_exact_ggml_against_float64(spec):
    """The ExactGGML mode (cpu.go:15-21, 117-140, 166-214, 298-299): within
    1e-6 of the float64 forward that quantises every matrix input the same way
    and keeps a binary16 cache, and at least 1000 times closer to it than to
    the unquantised float64 forward (measured: 4e-8 to 1.2e-7 against 3e-3 to
    9e-3), so a wrong rounding, scale or Q4_1 term fails."""
    path = synth.cached(spec)
    toks = list(synth.prompt(11, 40, spec.vocab))
    cpu = cpuref.CPU(path, 64, exact_ggml=True)
    for t in toks:
        got = cpu.forward(t)
    we, wp = _forward64(path, toks, exact=True), _forward64(path, toks)
    re_, rp = (np.max(np.abs(got - w)) / np.max(np.abs(w)) for w in (we, wp))
    assert re_ <= 1e-6 and rp >= 1000 * re_, (re_, rp)


@pytest.mark.parametrize("spec", [synth.tiny_llama(), synth.tiny_qwen()], ids=["llama", "qwen2"])
def test_forward_f16kv_against_float64(spec):
    """The F16KV mode (cpu.go:22-24, 298-299): within 1.5e-5 of a float64
    forward whose cache holds binary16-rounded K and V, and at least four times
    closer to it than to the float64 forward with an exact cache.  The f32
    mode sits 3.5e-5 to 1e-4 from the rounded forward, so a mode that did not
    round, or rounded something else, fails."""
    path = synth.cached(spec)
    toks = list(synth.prompt(11, 60, spec.vocab))
    cpu = cpuref.CPU(path, 64, f16kv=True)
    for t in toks:
        got = cpu.forward(t)
    want16, want32 = _forward64(path, toks, f16kv=True), _forward64(path, toks)
    scale = np.max(np.abs(want16))
    r16, r32 = np.max(np.abs(got - want16)) / scale, np.max(np.abs(got - want32)) / scale
    assert r16 <= 1.5e-5 and r32 >= 4 * r16, (r16, r32)


def test_forward_modes_and_layers():
    spec = synth.tiny_llama(layers=3)
    path = synth.cached(spec)
    cpu = cpuref.CPU(path, 32)
    cpu.set_max_layers(-1)  # no layers: the embedding row itself
    assert cpu.forward(7) is None
    t, _, _ = cpu.tensor("token_embd.weight")
    nb = spec.embd // 32
    row = cpuref.dequant(synth.Q4_0, t[7 * nb * 18:(7 + 1) * nb * 18], nb)
    assert np.array_equal(cpu.last_x().view(np.uint32), row.view(np.uint32))
    assert cpu.pos() == 1
    cpu.set_max_layers(0)
    cpu.reset()
    a = cpu.forward(3)
    # F16KV rounds the cache through binary16: close to, not equal to, f32
    c2 = cpuref.CPU(path, 32, f16kv=True)
    c2.forward(3)
    b = c2.forward(5)
    a = cpu.forward(5)
    assert not np.array_equal(a, b) and np.max(np.abs(a - b)) <= 1e-2 * np.max(np.abs(a))
    with pytest.raises(RuntimeError):
        full = cpuref.CPU(path, 1)
        full.forward(1)
        full.forward(2)  # context full (cpu.go:227-229)


def test_threaded_forward_bit_identical():
    """Row-parallel matvec and head-parallel attention keep every sum's order."""
    spec = synth.tiny_qwen()
    path = synth.cached(spec)
    toks = list(synth.prompt(8, 80, spec.vocab))
    a, b = cpuref.CPU(path, 128, threads=1), cpuref.CPU(path, 128, threads=4)
    for t in toks:
        la, lb = a.forward(t), b.forward(t)
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))


def test_config4_golden_consistent():
    """The committed config-4 fixtures agree with each other: the logits file
    is the one the JSON's hash names, its argmax (the oracle's Argmax rule) is
    the first greedy token, its 16 largest are the recorded ones."""
    import hashlib
    import json
    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    gold = json.load(open(os.path.join(here, "config4.json")))
    l = np.load(os.path.join(here, gold["logits_file"]))["logits"]
    assert hashlib.sha256(l.astype("<f4").tobytes()).hexdigest() == gold["logits_sha256"]
    assert cpuref.argmax(l) == gold["steps"][0]["tok"]
    assert [[int(i), float(v)] for i, v in gold["first_top16"]] == [[int(i), float(l[i])] for i, _ in gold["first_top16"]]
    assert float(np.max(np.abs(l))) == gold["steps"][0]["maxabs"]
