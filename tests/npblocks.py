"""The GGUF block formats and ggml's activation quantisation restated in
vectorised numpy, independently of the C oracle: the checks that pin it
(tests/test_oracle.py) and the error bounds of the GPU tests use them."""
import numpy as np

from llm_amd import synth


def dequant(qtype, raw, nblocks):
    """The GGUF block formats decoded in numpy, vectorised (ggml's layouts:
    Q4_0 byte j holds element j in the low nibble and j+16 in the high one)."""
    b = np.frombuffer(raw, np.uint8)
    if qtype == synth.Q4_0:
        blk = b.reshape(nblocks, 18)
        d = blk[:, :2].copy().view(np.float16).astype(np.float64)
        q = np.concatenate([blk[:, 2:] & 15, blk[:, 2:] >> 4], axis=1).astype(np.float64) - 8
        return (d * q).reshape(-1)
    if qtype == synth.Q4_1:
        blk = b.reshape(nblocks, 20)
        d = blk[:, :2].copy().view(np.float16).astype(np.float64)
        m = blk[:, 2:4].copy().view(np.float16).astype(np.float64)
        q = np.concatenate([blk[:, 4:] & 15, blk[:, 4:] >> 4], axis=1).astype(np.float64)
        return (d * q + m).reshape(-1)
    blk = b.reshape(nblocks, 34)
    d = blk[:, :2].copy().view(np.float16).astype(np.float64)
    return (d * blk[:, 2:].view(np.int8).astype(np.float64)).reshape(-1)


def blocks(qtype, raw, nblocks):
    """The GGUF blocks as (d, m, integer weights [nblocks][32]) in element order (Q4_0 minus 8)."""
    b = np.frombuffer(raw, np.uint8)
    if qtype == synth.Q4_0:
        blk = b.reshape(nblocks, 18)
        d = blk[:, :2].copy().view(np.float16).astype(np.float64)[:, 0]
        q = np.concatenate([blk[:, 2:] & 15, blk[:, 2:] >> 4], axis=1).astype(np.int64) - 8
        return d, np.zeros_like(d), q
    if qtype == synth.Q4_1:
        blk = b.reshape(nblocks, 20)
        d = blk[:, :2].copy().view(np.float16).astype(np.float64)[:, 0]
        m = blk[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
        return d, m, np.concatenate([blk[:, 4:] & 15, blk[:, 4:] >> 4], axis=1).astype(np.int64)
    blk = b.reshape(nblocks, 34)
    d = blk[:, :2].copy().view(np.float16).astype(np.float64)[:, 0]
    return d, np.zeros_like(d), blk[:, 2:].view(np.int8).astype(np.int64)


def quantize_q8(x):
    """Activation quantisation to Q8_0 / Q8_1 blocks in numpy float32
    arithmetic: d = amax / 127, q = round half away from zero of x * (1/d),
    scales rounded through binary16."""
    x = np.asarray(x, np.float32).reshape(-1, 32)
    d = (np.max(np.abs(x), axis=1) / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    v = (x * inv[:, None]).astype(np.float32).astype(np.float64)
    q = np.where(v >= 0, np.floor(v + 0.5), np.ceil(v - 0.5)).astype(np.int64)
    s = (d * q.sum(axis=1).astype(np.float32)).astype(np.float32)
    return d.astype(np.float16).astype(np.float64), s.astype(np.float16).astype(np.float64), q


def block_terms(qtype, raw, rows, k, x):
    """ggml's per-block terms p[row][b] = d_w d_x (w . x_q) (+ m_w s_x) in
    float64, for x (f32) quantised by quantize_q8: the summands of the
    ExactGGML product, whose f32 sum in any order is within (nb - 1) u sum|p|."""
    d, m, q = blocks(qtype, raw, rows * k // 32)
    dx, sx, qx = quantize_q8(x)
    si = np.einsum("obj,bj->ob", q.reshape(rows, k // 32, 32), qx).astype(np.float64)
    return d.reshape(rows, -1) * dx[None, :] * si + m.reshape(rows, -1) * sx[None, :]
