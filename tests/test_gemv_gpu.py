"""GPU parity of the quantised matrix kernels against the CPU oracle.

* dequantisation: bit-exact against cpuref_dequant (the weight values of
  cpu.go:233-251), every f16 scale pattern included (NaN compared by class);
* the isolated-kernel sweep: Q4_0 / Q8_0 (and Q4_1)
  weights x f32 activations ~N(0,1), shapes of both models, N = 1, 8, 64,
  checked against cpuref_matvec (cpu.go:143-222) within 1e-5 relative
  (max|gpu-cpu| / max|cpu|, the `check` metric of examples/generate/main.go:159-165);
* ragged shapes: rows not a multiple of 16, k with 1-3 trailing blocks.
"""
import functools

import numpy as np
import pytest

from llm_amd import synth
from tests import npblocks

pytestmark = pytest.mark.gpu

SWEEP = [(576, 576), (1536, 576), (576, 1536), (896, 896), (4864, 896), (896, 4864), (151936, 896)]
TOL = 1e-5


@functools.lru_cache(maxsize=4)
def _raw(qtype, rows, k, seed):
    rng = np.random.default_rng([seed, rows, k, qtype])
    return synth.quant_blocks(qtype, rows, k, rng, q8_div=8.0)


def _x(n, k, seed):
    return np.random.default_rng([seed, n, k]).standard_normal((n, k), dtype=np.float32)


def _rel(gpu, cpu):
    return float(np.max(np.abs(gpu.astype(np.float64) - cpu)) / max(np.max(np.abs(cpu)), 1e-30))


def _check_gemv(gpu, oracle, qtype, rows, k, n, seed=7, threads=16):
    from llm_amd.kernels import QMat
    print(f"gemv qtype={qtype} rows={rows} k={k} n={n}", flush=True)
    raw = _raw(qtype, rows, k, seed)
    m = QMat(qtype, rows, k, raw)
    x = _x(n, k, seed)
    y = m.gemv(x)
    want = np.stack([oracle.matvec(qtype, raw, rows, k, x[t], threads=threads) for t in range(n)])
    rel = _rel(y, want)
    assert rel <= TOL, f"rows={rows} k={k} n={n}: relative error {rel:.3e}"
    m.close()
    return rel


@pytest.mark.parametrize("qtype", [2, 8])
@pytest.mark.parametrize("rows,k", SWEEP)
@pytest.mark.parametrize("n", [1, 8, 64])
def test_sweep(gpu, oracle, qtype, rows, k, n):
    _check_gemv(gpu, oracle, qtype, rows, k, n)


@pytest.mark.parametrize("qtype", [2, 3, 8])
@pytest.mark.parametrize("rows,k,n", [(896, 896, 1), (1152, 896, 2), (896, 4864, 3), (4864, 896, 1), (37, 96, 1),
                                      (130, 224, 2), (33, 576, 4), (896, 896, 8), (9728, 896, 64), (896, 4864, 64),
                                      (130, 224, 5), (151936, 896, 1), (65541, 576, 1), (4100, 608, 37)])
def test_exact_ggml_gemv(gpu, oracle, qtype, rows, k, n):
    """The ExactGGML product (cpu.go:117-140, 166-214) against the oracle's,
    through the decode tile kernel (1-4 tokens), the streaming kernel (one
    token, >= 4096 tiles) and the prefill pair (>= 5 tokens).  Both sides
    quantise the same f32 inputs with the same f32 operations, so the codes,
    the integer block sums and each block's term p_b agree exactly; only the
    order of the f32 sum over the nb blocks differs, so every output is within
    2 (nb - 1) u sum_b |p_b| (u = 2^-24) of the oracle's -- for Q4_1, whose
    m_w s_x terms cancel, that is up to ~1e-5 of max|y|, otherwise ~1e-7.  The
    f32 product of the same inputs sits 1e-2 to 3e-2 away, so an input left
    unquantised fails."""
    from llm_amd.kernels import QMat
    print(f"gemv_q8 qtype={qtype} rows={rows} k={k} n={n}", flush=True)
    raw = _raw(qtype, rows, k, 11)
    m = QMat(qtype, rows, k, raw)
    x = _x(n, k, 11)
    x[0, :32] = np.concatenate([[127], np.arange(31) - 14.5])  # scale 1: halfway values round away from zero
    if k >= 64:
        x[0, 32:64] = 0  # an all-zero block: d = 0, every code 0
    y = m.gemv_q8(x)
    m.close()
    want = np.stack([oracle.matvec(qtype, raw, rows, k, x[t], threads=16, q8=True) for t in range(n)])
    plain = np.stack([oracle.matvec(qtype, raw, rows, k, x[t], threads=16) for t in range(min(n, 2))])
    rel = _rel(y, want)
    print(f"relative error {rel:.3e}; f32 product {_rel(plain, want[:len(plain)]):.3e} away", flush=True)
    nb = k // 32
    for t in range(n):
        bound = 2 * (nb - 1) * 2.0 ** -24 * np.abs(npblocks.block_terms(qtype, raw, rows, k, x[t])).sum(axis=1)
        err = np.abs(y[t].astype(np.float64) - want[t])
        assert np.all(err <= bound + 1e-30), (t, float(np.max(err / (bound + 1e-30))))
    assert rel <= 2e-5 and _rel(plain, want[:len(plain)]) >= 100 * max(rel, 1e-8)


@pytest.mark.parametrize("qtype", [2, 3, 8])
@pytest.mark.parametrize("rows,k,n", [(16, 32, 1), (37, 96, 1), (5, 160, 3), (33, 576, 2), (130, 224, 5),
                                      (64, 4864, 4), (1, 32, 1), (17, 1312, 7)])
def test_ragged(gpu, oracle, qtype, rows, k, n):
    _check_gemv(gpu, oracle, qtype, rows, k, n)


@pytest.mark.parametrize("qtype", [2, 3, 8])
@pytest.mark.parametrize("rows,k,n", [(4100, 608, 37), (4111, 4864, 13), (4096, 160, 64), (300, 1312, 9)])
def test_prefill_edges(gpu, oracle, qtype, rows, k, n):
    """The prefill product's clamped indices: an odd tile count on two-tile
    workgroups (257 tiles, the last workgroup half empty), a row count that
    is not a multiple of 16, trailing blocks (608 = 4 groups + 3 blocks,
    4864 = 38 groups, 160 = 1 group + 1 block, 1312 = 10 groups + 1), an odd
    number of 8-token groups (37 tokens: 5 groups on two-group workgroups)
    and a partial last group."""
    _check_gemv(gpu, oracle, qtype, rows, k, n)


@pytest.mark.parametrize("qtype", [3])
@pytest.mark.parametrize("rows,k", [(896, 4864), (4864, 896)])
@pytest.mark.parametrize("n", [1, 8])
def test_q41_shapes(gpu, oracle, qtype, rows, k, n):
    _check_gemv(gpu, oracle, qtype, rows, k, n)


@pytest.mark.parametrize("qtype", [2, 3, 8])
@pytest.mark.parametrize("rows,k", [(65541, 896), (70000, 512), (65536, 4864), (65541, 576), (70000, 224)])
def test_stream_shapes(gpu, oracle, qtype, rows, k):
    """One-token launches of 4096 tiles or more whose k is whole 4-block
    groups take the streaming kernel: ragged rows at k = 896 (one tile's 7
    groups in flight per wave), 4 groups per tile (the ring form), and a k
    that needs 8 waves per workgroup.  With tail blocks (576 = 4 groups + 2
    blocks, 224 = 7 blocks) the same launch takes the tile kernel."""
    _check_gemv(gpu, oracle, qtype, rows, k, 1)


def test_stream_accumulate(gpu, oracle):
    from llm_amd.kernels import QMat
    rows, k = 70001, 896
    raw = _raw(8, rows, k, 4)
    m = QMat(8, rows, k, raw)
    x = _x(1, k, 4)
    y0 = np.random.default_rng(6).standard_normal((1, rows), dtype=np.float32)
    y = m.gemv(x, y0, accumulate=True)
    want = y0.astype(np.float64) + oracle.matvec(8, raw, rows, k, x[0])[None]
    assert _rel(y, want) <= TOL


def test_accumulate(gpu, oracle):
    from llm_amd.kernels import QMat
    rows, k = 896, 4864
    raw = _raw(2, rows, k, 3)
    m = QMat(2, rows, k, raw)
    x = _x(2, k, 3)
    y0 = np.random.default_rng(5).standard_normal((2, rows), dtype=np.float32)
    y = m.gemv(x, y0, accumulate=True)
    want = y0.astype(np.float64) + np.stack([oracle.matvec(2, raw, rows, k, x[t]) for t in range(2)])
    assert _rel(y, want) <= TOL


@pytest.mark.parametrize("qtype", [2, 3, 8])
@pytest.mark.parametrize("rows,k", [(37, 96), (48, 576), (16, 160), (300, 896)])
def test_dequant_bit_exact(gpu, oracle, qtype, rows, k):
    from llm_amd.kernels import QMat
    print(f"dequant qtype={qtype} rows={rows} k={k}", flush=True)
    raw = _raw(qtype, rows, k, 11)
    m = QMat(qtype, rows, k, raw)
    got = m.dequant().reshape(-1)
    want = oracle.dequant(qtype, raw, rows * k // 32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("qtype", [2, 3, 8])
def test_dequant_every_scale(gpu, oracle, qtype):
    """All 65536 f16 scale patterns (and minima for Q4_1), bit for bit; NaN by class."""
    from llm_amd.kernels import QMat
    rows, k = 65536, 32
    bb = {2: 18, 3: 20, 8: 34}[qtype]
    rng = np.random.default_rng(13)
    blk = np.zeros((rows, bb), np.uint8)
    pat = np.arange(rows, dtype=np.uint16)
    blk[:, 0:2] = pat.view(np.uint8).reshape(rows, 2)
    if qtype == 3:
        blk[:, 2:4] = rng.permutation(pat).view(np.uint8).reshape(rows, 2)
    blk[:, (4 if qtype == 3 else 2):] = rng.integers(0, 256, size=(rows, bb - (4 if qtype == 3 else 2)),
                                                     dtype=np.uint8)
    raw = blk.tobytes()
    m = QMat(qtype, rows, k, raw)
    got = m.dequant().reshape(-1)
    want = oracle.dequant(qtype, raw, rows)
    nan_g, nan_w = np.isnan(got), np.isnan(want)
    assert np.array_equal(nan_g, nan_w)
    assert np.array_equal(got[~nan_g].view(np.uint32), want[~nan_w].view(np.uint32))


def test_gemv_scale_exact(gpu, oracle):
    """The matvec's hardware f16->f32 scale conversion is exact for every finite f16."""
    from llm_amd.kernels import QMat
    pat = np.arange(65536, dtype=np.uint16)
    pat = pat[((pat >> 10) & 0x1f) != 31]  # finite scales
    rows = pat.size
    blk = np.zeros((rows, 34), np.uint8)
    blk[:, 0:2] = pat.view(np.uint8).reshape(rows, 2)
    blk[:, 2] = 1  # element 0 is 1, the rest 0
    m = QMat(8, rows, 32, blk.tobytes())
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 1
    y = m.gemv(x).reshape(-1)
    # cpu.go sums from +0, so a -0 scale gives +0: compare with the oracle's matvec,
    # and with the scale itself elsewhere
    want = oracle.matvec(8, blk.tobytes(), rows, 32, x[0])
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
    nz = pat != 0x8000
    assert np.array_equal(y[nz].view(np.uint32), oracle.f16_to_f32(pat[nz]).view(np.uint32))


def test_upload_in_pieces(gpu, oracle):
    """Whole-block pieces in any order give the same matrix (the streaming loader's contract)."""
    from llm_amd.kernels import QMat
    rows, k, bb = 200, 896, 18
    raw = _raw(2, rows, k, 21)
    nblk = rows * k // 32
    m = QMat(2, rows, k)
    cuts = [0, 1, 57, 1000, 3001, nblk]
    for a, b in reversed(list(zip(cuts[:-1], cuts[1:]))):
        m.upload(np.frombuffer(raw, np.uint8)[a * bb:b * bb], byte_offset=a * bb)
    got = m.dequant().reshape(-1)
    want = oracle.dequant(2, raw, nblk)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    with pytest.raises(Exception):
        m.upload(np.zeros(17, np.uint8), byte_offset=0)  # not whole blocks
    x = _x(1, k, 1)
    y = m.gemv(x)
    assert _rel(y, oracle.matvec(2, raw, rows, k, x[0])[None]) <= TOL


@pytest.mark.parametrize("n", [1, 8])
def test_bench_graph(gpu, oracle, n):
    """The sweep's graph-replay measurement (llmhip_qmat_bench_graph) runs the
    same product: after the replays y holds the gemv of the last matrix."""
    from llm_amd import kernels
    qtype, rows, k = 2, 65541, 896  # 1-token launches take the streaming kernel
    raw = _raw(qtype, rows, k, 21)
    m = kernels.QMat(qtype, rows, k, raw)
    c = m.clone()
    x = _x(n, k, 21)
    xb = kernels.DeviceBuffer.from_numpy(x)
    yb = kernels.DeviceBuffer(n * rows * 4)
    us = kernels.bench([m, c], xb, yb, n, iters=40, warmup=2, graph=True)
    assert us > 0
    y = yb.numpy(np.float32, (n, rows))
    want = np.stack([oracle.matvec(qtype, raw, rows, k, x[t], threads=16) for t in range(n)])
    assert _rel(y, want) <= TOL
    for b in (xb, yb, c, m):
        b.close()
