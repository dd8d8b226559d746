"""The measurement plumbing on the CPU: the source fingerprint that ties a
counter summary under profiles/ to the kernels it measured, and bench.py's
refusal of a stale traffic or duration figure."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_sources_hash_stable():
    from llm_amd import profsum
    h = profsum.sources_hash()
    assert len(h) == 12 and int(h, 16) >= 0
    assert profsum.sources_hash() == h


def test_figures_only_for_matching_sources(tmp_path, monkeypatch):
    import bench
    from llm_amd import profsum
    good = tmp_path / "good.txt"
    good.write_text(f"header\nsources_hash {profsum.sources_hash()}\ntraffic_bytes k5 123\nduration_us pass 321.5\n")
    stale = tmp_path / "stale.txt"
    stale.write_text("sources_hash 000000000000\ntraffic_bytes k5 123\nduration_us pass 321.5\n")
    monkeypatch.setattr(bench, "PMC_SUMMARY", str(good))
    assert bench.pmc_value("traffic_bytes", "k5")[0] == 123
    assert bench.pmc_value("traffic_bytes", "k4")[0] is None
    assert bench.pmc_value("duration_us", "pass")[0] == 321.5
    assert bench.pmc_value("duration_us", "k5")[0] is None
    monkeypatch.setattr(bench, "PMC_SUMMARY", str(stale))
    for kind, cls in (("traffic_bytes", "k5"), ("duration_us", "pass")):
        value, why = bench.pmc_value(kind, cls)
        assert value is None and "000000000000" in why


def test_committed_summaries_name_their_sources():
    for name in ("decode_kernels_qwen25.md", "pmc_decode_qwen25.txt", "gemv_sweep_config1.md", "gemv_q40_vocab.md",
                 "mfma_util_qwen25.md"):
        text = open(os.path.join(ROOT, "profiles", name)).read()
        assert "ources" in text and "rocprofv3" in text, name


def test_sweep_blocks_split_in_order():
    """gemv_blocks assigns each --gemv shape the run of product launches it
    made (prep + product pairs summed for N > 1)."""
    from llm_amd import profsum
    rows = []
    t = 0
    for i in range(3):  # shape 0: 3 launches of 2 us
        rows.append((t, "gemv_kernel<2u, 1, 0, 0, 2>", 64, 1, 2.0))
        t += 1
    rows.append((t, "repack_kernel<2u>", 64, 1, 9.0))
    t += 1
    for i in range(2):  # shape 1: 2 launch pairs
        rows.append((t, "prep_kernel<0>", 64, 1, 1.0))
        rows.append((t + 1, "gemm_kernel<2u, 0, false, 1, 2>", 64, 4, 3.0))
        t += 2
    specs = [{"n": 1, "launches": 3}, {"n": 64, "launches": 2}]
    b = profsum.gemv_blocks(rows, specs)
    assert b[0]["median"] == 2.0 and b[0]["names"] == ["gemv_kernel<2u, 1, 0, 0, 2>"]
    assert b[1]["median"] == 4.0 and len(b[1]["names"]) == 2
