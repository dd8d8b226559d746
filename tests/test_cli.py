"""llm-generate (the native counterpart of examples/generate/main.go) on a
machine without a GPU: argument handling, the reference-file format shared
with llm_amd.reffile, and the "no GPU" exit (main.go:87-91) after the header."""
import os
import subprocess

import numpy as np
import pytest

from llm_amd import reffile, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "llm_amd", "llm-generate")


def run(*args):
    r = subprocess.run([CLI, *map(str, args)], capture_output=True, text=True, timeout=60)
    return r.returncode, r.stdout, r.stderr


@pytest.fixture(scope="module")
def cli():
    if not os.path.exists(CLI):  # nothing built yet: build it (and the library it links)
        from llm_amd import build
        build.build(verbose=False)
    return CLI


def test_usage_and_flags(cli):
    rc, out, err = run()
    assert rc == 1 and "usage: llm-generate run|check|bench|trace|dump" in err
    rc, out, err = run("serve")
    assert rc == 1 and 'unknown mode "serve"' in err
    rc, out, err = run("run", "-bogus", "1")
    assert rc == 1 and "flag provided but not defined: -bogus" in err
    rc, out, err = run("run", "-n", "x")
    assert rc == 1 and 'invalid value "x" for flag -n' in err
    rc, out, err = run("run", "-n")
    assert rc == 1 and "flag needs an argument: -n" in err
    rc, out, err = run("run", "-model", "/nonexistent.gguf")
    assert rc == 1 and "llm: cannot open /nonexistent.gguf" in err


def test_reference_files(cli, tmp_path):
    p = tmp_path / "r.llmref"
    recs = {"prompt": np.array([1, 2, 3], np.int32), "logits": np.linspace(-1, 1, 7, dtype=np.float32),
            "x.-1": np.arange(4, dtype=np.float32)}
    reffile.write(p, recs)
    back = reffile.read(p)
    assert set(back) == set(recs)
    for k in recs:
        assert back[k].dtype == recs[k].dtype and np.array_equal(back[k], recs[k])
    bad = tmp_path / "bad.llmref"
    bad.write_bytes(b"NOTAREF!")
    with pytest.raises(ValueError):
        reffile.read(bad)
    model = synth.cached(synth.tiny_llama())
    rc, out, err = run("check", "-model", model, "-ref", bad)
    assert rc == 1 and "not a reference file" in err
    rc, out, err = run("check", "-model", model, "-ref", p)  # no tokens record
    assert rc == 1 and "needs the records logits and tokens" in err
    rc, out, err = run("check", "-model", model)
    assert rc == 1 and "check needs -ref FILE" in err
    trunc = tmp_path / "trunc.llmref"
    trunc.write_bytes(p.read_bytes()[:-5])
    rc, out, err = run("trace", "-model", model, "-ref", trunc)
    assert rc == 1 and "truncated record" in err


def test_no_gpu_exit(cli):
    from llm_amd import _lib
    if _lib.device_count() > 0:
        pytest.skip("a GPU is present: the no-GPU exit cannot happen here")
    model = synth.cached(synth.tiny_llama())
    rc, out, err = run("run", "-model", model, "-ids", "1,2,3")
    assert rc == 2, (out, err)
    assert out.startswith("header: ") and "tensors" in out and "no GPU" in out
