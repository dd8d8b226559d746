"""The GGUF header parser and ConfigFrom (llm_amd/csrc/gguf.cpp, host code with
no HIP) built on their own with AddressSanitizer and UndefinedBehaviorSanitizer
(g++, CPU only) and run over the reference's fuzz corpus (216 inputs of
gguf/testdata/fuzz/FuzzParse), gguf_test.go's valid header, two synthetic
models, and seeded mutations of every one of them (tests/gguf_sanitized_driver.cpp):
no sanitizer report, every input parsed or refused with a typed error.  The
reference runs its parser under `go test -race` and a fuzz job
(.github/workflows/ci.yml:42,44-53); this is the C++ parser's counterpart."""
import glob
import os
import shutil
import subprocess

import pytest

from llm_amd import synth
from tests.test_gguf import GOLDEN, _go_bytes, build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "llm_amd", "csrc")
FLAGS = ["-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
         "-fno-omit-frame-pointer"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")


def _gxx():
    if not shutil.which("g++"):
        pytest.skip("no g++")
    return "g++"


def test_sanitizers_are_live(tmp_path):
    """The same flags report a planted heap read one past a vector's end."""
    src = tmp_path / "oob.cpp"
    src.write_text("#include <vector>\nint main(int c, char**) { std::vector<int> v(4); return v.data()[3 + c]; }\n")
    exe = str(tmp_path / "oob")
    subprocess.run([_gxx()] + FLAGS + [str(src), "-o", exe], check=True, capture_output=True)
    r = subprocess.run([exe], capture_output=True, text=True, env=ENV, timeout=60)
    assert r.returncode != 0 and "heap-buffer-overflow" in r.stderr


def test_parser_under_sanitizers(tmp_path):
    exe = str(tmp_path / "drv")
    r = subprocess.run([_gxx()] + FLAGS + [os.path.join(CSRC, "gguf.cpp"), os.path.join(CSRC, "errors.cpp"),
                                           os.path.join(ROOT, "tests", "gguf_sanitized_driver.cpp"), "-o", exe],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    inputs = []
    for i, p in enumerate(sorted(glob.glob(os.path.join(GOLDEN, "gguf_fuzz", "*")))):
        f = tmp_path / f"fuzz{i:03d}.gguf"
        f.write_bytes(_go_bytes(open(p, encoding="utf-8").read()))
        inputs.append(str(f))
    assert len(inputs) == 216
    (tmp_path / "valid.gguf").write_bytes(build())
    inputs.append(str(tmp_path / "valid.gguf"))
    inputs += [synth.cached(synth.tiny_llama()), synth.cached(synth.tiny_qwen())]
    r = subprocess.run([exe, "150"] + inputs, capture_output=True, text=True, env=ENV, timeout=600)
    print(r.stdout, r.stderr[-3000:])
    assert r.returncode == 0 and "runtime error" not in r.stderr and "Sanitizer" not in r.stderr
    parsed, refused = (int(w) for w in r.stdout.replace(",", "").split()[1::2])
    assert parsed >= 3 and parsed + refused == len(inputs) * 151
