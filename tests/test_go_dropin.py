"""The Go drop-in (go/*_hip.go) against the API surface of the reference's
WebGPU files (tests/golden/go_api.json, written from the reference by
tests/golden/go_api.py).

No Go toolchain exists here, so the files cannot be compiled; these checks
pin what a compile under `-tags hip` needs from them: the build tag, every
identifier the !hip files declare that the rest of the package or its callers
use (gpu.go:20-60,165-168,851,930-939,1046-1054, fused.go:17;
examples/generate/main.go), every package-level name the hip files
themselves use, and every C function they call being in include/llmhip.h.
"""
import importlib.util
import json
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GO = os.path.join(ROOT, "go")
FIXTURE = os.path.join(ROOT, "tests", "golden", "go_api.json")
PKG_FILES = ["api_hip.go", "gpu_hip.go"]

spec = importlib.util.spec_from_file_location("go_api", os.path.join(ROOT, "tests", "golden", "go_api.py"))
go_api = importlib.util.module_from_spec(spec)
spec.loader.exec_module(go_api)

# Go's predeclared identifiers and the packages the hip files import
PREDECLARED = {"bool", "byte", "error", "int", "int32", "int64", "uint32", "uint64", "uintptr", "float32", "float64",
               "string", "true", "false", "nil", "append", "len", "make", "min", "max", "copy", "new", "panic",
               "C", "errors", "fmt", "io", "os", "time", "unsafe", "gguf", "llm", "any"}


def _code(path):
    """The file without comments and string literals."""
    src = open(path).read()
    src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    src = re.sub(r'"(?:\\.|[^"\\])*"', '""', src)
    return re.sub(r"`[^`]*`", "``", src)


def _declared():
    out = {}
    for f in PKG_FILES:
        out.update(go_api.declarations(os.path.join(GO, f), f))
    for f in PKG_FILES:
        path = os.path.join(GO, f)
        for typ in ("GPU", "Limits", "Stats", "Timing", "Device"):
            if re.search(r"^type " + typ + r" struct \{", open(path).read(), re.M):
                for fl in go_api.struct_fields(path, typ):
                    out[f"{typ}.{fl}"] = {"kind": "field", "at": f}
    return out


@pytest.fixture(scope="module")
def fixture():
    return json.load(open(FIXTURE))


def test_build_tags():
    files = PKG_FILES + [os.path.join("examples", "generate", "device_hip.go")]
    for f in files:
        first = open(os.path.join(GO, f)).read().split("\n")[0]
        assert first == "//go:build hip", f


def test_required_names_declared(fixture):
    have = _declared()
    missing = [n for n in fixture["required"] if n not in have]
    assert not missing, f"declared by the WebGPU files and needed under -tags hip, missing in go/: {missing}"
    # the method receivers match (value receiver for Limits, pointer for GPU)
    api = open(os.path.join(GO, "api_hip.go")).read() + open(os.path.join(GO, "gpu_hip.go")).read()
    assert re.search(r"^func \(l Limits\) WorkgroupSize\(\) int \{", api, re.M)
    for m, sig in (("Generate", r"\(prompt \[\]int32, n int, eos int32, emit func\(int32\) bool\) \(Timing, error\)"),
                   ("PrefillLogits", r"\(prompt \[\]int32\) \(\[\]float32, error\)"),
                   ("Peek", r"\(name string, n int\) \(\[\]float32, error\)"), ("MemoryUsed", r"\(\) uint64")):
        assert re.search(r"^func \(g \*GPU\) " + m + sig, api, re.M), m
    assert re.search(r"^func NewGPU\(dev \*Device, lim Limits, f \*gguf\.File, r io\.ReaderAt, ctx int\) "
                     r"\(\*GPU, error\)", api, re.M)


def test_used_names_declared(fixture):
    """Every package-level name the hip files use is declared by them or by a
    file that stays in the hip build (cpu.go, config.go, f16.go, tokenizer.go)."""
    have = set(_declared()) | set(fixture["package_other"])
    fields = {n.split(".")[1] for n in have if "." in n}
    webgpu = set(fixture["declared"])
    for f in PKG_FILES + [os.path.join("examples", "generate", "device_hip.go")]:
        code = _code(os.path.join(GO, f))
        if "examples" not in f:
            for n in set(re.findall(r"(?<![\w.])([A-Za-z_]\w*)\b", code)):
                assert n not in webgpu or n in have, f"{f} uses {n}, which only the WebGPU files declare"
        # capitalised names not after a selector and not a keyed literal's key
        for n in set(re.findall(r"(?<![\w.])([A-Z]\w*)\b(?!\s*:[^=])", code)):
            assert n in PREDECLARED or n in have or n in fields, f"{f} uses {n}, declared nowhere in the hip build"


def test_c_calls_exist():
    header = open(os.path.join(ROOT, "include", "llmhip.h")).read()
    for f in PKG_FILES:
        code = _code(os.path.join(GO, f))
        for n in set(re.findall(r"\bC\.(llmhip_\w+)", code)):
            if n.startswith("llmhip_") and not re.search(r"\b" + n + r"\b", header):
                pytest.fail(f"{f} calls C.{n}, which include/llmhip.h does not declare")


def test_balanced():
    for f in PKG_FILES + [os.path.join("examples", "generate", "device_hip.go")]:
        code = _code(os.path.join(GO, f))
        for a, b in ("()", "{}", "[]"):
            assert code.count(a) == code.count(b), (f, a)
