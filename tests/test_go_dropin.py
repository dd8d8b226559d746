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


# C scalar types of the header and what each may become on the Go side (the
# conversions gpu_hip.go applies to a field it reads) and in ctypes
C_TO_GO = {"uint32_t": {"uint32", "uint64", "int", "int64"}, "uint64_t": {"uint64"}, "int64_t": {"int", "int64"},
           "int32_t": {"int", "int32", "int64"}, "float": {"float32", "float64"}}
C_TO_CTYPES = {"uint32_t": "c_uint32", "uint64_t": "c_uint64", "int64_t": "c_int64", "int32_t": "c_int32",
               "float": "c_float"}
CGO_STRUCTS = ("llmhip_limits", "llmhip_config", "llmhip_stats")


def _header_structs():
    """{struct: [(field, C type)]} of the typedef'd structs in include/llmhip.h, in declaration order."""
    src = re.sub(r"/\*.*?\*/", " ", open(os.path.join(ROOT, "include", "llmhip.h")).read(), flags=re.S)
    out = {}
    for body, name in re.findall(r"typedef struct \w+ \{(.*?)\} (\w+);", src, flags=re.S):
        fields = []
        for decl in body.split(";"):
            m = re.match(r"\s*(u?int(?:32|64)_t|float)\s+(.*)", decl, flags=re.S)
            if m:
                fields += [(f.strip(), m.group(1)) for f in m.group(2).split(",")]
        out[name] = fields
    return out


def test_cgo_struct_fields():
    """Every field of C.llmhip_limits / llmhip_config / llmhip_stats that
    gpu_hip.go reads, assigns or sets in a keyed literal exists in
    include/llmhip.h, with a C type that matches the conversion the Go code
    applies (gpu.go:28-36,56-60 are the Go types they fill)."""
    structs = _header_structs()
    code = _code(os.path.join(GO, "gpu_hip.go"))
    checked = 0
    for st in CGO_STRUCTS:
        fields = dict(structs[st])
        assert fields, st
        names = set(re.findall(r"var (\w+) C\." + st + r"\b", code))
        for var in names:
            # reads: goType(var.field)
            for goty, fl in re.findall(r"\b(\w+)\(" + var + r"\.(\w+)\)", code):
                assert fl in fields, f"gpu_hip.go reads {st}.{fl}, which include/llmhip.h does not declare"
                assert goty in C_TO_GO[fields[fl]], f"{st}.{fl} is {fields[fl]}, read as {goty}"
                checked += 1
            # writes: var.field = C.type(...)
            for fl, cty in re.findall(r"\b" + var + r"\.(\w+)\s*=\s*C\.(\w+)\(", code):
                assert fl in fields and fields[fl] == cty, f"{st}.{fl} assigned a C.{cty}, header has {fields.get(fl)}"
                checked += 1
        # keyed literals: C.st{field: C.type(...), ...}
        for body in re.findall(r"C\." + st + r"\{(.*?)\}", code, flags=re.S):
            keyed = re.findall(r"(\w+):\s*C\.(\w+)\(", body)
            assert {k for k, _ in keyed} == set(fields), f"the {st} literal sets {sorted(k for k, _ in keyed)}"
            for fl, cty in keyed:
                assert fields[fl] == cty, f"{st}.{fl} set from a C.{cty}, header has {fields[fl]}"
                checked += 1
    assert checked >= 7 + 14 + 3, checked  # limits read, config literal, stats read


def test_ctypes_structs_match_header():
    """The Python binding's ctypes mirrors of the same structs (llm_amd/_lib.py)
    hold the header's fields in the header's order with the same widths."""
    import ctypes
    from llm_amd import _lib
    structs = _header_structs()
    for st, cls in (("llmhip_limits", _lib.Limits), ("llmhip_config", _lib.Config), ("llmhip_stats", _lib.Stats)):
        want = [(f, getattr(ctypes, C_TO_CTYPES[t])) for f, t in structs[st]]
        assert [(f, t) for f, t in cls._fields_] == want, st
