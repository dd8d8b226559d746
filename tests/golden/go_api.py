"""The Go API surface the hip build of package llm must provide, as a fixture.

Reads the reference's Go sources once (in the build container, where
/root/reference exists) and writes tests/golden/go_api.json:

* `declared`: every package-level identifier of the WebGPU files that the hip
  build leaves out (gpu.go, fused.go, kernels.go, kernels_fused.go; they get
  `//go:build !hip`) -- functions, methods (as Type.Name), types, vars and
  consts, with file:line;
* `used`: every identifier of package llm that the rest of the package
  (cpu.go, config.go, f16.go, tokenizer.go and the tests) and its callers
  (examples/generate/main.go, cmd/*/main.go) use, with the file:line of the
  first use; `llm.X`, and the fields and methods callers reach on a *GPU or a
  Limits value;
* `required`: the names the hip files must declare: the exported names of
  the four files plus those any other file uses, minus the WebGPU-only ones
  listed in `webgpu_only` with the reason;
* `package_other`: what the files that stay in both builds declare (cpu.go,
  config.go, f16.go, tokenizer.go), which the hip files may use.

tests/test_go_dropin.py checks the committed go/*_hip.go files against it.
Run:  python tests/golden/go_api.py [reference dir]
"""
import json
import os
import re
import sys

GPU_FILES = ["gpu.go", "fused.go", "kernels.go", "kernels_fused.go"]
PKG_FILES = ["cpu.go", "config.go", "f16.go", "tokenizer.go", "oracle_test.go", "tokenizer_test.go"]
CALLERS = ["examples/generate/main.go", "cmd/ggufdump/main.go"]
# Left out of the hip build with their callers, which get `//go:build !hip` too.
WEBGPU_ONLY = {
    "Shaders": "WGSL text for browser validation (kernels.go:439-449); its only callers, cmd/wgsldump and "
               "kernels_test.go, are WebGPU tools and build with !hip",
}
# Files that test or dump the WGSL kernels and the WebGPU row permutation:
# they build with !hip, so their uses (Shaders, neoxMap, neoxRows) are not
# requirements of the hip build.
WEBGPU_ONLY_FILES = {
    "kernels_test.go": "TestShadersFullySubstituted (WGSL placeholders) and TestNeoxRowsEqualNeoxRope (the WebGPU "
                       "path's load-time row permutation, fused.go:331-344; the hip build places NEOX pairs in its "
                       "tile layout instead)",
    "cmd/wgsldump/main.go": "prints llm.Shaders as JSON for browser validation",
}

DECL_FUNC = re.compile(r"^func (?:\((\w+) \*?(\w+)\) )?(\w+)\s*[\[(]")
DECL_ONE = re.compile(r"^(type|var|const) (\w+)\b")
DECL_GROUP = re.compile(r"^(var|const|type) \($")
GROUP_ITEM = re.compile(r"^\t(\w+)\b")


def declarations(path, rel):
    out = {}
    lines = open(path).read().split("\n")
    group = None
    in_raw = False  # inside a `...` raw string (WGSL sources)
    for i, line in enumerate(lines, 1):
        if in_raw:
            if line.count("`") % 2 == 1:
                in_raw = False
            continue
        if group:
            if line.startswith(")"):
                group = None
            else:
                m = GROUP_ITEM.match(line)
                if m and not line.strip().startswith("//"):
                    out.setdefault(m.group(1), {"kind": group, "at": f"{rel}:{i}"})
            continue
        m = DECL_FUNC.match(line)
        if m:
            name = f"{m.group(2)}.{m.group(3)}" if m.group(2) else m.group(3)
            out.setdefault(name, {"kind": "method" if m.group(2) else "func", "at": f"{rel}:{i}"})
        else:
            m = DECL_GROUP.match(line)
            if m:
                group = m.group(1)
            else:
                m = DECL_ONE.match(line)
                if m:
                    out.setdefault(m.group(2), {"kind": m.group(1), "at": f"{rel}:{i}"})
        if line.count("`") % 2 == 1:
            in_raw = True
    return out


def struct_fields(path, typ):
    """Exported fields of `type typ struct { ... }`."""
    src = open(path).read()
    m = re.search(r"^type " + typ + r" struct \{\n(.*?)^\}", src, re.S | re.M)
    fields = []
    for line in m.group(1).split("\n"):
        line = line.split("//")[0].strip()
        if not line:
            continue
        names = line.split()[0:1]
        if "," in line.split()[0] or (len(line.split()) > 2 and line.split()[0].endswith(",")):
            names = [n.strip(",") for n in re.match(r"([\w, ]+?)\s+\S+$", line).group(1).split(",")]
        fields += [n.strip() for n in names if n.strip()[:1].isupper()]
    return fields


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    declared = {}
    for f in GPU_FILES:
        declared.update(declarations(os.path.join(ref, f), f))
    gpu_fields = struct_fields(os.path.join(ref, "gpu.go"), "GPU")
    limits_fields = struct_fields(os.path.join(ref, "gpu.go"), "Limits")
    for fl in gpu_fields:
        declared.setdefault(f"GPU.{fl}", {"kind": "field", "at": "gpu.go"})
    for fl in limits_fields:
        declared.setdefault(f"Limits.{fl}", {"kind": "field", "at": "gpu.go"})
    for t in ("Stats", "Timing"):
        for fl in struct_fields(os.path.join(ref, "gpu.go"), t):
            declared.setdefault(f"{t}.{fl}", {"kind": "field", "at": "gpu.go"})
    used = {}

    def note(name, at):
        used.setdefault(name, at)

    bare = {n for n in declared if "." not in n}
    for f in PKG_FILES:
        for i, line in enumerate(open(os.path.join(ref, f)).read().split("\n"), 1):
            code = line.split("//")[0]
            for n in bare:
                if re.search(r"(?<![\w.])" + re.escape(n) + r"\b", code):
                    note(n, f"{f}:{i}")
    for f in CALLERS:
        for i, line in enumerate(open(os.path.join(ref, f)).read().split("\n"), 1):
            code = line.split("//")[0]
            for m in re.finditer(r"\bllm\.([A-Z]\w*)", code):
                note(m.group(1), f"{f}:{i}")
            # fields and methods reached on the *GPU (g) and the Limits (lim) of examples/generate
            for var, typ in (("g", "GPU"), ("lim", "Limits")):
                for m in re.finditer(r"\b" + var + r"\.([A-Z]\w*)", code):
                    note(f"{typ}.{m.group(1)}", f"{f}:{i}")
    required = {}
    for n, d in declared.items():
        exported = n.split(".")[-1][:1].isupper()
        if (exported or n in used) and n not in WEBGPU_ONLY:
            owner = n.split(".")[0] if "." in n else None
            if owner and not owner[:1].isupper():
                continue  # methods of unexported types
            if d["kind"] == "field" and n not in used and owner == "GPU" and n.split(".")[1] not in ("Cfg", "Stats",
                                                                                                  "Layers", "Skip"):
                continue
            required[n] = {"declared": d["at"], "kind": d["kind"], "used": used.get(n)}
    for n in used:
        if n in declared and n not in WEBGPU_ONLY and n not in required:
            required[n] = {"declared": declared[n]["at"], "kind": declared[n]["kind"], "used": used[n]}
    # what the files that stay in the hip build declare (the hip files may use these)
    others = {}
    for f in PKG_FILES[:4]:
        others.update(declarations(os.path.join(ref, f), f))
    out = {"reference_files": GPU_FILES, "declared": declared, "used": used, "webgpu_only": WEBGPU_ONLY,
           "webgpu_only_files": WEBGPU_ONLY_FILES, "package_other": sorted(others),
           "required": dict(sorted(required.items()))}
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "go_api.json")
    json.dump(out, open(dst, "w"), indent=1, sort_keys=True)
    print(f"wrote {dst}: {len(declared)} declared, {len(used)} used, {len(required)} required")


if __name__ == "__main__":
    main()
