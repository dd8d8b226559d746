"""Builds libllmhip.so in-tree for gfx950 (hipcc, no JIT cache).

Each source compiles to an object under llm_amd/_build/ in parallel, then one
link step.  Every HIP compile disables packed-FP32 instruction selection
(-packed-fp32-ops): those forms have given wrong results on these machines.
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libllmhip.so")
ARCH = os.environ.get("LLMHIP_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
CLI = os.path.join(HERE, "llm-generate")

CFLAGS = ["-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", f"--offload-arch={ARCH}",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-function",
          "-Wno-unused-variable", "-Wno-unused-but-set-variable", "-Wno-unused-result"]


def sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _compile(src):
    obj = os.path.join(BUILD, src + ".o")
    cmd = [HIPCC] + CFLAGS + ["-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC] + CFLAGS + ["-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile {src} failed:\n{r.stdout}\n{r.stderr}")
    return obj


def build(jobs=None, verbose=True):
    """Compile every source and link llm_amd/libllmhip.so; always rebuilds."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", "-o", tmp] + objs,
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    build_cli()
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources and {CLI}", file=sys.stderr)
    return LIB


def build_cli():
    """The llm-generate tool (cli/generate.cpp): host code only, linked against
    libllmhip.so next to it (rpath $ORIGIN)."""
    tmp = CLI + ".tmp"
    r = subprocess.run([CXX, "-O2", "-std=c++17", "-Wall", "-I", os.path.join(os.path.dirname(HERE), "include"),
                        os.path.join(HERE, "cli", "generate.cpp"), "-L", HERE, "-lllmhip", "-Wl,-rpath,$ORIGIN",
                        "-o", tmp], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"llm-generate failed to build:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, CLI)
    return CLI


if __name__ == "__main__":
    build()
