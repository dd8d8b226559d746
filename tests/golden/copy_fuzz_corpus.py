"""Copies the reference's GGUF fuzz corpus (gguf/testdata/fuzz/FuzzParse/*,
Go's `go test fuzz v1` text format: data, not code) into tests/golden/gguf_fuzz/
so the parser tests run where /root/reference is absent.  Run once:
    python tests/golden/copy_fuzz_corpus.py [/root/reference]
"""
import os
import shutil
import sys

src = os.path.join(sys.argv[1] if len(sys.argv) > 1 else "/root/reference", "gguf", "testdata", "fuzz", "FuzzParse")
dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gguf_fuzz")
os.makedirs(dst, exist_ok=True)
n = 0
for name in sorted(os.listdir(src)):
    shutil.copyfile(os.path.join(src, name), os.path.join(dst, name))
    n += 1
print(f"copied {n} corpus files to {dst}")
