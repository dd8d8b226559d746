"""Reference files of llm-generate (cli/generate.cpp): the records a CPU path
writes for `check` and `trace`, and what `dump` writes from the GPU.

Format: the 8 bytes b"LLMREF01", then records until the end of the file:
u32 name length, the name (UTF-8), u32 kind (0 f32, 1 i32), u64 count, count
little-endian 4-byte values.  Names used by the tool: "prompt" (i32 ids),
"logits" (f32 logits after the prompt), "tokens" (i32 greedy tokens),
"x.<k>" (f32 residual stream after k layers for the prompt's first token).
"""
import struct

import numpy as np

MAGIC = b"LLMREF01"
KINDS = {0: np.float32, 1: np.int32}


def write(path, records):
    """records: {name: array}; float arrays are stored as f32, integer ones as i32."""
    with open(path, "wb") as fp:
        fp.write(MAGIC)
        for name, arr in records.items():
            a = np.asarray(arr)
            kind = 1 if np.issubdtype(a.dtype, np.integer) else 0
            a = np.ascontiguousarray(a.ravel(), dtype="<i4" if kind else "<f4")
            nb = name.encode()
            fp.write(struct.pack("<I", len(nb)) + nb + struct.pack("<IQ", kind, a.size))
            fp.write(a.tobytes())


def read(path):
    """{name: numpy array} of a reference file."""
    data = open(path, "rb").read()
    if data[:8] != MAGIC:
        raise ValueError(f"{path}: not a reference file (LLMREF01)")
    out, i = {}, 8
    while i < len(data):
        (nl,) = struct.unpack_from("<I", data, i)
        name = data[i + 4:i + 4 + nl].decode()
        kind, count = struct.unpack_from("<IQ", data, i + 4 + nl)
        i += 4 + nl + 12
        if kind not in KINDS or i + 4 * count > len(data):
            raise ValueError(f"{path}: bad record {name}")
        out[name] = np.frombuffer(data, dtype="<i4" if kind else "<f4", count=count, offset=i).astype(KINDS[kind])
        i += 4 * count
    return out
