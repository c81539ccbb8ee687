"""Writes tests/golden/tiny.gguf and tiny_gguf_expected.json.

No GGUF reader or file exists in the reference (it plans one:
docs/tensor-design.md:443-459), so this fixture is written here from the
published GGUF layout (version 3, little endian): magic, version, tensor
count, metadata count, metadata entries, tensor infos (ne[0] innermost),
padding to general.alignment, tensor data at aligned offsets.  The manifest
records what a reader must return.  Also importable: tests use ``write_gguf``
to build files of other shapes and broken ones.

Run: ``python tests/golden/make_gguf_fixture.py``.
"""

from __future__ import annotations

import hashlib
import json
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}


def _string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STR:
        return _string(v)
    if vtype == ARR:
        etype, items = v
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, x) for x in items)
    return struct.pack(_FMT[vtype], v)


def write_gguf(path, metadata, tensors, alignment=32, version=3, magic=b"GGUF"):
    """metadata: list of (key, vtype, value); tensors: list of (name, shape
    outermost first, ggml_type, bytes).  Returns {name: absolute offset}."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(metadata))
    for key, vtype, v in metadata:
        head += _string(key) + struct.pack("<I", vtype) + _value(vtype, v)
    rel, offsets = 0, []
    for name, shape, ggml_type, data in tensors:
        offsets.append(rel)
        head += _string(name) + struct.pack("<I", len(shape))
        head += b"".join(struct.pack("<Q", d) for d in reversed(shape))
        head += struct.pack("<IQ", ggml_type, rel)
        rel += -(-len(data) // alignment) * alignment
    data_offset = -(-len(head) // alignment) * alignment
    out = bytearray(head + b"\0" * (data_offset - len(head)))
    for (name, shape, ggml_type, data), off in zip(tensors, offsets):
        out += b"\0" * (data_offset + off - len(out)) + bytes(data)
    with open(path, "wb") as f:
        f.write(out)
    return {t[0]: data_offset + off for t, off in zip(tensors, offsets)}


def fixture_tensors():
    rng = np.random.default_rng(20261201)
    def q4_0(n, k):  # f16 scale 1.0 + deterministic nibbles
        blocks = rng.integers(0, 256, size=(n * k // 32, 18), dtype=np.uint8)
        blocks[:, 0:2] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
        return blocks.reshape(-1).tobytes()
    def q8_0(n, k):
        blocks = rng.integers(0, 256, size=(n * k // 32, 34), dtype=np.uint8)
        blocks[:, 0:2] = np.frombuffer(np.float16(0.125).tobytes(), np.uint8)
        return blocks.reshape(-1).tobytes()
    return [
        ("blk.0.ffn_up.weight", (3, 64), 2, q4_0(3, 64)),
        ("blk.0.ffn_down.weight", (2, 64), 8, q8_0(2, 64)),
        ("token_embd.weight", (4, 8), 1, np.arange(32, dtype=np.float16).tobytes()),
        ("output_norm.weight", (8,), 0, np.linspace(0.5, 1.5, 8, dtype=np.float32).tobytes()),
    ]


def fixture_metadata():
    return [
        ("general.architecture", STR, "llama"),
        ("general.name", STR, "mote tiny fixture"),
        ("general.alignment", U32, 32),
        ("llama.embedding_length", U32, 64),
        ("llama.rope.freq_base", F32, 500000.0),
        ("tokenizer.ggml.scores", ARR, (F32, [0.0, -1.5, 2.25])),
        ("general.quantized", BOOL, True),
    ]


def main() -> None:
    tensors = fixture_tensors()
    offsets = write_gguf(os.path.join(HERE, "tiny.gguf"), fixture_metadata(), tensors)
    manifest = {
        "metadata": {"general.architecture": "llama", "general.name": "mote tiny fixture",
                     "general.alignment": 32, "llama.embedding_length": 64,
                     "llama.rope.freq_base": 500000.0, "tokenizer.ggml.scores": [0.0, -1.5, 2.25],
                     "general.quantized": True},
        "tensors": [{"name": n, "shape": list(s), "ggml_type": t, "offset": offsets[n], "nbytes": len(d),
                     "sha256": hashlib.sha256(d).hexdigest()} for n, s, t, d in tensors],
    }
    with open(os.path.join(HERE, "tiny_gguf_expected.json"), "w") as f:
        json.dump(manifest, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
