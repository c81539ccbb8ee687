"""GGUF loader (host side): parsing, the reference's span rules, error cases.

No GGUF reader or fixture exists in the reference (docs/tensor-design.md:
443-459 plans one), so the file format is pinned only by the committed
fixture written from the published layout (tests/golden/make_gguf_fixture.py)
and by the span rules of crates/mote-types/src/tensor_desc.rs:52-101 and the
block geometry of crates/mote-types/src/lib.rs:39-74: parity unpinned against
the reference.
"""

from __future__ import annotations

import hashlib
import json
import os
import struct
import sys

import numpy as np
import pytest

from mote_amd import gguf

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_gguf_fixture as fx  # noqa: E402


def test_fixture_parses_to_the_manifest():
    with open(os.path.join(GOLDEN, "tiny_gguf_expected.json")) as f:
        want = json.load(f)
    with gguf.read(os.path.join(GOLDEN, "tiny.gguf")) as g:
        assert g.version == 3 and g.alignment == 32
        meta = dict(g.metadata)
        assert meta["llama.rope.freq_base"] == pytest.approx(500000.0)
        assert [pytest.approx(v) for v in want["metadata"]["tokenizer.ggml.scores"]] == meta["tokenizer.ggml.scores"]
        for key in ("general.architecture", "general.name", "general.alignment", "llama.embedding_length",
                    "general.quantized"):
            assert meta[key] == want["metadata"][key]
        assert list(g.tensors) == [t["name"] for t in want["tensors"]]
        for t in want["tensors"]:
            info = g.tensors[t["name"]]
            assert list(info.shape) == t["shape"] and info.ggml_type == t["ggml_type"]
            assert info.offset == t["offset"] and info.nbytes == t["nbytes"]
            data = g.tensor_bytes(t["name"])
            assert hashlib.sha256(data.tobytes()).hexdigest() == t["sha256"]
            assert not data.flags.writeable


def test_fixture_tensor_bytes_are_the_generators():
    with gguf.read(os.path.join(GOLDEN, "tiny.gguf")) as g:
        for name, shape, ggml_type, data in fx.fixture_tensors():
            assert g.tensor_bytes(name).tobytes() == data
        assert g.tensors["blk.0.ffn_up.weight"].encoding == "q4_0"
        assert g.tensors["blk.0.ffn_down.weight"].quantized
        assert not g.tensors["token_embd.weight"].quantized


@pytest.mark.parametrize("shape,ggml_type,nbytes", [
    ((14336, 4096), 2, 14336 * 128 * 18),  # the reference's 33 030 144-byte span
    ((2, 3, 64), 8, 2 * 3 * 2 * 34),        # outer dimensions count whole rows
    ((0, 64), 2, 0),
    ((4096,), 1, 8192),
    ((7, 256), 12, 7 * 144),
    ((5, 512), 14, 5 * 2 * 210),
    # crates/mote-types/tests/tensor_desc.rs:80-202, case by case
    ((32,), 2, 18), ((32,), 8, 34), ((256,), 12, 144), ((256,), 14, 210),
    ((2, 3, 64), 8, 408), ((5, 256), 14, 1050),
    ((0, 64), 8, 0), ((2, 0), 2, 0), ((3, 0, 256), 14, 0),
])
def test_span_rules_of_the_reference(shape, ggml_type, nbytes):
    assert gguf.span_bytes(shape, ggml_type) == nbytes


@pytest.mark.parametrize("shape,ggml_type,message", [
    ((3, 48), 2, "whole number"),       # QuantizedRowMisaligned
    ((), 8, "scalar"),                  # QuantizedScalarShape
    ((4, 128), 12, "whole number"),     # K-quants: 256-element blocks
    ((4, 32), 3, "unsupported"),        # Q4_1 is not a format of the path
    ((2, 260), 12, "whole number"),     # crates/mote-types/tests/tensor_desc.rs:130-143
    ((0, 33), 8, "whole number"),       # :145-156, a zero outer dimension does not waive it
])
def test_span_rule_errors(shape, ggml_type, message):
    with pytest.raises(gguf.GGUFError, match=message):
        gguf.span_bytes(shape, ggml_type)


def _write(tmp_path, name="f.gguf", **kw):
    path = tmp_path / name
    tensors = kw.pop("tensors", [("w", (2, 32), 2, bytes(2 * 18))])
    fx.write_gguf(path, kw.pop("metadata", []), tensors, **kw)
    return path


def test_default_alignment_and_large_alignment(tmp_path):
    with gguf.read(_write(tmp_path)) as g:
        assert g.alignment == 32 and g.data_offset % 32 == 0
    p = tmp_path / "a.gguf"
    fx.write_gguf(p, [("general.alignment", fx.U32, 256)], [("a", (1, 32), 2, bytes(18)), ("b", (1, 32), 8, bytes(34))],
                  alignment=256)
    with gguf.read(p) as g:
        assert g.data_offset % 256 == 0 and g.tensors["b"].offset - g.tensors["a"].offset == 256


@pytest.mark.parametrize("mutate,message", [
    (lambda b: b"GGUX" + b[4:], "bad magic"),
    (lambda b: b[:4] + struct.pack("<I", 1) + b[8:], "version 1"),
    (lambda b: b[:-10], "extends past the end"),
    (lambda b: b[:20], "truncated"),
    (lambda b: b"", "empty"),
])
def test_malformed_files_raise(tmp_path, mutate, message):
    good = _write(tmp_path).read_bytes()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(mutate(good))
    with pytest.raises(gguf.GGUFError, match=message):
        gguf.read(bad)


def test_misaligned_quantized_row_and_unsupported_type_raise(tmp_path):
    with pytest.raises(gguf.GGUFError, match="whole number"):
        gguf.read(_write(tmp_path, tensors=[("w", (2, 40), 2, bytes(64))]))
    with pytest.raises(gguf.GGUFError, match="unsupported"):
        gguf.read(_write(tmp_path, "u.gguf", tensors=[("w", (2, 32), 3, bytes(40))]))


def test_unknown_tensor_name(tmp_path):
    with gguf.read(_write(tmp_path)) as g, pytest.raises(KeyError):
        g.tensor_bytes("missing")
