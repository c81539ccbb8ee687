"""GGUF weights uploaded by the loader feed the quantized linear unchanged.

A GGUF file holding a Q4_0 [512, 4096] and a Q8_0 [256, 4096] weight (rows
written in the reference's GGML block layout, crates/mote-types/src/lib.rs:
39-74) is written to a temporary directory, memory-mapped, uploaded verbatim
(as ``HipStorage::from_bytes`` takes GGML bytes, crates/mote-backend-hip/src/
storage.rs:15-45) and used as the weight of the linear.  The bytes on the
device must equal the file's, and the outputs must be bit-identical to those
from the same bytes uploaded directly, and within the Q4_0/Q8_0 tolerance of
the f64 oracle.  Every call goes through the C ABI of libmote_hip.so.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

from helpers import assert_linear_close, bits_to_f32
from mote_amd import gguf, ops, workloads as wl
from mote_amd.device import DeviceBuffer

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_gguf_fixture as fx  # noqa: E402

pytestmark = pytest.mark.gpu

K = 4096


def _scales(w: np.ndarray, block: int) -> np.ndarray:
    return w.reshape(-1, block)[:, 0:2].copy().view("<u2")[:, 0].view(np.float16).astype(np.float32)


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    q4 = wl.q4_0_weights(41, 512, K)
    q8 = wl.q8_0_weights(42, 256, K)
    path = tmp_path_factory.mktemp("gguf") / "two_linears.gguf"
    meta = [("general.architecture", fx.STR, "llama"), ("general.alignment", fx.U32, 64)]
    fx.write_gguf(str(path), meta, [
        ("output_norm.weight", (K,), 0, np.ones(K, dtype=np.float32).tobytes()),
        ("blk.0.ffn_up.weight", (512, K), 2, q4.tobytes()),
        ("blk.0.ffn_down.weight", (256, K), 8, q8.tobytes()),
    ], alignment=64)
    return str(path), {"blk.0.ffn_up.weight": q4, "blk.0.ffn_down.weight": q8}


def _linear(encoding, x_bits, w_ptr, m, n, stream):
    xb = DeviceBuffer.from_array(x_bits)
    yb = DeviceBuffer(m * n * 4)
    yb.upload(np.full(m * n * 4, 0xA5, dtype=np.uint8))
    fn = ops.quantized_linear_q4_0_f32 if encoding == "q4_0" else ops.quantized_linear_q8_0_f32
    fn(xb.ptr, w_ptr, yb.ptr, m, n, K, stream)
    stream.synchronize()
    return yb.download(np.float32).reshape(m, n)


@pytest.mark.parametrize("name", ["blk.0.ffn_up.weight", "blk.0.ffn_down.weight"])
@pytest.mark.parametrize("m", [1, 4, 64])
def test_uploaded_gguf_weight_drives_the_linear(stream, oracle, model_file, name, m):
    path, expected = model_file
    with gguf.read(path) as g:
        assert g.alignment == 64 and g.tensors[name].offset % 64 == 0
        wbuf, info = g.upload(name)
    w = expected[name]
    n = info.shape[0]
    assert info.shape == (n, K) and info.nbytes == w.nbytes
    np.testing.assert_array_equal(wbuf.download(np.uint8), w)

    direct = DeviceBuffer.from_array(w)
    x = wl.normal_f16(7 + m, m * K)
    y_file = _linear(info.encoding, x, wbuf.ptr, m, n, stream)
    y_direct = _linear(info.encoding, x, direct.ptr, m, n, stream)
    np.testing.assert_array_equal(y_file.view(np.uint32), y_direct.view(np.uint32))

    fmt = oracle.Q4_0 if info.encoding == "q4_0" else oracle.Q8_0
    block = 18 if info.encoding == "q4_0" else 34
    y64 = oracle.quantized_linear_f64(bits_to_f32(x), w, m, n, K, None, fmt=fmt)
    assert_linear_close(y_file, y64, K, float(np.max(np.abs(_scales(w, block)))),
                        float(np.max(np.abs(bits_to_f32(x)))), what=f"{name} m={m}")
