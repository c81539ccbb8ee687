"""GPU parity of the linears at K above 2^31 - 1, where the reference's
kernel takes 64-bit sizes and launches
(crates/mote-backend-hip/src/quantized_linear.hip:13-52, 56-91) and this
library runs its 64-bit K-part path.

A row of x is 4 GiB here, so the operands are zero except for three windows of
blocks: the start of each row, a run that straddles a boundary between the K
parts of a 6-output launch, and the end of each row, which crosses element
2^31 (byte 2^32 of the row).  Zero weight bytes decode to (0 - 8) * 0 = -0 and
zero activations give +-0 products, so every term outside the windows adds an
exact zero and the result is the oracle's linear over the windows alone, to
the path's tolerance (f64 oracle, |y - y64| <= 1e-3 |y64| or the sqrt(K)
bound).  Rows m >= 1 start past byte 2^32 of x.  The allocation-free entry
point must agree bit for bit with the allocating one, and two runs with each
other.
"""

from __future__ import annotations

import numpy as np
import pytest

from mote_amd import ops, workloads as wl
from mote_amd.device import DeviceBuffer
from test_gpu_q4_0 import check_against_oracle, check_gate_up
import test_gpu_q8_0 as q8

pytestmark = pytest.mark.gpu

M, N = 2, 3
K = (1 << 31) + 64
BLOCKS = K // 32
# (first block, block count): a row's start, a run across the boundary of
# two K parts (a launch of 6 outputs cuts K into 1024 runs of 65 537 blocks),
# and a row's end, across element 2^31.
WINDOWS = [(0, 64), (65537 - 16, 32), (BLOCKS - 64, 64)]
KC = 32 * sum(c for _, c in WINDOWS)  # K of the windows side by side
_ZERO = np.zeros(1 << 28, dtype=np.uint8)


def zeroed(nbytes: int) -> DeviceBuffer:
    b = DeviceBuffer(nbytes)
    for off in range(0, nbytes, _ZERO.nbytes):
        b.upload(_ZERO[: min(_ZERO.nbytes, nbytes - off)], offset=off)
    return b


@pytest.fixture(scope="module")
def x_operand():
    """(device x [M, K] f16, zero outside the windows; the windows side by
    side [M, KC] on the host)."""
    xc = wl.normal_f16(wl.seed_for(61, 1), M * KC).reshape(M, KC)
    xb = zeroed(M * K * 2)
    for m in range(M):
        c = 0
        for b0, cnt in WINDOWS:
            xb.upload(xc[m, c: c + 32 * cnt], offset=(m * K + 32 * b0) * 2)
            c += 32 * cnt
    yield xb, np.ascontiguousarray(xc).reshape(-1)
    xb.free()


def weights_operand(wc: np.ndarray, rows: int, block_bytes: int) -> DeviceBuffer:
    """Device [rows, K] weights, zero outside the windows, from the windows
    side by side (wc: [rows, KC] in blocks of block_bytes)."""
    wc = wc.reshape(rows, KC // 32, block_bytes)
    row_bytes = BLOCKS * block_bytes
    wb = zeroed(rows * row_bytes)
    for n in range(rows):
        c = 0
        for b0, cnt in WINDOWS:
            wb.upload(wc[n, c: c + cnt], offset=n * row_bytes + b0 * block_bytes)
            c += cnt
    return wb


def run(fn, *ptrs, stream, f16_out=False):
    out_bytes = M * N * (2 if f16_out else 4)
    yb = DeviceBuffer(out_bytes)
    yb.upload(np.full(out_bytes, 0xA5, dtype=np.uint8))  # sentinel: every element must be written
    fn(*ptrs, yb.ptr, M, N, K, stream)
    stream.synchronize()
    y = yb.download(np.uint16 if f16_out else np.float32)
    yb.free()
    if f16_out:
        y = y.view(np.float16).astype(np.float32)
    return y.reshape(M, N)


def test_q4_0_linear(stream, oracle, x_operand):
    xb, xc = x_operand
    wc = wl.q4_0_weights(wl.seed_for(61, 2), N, KC)
    wb = weights_operand(wc, N, 18)
    try:
        y = run(ops.quantized_linear_q4_0_f32, xb.ptr, wb.ptr, stream=stream)
        check_against_oracle(oracle, y, xc, wc, M, N, KC, what="Q4_0 f32, K = 2^31 + 64")
        assert np.array_equal(y, run(ops.quantized_linear_q4_0_f32, xb.ptr, wb.ptr, stream=stream))
        y_na = run(ops.quantized_linear_q4_0_f32_no_alloc, xb.ptr, wb.ptr, stream=stream)
        assert np.array_equal(y, y_na), "allocation-free entry point differs"
        y16 = run(ops.quantized_linear_q4_0_f16, xb.ptr, wb.ptr, stream=stream, f16_out=True)
        check_against_oracle(oracle, y16, xc, wc, M, N, KC, f16_out=True, what="Q4_0 f16, K = 2^31 + 64")
        assert np.array_equal(y16, y.astype(np.float16).astype(np.float32)), "f16 output is not the f32 sum rounded once"
    finally:
        wb.free()


def test_q8_0_linear(stream, oracle, x_operand):
    xb, xc = x_operand
    wc = wl.q8_0_weights(wl.seed_for(61, 3), N, KC)
    wb = weights_operand(wc, N, 34)
    try:
        y = run(ops.quantized_linear_q8_0_f32, xb.ptr, wb.ptr, stream=stream)
        q8.check(oracle, y, xc, wc, M, N, KC, what="Q8_0 f32, K = 2^31 + 64")
    finally:
        wb.free()


def test_fused_gate_up(stream, oracle, x_operand):
    """Gate and up rows in one concatenated [2N, K] buffer (up = NULL), so the
    up rows start past byte 2^32 of the weights."""
    xb, xc = x_operand
    wg = wl.q4_0_weights(wl.seed_for(61, 4), N, KC)
    wu = wl.q4_0_weights(wl.seed_for(61, 5), N, KC)
    wb = weights_operand(np.concatenate([wg, wu]), 2 * N, 18)
    try:
        y = run(ops.q4_0_gate_up_silu_f32, xb.ptr, wb.ptr, None, stream=stream)
        check_gate_up(oracle, y, xc, wg, wu, M, N, KC, what="gate/up, K = 2^31 + 64")
    finally:
        wb.free()
