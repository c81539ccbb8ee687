"""The entry point that allocates nothing, mote_hip_quantized_linear_q4_0_f32
_no_alloc, against mote_hip_quantized_linear_q4_0_f32 through the C ABI.

Both run the same plans and kernels; the no-allocation entry point keeps the
split-K partial tiles in the library's static 16 MiB device array instead of
the per-stream pool.  Two calls in a row on split-K shapes (the K = 14336 down
projection at 16 tokens, then a smaller 4 x 8192 x 2048 problem, so the
second call reads an array that still holds the first call's partial tiles)
must reproduce the existing entry point bit for bit and meet the oracle's
tolerance; a decode shape (no scratch) must too; a problem whose partial
tiles exceed 16 MiB must return 2 before launching, leaving the output
untouched."""

from __future__ import annotations

import numpy as np
import pytest

from mote_amd import _ffi, ops, workloads as wl
from mote_amd.device import DeviceBuffer
from test_gpu_q4_0 import check_against_oracle

pytestmark = pytest.mark.gpu


def _run(stream, fn, x, w, m, n, k):
    xb, wb = DeviceBuffer.from_array(x), DeviceBuffer.from_array(w)
    yb = DeviceBuffer(m * n * 4)
    yb.upload(np.full(m * n * 4, 0xA5, dtype=np.uint8))
    fn(xb.ptr, wb.ptr, yb.ptr, m, n, k, stream)
    stream.synchronize()
    return yb.download(np.float32).reshape(m, n)


@pytest.mark.parametrize("m,k,n", [(16, 14336, 4096), (4, 2048 * 4, 2048), (1, 4096, 14336)])
def test_no_alloc_matches_the_allocating_entry_point(stream, oracle, m, k, n):
    x = wl.normal_f16(wl.seed_for(31, m), m * k)
    w = wl.q4_0_weights(wl.seed_for(31, n), n, k)
    want = _run(stream, ops.quantized_linear_q4_0_f32, x, w, m, n, k)
    got = _run(stream, ops.quantized_linear_q4_0_f32_no_alloc, x, w, m, n, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    check_against_oracle(oracle, got, x, w, m, n, k, what=f"no-alloc {m}x{n}x{k}")


def test_two_calls_in_a_row_second_smaller(stream, oracle):
    d = ops.Q4_0Dispatch()
    for m, k, n in [(16, 14336, 4096), (4, 8192, 2048)]:
        assert d.select(m, n, k).endswith("_sk"), (m, k, n)  # both use the scratch array
    shapes = [(16, 14336, 4096), (4, 8192, 2048)]
    inputs = [(wl.normal_f16(wl.seed_for(32, m), m * k), wl.q4_0_weights(wl.seed_for(32, n + k), n, k))
              for m, k, n in shapes]
    got = [_run(stream, ops.quantized_linear_q4_0_f32_no_alloc, x, w, m, n, k)
           for (m, k, n), (x, w) in zip(shapes, inputs)]
    for (m, k, n), (x, w), y in zip(shapes, inputs, got):
        want = _run(stream, ops.quantized_linear_q4_0_f32, x, w, m, n, k)
        assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), (m, k, n)
        check_against_oracle(oracle, y, x, w, m, n, k, what=f"no-alloc {m}x{n}x{k}")


def test_partial_tiles_beyond_the_array_are_rejected_before_launch(stream):
    """64 tokens x N = 9216 x K = 32768 on the split-K tiles (eight K parts
    of 4096; 144 64 x 64 tiles, too few for the prefill tiles) needs 64 x
    9216 x 8 x 4 bytes = 18 MiB > 16 MiB: status 2, output untouched."""
    m, n, k = 64, 9216, 32768
    d = ops.Q4_0Dispatch()
    assert d.select(m, n, k).endswith("_sk")
    xb, wb = DeviceBuffer(m * k * 2), DeviceBuffer(n * (k // 32) * 18)
    yb = DeviceBuffer(m * n * 4)
    yb.upload(np.full(m * n * 4, 0xA5, dtype=np.uint8))
    status = _ffi.lib().mote_hip_quantized_linear_q4_0_f32_no_alloc(xb.ptr, wb.ptr, yb.ptr, m, n, k, stream.handle)
    stream.synchronize()
    assert status == 2
    assert np.all(yb.download(np.uint8) == 0xA5)


def test_split_k_calls_allocate_nothing(stream, oracle):
    """On a fresh stream of the caller's own (hipStreamCreate: the library
    has reserved no scratch for it) that no allocating call has used, the
    no-allocation entry point's split-K calls (64 x 14336 x 4096: 7 K parts,
    7.3 MB of partial tiles) leave the device's free memory unchanged; the
    per-stream pool of the allocating entry point would allocate that buffer
    on the stream's first split-K call.  The same call through the allocating
    entry point on another stream loads every kernel first, and one decode
    call (no scratch) pays any per-stream cost of the runtime before the
    measurement."""
    from mote_amd.device import memory_info
    from mote_amd.hip_runtime import HipRuntime

    m, k, n = 64, 14336, 4096
    assert ops.Q4_0Dispatch().select(m, n, k).endswith("_sk")
    x = wl.normal_f16(wl.seed_for(33, m), m * k)
    w = wl.q4_0_weights(wl.seed_for(33, n), n, k)
    want = _run(stream, ops.quantized_linear_q4_0_f32, x, w, m, n, k)
    fresh = HipRuntime().foreign_stream()
    try:
        xb, wb, yb = DeviceBuffer.from_array(x), DeviceBuffer.from_array(w), DeviceBuffer(m * n * 4)
        ops.quantized_linear_q4_0_f32_no_alloc(xb.ptr, wb.ptr, yb.ptr, 1, n, k, fresh)
        fresh.synchronize()
        before = memory_info()[0]
        for _ in range(2):
            ops.quantized_linear_q4_0_f32_no_alloc(xb.ptr, wb.ptr, yb.ptr, m, n, k, fresh)
        fresh.synchronize()
        after = memory_info()[0]
        got = yb.download(np.float32).reshape(m, n)
    finally:
        fresh.close()
    assert after == before, f"free device memory changed by {before - after} bytes"
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
