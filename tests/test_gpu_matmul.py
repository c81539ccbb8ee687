"""Dense F16 x F16 -> F32 matmul through the hipBLASLt boundary.

The reference's matmul_f16_f32 (crates/mote-backend-hip/src/matmul.rs:10-52,
exported by crates/mote-backend-hip/src/hipblaslt_shim.cpp:326-408) is a
library GEMM; this library keeps its C ABI and plan-cache contract.  Checks:
the reference's own fixture and tolerance (crates/mote-backend-hip/tests/
matmul.rs:13-50: 48 x 64 x 32 closed-form values, |y - e| <= max(0.05,
0.002 |e|) against the f32 oracle matmul_f32, crates/mote-reference/src/
lib.rs:105-156); seeded shapes against a float64 product, within the
recursive-summation bound K 2^-24 sum_k |a_k b_k| (products of binary16
values are exact in f32); k = 0, empty outputs, plan reuse (bit-identical
repeat) and argument errors.  Every call goes through the C ABI.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import bits_to_f32, f16_bits
from mote_amd import HipError, ops, workloads as wl
from mote_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu

WS = ops.DenseMatmul.WORKSPACE_BYTES


@pytest.fixture(scope="module")
def ctx():
    c = ops.DenseMatmul()
    yield c
    c.close()


@pytest.fixture(scope="module")
def workspace():
    return DeviceBuffer(WS)


def matmul(ctx, workspace, stream, a_bits, b_bits, m, n, k):
    ab = DeviceBuffer.from_array(a_bits) if a_bits.size else DeviceBuffer(16)
    bb = DeviceBuffer.from_array(b_bits) if b_bits.size else DeviceBuffer(16)
    cb = DeviceBuffer(max(m * n * 4, 16))
    cb.upload(np.full(max(m * n * 4, 16), 0xA5, dtype=np.uint8))  # sentinel: every element must be written
    ctx.matmul_f16_f32(m, n, k, ab.ptr, bb.ptr, cb.ptr, workspace.ptr, WS, stream)
    stream.synchronize()
    return cb.download(np.float32, count=m * n).reshape(m, n)


def test_reference_fixture(ctx, workspace, stream, oracle):
    m, n, k = 48, 64, 32
    lhs = np.array([[((r * 7 + c * 3) % 17) / 8.0 - 1.0 for c in range(k)] for r in range(m)], np.float32)
    rhs = np.array([[((r * 5 + c * 11) % 19) / 8.0 - 1.0 for c in range(n)] for r in range(k)], np.float32)
    a, b = f16_bits(lhs), f16_bits(rhs)
    y = matmul(ctx, workspace, stream, a, b, m, n, k)
    e = oracle.matmul_f32(bits_to_f32(a), bits_to_f32(b), m, n, k).reshape(m, n)
    assert np.all(np.abs(y - e) <= np.maximum(0.05, 0.002 * np.abs(e)))
    assert ctx.last_error() == ""


@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (5, 64, 128), (64, 1024, 4096), (512, 14336, 4096),
                                   (256, 4096, 14336)])
def test_seeded_shapes_against_float64(ctx, workspace, stream, m, n, k):
    a = wl.normal_f16(wl.seed_for(30, m), m * k)
    b = wl.normal_f16(wl.seed_for(31, n), k * n, std=0.05)
    y = matmul(ctx, workspace, stream, a, b, m, n, k)
    cols = np.arange(n) if n <= 1024 else np.random.default_rng(3).choice(n, 192, replace=False)
    A = bits_to_f32(a).reshape(m, k).astype(np.float64)
    B = bits_to_f32(b).reshape(k, n)[:, cols].astype(np.float64)
    exact = A @ B
    bound = k * 2.0 ** -24 * (np.abs(A) @ np.abs(B)) + 1e-30
    err = np.abs(y[:, cols] - exact)
    assert np.all(err <= bound), float(np.max(err / bound))
    # the cached plan: a second call gives the same bits
    again = matmul(ctx, workspace, stream, a, b, m, n, k)
    assert np.array_equal(y.view(np.uint32), again.view(np.uint32))


def test_empty_inner_dimension_writes_zeros_and_empty_outputs_do_nothing(ctx, workspace, stream):
    y = matmul(ctx, workspace, stream, np.zeros(0, np.uint16), np.zeros(0, np.uint16), 3, 8, 0)
    assert np.array_equal(y, np.zeros((3, 8), np.float32))
    y = matmul(ctx, workspace, stream, np.zeros(8, np.uint16), np.zeros(8, np.uint16), 0, 8, 1)
    assert y.size == 0


def test_argument_errors_set_last_error(ctx, workspace, stream):
    buf = DeviceBuffer(64)
    with pytest.raises(HipError) as e:
        ctx.matmul_f16_f32(2, 2, 2, None, buf.ptr, buf.ptr, workspace.ptr, WS, stream)
    assert e.value.status == -1 and "null" in ctx.last_error()
    with pytest.raises(HipError):
        ctx.matmul_f16_f32(2, 2, 2, buf.ptr, buf.ptr, buf.ptr, None, WS, stream)
