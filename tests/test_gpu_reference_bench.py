"""The reference benchmark's own cases through the F16-output entry point.

crates/mote-backend-hip/benches/quantized_linear.rs:8-13 times (rows, N, K) in
{(1, 4096, 4096), (1, 11008, 4096), (1, 4096, 11008), (16, 4096, 4096)} with
its closed-form generators (:128-152), and validates three outputs against the
CPU decoder's sequential f32 sum rounded to f16 with tolerance max(0.25,
0.005 |e|) (:89-126).  Those are the only shapes behind the reference's one
published number for this path.  Here the same inputs run through
mote_hip_quantized_linear_q4_0_f16 (the symbol the reference benchmarks) and
the f32 entry point; the reference's three-position validation is applied as
written, and every output is also judged against the f64 oracle with the
path's tolerance."""

from __future__ import annotations

import numpy as np
import pytest

from helpers import bits_to_f32
from mote_amd import ops, workloads as wl
from test_gpu_q4_0 import check_against_oracle, run_linear

pytestmark = pytest.mark.gpu

CASES = [(1, 4096, 4096), (1, 11008, 4096), (1, 4096, 11008), (16, 4096, 4096)]


@pytest.mark.parametrize("rows,n,k", CASES, ids=[f"{r}x{n}x{k}" for r, n, k in CASES])
def test_reference_bench_case(stream, oracle, rows, n, k):
    x = wl.reference_bench_inputs(rows, k)
    w = wl.reference_bench_q4_0_weights(n, k)
    y16 = run_linear(stream, x, w, rows, n, k, f16_out=True)
    expected32 = oracle.quantized_linear_f32(bits_to_f32(x), w, oracle.Q4_0, rows, n, k).reshape(rows, n)
    for r, c in [(0, 0), (rows // 2, n // 3), (rows - 1, n - 1)]:
        e = float(np.float16(expected32[r, c]))
        assert abs(e - float(y16[r, c])) <= max(0.25, 0.005 * abs(e)), (r, c, e, float(y16[r, c]))
    check_against_oracle(oracle, y16, x, w, rows, n, k, f16_out=True, what="f16 entry point")
    y = run_linear(stream, x, w, rows, n, k)
    check_against_oracle(oracle, y, x, w, rows, n, k, what="f32 entry point")
    d = ops.Q4_0Dispatch()
    assert d.select(rows, n, k) in ops.variant_names()
