"""GPU parity of the streaming GEMV run as passes of up to four tokens
(`stream_m4x_d1q_g1`, `stream_s<S>_m4x_d1q_g1`, `q8_stream_s<S>_m4x_d1q_g1`:
5-16 tokens, rows whole or split over S waves, for K with no split-K slicing
such as 3584, 11 008 and 13 824).

Each pass computes its tokens exactly as the one-token split-row GEMV does (the
operands of a pair are unpacked once and fed to every token's dot chain in
the same order), so every output row must equal that GEMV run on its token
alone, bit for bit, and the oracle's tolerance holds.  Token counts cover
whole passes (8, 12, 16) and every remainder (5, 6, 7, 9); K covers both
split widths and a last slice shorter than the others; f32 and f16 outputs.
"""

from __future__ import annotations

import re

import numpy as np
import pytest

from mote_amd import ops, workloads as wl
from test_gpu_q4_0 import check_against_oracle, normal_x, run_linear, sample_columns, weights

pytestmark = pytest.mark.gpu

CASES = [(5, 300, 11008), (6, 257, 13824), (7, 64, 8320), (8, 4096, 11008), (9, 130, 5376), (12, 33, 16384),
         (16, 700, 13824), (6, 96, 6144), (13, 40, 7424), (8, 1000, 8192),
         (5, 300, 3584), (7, 129, 2560), (9, 1000, 3584), (16, 64, 4096)]


def _split(variant: str) -> int:
    m = re.search(r"_s(\d+)_m4x_", variant)
    return int(m.group(1)) if m else 1


@pytest.mark.parametrize("variant", ["stream_m4x_d1q_g1", "stream_s2_m4x_d1q_g1", "stream_s4_m4x_d1q_g1"])
def test_q4_0_token_passes(stream, oracle, variant):
    split = _split(variant)
    d = ops.Q4_0Dispatch()
    d.force(variant)
    one = ops.Q4_0Dispatch()
    one.force({1: "stream_d1q_g1", 2: "stream_s2_d1_g1", 4: "stream_s4_d1q_g1"}[split])
    for m, n, k in CASES:
        if not (4096 * (split // 2) < k <= 4096 * split):
            continue
        print(f"{variant} {m}x{n}x{k}", flush=True)
        x = normal_x(wl.seed_for(31, m * k), m, k)
        w = weights(wl.seed_for(31, n + k), n, k)
        for f16_out in (False, True):
            y = run_linear(stream, x, w, m, n, k, dispatch=d, f16_out=f16_out)
            want = np.concatenate([run_linear(stream, x[t * k:(t + 1) * k], w, 1, n, k, dispatch=one,
                                              f16_out=f16_out) for t in range(m)])
            assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), (variant, m, n, k, f16_out)
            cols = None if n < 2000 else sample_columns(n, 256)
            check_against_oracle(oracle, y, x, w, m, n, k, columns=cols, f16_out=f16_out,
                                 what=f"{variant} {m}x{n}x{k}")


@pytest.mark.parametrize("variant", ["q8_stream_s2_m4x_d1q_g1", "q8_stream_s4_m4x_d1q_g1"])
def test_q8_0_token_passes(stream, oracle, variant):
    from test_gpu_q8_0 import check as check_q8, run as run_q8, weights as q8_weights

    split = _split(variant)
    d = ops.Q4_0Dispatch()
    d.force(variant)
    one = ops.Q4_0Dispatch()
    one.force(f"q8_stream_s{split}_d1_g1")
    for m, n, k in CASES:
        if not (4096 * (split // 2) < k <= 4096 * split):
            continue
        print(f"{variant} {m}x{n}x{k}", flush=True)
        x = normal_x(wl.seed_for(32, m * k), m, k)
        w = q8_weights(wl.seed_for(32, n + k), n, k)
        for f16_out in (False, True):
            y = run_q8(stream, x, w, m, n, k, dispatch=d, f16_out=f16_out)
            want = np.concatenate([run_q8(stream, x[t * k:(t + 1) * k], w, 1, n, k, dispatch=one, f16_out=f16_out)
                                   for t in range(m)])
            assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), (variant, m, n, k, f16_out)
            cols = None if n < 2000 else sample_columns(n, 256)
            check_q8(oracle, y, x, w, m, n, k, columns=cols, f16_out=f16_out, what=f"{variant} {m}x{n}x{k}")


def test_token_passes_reject_what_they_cannot_run(stream):
    """4 and 17 tokens fall outside the pass variants: forcing them is an error."""
    from mote_amd import HipError

    d = ops.Q4_0Dispatch()
    d.force("stream_s4_m4x_d1q_g1")
    for m in (4, 17):
        x = normal_x(wl.seed_for(33, m), m, 11008)
        w = weights(wl.seed_for(33, 1), 64, 11008)
        with pytest.raises(HipError):
            run_linear(stream, x, w, m, 64, 11008, dispatch=d)
