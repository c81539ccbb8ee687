"""GPU parity of every matrix-core kernel for block scales across the whole
binary16 range.

The matrix-core kernels round each dequantised weight to binary16 before the
MFMA; a product (q - 8) d past 65504 (|d| >= 8192 for Q4_0, |d| >= 512 for
Q8_0) would overflow there, while the reference decodes in f32
(crates/mote-reference/src/quantized.rs:187-195) and stays finite.  The
kernels run such a step with every scale times 2^-S and rescale the
accumulators.  Every skinny, split-K and prefill variant (linear, fused
gate/up, Q8_0) runs here on weights whose scales are
* "full": every finite binary16 magnitude, subnormals to 65504, both signs;
* "big": only magnitudes whose products overflow binary16;
* "subnormal": only nonzero subnormals (the products the binary16 operands
  must carry exactly at the bottom of the range);
* "special": "full" plus one scale in 64 set to +inf, -inf or NaN;
against the f64 judge (oracle-decoded weights, every output): NaN and
infinities must appear exactly where the judge has them, and every finite
output must meet the path's tolerance, |y - y64| <= 1e-3 |y64| or
<= 2e-3 sqrt(K) max|d| max|x| with max|d| over the finite scales (f16 outputs,
checked for the subnormal scales whose results fit binary16, get 2^-11 |y64|
more).
"""

from __future__ import annotations

import zlib

import numpy as np
import pytest

from helpers import (
    bits_to_f32,
    block_scales,
    linear_f64_full,
    linear_tolerance,
    wide_q4_0_weights,
    wide_q8_0_weights,
)
from mote_amd import ops, workloads as wl
from test_gpu_q4_0 import run_gate_up, run_linear
from test_gpu_q8_0 import run as run_q8

pytestmark = pytest.mark.gpu

MODES = ["full", "big", "subnormal", "special"]
F16_REL = 2.0 ** -11


def _names(*prefixes):
    return [v for v in ops.variant_names() if v.startswith(prefixes)]


def _slice_k(variant: str) -> int:
    """K of one slice of a skinny variant (KS waves x STEPS steps x 256)."""
    ks, rest = variant.split("_k", 1)[1].split("_s", 1)
    return int(ks) * int(rest.split("_t")[0]) * 256


def _shape(variant: str) -> tuple[int, int, int]:
    """A shape the variant runs: tokens padded in a 16-token tile, N ragged
    against the row tiles; split K with three parts; prefill tiles partial."""
    if "skinny" in variant:
        k = _slice_k(variant)
        if variant.endswith("_sk"):
            k *= 3
        return 17, 70, k
    return 70, 200, 512


def _finite_max(values: np.ndarray) -> float:
    v = np.abs(values[np.isfinite(values)])
    return float(v.max()) if v.size else 0.0


def assert_matches(got, want, tol, what):
    """NaN and signed infinities exactly where `want` has them; finite
    elements within `tol`."""
    got = np.asarray(got, dtype=np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(want)), f"{what}: NaN positions differ"
    inf = np.isinf(want)
    assert np.array_equal(got[inf], want[inf]), f"{what}: infinities differ"
    fin = np.isfinite(want)
    assert np.all(np.isfinite(got[fin])), f"{what}: non-finite output where the judge is finite"
    err = np.abs(got[fin] - want[fin])
    excess = err - np.asarray(tol)[fin]
    assert np.all(excess <= 0), f"{what}: {int((excess > 0).sum())} elements out of tolerance, max excess {excess.max()}"


def _seed(variant: str, mode: str) -> int:
    return zlib.crc32(f"{variant}/{mode}".encode())


def _x(m, k):
    return wl.normal_f16(wl.seed_for(21, m * 7 + k), m * k)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("variant", _names("skinny_mfma_", "mfma_"))
def test_q4_0_linear_wide_scales(stream, oracle, variant, mode):
    m, n, k = _shape(variant)
    x = _x(m, k)
    w = wide_q4_0_weights(_seed(variant, mode), n, k, mode)
    d = ops.Q4_0Dispatch()
    d.force(variant)
    y = run_linear(stream, x, w, m, n, k, dispatch=d)
    y64 = linear_f64_full(oracle, x, w, m, n, k, oracle.Q4_0)
    max_d = _finite_max(block_scales(w, n, k))
    max_x = float(np.abs(bits_to_f32(x)).max())
    tol = linear_tolerance(y64, k, max_d, max_x)
    assert_matches(y, y64, tol, f"{variant} {mode} {m}x{n}x{k}")
    if mode == "subnormal":
        y16 = run_linear(stream, x, w, m, n, k, dispatch=d, f16_out=True)
        assert_matches(y16, y64, tol + F16_REL * np.abs(y64), f"{variant} {mode} f16")


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("variant", _names("q8_skinny_", "q8_mfma_"))
def test_q8_0_linear_wide_scales(stream, oracle, variant, mode):
    m, n, k = _shape(variant)
    x = _x(m, k)
    w = wide_q8_0_weights(_seed(variant, mode), n, k, mode)
    d = ops.Q4_0Dispatch()
    d.force(variant)
    y = run_q8(stream, x, w, m, n, k, dispatch=d)
    y64 = linear_f64_full(oracle, x, w, m, n, k, oracle.Q8_0)
    max_d = _finite_max(block_scales(w, n, k, block_bytes=34))
    max_x = float(np.abs(bits_to_f32(x)).max())
    tol = linear_tolerance(y64, k, max_d, max_x)
    assert_matches(y, y64, tol, f"{variant} {mode} {m}x{n}x{k}")
    if mode == "subnormal":
        y16 = run_q8(stream, x, w, m, n, k, dispatch=d, f16_out=True)
        assert_matches(y16, y64, tol + F16_REL * np.abs(y64), f"{variant} {mode} f16")


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("variant", _names("gateup_skinny_", "gateup_mfma_"))
def test_gate_up_wide_scales(stream, oracle, variant, mode):
    """silu(g) u against the f64 judge, the linear bound of g and u propagated
    through the product (|d silu / dg| <= 1.1)."""
    m, n, k = _shape(variant)
    x = _x(m, k)
    seed = _seed(variant, mode)
    wg, wu = wide_q4_0_weights(seed, n, k, mode), wide_q4_0_weights(seed + 1, n, k, mode)
    d = ops.Q4_0Dispatch()
    d.force(variant)
    y = run_gate_up(stream, x, wg, wu, m, n, k, dispatch=d)
    g64 = linear_f64_full(oracle, x, wg, m, n, k, oracle.Q4_0)
    u64 = linear_f64_full(oracle, x, wu, m, n, k, oracle.Q4_0)
    with np.errstate(over="ignore", invalid="ignore"):
        silu = g64 / (1.0 + np.exp(-g64))
        y64 = silu * u64
    max_d = max(_finite_max(block_scales(wg, n, k)), _finite_max(block_scales(wu, n, k)))
    max_x = float(np.abs(bits_to_f32(x)).max())
    with np.errstate(over="ignore", invalid="ignore"):
        tol = 1.1 * np.abs(u64) * linear_tolerance(g64, k, max_d, max_x) + np.abs(silu) * linear_tolerance(
            u64, k, max_d, max_x)
        tol = np.maximum(tol, 1e-3 * np.abs(y64))
    assert_matches(y, y64, tol, f"{variant} {mode} {m}x{n}x{k}")
