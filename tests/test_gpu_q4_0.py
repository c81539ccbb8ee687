"""GPU parity of the Q4_0 quantized linear against the oracle.

Mirrors crates/mote-backend-hip/tests/quantized_linear.rs (fixture, empty and
K == 0 cases) and adds the seeded workloads: decode GEMV (M = 1), the skinny
sweep (M <= 32), the prefill MFMA path (M >= 64) and the fused gate/up.
Every call goes through the C ABI of libmote_hip.so.

Tolerance (stated by the path's specification): an element passes if
|y - y64| <= 1e-3 |y64| or |y - y64| <= 2e-3 sqrt(K) max|d| max|x|, y64 being
the f64-accumulated oracle.  Outputs rounded to f16 get an extra 2^-11 |y64|.
"""

from __future__ import annotations

import functools
import re

import numpy as np
import pytest

from helpers import (
    assert_linear_close,
    bits_to_f32,
    f16_bits,
    linear_f64_full,
    q4_0_scales,
    ref_test_q4_0_inputs,
    ref_test_q4_0_weights,
    row_bytes,
)
from mote_amd import ops, workloads as wl
from mote_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu

F16_REL = 2.0 ** -11


@functools.lru_cache(maxsize=None)
def weights(seed: int, n: int, k: int) -> np.ndarray:
    return wl.q4_0_weights(seed, n, k)


@functools.lru_cache(maxsize=None)
def normal_x(seed: int, m: int, k: int) -> np.ndarray:
    return wl.normal_f16(seed, m * k)


def run_linear(stream, x_bits, w, m, n, k, f16_out=False, dispatch=None, fn=None, w_offset=0, x_offset=0):
    """Uploads, launches through the C ABI, synchronises, reads back."""
    xb = DeviceBuffer(x_bits.nbytes + x_offset)
    xb.upload(x_bits, offset=x_offset)
    wb = DeviceBuffer(w.nbytes + w_offset)
    wb.upload(w, offset=w_offset)
    out_bytes = m * n * (2 if f16_out else 4)
    yb = DeviceBuffer(out_bytes)
    yb.upload(np.full(out_bytes, 0xA5, dtype=np.uint8))  # sentinel: every element must be written
    args = (xb.ptr + x_offset, wb.ptr + w_offset, yb.ptr, m, n, k)
    if fn is not None:
        fn(*args, stream)
    elif dispatch is not None:
        dispatch.linear(*args, stream, f16_out=f16_out)
    elif f16_out:
        ops.quantized_linear_q4_0_f16(*args, stream)
    else:
        ops.quantized_linear_q4_0_f32(*args, stream)
    stream.synchronize()
    y = yb.download(np.uint16 if f16_out else np.float32)
    if f16_out:
        y = bits_to_f32(y)
    return y.reshape(m, n)


FULL_JUDGE_MACS = 1 << 26  # above this, every output is judged by the BLAS f64 judge


def oracle_f64(oracle, x_bits, w, m, n, k, columns=None):
    """The f64 linear: the oracle's sequential sum, or for large problems
    judged in full the BLAS f64 judge over oracle-decoded weights (held to the
    oracle by tests/test_oracle.py)."""
    if columns is None and m * n * k > FULL_JUDGE_MACS:
        return linear_f64_full(oracle, x_bits, w, m, n, k, oracle.Q4_0)
    return oracle.quantized_linear_f64(bits_to_f32(x_bits), w, m, n, k, columns)


def check_against_oracle(oracle, y, x_bits, w, m, n, k, columns=None, f16_out=False, what="output"):
    y64 = oracle_f64(oracle, x_bits, w, m, n, k, columns)
    got = y if columns is None else y[:, columns]
    max_d = float(np.max(np.abs(q4_0_scales(w, n, k)))) if k else 0.0
    max_x = float(np.max(np.abs(bits_to_f32(x_bits)))) if x_bits.size else 0.0
    assert_linear_close(got, y64, k, max_d, max_x, extra_rel=F16_REL if f16_out else 0.0, what=what)


def sample_columns(n: int, count: int = 256, seed: int = 7) -> np.ndarray:
    rng = np.random.default_rng(seed)
    cols = np.unique(np.concatenate([[0, n - 1], rng.choice(n, size=min(count, n), replace=False)]))
    return cols.astype(np.uint64)


# --- the reference's own fixture ----------------------------------------------

def test_reference_fixture_matches_cpu_oracle(stream, oracle):
    """crates/mote-backend-hip/tests/quantized_linear.rs:13-62: M=3, N=5, K=64,
    F16 output, tolerance max(0.01, 0.002 |e|) against f16(oracle f32)."""
    m, n, k = 3, 5, 64
    x = ref_test_q4_0_inputs(m, k)
    w = ref_test_q4_0_weights(n, k)
    wb = DeviceBuffer.from_array(w)
    assert bytes(wb.download(np.uint8)) == bytes(w)  # stored verbatim
    y = run_linear(stream, x, w, m, n, k, f16_out=True)
    expected = oracle.quantized_linear_f32(bits_to_f32(x), w, oracle.Q4_0, m, n, k).reshape(m, n)
    expected = expected.astype(np.float16).astype(np.float32)
    tol = np.maximum(0.01, np.abs(expected) * 0.002)
    assert np.all(np.abs(y - expected) <= tol), (y, expected)
    check_against_oracle(oracle, y, x, w, m, n, k, f16_out=True)


def test_empty_outputs_return_without_a_launch(stream):
    """crates/mote-backend-hip/tests/quantized_linear.rs:124-140."""
    w = ref_test_q4_0_weights(2, 32)
    wb = DeviceBuffer.from_array(w)
    xb = DeviceBuffer(0)
    yb = DeviceBuffer(0)
    for fn in (ops.quantized_linear_q4_0_f16, ops.quantized_linear_q4_0_f32):
        fn(xb.ptr, wb.ptr, yb.ptr, 0, 2, 32, stream)
        fn(xb.ptr, wb.ptr, yb.ptr, 3, 0, 32, stream)
    stream.synchronize()


def test_zero_input_features_writes_zeros(stream):
    """crates/mote-backend-hip/tests/quantized_linear.rs:142-158: K == 0 with
    M, N > 0 launches and writes zeros."""
    for f16_out in (True, False):
        y = run_linear(stream, np.zeros(0, np.uint16), np.zeros(0, np.uint8), 3, 2, 0, f16_out=f16_out)
        assert np.array_equal(y, np.zeros((3, 2), np.float32))
        assert not np.signbit(y).any()


# --- seeded workloads -------------------------------------------------------------

def test_decode_gemv_4096x4096_uniform_activations(stream, oracle):
    m, k, n = 1, 4096, 4096
    x = wl.uniform_f16(wl.seed_for(0, 0), m * k)
    w = weights(wl.seed_for(0, 1), n, k)
    y = run_linear(stream, x, w, m, n, k)
    check_against_oracle(oracle, y, x, w, m, n, k)


@pytest.mark.parametrize("k,n", [(4096, 14336), (14336, 4096), (28672, 8192)], ids=["up_gate", "down", "down_70b"])
def test_decode_gemv_llama_mlp_shapes(stream, oracle, k, n):
    m = 1
    x = normal_x(wl.seed_for(1, 0), m, k)
    w = weights(wl.seed_for(1, 1), n, k)
    cols = None if n * k <= 14336 * 4096 else sample_columns(n, 512)
    y = run_linear(stream, x, w, m, n, k)
    check_against_oracle(oracle, y, x, w, m, n, k, columns=cols)
    y16 = run_linear(stream, x, w, m, n, k, f16_out=True)
    check_against_oracle(oracle, y16, x, w, m, n, k, columns=cols, f16_out=True, what="f16 output")


@pytest.mark.parametrize("n", [4096, 6144, 14336])
@pytest.mark.parametrize("m", [2, 4, 8, 16, 32])
def test_skinny_sweep(stream, oracle, m, n):
    k = 4096
    x = normal_x(wl.seed_for(2, 0), m, k)
    w = weights(wl.seed_for(2, 1), n, k)
    y = run_linear(stream, x, w, m, n, k)
    check_against_oracle(oracle, y, x, w, m, n, k)  # every output


@pytest.mark.parametrize("m", [64, 256, 512])
def test_prefill_mfma(stream, oracle, m):
    k, n = 4096, 14336
    x = normal_x(wl.seed_for(4, 0), m, k)
    w = weights(wl.seed_for(4, 1), n, k)
    y = run_linear(stream, x, w, m, n, k)
    check_against_oracle(oracle, y, x, w, m, n, k)  # every output


def run_gate_up(stream, x, wg, wu, m, n, k, dispatch=None, f16_out=False, concatenated=False):
    """The fused gate/up through the C ABI (gate and up buffers, or one
    concatenated [2N, K] buffer with up = NULL); returns y as f32 [m, n]."""
    xb = DeviceBuffer.from_array(x)
    if concatenated:
        gb, ub = DeviceBuffer.from_array(np.concatenate([wg, wu])), None
    else:
        gb, ub = DeviceBuffer.from_array(wg), DeviceBuffer.from_array(wu)
    out_bytes = m * n * (2 if f16_out else 4)
    yb = DeviceBuffer(out_bytes)
    yb.upload(np.full(out_bytes, 0xA5, dtype=np.uint8))  # sentinel: every element must be written
    up = None if ub is None else ub.ptr
    if dispatch is not None:
        dispatch.gate_up_silu(xb.ptr, gb.ptr, up, yb.ptr, m, n, k, stream, f16_out=f16_out)
    else:
        assert not f16_out
        ops.q4_0_gate_up_silu_f32(xb.ptr, gb.ptr, up, yb.ptr, m, n, k, stream)
    stream.synchronize()
    y = yb.download(np.uint16 if f16_out else np.float32)
    return (bits_to_f32(y) if f16_out else y).reshape(m, n)


def check_gate_up(oracle, y, x, wg, wu, m, n, k, cols=None, f16_out=False, what="gate/up"):
    """silu(g) u against the f64 oracle: the linear bound of g and of u
    propagated through the product (|d silu/dg| <= 1.1), so
    |dy| <= 1.1 |u| tol_g + |silu(g)| tol_u (+2^-11 |y| for f16 outputs)."""
    from helpers import linear_tolerance

    if cols is None and m * n * k > FULL_JUDGE_MACS:
        g64 = linear_f64_full(oracle, x, wg, m, n, k, oracle.Q4_0)
        u64 = linear_f64_full(oracle, x, wu, m, n, k, oracle.Q4_0)
        y64 = g64 / (1.0 + np.exp(-g64)) * u64  # the oracle's f64 SiLU composition
    else:
        y64 = oracle.gate_up_silu_f64(bits_to_f32(x), wg, wu, m, n, k, cols)
        g64 = oracle.quantized_linear_f64(bits_to_f32(x), wg, m, n, k, cols)
        u64 = oracle.quantized_linear_f64(bits_to_f32(x), wu, m, n, k, cols)
    max_d = float(max(np.abs(q4_0_scales(wg, n, k)).max(), np.abs(q4_0_scales(wu, n, k)).max()))
    max_x = float(np.abs(bits_to_f32(x)).max())
    silu = g64 / (1.0 + np.exp(-g64))
    tol = 1.1 * np.abs(u64) * linear_tolerance(g64, k, max_d, max_x) + np.abs(silu) * linear_tolerance(
        u64, k, max_d, max_x
    )
    tol = np.maximum(tol, 1e-3 * np.abs(y64)) + (F16_REL * np.abs(y64) if f16_out else 0.0)
    got = y if cols is None else y[:, cols]
    err = np.abs(got - y64)
    assert np.all(err <= tol), f"{what}: max excess {float(np.max(err - tol))}"


@pytest.mark.parametrize("m", [1, 2, 4, 16, 32, 64, 256, 512])
def test_fused_gate_up_silu(stream, oracle, m):
    """Default entry point at every token count of the path (the skinny gate/up
    up to 64 tokens, the prefill tiles above), separate and concatenated
    weight buffers giving identical outputs."""
    k, n = 4096, 14336
    x = normal_x(wl.seed_for(4, 0), m, k)
    wg = weights(wl.seed_for(4, 1), n, k)
    wu = weights(wl.seed_for(4, 2), n, k)
    y = run_gate_up(stream, x, wg, wu, m, n, k)
    yc = run_gate_up(stream, x, wg, wu, m, n, k, concatenated=True)
    assert np.array_equal(y, yc)
    check_gate_up(oracle, y, x, wg, wu, m, n, k, what=f"gate/up M={m}")  # every output


# --- every kernel variant, ragged and misaligned shapes ------------------------------

def _variants(prefix):
    return [v for v in ops.variant_names() if v.startswith(prefix)]


@pytest.mark.parametrize("variant", _variants("gemv_") + ["generic"])
def test_every_vector_variant(stream, oracle, variant):
    d = ops.Q4_0Dispatch()
    d.force(variant)
    for m, n, k in [(1, 257, 1024), (5, 61, 4480), (3, 130, 64)]:
        x = normal_x(wl.seed_for(9, m), m, k)
        w = weights(wl.seed_for(9, 100 + n), n, k)
        y = run_linear(stream, x, w, m, n, k, dispatch=d)
        check_against_oracle(oracle, y, x, w, m, n, k, what=f"{variant} {m}x{n}x{k}")


def _rows_shapes(variant):
    """M = 1 shapes a row-streaming variant rows_r<R>_k<KS> can run: ragged N,
    idle lanes (K below 4096 KS) and a row exactly filling the K slices."""
    ks = int(variant.split("_k")[1])
    shapes = []
    for n, k in [(257, 1024), (130, 64), (61, 4480), (1000, 14336), (67, 28672), (33, 4096 * ks)]:
        if k <= 4096 * ks and (k // 64) * 144 <= 65536:
            shapes.append((1, n, k))
    return shapes


@pytest.mark.parametrize("variant", _variants("rows_"))
def test_every_rows_variant(stream, oracle, variant):
    d = ops.Q4_0Dispatch()
    d.force(variant)
    for m, n, k in _rows_shapes(variant):
        x = normal_x(wl.seed_for(9, k), m, k)
        w = weights(wl.seed_for(9, 100 + n), n, k)
        y = run_linear(stream, x, w, m, n, k, dispatch=d)
        check_against_oracle(oracle, y, x, w, m, n, k, what=f"{variant} {m}x{n}x{k}")
        y16 = run_linear(stream, x, w, m, n, k, dispatch=d, f16_out=True)
        check_against_oracle(oracle, y16, x, w, m, n, k, f16_out=True, what=f"{variant} f16 {m}x{n}x{k}")


@pytest.mark.parametrize("variant", [v for v in _variants("stream_") if "_m4x_" not in v])
def test_every_stream_variant(stream, oracle, variant):
    """Persistent pipelined GEMV: N below one workgroup, ragged N, idle lanes
    (K < 4096), and N = 140001 at K = 64, where waves own more than 64 rows
    and flush their register-held sums mid-loop.  Variants with P pair slots
    per lane, or rows split over S waves, also run K filling all of the P S
    64-pair slots, K one pair past P S - 1 slots, and the 14336 -> 4096 down
    projection where it fits.  Multi-token variants run every shape with
    their M."""
    d = ops.Q4_0Dispatch()
    d.force(variant)
    slots = int(variant.split("_p")[1].split("_")[0]) if "_p" in variant else 1
    slots *= int(variant.split("_s")[1].split("_")[0]) if "_s" in variant else 1
    tokens = int(variant.split("_m")[1].split("_")[0]) if "_m" in variant else 1
    shapes = [(1, 64), (7, 4096), (257, 1024), (130, 64), (140001, 64)]
    if slots > 1:
        shapes += [(61, 4096 * slots), (1000, 4096 * (slots - 1) + 64)]
        if 14336 <= 4096 * slots:
            shapes.append((4096, 14336))
    shapes.append((14336, 4096))
    shapes = [(tokens, n, k) for n, k in shapes]
    for m, n, k in shapes:
        x = normal_x(wl.seed_for(13, k), m, k)
        w = weights(wl.seed_for(13, 100 + n), n, k)
        y = run_linear(stream, x, w, m, n, k, dispatch=d)
        cols = None if n < 2000 else sample_columns(n, 512)
        check_against_oracle(oracle, y, x, w, m, n, k, columns=cols, what=f"{variant} {m}x{n}x{k}")
    y16 = run_linear(stream, x, w, m, n, k, dispatch=d, f16_out=True)
    check_against_oracle(oracle, y16, x, w, m, n, k, columns=cols, f16_out=True, what=f"{variant} f16")


def _skinny_k(variant):
    ks, rest = variant.split("_k", 1)[1].split("_s", 1)
    return int(ks) * int(rest.split("_t")[0]) * 256


@pytest.mark.parametrize("variant", [v for v in _variants("skinny_mfma_") if not v.endswith("_sk")])
def test_every_skinny_mfma_variant(stream, oracle, variant):
    """Matrix-core skinny GEMM: tokens padded inside a 16-token tile (M = 2, 5),
    exactly one and two tiles (16, 32), one token over (17, 33), the 64-token
    maximum, N ragged against the 16-row tiles, f32 and f16 outputs; 20 x
    14336 gives every workgroup several items (the item ring and the deferred
    reduction over several items)."""
    d = ops.Q4_0Dispatch()
    d.force(variant)
    k = _skinny_k(variant)
    for m, n in [(2, 100), (5, 33), (16, 16), (17, 130), (32, 61), (33, 7), (64, 80), (20, 14336), (3, 4096)]:
        x = normal_x(wl.seed_for(14, m), m, k)
        w = weights(wl.seed_for(14, 100 + n), n, k)
        y = run_linear(stream, x, w, m, n, k, dispatch=d)
        cols = None if n < 1000 else sample_columns(n, 256)
        check_against_oracle(oracle, y, x, w, m, n, k, columns=cols, what=f"{variant} {m}x{n}x{k}")
    y16 = run_linear(stream, x, w, m, n, k, dispatch=d, f16_out=True)
    check_against_oracle(oracle, y16, x, w, m, n, k, columns=cols, f16_out=True, what=f"{variant} f16")


@pytest.mark.parametrize("variant", _variants("mfma_"))
def test_every_mfma_variant(stream, oracle, variant):
    d = ops.Q4_0Dispatch()
    d.force(variant)
    # `_k<P>` tiles take P block pairs (64 P of K) per step: the shapes they
    # can run, plus K = 768 (12 pairs: 6 or 3 steps); K = 448 is seven steps
    # of one pair
    kp = int(re.search(r"_k(\d+)$", variant).group(1)) if re.search(r"_k(\d+)$", variant) else 1
    shapes = [(70, 200, 512), (130, 67, 1024), (64, 128, 64), (96, 160, 448), (96, 160, 768)]
    for m, n, k in [sh for sh in shapes if sh[2] % (64 * kp) == 0]:
        x = normal_x(wl.seed_for(10, m), m, k)
        w = weights(wl.seed_for(10, 100 + n), n, k)
        y = run_linear(stream, x, w, m, n, k, dispatch=d)
        check_against_oracle(oracle, y, x, w, m, n, k, what=f"{variant} {m}x{n}x{k}")


@pytest.mark.parametrize(
    "variant", [v for v in _variants("gateup_") if not v.startswith(("gateup_skinny_", "gateup_stream_"))]
)
def test_every_gate_up_variant(stream, oracle, variant):
    d = ops.Q4_0Dispatch()
    d.force(variant)
    m, n, k = 70, 100, 512
    x = normal_x(wl.seed_for(11, 0), m, k)
    wg, wu = weights(wl.seed_for(11, 1), n, k), weights(wl.seed_for(11, 2), n, k)
    xb, gb, ub = DeviceBuffer.from_array(x), DeviceBuffer.from_array(wg), DeviceBuffer.from_array(wu)
    yb = DeviceBuffer(m * n * 4)
    d.gate_up_silu(xb.ptr, gb.ptr, ub.ptr, yb.ptr, m, n, k, stream)
    stream.synchronize()
    y = yb.download(np.float32).reshape(m, n)
    y64 = oracle.gate_up_silu_f64(bits_to_f32(x), wg, wu, m, n, k)
    assert np.all(np.abs(y - y64) <= np.maximum(2e-2, 2e-3 * np.abs(y64))), float(np.max(np.abs(y - y64)))


@pytest.mark.parametrize("variant", _variants("gateup_stream_"))
def test_every_stream_gate_up_variant(stream, oracle, variant):
    """Gate/up on the streaming GEMV (both rows per step, one or two tokens per
    row read, rows whole or split over S waves): N below one workgroup, ragged N, idle lanes (K < 4096), N =
    140001 at K = 64 (waves flush register-held results mid-loop), K filling
    all P 64-pair slots and one pair past P - 1 slots, the 4096 x 14336 MLP
    shape; f32 and f16."""
    d = ops.Q4_0Dispatch()
    d.force(variant)
    slots = int(variant.split("_p")[1].split("_")[0]) if "_p" in variant else 1
    slots *= int(variant.split("_s")[2].split("_")[0]) if variant.count("_s") > 1 else 1  # rows split over S waves
    m = int(variant.split("_m")[1].split("_")[0]) if "_m" in variant else 1
    shapes = [(100, 4096), (4099, 1024), (140001, 64), (7, 4096 * slots), (14336, 4096)]
    if slots > 1:
        shapes.append((513, 4096 * (slots - 1) + 64))
    for n, k in shapes:
        x = normal_x(wl.seed_for(16, k), m, k)
        wg, wu = weights(wl.seed_for(16, 100 + n), n, k), weights(wl.seed_for(16, 300 + n), n, k)
        cols = None if n < 5000 else sample_columns(n, 128)
        y = run_gate_up(stream, x, wg, wu, m, n, k, dispatch=d)
        check_gate_up(oracle, y, x, wg, wu, m, n, k, cols=cols, what=f"{variant} {m}x{n}x{k}")
        y16 = run_gate_up(stream, x, wg, wu, m, n, k, dispatch=d, f16_out=True)
        check_gate_up(oracle, y16, x, wg, wu, m, n, k, cols=cols, f16_out=True, what=f"{variant} f16 {m}x{n}x{k}")


@pytest.mark.parametrize("variant", [v for v in _variants("gateup_skinny_") if not v.endswith("_sk")])
def test_every_skinny_gate_up_variant(stream, oracle, variant):
    """Skinny gate/up items (one gate and one up row tile): one token, tokens
    padded inside a tile, one over a tile, the 64-token maximum, N ragged
    against the 16-row tiles, several items per workgroup (20 x 14336), f32
    and f16 outputs."""
    d = ops.Q4_0Dispatch()
    d.force(variant)
    k = _skinny_k(variant)
    for m, n in [(1, 100), (5, 33), (16, 16), (17, 130), (33, 7), (64, 80), (20, 14336)]:
        x = normal_x(wl.seed_for(15, m), m, k)
        wg, wu = weights(wl.seed_for(15, 100 + n), n, k), weights(wl.seed_for(15, 200 + n), n, k)
        y = run_gate_up(stream, x, wg, wu, m, n, k, dispatch=d)
        cols = None if n < 1000 else sample_columns(n, 96)
        check_gate_up(oracle, y, x, wg, wu, m, n, k, cols=cols, what=f"{variant} {m}x{n}x{k}")
    y16 = run_gate_up(stream, x, wg, wu, m, n, k, dispatch=d, f16_out=True)
    check_gate_up(oracle, y16, x, wg, wu, m, n, k, cols=cols, f16_out=True, what=f"{variant} f16")


@pytest.mark.parametrize(
    "m,n,k,w_offset,x_offset",
    [(7, 13, 96, 0, 0), (2, 33, 4096, 2, 0), (1, 40, 1024, 0, 2), (65, 50, 512, 2, 0), (9, 1, 32, 0, 0)],
    ids=["k96", "w_misaligned", "x_misaligned", "prefill_w_misaligned", "k32_n1"],
)
def test_ragged_and_misaligned(stream, oracle, m, n, k, w_offset, x_offset):
    x = normal_x(wl.seed_for(12, m), m, k)
    w = weights(wl.seed_for(12, n), n, k)
    y = run_linear(stream, x, w, m, n, k, w_offset=w_offset, x_offset=x_offset)
    check_against_oracle(oracle, y, x, w, m, n, k)


# --- bit-exact decode ----------------------------------------------------------------

def _all_scale_weights(k: int) -> np.ndarray:
    """One block per binary16 scale pattern (all 65536), nibble bytes covering
    every low and high nibble value at every position."""
    blocks = 65536
    out = np.empty((blocks, 18), dtype=np.uint8)
    out[:, 0:2] = np.arange(blocks, dtype="<u2").view(np.uint8).reshape(blocks, 2)
    j = np.arange(16)
    b = np.arange(blocks)[:, None]
    out[:, 2:] = ((j + b) % 16 | (((15 - j) + 3 * b) % 16) << 4).astype(np.uint8)
    return out.reshape(-1)


@pytest.mark.parametrize("k,offset", [(4096, 0), (4096, 2), (32, 0)], ids=["pairs", "misaligned", "k32"])
def test_decode_is_bit_exact_for_every_scale(stream, oracle, k, offset):
    w = _all_scale_weights(k)
    rows = w.size // row_bytes(k)
    wb = DeviceBuffer(w.nbytes + offset)
    wb.upload(w, offset=offset)
    ob = DeviceBuffer(rows * k * 4)
    ops.dequantize_q4_0_f32(wb.ptr + offset, ob.ptr, rows, k, stream)
    stream.synchronize()
    got = ob.download(np.float32).reshape(rows, k)
    rb = row_bytes(k)
    want = np.stack([oracle.dequantize_row(w[r * rb:(r + 1) * rb], oracle.Q4_0, k) for r in range(rows)])
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn)
    assert np.array_equal(got[~gn].view(np.uint32), want[~wn].view(np.uint32))


# --- size-independent properties at full size ------------------------------------------

@pytest.mark.parametrize("m,k,n", [(1, 4096, 14336), (1, 14336, 4096), (2, 4096, 4096), (8, 4096, 14336),
                                   (256, 4096, 14336)])
def test_exact_properties_at_full_size(stream, m, k, n):
    """Doubling x doubles y, negating every scale negates y, and zeroing the
    scales of one K block equals zeroing those 32 activations: all exact in
    the kernels' f32 arithmetic, so compared bit for bit.  Repeated runs are
    bitwise identical (no atomics)."""
    x = normal_x(wl.seed_for(1, 0), m, k)
    w = weights(wl.seed_for(1, 1), n, k)
    d = ops.Q4_0Dispatch()
    y = run_linear(stream, x, w, m, n, k, dispatch=d)
    matrix_cores = "mfma" in d.plan(m, n, k)
    assert np.array_equal(y, run_linear(stream, x, w, m, n, k, dispatch=d)), "non-deterministic"
    x2 = f16_bits(bits_to_f32(x) * 2.0)
    assert np.array_equal(run_linear(stream, x2, w, m, n, k, dispatch=d), 2.0 * y)
    wneg = w.copy().reshape(n, k // 32, 18)
    wneg[:, :, 1] ^= 0x80
    yneg = run_linear(stream, x, wneg.reshape(-1), m, n, k, dispatch=d)
    if not matrix_cores:
        assert np.array_equal(yneg, -y)
    else:
        # The matrix cores' f32 accumulation is not symmetric under negation
        # (measured: differences of a few ulps of the partial sums, which can
        # exceed the result's own ulp after cancellation), so the MFMA path is
        # held to 2^-20 of the accumulation scale sqrt(K) max|d| max|x| * 8.
        scale = 8 * np.sqrt(k) * float(np.abs(q4_0_scales(w, n, k)).max()) * float(np.abs(bits_to_f32(x)).max())
        assert np.all(np.abs(yneg + y) <= 2.0 ** -20 * scale)
    blk = 5
    wz = w.copy().reshape(n, k // 32, 18)
    wz[:, blk, 0:2] = 0
    xz = x.copy().reshape(m, k)
    xz[:, 32 * blk:32 * blk + 32] = 0
    assert np.array_equal(run_linear(stream, x, wz.reshape(-1), m, n, k, dispatch=d),
                          run_linear(stream, xz.reshape(-1), w, m, n, k, dispatch=d))


def test_autotuned_dispatch_caches_a_plan(stream, oracle):
    m, k, n = 1, 4096, 4096
    d = ops.Q4_0Dispatch(autotune=True)
    x = normal_x(wl.seed_for(1, 0), m, k)
    w = weights(wl.seed_for(0, 1), n, k)
    assert d.plan(m, n, k) is None
    y = run_linear(stream, x, w, m, n, k, dispatch=d)
    assert d.plan(m, n, k) in ops.variant_names()
    check_against_oracle(oracle, y, x, w, m, n, k)


def test_autotuner_times_the_heuristic_pick(stream, oracle):
    """16 tokens at K = 11008 (no K slicing): the heuristic takes the prefill
    tiles, a kind the autotuner's own list holds only from 64 tokens; the
    autotuner times that pick beside its list, so its plan is a variant of
    the list or that pick, and the result is within the oracle's tolerance."""
    m, k, n = 16, 11008, 512
    x = normal_x(wl.seed_for(1, 2), m, k)
    w = weights(wl.seed_for(0, 3), n, k)
    plain = ops.Q4_0Dispatch()
    run_linear(stream, x, w, m, n, k, dispatch=plain)
    assert plain.plan(m, n, k).startswith("mfma_")
    d = ops.Q4_0Dispatch(autotune=True)
    y = run_linear(stream, x, w, m, n, k, dispatch=d)
    assert d.plan(m, n, k) in ops.variant_names()
    check_against_oracle(oracle, y, x, w, m, n, k)
