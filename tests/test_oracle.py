"""Pins the CPU oracle (test infrastructure) before it judges the HIP path.

Each check is independent of the oracle's own code:
* the reference's known-answer tests, transcribed into
  tests/golden/reference_kats.json (crates/mote-reference/tests/*.rs);
* binary16 conversion against numpy's independent implementation for all
  65536 patterns (decode) and for edge and random binary32 values (rounding);
* the Q4_0 decode against a from-the-definition numpy decoder for every scale
  pattern, including subnormals, signed zeros, infinities and NaN;
* the f64 linear against exact rational arithmetic on small inputs, the f32
  linear against a sequential numpy.float32 loop (which pins the rounding
  order) and against linearity / sign / zero-block invariants;
* RMSNorm / fused add + RMSNorm against independent f64 formulas and the
  reference's hand-computed anchors;
* the RoPE table builder against the closed form.
"""

from __future__ import annotations

import hashlib
import json
import math
import os
from fractions import Fraction

import numpy as np
import pytest

from helpers import bits_to_f32, f16_bits, ref_test_q4_0_inputs, ref_test_q4_0_weights, row_bytes

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_kats():
    with open(os.path.join(GOLDEN, "reference_kats.json"), encoding="utf-8") as f:
        return json.load(f)


KATS = load_kats()


def block(scale_bits: int, quants) -> bytes:
    return int(scale_bits).to_bytes(2, "little") + bytes(quants)


# --- reference known-answer tests ------------------------------------------------------

@pytest.mark.parametrize("case", KATS["dequantize_q4_0"], ids=lambda c: c["name"])
def test_kat_dequantize(oracle, case):
    data = b"".join(block(b["scale_bits"], b["quants"]) for b in case["blocks"])
    got = oracle.dequantize_row(data, oracle.Q4_0, case["row_elements"])
    assert got.tolist() == case["expected"]


def test_kat_dequantize_q8_0(oracle):
    case = KATS["dequantize_q8_0"]
    quants = [q & 0xFF for q in case["quants"]]
    got = oracle.dequantize_row(block(case["scale_bits"], quants), oracle.Q8_0, 32)
    assert got.tolist() == case["expected"]


@pytest.mark.parametrize("case", KATS["quantized_linear"], ids=lambda c: c["name"])
def test_kat_quantized_linear(oracle, case):
    fmt = getattr(oracle, case["format"])
    data = b"".join(block(b["scale_bits"], [q & 0xFF for q in b["quants"]]) for b in case["blocks"])
    got = oracle.quantized_linear_f32(case["input"], data, fmt, case["rows"], case["output_features"],
                                      case["input_features"])
    assert got.tolist() == case["expected"]


@pytest.mark.parametrize("case", KATS["errors"], ids=lambda c: c["name"])
def test_kat_error_taxonomy(oracle, case):
    fmt = getattr(oracle, case["format"])
    big = lambda v: (2 ** 64 - 1) if v == "usize::MAX" else (((2 ** 64 - 1) // 32) * 32 if v == "huge_q8_row" else v)
    with pytest.raises(oracle.OracleError) as err:
        if case["op"] == "dequantize_row":
            oracle.dequantize_row(bytes(case["bytes"]), fmt, big(case["row_elements"]))
        else:
            oracle.quantized_linear_f32(np.zeros(case["input_len"], np.float32), bytes(case["weights_len"]),
                                        fmt, big(case["rows"]), case["output_features"], case["input_features"])
    assert err.value.kind == case["kind"]
    want = {k: big(v) for k, v in case["fields"].items()}
    assert err.value.fields == want


def test_kat_empty_geometries(oracle):
    """quantized_rows.rs:85-102."""
    assert oracle.quantized_linear_f32([], b"", oracle.Q4_0, 3, 2, 0).tolist() == [0.0] * 6
    zeros = block(0x3C00, [0] * 32) * 2
    assert oracle.quantized_linear_f32([], zeros, oracle.Q8_0, 0, 2, 32).size == 0
    assert oracle.dequantize_row(b"", oracle.Q8_0, 0).size == 0


def test_kat_matmul(oracle):
    """crates/mote-reference/tests/matmul_f32.rs."""
    for case in KATS["matmul"]:
        got = oracle.matmul_f32(case["lhs"], case["rhs"], case["m"], case["n"], case["k"])
        assert got.tolist() == case["expected"], case["name"]
    with pytest.raises(oracle.OracleError) as e:
        oracle.matmul_f32([1.0], [1.0] * 6, 2, 2, 3)
    assert e.value.kind == "LhsLengthMismatch" and e.value.fields == {"expected": 6, "actual": 1}
    with pytest.raises(oracle.OracleError) as e:
        oracle.matmul_f32([1.0] * 6, [1.0], 2, 2, 3)
    assert e.value.kind == "RhsLengthMismatch"
    with pytest.raises(oracle.OracleError) as e:
        oracle.matmul_f32([], [], 2 ** 64 - 1, 1, 2)
    assert e.value.kind == "DimensionsOverflow"


@pytest.mark.parametrize("case", KATS["rope"], ids=lambda c: c["name"])
def test_kat_rope(oracle, case):
    layout = getattr(oracle, case["layout"])
    got = oracle.rope_f32(case["input"], case["cos"], case["sin"], case["tokens"], case["heads"],
                          case["head_dim"], case["rotary_dim"], layout)
    assert got.tolist() == case["expected"]


@pytest.mark.parametrize("case", KATS["rope_errors"], ids=lambda c: c["name"])
def test_kat_rope_errors(oracle, case):
    with pytest.raises(oracle.OracleError) as e:
        oracle.rope_f32(case["input"], case["cos"], case["sin"], case["tokens"], case["heads"],
                        case["head_dim"], case["rotary_dim"], oracle.HALF_SPLIT)
    assert e.value.kind == case["kind"]
    assert e.value.fields == case["fields"]


def _rms_f64(x, w, hidden, eps):
    """Independent f64 RMSNorm (crates/mote-reference/tests/rms_norm_f32.rs:13-24)."""
    out = []
    for r in range(len(x) // hidden):
        row = [float(v) for v in x[r * hidden:(r + 1) * hidden]]
        inv = 1.0 / math.sqrt(sum(v * v for v in row) / hidden + float(np.float32(eps)))
        out += [float(np.float32(v * inv * float(wv))) for v, wv in zip(row, w)]
    return np.array(out, dtype=np.float64)


def test_kat_rms_norm(oracle):
    k = KATS["rms_norm"]
    got = oracle.rms_norm_f32(k["input"], k["weight"], k["hidden"], k["epsilon"])
    assert np.all(np.abs(got - _rms_f64(k["input"], k["weight"], k["hidden"], k["epsilon"])) < 1e-5)
    for i, want in k["anchors"]:
        assert abs(got[i] - want) < 1e-4
    assert oracle.rms_norm_f32([], k["weight"], 4, 1e-6).size == 0
    for args, kind in [(([1.0, 2.0], [1.0, 1.0], 0, 1e-6), "ZeroHiddenSize"),
                       (([1.0, 2.0], [1.0], 2, 1e-6), "WeightLengthMismatch"),
                       (([1.0, 2.0, 3.0], [1.0, 1.0], 2, 1e-6), "InputNotMultiple"),
                       (([1.0, 2.0], [1.0, 1.0], 2, -1e-6), "InvalidEpsilon"),
                       (([1.0, 2.0], [1.0, 1.0], 2, float("nan")), "InvalidEpsilon"),
                       (([1.0, 2.0], [1.0, 1.0], 2, float("inf")), "InvalidEpsilon")]:
        with pytest.raises(oracle.OracleError) as e:
            oracle.rms_norm_f32(*args)
        assert e.value.kind == kind


def test_kat_fused_add_rms_norm(oracle):
    k = KATS["fused_add_rms_norm"]
    normalized, residual = oracle.fused_add_rms_norm_f32(k["input"], k["residual"], k["weight"], k["hidden"],
                                                         k["epsilon"])
    sums = [a + b for a, b in zip(k["input"], k["residual"])]
    assert np.all(np.abs(normalized - _rms_f64(sums, k["weight"], k["hidden"], k["epsilon"])) < 1e-5)
    for i, want in k["anchors"]:
        assert abs(normalized[i] - want) < 1e-4
    assert residual.tolist() == k["expected_residual"]
    n, r = oracle.fused_add_rms_norm_f32([1.0, 2.0, -3.0, 4.0], [4.0, -3.0, 2.0, -1.0], [0.0] * 4, 4, 1e-6)
    assert n.tolist() == [0.0] * 4 and r.tolist() == [5.0, -1.0, -1.0, 3.0]
    n, r = oracle.fused_add_rms_norm_f32([3.0], [1.0], [2.0], 1, 0.0)
    assert n.tolist() == [2.0] and r.tolist() == [4.0]
    with pytest.raises(oracle.OracleError) as e:
        oracle.fused_add_rms_norm_f32([1.0, 2.0], [1.0], [1.0, 1.0], 2, 1e-6)
    assert e.value.kind == "ResidualLengthMismatch" and e.value.fields == {"residual_len": 1, "input_len": 2}


# --- binary16, independent of the oracle's code -----------------------------------------

def test_f16_decode_all_patterns(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    got = oracle.f16_bits_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_round_to_nearest_even(oracle):
    rng = np.random.default_rng(1)
    raw = rng.integers(0, 2 ** 32, size=200000, dtype=np.uint64).astype(np.uint32)
    edge = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                     2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, np.inf, -np.inf], dtype=np.float32)
    vals = np.concatenate([raw.view(np.float32), edge])
    vals = vals[~np.isnan(vals)]
    got = oracle.f32_to_f16_bits(vals)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# --- Q4_0 decode: every scale pattern, from the definition -------------------------------

def test_q4_0_decode_every_scale_pattern(oracle):
    scales = np.arange(65536, dtype=np.uint16)
    j = np.arange(16)
    quants = ((j[None, :] + scales[:, None]) % 16 | ((15 - j[None, :] + 3 * scales[:, None]) % 16) << 4)
    quants = quants.astype(np.uint8)
    blocks = np.empty((65536, 18), np.uint8)
    blocks[:, 0:2] = scales.astype("<u2").view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = quants
    k = 4096
    rb = row_bytes(k)
    data = blocks.reshape(-1)
    got = np.concatenate([oracle.dequantize_row(data[r * rb:(r + 1) * rb], oracle.Q4_0, k)
                          for r in range(data.size // rb)]).reshape(65536, 32)
    d = scales.view(np.float16).astype(np.float32)[:, None]
    lo = (quants & 15).astype(np.float32) - 8.0
    hi = (quants >> 4).astype(np.float32) - 8.0
    with np.errstate(invalid="ignore"):
        want = np.concatenate([lo * d, hi * d], axis=1).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # 0 x negative scale keeps the sign of zero
    assert np.signbit(got[0x8000 + 0x3C00, :][want[0x8000 + 0x3C00, :] == 0]).all()


# --- the linear: exact arithmetic, rounding order and invariants --------------------------

def _decode_fraction(w, n, k):
    """Exact rational decode of a Q4_0 matrix."""
    rows = []
    blocks = w.reshape(n, k // 32, 18)
    for r in range(n):
        row = []
        for b in range(k // 32):
            bits = int(blocks[r, b, 0]) | (int(blocks[r, b, 1]) << 8)
            d = Fraction(float(np.uint16(bits).view(np.float16)))
            q = blocks[r, b, 2:]
            row += [(int(v & 15) - 8) * d for v in q] + [(int(v >> 4) - 8) * d for v in q]
        rows.append(row)
    return rows


@pytest.mark.parametrize("m,n,k", [(3, 5, 64), (2, 7, 96)])
def test_linear_f64_against_exact_rationals(oracle, m, n, k):
    from mote_amd import workloads as wl

    x = wl.normal_f16(11, m * k)
    w = wl.q4_0_weights(12, n, k)
    xf = [Fraction(float(v)) for v in x.view(np.float16)]
    dec = _decode_fraction(w, n, k)
    exact = np.array([[float(sum(xf[r * k + i] * dec[c][i] for i in range(k))) for c in range(n)]
                      for r in range(m)])
    got = oracle.quantized_linear_f64(bits_to_f32(x), w, m, n, k)
    assert np.all(np.abs(got - exact) <= 1e-12 * np.maximum(1.0, np.abs(exact)))
    cols = np.array([4, 0, 2], np.uint64)[: min(3, n)]
    cols = cols[cols < n]
    assert np.array_equal(oracle.quantized_linear_f64(bits_to_f32(x), w, m, n, k, cols), got[:, cols.astype(int)])


def test_linear_f32_rounding_order_is_sequential(oracle):
    """The f32 oracle equals a sequential binary32 multiply-then-add over K
    (the reference's loop, quantized.rs:134-141), bit for bit."""
    from mote_amd import workloads as wl

    m, n, k = 2, 3, 128
    x = bits_to_f32(wl.normal_f16(21, m * k))
    w = wl.q4_0_weights(22, n, k)
    got = oracle.quantized_linear_f32(x, w, oracle.Q4_0, m, n, k).reshape(m, n)
    blocks = w.reshape(n, k // 32, 18)
    for c in range(n):
        d = blocks[c, :, 0:2].copy().view("<u2")[:, 0].view(np.float16).astype(np.float32)
        q = blocks[c, :, 2:]
        dec = np.concatenate([np.concatenate([((q[b] & 15).astype(np.float32) - 8) * d[b],
                                              ((q[b] >> 4).astype(np.float32) - 8) * d[b]])
                              for b in range(k // 32)])
        for r in range(m):
            s = np.float32(0.0)
            for i in range(k):
                s = np.float32(s + np.float32(x[r * k + i] * dec[i]))
            assert got[r, c].view(np.uint32) == s.view(np.uint32)


def test_linear_invariants(oracle):
    from mote_amd import workloads as wl

    m, n, k = 2, 4, 256
    x = bits_to_f32(wl.normal_f16(31, m * k))
    w = wl.q4_0_weights(32, n, k)
    y = oracle.quantized_linear_f64(x, w, m, n, k)
    assert np.array_equal(oracle.quantized_linear_f64(2 * x, w, m, n, k), 2 * y)
    wneg = w.reshape(n, k // 32, 18).copy()
    wneg[:, :, 1] ^= 0x80
    assert np.array_equal(oracle.quantized_linear_f64(x, wneg.reshape(-1), m, n, k), -y)
    wz = w.reshape(n, k // 32, 18).copy()
    wz[:, 3, 0:2] = 0
    xz = x.reshape(m, k).copy()
    xz[:, 96:128] = 0
    assert np.allclose(oracle.quantized_linear_f64(x, wz.reshape(-1), m, n, k),
                       oracle.quantized_linear_f64(xz.reshape(-1), w, m, n, k), rtol=1e-14, atol=1e-14)
    # the f32 and f64 oracles agree to f32 summation error
    y32 = oracle.quantized_linear_f32(x, w, oracle.Q4_0, m, n, k).reshape(m, n)
    assert np.all(np.abs(y32 - y) <= 1e-5 * np.abs(x).sum() * 0.2)


def test_gate_up_silu_composition(oracle):
    from mote_amd import workloads as wl

    m, n, k = 3, 6, 128
    x = bits_to_f32(wl.normal_f16(41, m * k))
    g, u = wl.q4_0_weights(42, n, k), wl.q4_0_weights(43, n, k)
    yg = oracle.quantized_linear_f64(x, g, m, n, k)
    yu = oracle.quantized_linear_f64(x, u, m, n, k)
    want = yg / (1.0 + np.exp(-yg)) * yu
    assert np.allclose(oracle.gate_up_silu_f64(x, g, u, m, n, k), want, rtol=1e-15, atol=0)


def test_reference_test_fixture_generator(oracle):
    """The reference GPU test's closed-form fixture (quantized_linear.rs:160-177)
    regenerated here matches the committed golden bytes and expected output."""
    with open(os.path.join(GOLDEN, "q4_0_fixture_3x5x64.json"), encoding="utf-8") as f:
        g = json.load(f)
    w = ref_test_q4_0_weights(5, 64)
    x = ref_test_q4_0_inputs(3, 64)
    assert w.tolist() == g["weights"]
    assert x.tolist() == g["input_f16_bits"]
    got = oracle.quantized_linear_f32(bits_to_f32(x), w, oracle.Q4_0, 3, 5, 64)
    assert got.tolist() == g["expected_f32"]


# --- RoPE tables --------------------------------------------------------------------------

def test_rope_tables_closed_form(oracle):
    pos = np.array([0, 1, 7, 8191], np.int64)
    c, s = oracle.rope_tables(pos, 128, 500000.0)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    assert c[1, 0] == np.float32(math.cos(1.0)) and s[1, 0] == np.float32(math.sin(1.0))
    i = np.arange(64)
    inv = 500000.0 ** (-(2.0 * i) / 128.0)
    ang = pos[:, None].astype(np.float64) * inv[None, :]
    assert np.array_equal(c, np.cos(ang).astype(np.float32))
    assert np.array_equal(s, np.sin(ang).astype(np.float32))


def test_geometry(oracle):
    """crates/mote-types/src/lib.rs:48-73."""
    assert oracle.block_geometry(oracle.Q4_0) == (32, 18, 2)
    assert oracle.block_geometry(oracle.Q8_0) == (32, 34, 2)
    assert oracle.block_geometry(oracle.Q4_K) == (256, 144, 4)
    assert oracle.block_geometry(oracle.Q6_K) == (256, 210, 2)


def test_regression_vectors(oracle):
    """Small regression vectors written by tests/golden/make_golden.py from the
    oracle itself: they pin the oracle against later changes (not ground truth)."""
    from mote_amd import workloads as wl

    with open(os.path.join(GOLDEN, "oracle_regression.json"), encoding="utf-8") as f:
        g = json.load(f)
    for case in g["linear"]:
        m, n, k = case["m"], case["n"], case["k"]
        x = (wl.uniform_f16 if case["x"] == "uniform" else wl.normal_f16)(case["x_seed"], m * k)
        w = wl.q4_0_weights(case["w_seed"], n, k)
        assert hashlib.sha256(w.tobytes()).hexdigest() == case["w_sha256"]
        y = oracle.quantized_linear_f32(bits_to_f32(x), w, oracle.Q4_0, m, n, k)
        assert y.view(np.uint32).tolist() == case["y_f32_bits"]


@pytest.mark.parametrize("mode", ["full", "big", "subnormal", "special"])
def test_full_output_judge_matches_the_f64_linear(oracle, mode):
    """The BLAS float64 judge of the full-size GPU checks (oracle-decoded
    weights times the f16 activations) equals the oracle's sequential f64
    linear to 1e-13 of the absolute sum, on weights whose scales span the
    whole binary16 range; NaN where the oracle has NaN."""
    from helpers import linear_f64_full, wide_q4_0_weights, wide_q8_0_weights

    m, n, k = 3, 19, 512
    x = f16_bits(np.random.default_rng(3).standard_normal(m * k))
    for fmt, gen in ((oracle.Q4_0, wide_q4_0_weights), (oracle.Q8_0, wide_q8_0_weights)):
        w = gen(11, n, k, mode)
        got = linear_f64_full(oracle, x, w, m, n, k, fmt)
        want = oracle.quantized_linear_f64(bits_to_f32(x), w, m, n, k, fmt=fmt).reshape(m, n)
        assert np.array_equal(np.isnan(got), np.isnan(want))
        fin = ~np.isnan(want)
        absum = np.abs(bits_to_f32(x).astype(np.float64).reshape(m, k)) @ np.abs(
            oracle.dequantize_row(w, fmt, n * k).astype(np.float64).reshape(n, k)).T
        assert np.all(np.abs(got[fin] - want[fin]) <= 1e-13 * absum[fin])
