"""Pins the oracle's Q4_K / Q6_K decode (ggml-common.h block_q4_K / block_q6_K,
ggml-quants.c dequantize_row_q4_K / dequantize_row_q6_K).

The reference has the geometry of these formats only
(crates/mote-types/src/lib.rs:39-74) and its oracle rejects them
(crates/mote-reference/src/quantized.rs:154-156), so there are no reference
vectors: parity against the reference is unpinned.  The oracle is pinned
instead by
* known-answer blocks whose bytes and decoded values were worked out by hand
  from the GGML definition (sub-block scales and mins in both halves of the
  12-byte field, every nibble / bit-pair position class of Q6_K, a negative
  Q6_K scale);
* the exact-rational value of every element of random blocks over all finite
  binary16 scales: Q4_K rounds d sc q - dmin m once to binary32 (d sc, dmin m
  and d sc q are exact in binary32), Q6_K is exact (at most 11 + 7 + 5
  significant bits);
* decode(pack(parameters)) against the parameters, with the packer written
  from the encoder's side (quantize_row_q*_K_ref's bit placement), over every
  6-bit scale and min in every sub-block slot.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from kquant_blocks import (
    SUPER,
    pack_q4_k,
    pack_q6_k,
    q4_k_exact,
    q6_k_exact,
    random_q4_k,
    random_q6_k,
    round_f32,
)


def _decode(fmt, data, elements):
    if isinstance(data, bytes):
        data = np.frombuffer(data, dtype=np.uint8)
    return oracle.dequantize_kquant_row(np.asarray(data, dtype=np.uint8), fmt, elements)


def test_geometry_matches_the_reference():
    # crates/mote-types/src/lib.rs:48-73
    assert oracle.block_geometry(oracle.Q4_K) == (256, 144, 4)
    assert oracle.block_geometry(oracle.Q6_K) == (256, 210, 2)


def test_reference_oracle_functions_still_reject_k_quants():
    # crates/mote-reference/src/quantized.rs:154-156: UnsupportedFormat
    for fmt in (oracle.Q4_K, oracle.Q6_K):
        with pytest.raises(oracle.OracleError) as e:
            oracle.dequantize_row(np.zeros(oracle.block_geometry(fmt)[1], np.uint8), fmt, 256)
        assert e.value.kind == "UnsupportedFormat"


def test_q4_k_known_answer_low_scale_bytes():
    """sc = 1..8, m = 0,1,0,1,...; d = 1, dmin = 0.5; every qs byte 0x21
    (low nibble 1, high nibble 2).  Scales of sub-blocks 4..7 sit in the
    nibbles of bytes 8..11, mins 4..7 in their high nibbles."""
    block = bytes([0x00, 0x3C, 0x00, 0x38,
                   1, 2, 3, 4, 0, 1, 0, 1, 0x05, 0x16, 0x07, 0x18]) + bytes([0x21]) * 128
    want = np.repeat(np.array([1.0, 3.5, 3.0, 7.5, 5.0, 11.5, 7.0, 15.5], np.float32), 32)
    np.testing.assert_array_equal(_decode(oracle.Q4_K, block, 256), want)


def test_q4_k_known_answer_high_scale_bits():
    """sc_0 = 1, sc_4 = 63 (low bits 0xF in byte 8, high bits 3 in byte 0's
    top two), m_7 = 42 (low bits 0xA in byte 11's high nibble, high bits 2
    in byte 7's top two); d = 2, dmin = 0.25; qs[32p + l] = (l % 16) |
    (15 - l % 16) << 4."""
    scales = [0xC1, 0, 0, 0, 0, 0, 0, 0x80, 0x0F, 0, 0, 0xA0]
    qs = [(l % 16) | ((15 - l % 16) << 4) for _ in range(4) for l in range(32)]
    block = bytes([0x00, 0x40, 0x00, 0x34] + scales + qs)
    l16 = np.arange(32) % 16
    want = np.concatenate([
        2.0 * l16,              # sub-block 0: d 1 q
        np.zeros(32),           # 1: sc = m = 0
        np.zeros(64),           # 2, 3
        126.0 * l16,            # 4: d 63 q
        np.zeros(32),           # 5
        np.zeros(32),           # 6
        np.full(32, -10.5),     # 7: 0 q - dmin 42
    ]).astype(np.float32)
    np.testing.assert_array_equal(_decode(oracle.Q4_K, block, 256), want)


def test_q6_k_known_answer():
    """d = 0.5, scales[i] = i + 1 except scales[15] = -3; ql[0] = 0x21,
    ql[32] = 0x43, ql[64] = 0x65, ql[96] = 0x87, qh[0] = 0xE4, qh[32] = 0x1B,
    every other byte 0 (value 0 - 32 = -32)."""
    ql = [0] * 128
    ql[0], ql[32], ql[64], ql[96] = 0x21, 0x43, 0x65, 0x87
    qh = [0] * 64
    qh[0], qh[32] = 0xE4, 0x1B
    sc = list(range(1, 16)) + [0xFD]
    block = bytes(ql + qh + sc + [0x00, 0x38])
    scales = np.array(list(range(1, 16)) + [-3], np.float32)
    want = -16.0 * scales[np.arange(256) // 16]
    # q = ql nibble | qh bit pair << 4, minus 32, times d scales[e / 16]
    want[0] = 0.5 * 1 * (1 - 32)             # ql[0] low 1, qh[0] bits 0-1 = 0
    want[32] = 0.5 * 3 * ((3 | 1 << 4) - 32)   # ql[32] low 3, qh[0] bits 2-3 = 1
    want[64] = 0.5 * 5 * ((2 | 2 << 4) - 32)   # ql[0] high 2, qh[0] bits 4-5 = 2
    want[96] = 0.5 * 7 * ((4 | 3 << 4) - 32)   # ql[32] high 4, qh[0] bits 6-7 = 3
    want[128] = 0.5 * 9 * ((5 | 3 << 4) - 32)  # second half: ql[64], qh[32]
    want[160] = 0.5 * 11 * ((7 | 2 << 4) - 32)
    want[192] = 0.5 * 13 * ((6 | 1 << 4) - 32)
    want[224] = 0.5 * 15 * ((8 | 0 << 4) - 32)
    assert want[240] == 48.0  # the negative scale: 0.5 * -3 * -32
    np.testing.assert_array_equal(_decode(oracle.Q6_K, block, 256), want.astype(np.float32))


def test_q4_k_every_element_is_the_rounded_exact_value():
    rng = np.random.default_rng(401)
    data, params = random_q4_k(rng, 48)
    got = _decode(oracle.Q4_K, data, 48 * SUPER)
    for b, p in enumerate(params):
        want = np.array([round_f32(v) for v in q4_k_exact(*p)], dtype=np.float32)
        np.testing.assert_array_equal(got[b * SUPER:(b + 1) * SUPER], want, err_msg=f"block {b}")


def test_q4_k_rounding_is_a_single_rounding():
    """A block whose values need rounding (d sc q and dmin m of very
    different magnitude): d sc, dmin m and d sc q are exact in binary32, so
    the subtraction is the one rounding, to nearest even, of the exact
    value."""
    d_bits, dmin_bits = 0x7BFF, 0x0001  # 65504 and 2^-24
    sc, m = np.full(8, 63), np.full(8, 63)
    q = np.arange(256) % 16
    got = _decode(oracle.Q4_K, pack_q4_k(d_bits, dmin_bits, sc, m, q), 256)
    want = np.array([round_f32(v) for v in q4_k_exact(d_bits, dmin_bits, sc, m, q)], dtype=np.float32)
    np.testing.assert_array_equal(got, want)
    assert not all(float(v) == float(np.float32(float(v))) for v in q4_k_exact(d_bits, dmin_bits, sc, m, q))


def test_q6_k_every_element_is_exact():
    rng = np.random.default_rng(402)
    data, params = random_q6_k(rng, 48)
    got = _decode(oracle.Q6_K, data, 48 * SUPER)
    for b, p in enumerate(params):
        exact = q6_k_exact(*p)
        assert all(np.float64(np.float32(float(v))) == v for v in exact)  # representable
        np.testing.assert_array_equal(got[b * SUPER:(b + 1) * SUPER], np.array([float(v) for v in exact], np.float32))


@pytest.mark.parametrize("slot", range(8))
def test_q4_k_every_scale_and_min_in_every_slot(slot):
    """Only sub-block `slot` carries a scale and a min, each of the 64
    values: the decode sees them in that sub-block and nowhere else."""
    q = np.arange(256) % 16
    blocks, want = [], []
    for v in range(64):
        sc, m = np.zeros(8, np.int64), np.zeros(8, np.int64)
        sc[slot], m[slot] = v, 63 - v
        blocks.append(pack_q4_k(0x3C00, 0x3800, sc, m, q))  # d = 1, dmin = 0.5
        w = np.zeros(256)
        e = slice(32 * slot, 32 * slot + 32)
        w[e] = v * q[e] - 0.5 * (63 - v)
        want.append(w)
    got = _decode(oracle.Q4_K, np.concatenate(blocks), 64 * SUPER)
    np.testing.assert_array_equal(got, np.concatenate(want).astype(np.float32))


def test_q6_k_every_position():
    """One element at a time carries the value 63 (all other 0): each of the
    256 positions decodes at its own index with its own group's scale."""
    scales = np.arange(16) - 8
    blocks, want = [], []
    for e in range(256):
        q = np.zeros(256, np.int64)
        q[e] = 63
        blocks.append(pack_q6_k(0x3C00, scales, q))
        w = (-32.0 * scales[np.arange(256) // 16]).astype(np.float64)
        w[e] = 31.0 * scales[e // 16]
        want.append(w)
    got = _decode(oracle.Q6_K, np.concatenate(blocks), 256 * SUPER)
    np.testing.assert_array_equal(got, np.concatenate(want).astype(np.float32))


def test_special_scales():
    """inf and NaN scales follow IEEE arithmetic: NaN d -> every element NaN;
    +inf d with sc q > 0 -> +inf; sc q = 0 -> inf * 0 = NaN."""
    q = np.arange(256) % 16
    sc, m = np.full(8, 1), np.zeros(8, np.int64)
    got = _decode(oracle.Q4_K, pack_q4_k(0x7E00, 0x3C00, sc, m, q), 256)
    assert np.isnan(got).all()
    got = _decode(oracle.Q4_K, pack_q4_k(0x7C00, 0x3C00, sc, m, q), 256)
    assert np.array_equal(np.isnan(got), q == 0) and np.all(got[q > 0] == np.inf)
    got = _decode(oracle.Q6_K, pack_q6_k(0xFC00, np.full(16, 2), np.arange(256) % 64), 256)
    vals = np.arange(256) % 64 - 32
    assert np.array_equal(np.isnan(got), vals == 0)
    assert np.all(got[vals > 0] == -np.inf) and np.all(got[vals < 0] == np.inf)


def test_rejections():
    with pytest.raises(oracle.OracleError):
        _decode(oracle.Q4_K, np.zeros(144, np.uint8), 128)  # K % 256
    with pytest.raises(oracle.OracleError):
        _decode(oracle.Q6_K, np.zeros(209, np.uint8), 256)  # byte length
    with pytest.raises(oracle.OracleError):
        _decode(oracle.Q4_0, np.zeros(144, np.uint8), 256)  # not a K-quant


@pytest.mark.parametrize("fmt", [oracle.Q4_K, oracle.Q6_K])
def test_linear_f64_is_the_exact_sum_on_tiny_inputs(fmt):
    """Brute force: every output of a 3 x 4 x 512 problem against the exact
    rational sum of x w over the exactly decoded weights (the f64 judge may
    differ by its summation rounding only)."""
    from fractions import Fraction

    rng = np.random.default_rng(403 + fmt)
    n, k, rows = 4, 512, 3
    if fmt == oracle.Q4_K:
        w, params = random_q4_k(rng, n * k // SUPER, lambda r: (0x2C00 + int(r.integers(0, 0x400)), 0x2400))
        exact = [v for p in params for v in q4_k_exact(*p)]
    else:
        w, params = random_q6_k(rng, n * k // SUPER, lambda r: 0x2000 + int(r.integers(0, 0x400)))
        exact = [v for p in params for v in q6_k_exact(*p)]
    x = rng.standard_normal(rows * k).astype(np.float16).astype(np.float32)
    got = oracle.kquant_linear_f64(x, w, fmt, rows, n, k)
    for r in range(rows):
        for c in range(n):
            ws = exact[c * k:(c + 1) * k]
            # the oracle decodes in f32: Q4_K elements round once
            wf = [Fraction(round_f32(v)) for v in ws]
            s = sum(Fraction(float(x[r * k + i])) * wf[i] for i in range(k))
            bound = sum(abs(Fraction(float(x[r * k + i])) * wf[i]) for i in range(k))
            assert abs(Fraction(got[r, c]) - s) <= bound * Fraction(k, 1 << 52), (r, c)
