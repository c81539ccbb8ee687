"""GPU parity of the Q4_K / Q6_K kernels, called through the C ABI.

Decode (mote_hip_dequantize_q{4,6}_k_f32) must be bit-identical to the
oracle's GGML decode, which tests/test_kquant_oracle.py pins (hand-derived
known-answer blocks, exact-rational element values, an encoder-side packer):
every finite binary16 d and dmin, inf and NaN scales, Q6_K blocks at 2-byte
offsets, unaligned outputs.

The linears are judged on every output against the oracle's f64 linear over
the oracle-decoded weights: |y - y64| <= 1e-3 |y64| or
<= 2.5e-4 sqrt(K) max|w| max|x|, the Q4_0 bound (2e-3 sqrt(K) max|d| max|x|
with |w| <= 8 |d|) written in terms of the largest decoded weight; f16
outputs get 2^-11 |y64| more.  Parity against the reference is unpinned (the
reference has no oracle for these formats,
crates/mote-reference/src/quantized.rs:154-156).
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from helpers import bits_to_f32
from kquant_blocks import Q4_K_BYTES, Q6_K_BYTES, SUPER, random_q4_k, random_q6_k
from mote_amd import ops, workloads as wl
from mote_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu

FORMATS = {
    "q4_k": (Q4_K_BYTES, ops.dequantize_q4_k_f32, ops.quantized_linear_q4_k_f32, ops.quantized_linear_q4_k_f16),
    "q6_k": (Q6_K_BYTES, ops.dequantize_q6_k_f32, ops.quantized_linear_q6_k_f32, ops.quantized_linear_q6_k_f16),
}


def _fmt(oracle, name):
    return oracle.Q4_K if name == "q4_k" else oracle.Q6_K


def _blocks(name, seed, count, scale_bits=None):
    rng = np.random.default_rng(seed)
    return (random_q4_k if name == "q4_k" else random_q6_k)(rng, count, scale_bits)[0]


def _decode_gpu(stream, name, w, rows, k, w_offset=0, out_offset=0):
    wb = DeviceBuffer(w.nbytes + w_offset)
    wb.upload(w, offset=w_offset)
    ob = DeviceBuffer(rows * k * 4 + out_offset)
    ob.upload(np.full(rows * k * 4 + out_offset, 0xA5, dtype=np.uint8))
    FORMATS[name][1](wb.ptr + w_offset, ob.ptr + out_offset, rows, k, stream)
    stream.synchronize()
    return ob.download(np.uint8, offset=out_offset).view(np.float32)


def _same_bits(got, want):
    """Bit-identical, NaN payloads aside (any NaN matches any NaN)."""
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"NaN positions differ ({int((gn != wn).sum())})"
    g, w = got[~gn].view(np.uint32), want[~wn].view(np.uint32)
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, f"{bad.size} elements differ, first at {bad[0]}: {got[~gn][bad[0]]} vs {want[~wn][bad[0]]}"


@pytest.mark.parametrize("name", list(FORMATS))
def test_decode_every_finite_scale(stream, oracle, name):
    rows, k = 24, 2048
    w = _blocks(name, 501 if name == "q4_k" else 502, rows * k // SUPER)
    got = _decode_gpu(stream, name, w, rows, k)
    want = oracle.dequantize_kquant_row(w, _fmt(oracle, name), rows * k)
    _same_bits(got, want)


@pytest.mark.parametrize("name", list(FORMATS))
def test_decode_special_scales(stream, oracle, name):
    """One block in four with an inf, -inf or NaN d (and dmin for Q4_K)."""
    specials = [0x7C00, 0xFC00, 0x7E00, 0x3C00]

    def bits(r):
        if name == "q4_k":
            return int(r.choice(specials)), int(r.choice(specials))
        return int(r.choice(specials))

    rows, k = 8, 1024
    w = _blocks(name, 503, rows * k // SUPER, bits)
    got = _decode_gpu(stream, name, w, rows, k)
    _same_bits(got, oracle.dequantize_kquant_row(w, _fmt(oracle, name), rows * k))


@pytest.mark.parametrize("name,w_offset,out_offset", [("q4_k", 4, 4), ("q6_k", 2, 4), ("q6_k", 6, 8)])
def test_decode_offsets(stream, oracle, name, w_offset, out_offset):
    """Weights at their format's minimum alignment (Q6_K rows of 3 blocks
    start at alternating 2 and 0 mod 4), outputs off the 16-byte grid."""
    rows, k = 5, 768
    w = _blocks(name, 504 + w_offset, rows * k // SUPER)
    got = _decode_gpu(stream, name, w, rows, k, w_offset, out_offset)
    _same_bits(got, oracle.dequantize_kquant_row(w, _fmt(oracle, name), rows * k))


def _judge(oracle, name, x_bits, w, m, n, k):
    fmt = _fmt(oracle, name)
    x32 = bits_to_f32(x_bits)
    y64 = oracle.kquant_linear_f64(x32, w, fmt, m, n, k)
    max_w = float(np.abs(oracle.dequantize_kquant_row(w, fmt, n * k)).max())
    max_x = float(np.abs(x32).max())
    return y64, max_w, max_x


def _run(stream, name, x_bits, w, m, n, k, f16_out=False, w_offset=0, x_offset=0):
    xb = DeviceBuffer(x_bits.nbytes + x_offset)
    xb.upload(x_bits, offset=x_offset)
    wb = DeviceBuffer(w.nbytes + w_offset)
    wb.upload(w, offset=w_offset)
    out_bytes = m * n * (2 if f16_out else 4)
    yb = DeviceBuffer(out_bytes)
    yb.upload(np.full(out_bytes, 0xA5, dtype=np.uint8))  # sentinel: every element must be written
    FORMATS[name][3 if f16_out else 2](xb.ptr + x_offset, wb.ptr + w_offset, yb.ptr, m, n, k, stream)
    stream.synchronize()
    y = yb.download(np.uint16 if f16_out else np.float32)
    return (bits_to_f32(y) if f16_out else y).reshape(m, n).astype(np.float64)


def _check(y, y64, k, max_w, max_x, extra_rel=0.0, what=""):
    tol = np.maximum(1e-3 * np.abs(y64), 2.5e-4 * math.sqrt(k) * max_w * max_x) + extra_rel * np.abs(y64)
    err = np.abs(y - y64)
    bad = ~(err <= tol)
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} out of tolerance, worst {float((err - tol).max())}"


SHAPES = [
    # (M, N, K): ragged N against the 8-row groups, every token-group width,
    # K of one block, odd block counts (Q6_K rows at 2 mod 4), and K past
    # one LDS chunk for multi-token groups
    (1, 7, 256),
    (1, 100, 768),
    (1, 4096, 4096),
    (2, 33, 1280),
    (3, 64, 4096),
    (4, 130, 2304),
    (5, 9, 512),
    (8, 200, 4096),
    (9, 17, 3840),
    (17, 24, 1024),
    (2, 96, 14336),
    (8, 40, 14336),
    (1, 24, 36864),
    # the ring kernel's K slices: 2, 4 and 8 ways, Q6_K slices padded to 8
    # blocks (10 blocks per slice -> an empty fourth slice at K = 10240)
    (1, 33, 8192),
    (3, 70, 10240),
    (2, 45, 20480),
    (1, 18, 28672),
    (4, 1000, 4096),
    (5, 12, 6144),
    # the matrix-core tiles (2 for Q4_K, 3 past K = 4096, 5 for Q6_K, to 64
    # tokens):
    # four full 16-token tiles, and two and a bit over odd-block rows (Q6_K
    # rows at 2 mod 4: the five-dword reads)
    (64, 40, 4096),
    (33, 50, 2304),
    # split K (parts of 16 super-blocks): four parts, a short last part of one
    # block over odd-block rows, and nine parts (Q6_K rows of whole 16-byte
    # units at K % 2048 == 0, five-dword reads otherwise)
    (64, 40, 14336),
    (21, 30, 8448),
    (16, 20, 36864),
]


@pytest.mark.parametrize("name", list(FORMATS))
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_linear(stream, oracle, name, m, n, k):
    seed = 600 + m * 7 + n + k
    w = (wl.q4_k_weights if name == "q4_k" else wl.q6_k_weights)(seed, n, k)
    x = wl.normal_f16(wl.seed_for(31, seed), m * k)
    y64, max_w, max_x = _judge(oracle, name, x, w, m, n, k)
    y = _run(stream, name, x, w, m, n, k)
    _check(y, y64, k, max_w, max_x, what=f"{name} {m}x{n}x{k} f32")
    y16 = _run(stream, name, x, w, m, n, k, f16_out=True)
    _check(y16, y64, k, max_w, max_x, 2.0 ** -11, what=f"{name} {m}x{n}x{k} f16")


@pytest.mark.parametrize("name", list(FORMATS))
@pytest.mark.parametrize("m,n,k", [(1, 300, 4096), (2, 64, 14336), (4, 50, 8192), (3, 20, 2048)])
def test_linear_unaligned_activations(stream, oracle, name, m, n, k):
    """Activations off the 16-byte grid take the LDS-staged kernel instead of
    the ring kernel (which loads a lane's activations 16 bytes at a time):
    the same shapes judged the same way."""
    seed = 700 + m + n + k
    w = (wl.q4_k_weights if name == "q4_k" else wl.q6_k_weights)(seed, n, k)
    x = wl.normal_f16(wl.seed_for(34, seed), m * k)
    y64, max_w, max_x = _judge(oracle, name, x, w, m, n, k)
    _check(_run(stream, name, x, w, m, n, k, x_offset=2), y64, k, max_w, max_x, what=f"{name} x at 2 mod 16")


@pytest.mark.parametrize("name", list(FORMATS))
@pytest.mark.parametrize("m,k", [(3, 1536), (20, 8192)])
def test_linear_every_finite_scale(stream, oracle, name, m, k):
    """Scales over every finite binary16 magnitude, subnormal to 65504 (the
    kernel computes in f32: no binary16 product can overflow), also through
    the split-K tiles."""
    n = 40
    w = _blocks(name, 610 + k, n * k // SUPER)
    x = wl.normal_f16(wl.seed_for(32, 1), m * k)
    y64, max_w, max_x = _judge(oracle, name, x, w, m, n, k)
    assert np.isfinite(y64).all()
    _check(_run(stream, name, x, w, m, n, k), y64, k, max_w, max_x, what=f"{name} wide scales")


@pytest.mark.parametrize("name", list(FORMATS))
@pytest.mark.parametrize("m", [2, 6, 20])
def test_linear_non_finite_activations(stream, oracle, name, m):
    """inf, -inf and NaN activations in different K parts of different tokens
    (K = 12288: three parts on the split-K tiles; the ring for Q6_K at 2
    tokens): those tokens' outputs are what the f64 definition gives (+-inf
    where one infinity meets nonzero weights, NaN where it meets a zero weight
    or a NaN), every other output is judged as usual."""
    n, k = 24, 12288
    w = (wl.q4_k_weights if name == "q4_k" else wl.q6_k_weights)(620 + m, n, k)
    x = wl.normal_f16(wl.seed_for(35, m), m * k).copy()
    x[5000] = 0x7C00  # token 0, part 1: +inf
    x[(m - 1) * k + 9000] = 0xFC00  # the last token, part 2: -inf
    if m > 2:
        x[k + 100] = 0x7E00  # token 1, part 0: NaN
    y64 = oracle.kquant_linear_f64(bits_to_f32(x), w, _fmt(oracle, name), m, n, k)
    finite_x = bits_to_f32(x)[np.isfinite(bits_to_f32(x))]
    max_w = float(np.abs(oracle.dequantize_kquant_row(w, _fmt(oracle, name), n * k)).max())
    for f16_out in (False, True):
        y = _run(stream, name, x, w, m, n, k, f16_out=f16_out)
        for cls in (np.isnan, np.isposinf, np.isneginf):
            assert np.array_equal(cls(y), cls(y64)), f"{name} {m} tokens: {cls.__name__} positions differ"
        assert not np.isfinite(y64[0]).any() and not np.isfinite(y64[m - 1]).any()
        ok = np.isfinite(y64)
        _check(y[ok], y64[ok], k, max_w, float(np.abs(finite_x).max()), 2.0 ** -11 if f16_out else 0.0,
               what=f"{name} {m} tokens, finite outputs")


def test_q6_k_weights_at_two_byte_offset(stream, oracle):
    m, n, k = 2, 50, 1280
    w = wl.q6_k_weights(611, n, k)
    x = wl.normal_f16(wl.seed_for(33, 1), m * k)
    y64, max_w, max_x = _judge(oracle, "q6_k", x, w, m, n, k)
    _check(_run(stream, "q6_k", x, w, m, n, k, w_offset=2), y64, k, max_w, max_x, what="q6_k at 2 mod 4")


@pytest.mark.parametrize("name", list(FORMATS))
def test_linear_k0_writes_zeros(stream, name):
    yb = DeviceBuffer(3 * 5 * 4)
    yb.upload(np.full(60, 0xA5, dtype=np.uint8))
    xb, wb = DeviceBuffer(16), DeviceBuffer(16)
    FORMATS[name][2](xb.ptr, wb.ptr, yb.ptr, 3, 5, 0, stream)
    stream.synchronize()
    assert np.array_equal(yb.download(np.float32), np.zeros(15, np.float32))
