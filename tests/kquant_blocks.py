"""Q4_K / Q6_K super-block helpers for the tests: an encoder-side packer for
each format (the bit placement of GGML's quantize_row_q4_K_ref /
quantize_row_q6_K_ref, written from the encoder's side so that a decoder
index mistake does not cancel against it), random blocks, and the
exact-rational value of every element.

Q4_K (144 bytes): f16 d, f16 dmin, 12 scale bytes, 128 nibble bytes; 8
sub-blocks of 32 elements with 6-bit scale sc_j and min m_j, value
d sc_j q - dmin m_j.  Q6_K (210 bytes): ql[128], qh[64], int8 scales[16],
f16 d; 16 groups of 16 elements, value d scales[g] (q - 32), q in 0..63.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np

Q4_K_BYTES, Q6_K_BYTES, SUPER = 144, 210, 256


def pack_q4_k(d_bits: int, dmin_bits: int, sc, m, q) -> np.ndarray:
    """One Q4_K block from its parameters: sc, m (8 values in 0..63 each),
    q (256 nibbles in element order)."""
    sc, m, q = (np.asarray(v, dtype=np.int64) for v in (sc, m, q))
    assert sc.shape == (8,) and m.shape == (8,) and q.shape == (SUPER,)
    assert sc.min() >= 0 and sc.max() < 64 and m.min() >= 0 and m.max() < 64 and q.min() >= 0 and q.max() < 16
    s = np.zeros(12, dtype=np.int64)
    for j in range(8):
        if j < 4:
            s[j] |= sc[j]
            s[j + 4] |= m[j]
        else:
            s[j + 4] = (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (m[j] >> 4) << 6
    # element 64p + 32h + l -> nibble h of qs[32p + l]
    qp = q.reshape(4, 2, 32)
    qs = qp[:, 0, :] | (qp[:, 1, :] << 4)
    out = np.concatenate([
        np.array([d_bits & 0xFF, d_bits >> 8, dmin_bits & 0xFF, dmin_bits >> 8]),
        s,
        qs.reshape(-1),
    ]).astype(np.uint8)
    assert out.size == Q4_K_BYTES
    return out


def pack_q6_k(d_bits: int, scales, q) -> np.ndarray:
    """One Q6_K block from its parameters: scales (16 values in -128..127),
    q (256 values in 0..63, element order; the stored value is q - 32)."""
    scales, q = np.asarray(scales, dtype=np.int64), np.asarray(q, dtype=np.int64)
    assert scales.shape == (16,) and q.shape == (SUPER,)
    assert q.min() >= 0 and q.max() < 64 and scales.min() >= -128 and scales.max() < 128
    ql = np.zeros(128, dtype=np.int64)
    qh = np.zeros(64, dtype=np.int64)
    for half in range(2):
        L = q[128 * half: 128 * half + 128]
        lo, hi = L & 0xF, L >> 4
        ql[64 * half: 64 * half + 32] = lo[0:32] | (lo[64:96] << 4)
        ql[64 * half + 32: 64 * half + 64] = lo[32:64] | (lo[96:128] << 4)
        qh[32 * half: 32 * half + 32] = hi[0:32] | (hi[32:64] << 2) | (hi[64:96] << 4) | (hi[96:128] << 6)
    out = np.concatenate([ql, qh, scales & 0xFF, np.array([d_bits & 0xFF, d_bits >> 8])]).astype(np.uint8)
    assert out.size == Q6_K_BYTES
    return out


def _half(bits: int) -> Fraction:
    """Exact value of a finite binary16 pattern."""
    sign = -1 if bits & 0x8000 else 1
    e, f = (bits >> 10) & 0x1F, bits & 0x3FF
    assert e != 0x1F, "finite patterns only"
    if e == 0:
        return sign * Fraction(f, 1 << 24)
    return sign * Fraction(1024 + f, 1 << 10) * Fraction(2) ** (e - 15)


def round_f32(v: Fraction) -> float:
    """Round an exact value that is an integer multiple of 2^-24 with
    |v| < 2^40 to binary32, to nearest, ties to even (such values are never
    binary32 subnormals)."""
    n = v * (1 << 24)
    assert n.denominator == 1
    i = n.numerator
    sign = -1 if i < 0 else 1
    i = abs(i)
    if i == 0:
        return 0.0
    shift = max(0, i.bit_length() - 24)
    q, r = divmod(i, 1 << shift)
    half = 1 << shift >> 1 if shift else 0
    if shift and (r > half or (r == half and q & 1)):
        q += 1
    return sign * float(Fraction(q << shift, 1 << 24))


def q4_k_exact(d_bits: int, dmin_bits: int, sc, m, q) -> list[Fraction]:
    d, dmin = _half(d_bits), _half(dmin_bits)
    return [d * int(sc[e // 32]) * int(q[e]) - dmin * int(m[e // 32]) for e in range(SUPER)]


def q6_k_exact(d_bits: int, scales, q) -> list[Fraction]:
    d = _half(d_bits)
    return [d * int(scales[e // 16]) * (int(q[e]) - 32) for e in range(SUPER)]


def finite_half_bits(rng: np.random.Generator, count: int) -> np.ndarray:
    """Uniform over every finite binary16 pattern, both signs."""
    return ((rng.integers(0, 2, count) << 15) | rng.integers(0, 0x7C00, count)).astype(np.int64)


def random_q4_k(rng: np.random.Generator, blocks: int, scale_bits=None):
    """`blocks` Q4_K blocks with their parameters: (bytes, params list)."""
    out, params = [], []
    for b in range(blocks):
        if scale_bits is None:
            d_bits, dmin_bits = (int(v) for v in finite_half_bits(rng, 2))
        else:
            d_bits, dmin_bits = scale_bits(rng)
        sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        q = rng.integers(0, 16, SUPER)
        out.append(pack_q4_k(d_bits, dmin_bits, sc, m, q))
        params.append((d_bits, dmin_bits, sc, m, q))
    return np.concatenate(out), params


def random_q6_k(rng: np.random.Generator, blocks: int, scale_bits=None):
    out, params = [], []
    for b in range(blocks):
        d_bits = int(finite_half_bits(rng, 1)[0]) if scale_bits is None else scale_bits(rng)
        scales = rng.integers(-128, 128, 16)
        q = rng.integers(0, 64, SUPER)
        out.append(pack_q6_k(d_bits, scales, q))
        params.append((d_bits, scales, q))
    return np.concatenate(out), params
