"""Shared test helpers: the reference's closed-form fixture generators, binary16
utilities, the parity tolerance, and GPU round-trip helpers."""

from __future__ import annotations

import math

import numpy as np

BLOCK_ELEMENTS = 32
BLOCK_BYTES = 18


def f16_bits(values) -> np.ndarray:
    """Round to binary16 (RNE, numpy) and return the bit patterns."""
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def bits_to_f32(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def row_bytes(k: int) -> int:
    return (k // BLOCK_ELEMENTS) * BLOCK_BYTES


# --- closed-form fixtures of the reference tests ---------------------------

def ref_test_q4_0_weights(n: int, k: int) -> np.ndarray:
    """crates/mote-backend-hip/tests/quantized_linear.rs:160-177."""
    out = bytearray()
    for o in range(n):
        for b in range(k // 32):
            scale = np.float16(0.125 * ((o + b) % 4 + 1)).view(np.uint16)
            out += int(scale).to_bytes(2, "little")
            for j in range(16):
                low = (o * 3 + b * 5 + j) % 16
                high = (o * 7 + b * 2 + j * 3 + 1) % 16
                out.append(low | (high << 4))
    return np.frombuffer(bytes(out), dtype=np.uint8).copy()


def ref_test_q4_0_inputs(rows: int, k: int) -> np.ndarray:
    """crates/mote-backend-hip/tests/quantized_linear.rs:16-18 (f16 bits)."""
    i = np.arange(rows * k)
    return f16_bits((i % 23).astype(np.float32) / 7.0 - 1.5)


def ref_bench_q4_0_weights(n: int, k: int) -> np.ndarray:
    """crates/mote-backend-hip/benches/quantized_linear.rs:134-152 (the
    generator the benchmark shares, mote_amd.workloads)."""
    from mote_amd.workloads import reference_bench_q4_0_weights

    return reference_bench_q4_0_weights(n, k)


def ref_bench_q4_0_inputs(rows: int, k: int) -> np.ndarray:
    """crates/mote-backend-hip/benches/quantized_linear.rs:128-132."""
    from mote_amd.workloads import reference_bench_inputs

    return reference_bench_inputs(rows, k)


def ref_norm_input(count: int) -> np.ndarray:
    """crates/mote-backend-hip/tests/rms_norm.rs:161-163 (also rope.rs:456-458)."""
    i = np.arange(count)
    return f16_bits(((i * 37 + 5) % 19).astype(np.float32) / 6.0 - 1.5)


def ref_norm_weight(count: int) -> np.ndarray:
    """crates/mote-backend-hip/tests/rms_norm.rs:165-167."""
    i = np.arange(count)
    return f16_bits(0.5 + ((i * 7 + 3) % 13).astype(np.float32) / 12.0)


def ref_residual(count: int) -> np.ndarray:
    """crates/mote-backend-hip/tests/fused_add_rms_norm.rs:485-487."""
    i = np.arange(count)
    return f16_bits(((i * 11 + 7) % 23).astype(np.float32) / 8.0 - 1.4)


def ref_rope_cos(count: int) -> np.ndarray:
    """crates/mote-backend-hip/tests/rope.rs:460-462."""
    i = np.arange(count)
    return ((i * 11 + 3) % 13).astype(np.float32) / 12.0


def ref_rope_sin(count: int) -> np.ndarray:
    """crates/mote-backend-hip/tests/rope.rs:464-466."""
    i = np.arange(count)
    return ((i * 7 + 1) % 17).astype(np.float32) / 16.0


# --- Q4_0 facts used by the checks -------------------------------------------

def q4_0_scales(w: np.ndarray, n: int, k: int) -> np.ndarray:
    blocks = w.reshape(n, k // 32, BLOCK_BYTES)
    return bits_to_f32(blocks[:, :, 0:2].copy().view("<u2")[..., 0])


def linear_tolerance(y64: np.ndarray, k: int, max_d: float, max_x: float) -> np.ndarray:
    """Per-element bound of the parity criterion: an element passes if
    |y - y64| <= 1e-3 |y64| or |y - y64| <= 2e-3 sqrt(K) max|d| max|x|."""
    return np.maximum(1e-3 * np.abs(y64), 2e-3 * math.sqrt(k) * max_d * max_x)


def assert_linear_close(y, y64, k, max_d, max_x, extra_rel: float = 0.0, what: str = "output"):
    y = np.asarray(y, dtype=np.float64)
    y64 = np.asarray(y64, dtype=np.float64)
    assert y.shape == y64.shape, (y.shape, y64.shape)
    tol = linear_tolerance(y64, k, max_d, max_x) + extra_rel * np.abs(y64)
    err = np.abs(y - y64)
    bad = ~(err <= tol)
    if bad.any():
        idx = np.argwhere(bad)[:5]
        details = ", ".join(f"{tuple(i)}: got {y[tuple(i)]!r} want {y64[tuple(i)]!r}" for i in idx)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} elements out of tolerance; {details}")


# --- weights whose scales span the binary16 range ------------------------------

def wide_scale_bits(rng: np.random.Generator, count: int, mode: str, big_limit: int) -> np.ndarray:
    """`count` binary16 scale patterns, both signs:
    * "full": magnitude field uniform over every finite pattern (subnormals
      from 2^-24 up to 65504);
    * "big": every magnitude from `big_limit` (the first binary16 whose
      products can overflow) up to 65504;
    * "subnormal": nonzero subnormals only;
    * "special": "full" with one pattern in 64 replaced by +inf, -inf or NaN."""
    sign = (rng.integers(0, 2, count) << 15).astype(np.uint32)
    if mode in ("full", "special"):
        mag = rng.integers(1, 0x7C00, count)
    elif mode == "big":
        mag = rng.integers(big_limit, 0x7C00, count)
    elif mode == "subnormal":
        mag = rng.integers(1, 0x0400, count)
    else:
        raise ValueError(mode)
    bits = (sign | mag.astype(np.uint32)).astype(np.uint16)
    if mode == "special":
        idx = rng.choice(count, size=max(1, count // 64), replace=False)
        bits[idx] = rng.choice(np.array([0x7C00, 0xFC00, 0x7E00], dtype=np.uint16), size=idx.size)
    return bits


def wide_q4_0_weights(seed: int, n: int, k: int, mode: str) -> np.ndarray:
    """Q4_0 [n, k] with uniform nibbles and scales from wide_scale_bits
    (products overflow binary16 from |d| = 8192, pattern 0x7000)."""
    rng = np.random.default_rng(seed)
    blocks = n * (k // 32)
    out = np.empty((blocks, 18), dtype=np.uint8)
    out[:, 0:2] = wide_scale_bits(rng, blocks, mode, 0x7000).astype("<u2").view(np.uint8).reshape(blocks, 2)
    out[:, 2:] = rng.integers(0, 256, (blocks, 16), dtype=np.uint8)
    return out.reshape(-1)


def wide_q8_0_weights(seed: int, n: int, k: int, mode: str) -> np.ndarray:
    """Q8_0 [n, k] with uniform bytes and scales from wide_scale_bits
    (products overflow binary16 from |d| = 512, pattern 0x6000)."""
    rng = np.random.default_rng(seed)
    blocks = n * (k // 32)
    out = np.empty((blocks, 34), dtype=np.uint8)
    out[:, 0:2] = wide_scale_bits(rng, blocks, mode, 0x6000).astype("<u2").view(np.uint8).reshape(blocks, 2)
    out[:, 2:] = rng.integers(0, 256, (blocks, 32), dtype=np.uint8)
    return out.reshape(-1)


def block_scales(w: np.ndarray, n: int, k: int, block_bytes: int = BLOCK_BYTES) -> np.ndarray:
    """The f32 value of every block's scale, [n, k / 32]."""
    blocks = w.reshape(n, k // 32, block_bytes)
    return bits_to_f32(blocks[:, :, 0:2].copy().view("<u2")[..., 0])


# --- full-output f64 judge ---------------------------------------------------------

_DECODED: dict = {}


def decoded_f64(oracle, w: np.ndarray, n: int, k: int, fmt: int) -> np.ndarray:
    """The weights decoded by the oracle's block decoder (bit-exact, pinned by
    its own tests) as float64 [n, k].  The matrix is one run of whole blocks,
    so it decodes as one long row.  A few matrices are kept for reuse."""
    key = (w.ctypes.data, w.nbytes, n, k, fmt)
    hit = _DECODED.get(key)
    if hit is not None and hit[0] is w:  # the entry holds `w`, so its address cannot be reused
        return hit[1]
    if len(_DECODED) >= 4:
        _DECODED.pop(next(iter(_DECODED)))
    decoded = oracle.dequantize_row(w, fmt, n * k).astype(np.float64).reshape(n, k)
    _DECODED[key] = (w, decoded)
    return decoded


def linear_f64_full(oracle, x_bits: np.ndarray, w: np.ndarray, m: int, n: int, k: int, fmt: int) -> np.ndarray:
    """Every output of the linear in float64: the f16 activations times the
    oracle-decoded weights (each product exact in binary64), summed by the
    host BLAS, whose rounding (about K 2^-53 of the absolute sum) is many
    orders below the parity tolerance.  A CPU test holds it to the oracle's
    own f64 linear."""
    x64 = bits_to_f32(x_bits).astype(np.float64).reshape(m, k)
    with np.errstate(invalid="ignore", over="ignore"):  # inf and NaN scales give NaN, as in the oracle
        return x64 @ decoded_f64(oracle, w, n, k, fmt).T
