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
    """crates/mote-backend-hip/benches/quantized_linear.rs:134-152 (vectorised)."""
    blocks = k // 32
    o = np.arange(n)[:, None]
    b = np.arange(blocks)[None, :]
    scale = f16_bits(0.015625 * (((o * 3 + b) % 4) + 1).astype(np.float32))
    out = np.empty((n, blocks, BLOCK_BYTES), dtype=np.uint8)
    out[:, :, 0:2] = scale.astype("<u2").view(np.uint8).reshape(n, blocks, 2)
    j = np.arange(16)[None, None, :]
    low = (o[:, :, None] * 5 + b[:, :, None] * 3 + j) % 16
    high = (o[:, :, None] * 7 + b[:, :, None] + j * 3 + 1) % 16
    out[:, :, 2:] = (low | (high << 4)).astype(np.uint8)
    return out.reshape(-1)


def ref_bench_q4_0_inputs(rows: int, k: int) -> np.ndarray:
    """crates/mote-backend-hip/benches/quantized_linear.rs:128-132."""
    i = np.arange(rows * k)
    return f16_bits((i % 29).astype(np.float32) / 14.0 - 1.0)


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
