"""Seeded synthetic inputs for the Q4_0 linear, RMSNorm and RoPE workloads.

The reference has no random generator: its fixtures are closed-form modular
sequences (``crates/mote-backend-hip/tests/quantized_linear.rs:160-177``,
``crates/mote-backend-hip/benches/quantized_linear.rs:128-152``).  The seeded
workloads here are defined by this package:

* SplitMix64 (Steele, Lea and Flood, 2014), counter form: draw ``i`` of a
  stream seeded with ``s`` is ``mix(s + (i + 1) * 0x9E3779B97F4A7C15)``.
* A uniform double is ``(z >> 11) * 2**-53``.
* A normal sample is Box-Muller in float64 on two consecutive draws,
  ``sqrt(-2 ln(1 - u1)) * cos(2 pi u2)``, rounded to binary16 once (RNE).
* A Q4_0 block takes four draws: two for ``d = f16(|0.02 * N(0, 1)|)`` and two
  whose 16 little-endian bytes are the nibble bytes, so both nibbles of every
  byte are independent and uniform over 0..15.
* Each (workload, tensor) pair has its own stream, seeded
  ``20261201 + 1000 * workload + tensor``.

Every function returns numpy arrays; f16 data is returned as raw ``uint16``
bit patterns, which is what the device buffers hold.
"""

from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
MIX1 = np.uint64(0xBF58476D1CE4E5B9)
MIX2 = np.uint64(0x94D049BB133111EB)
BASE_SEED = 20261201

Q4_0_BLOCK_ELEMENTS = 32
Q4_0_BLOCK_BYTES = 18
Q8_0_BLOCK_BYTES = 34


def seed_for(workload: int, tensor: int) -> int:
    return BASE_SEED + 1000 * workload + tensor


def splitmix64(seed: int, count: int, offset: int = 0) -> np.ndarray:
    """Draws ``offset .. offset + count`` of the SplitMix64 stream ``seed``."""
    i = np.arange(offset + 1, offset + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + i * GAMMA
        z = (z ^ (z >> np.uint64(30))) * MIX1
        z = (z ^ (z >> np.uint64(27))) * MIX2
    return z ^ (z >> np.uint64(31))


def uniform01(draws: np.ndarray) -> np.ndarray:
    return (draws >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def _box_muller(u1: np.ndarray, u2: np.ndarray) -> np.ndarray:
    return np.sqrt(-2.0 * np.log1p(-u1)) * np.cos(2.0 * np.pi * u2)


def normal_f16(seed: int, count: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """``count`` f16 bit patterns of ``f16(mean + std * N(0, 1))``."""
    u = uniform01(splitmix64(seed, 2 * count)).reshape(count, 2) if count else np.zeros((0, 2))
    z = mean + std * _box_muller(u[:, 0], u[:, 1])
    return z.astype(np.float16).view(np.uint16)


def uniform_f16(seed: int, count: int, low: float = -1.0, high: float = 1.0) -> np.ndarray:
    u = uniform01(splitmix64(seed, count))
    return (low + (high - low) * u).astype(np.float16).view(np.uint16)


def q4_0_weights(seed: int, rows: int, cols: int, std: float = 0.02) -> np.ndarray:
    """GGML Q4_0 bytes for a ``[rows, cols]`` matrix, row-major blocks."""
    if cols % Q4_0_BLOCK_ELEMENTS:
        raise ValueError("cols must be a multiple of 32")
    blocks = rows * (cols // Q4_0_BLOCK_ELEMENTS)
    draws = splitmix64(seed, 4 * blocks).reshape(blocks, 4) if blocks else np.zeros((0, 4), np.uint64)
    u = uniform01(draws[:, :2])
    d = np.abs(std * _box_muller(u[:, 0], u[:, 1])).astype(np.float16).view(np.uint16)
    out = np.empty((blocks, Q4_0_BLOCK_BYTES), dtype=np.uint8)
    out[:, 0:2] = d.astype("<u2").view(np.uint8).reshape(blocks, 2)
    out[:, 2:18] = np.ascontiguousarray(draws[:, 2:4]).astype("<u8").view(np.uint8).reshape(blocks, 16)
    return out.reshape(-1)


def q8_0_weights(seed: int, rows: int, cols: int, std: float = 0.02) -> np.ndarray:
    """GGML Q8_0 bytes for a ``[rows, cols]`` matrix: per 32-element block an
    f16 scale ``|N(0, std)|`` and 32 uniform two's-complement bytes."""
    if cols % Q4_0_BLOCK_ELEMENTS:
        raise ValueError("cols must be a multiple of 32")
    blocks = rows * (cols // Q4_0_BLOCK_ELEMENTS)
    draws = splitmix64(seed, 6 * blocks).reshape(blocks, 6) if blocks else np.zeros((0, 6), np.uint64)
    u = uniform01(draws[:, :2])
    d = np.abs(std * _box_muller(u[:, 0], u[:, 1])).astype(np.float16).view(np.uint16)
    out = np.empty((blocks, Q8_0_BLOCK_BYTES), dtype=np.uint8)
    out[:, 0:2] = d.astype("<u2").view(np.uint8).reshape(blocks, 2)
    out[:, 2:34] = np.ascontiguousarray(draws[:, 2:6]).astype("<u8").view(np.uint8).reshape(blocks, 32)
    return out.reshape(-1)


Q4_K_BLOCK_BYTES, Q6_K_BLOCK_BYTES, K_SUPER = 144, 210, 256


def _random_blocks(seed: int, blocks: int, block_bytes: int) -> np.ndarray:
    words = (block_bytes + 7) // 8
    draws = splitmix64(seed, words * blocks) if blocks else np.zeros(0, np.uint64)
    raw = draws.astype("<u8").view(np.uint8).reshape(blocks, words * 8)
    return np.ascontiguousarray(raw[:, :block_bytes])


def q4_k_weights(seed: int, rows: int, cols: int, std: float = 0.002) -> np.ndarray:
    """GGML Q4_K bytes for a ``[rows, cols]`` matrix (144-byte blocks of 256
    elements): per block d and dmin ``|N(0, std)|`` in f16, then 12 scale
    bytes and 128 nibble bytes uniform (every byte pattern is a valid block)."""
    if cols % K_SUPER:
        raise ValueError("cols must be a multiple of 256")
    blocks = rows * (cols // K_SUPER)
    out = _random_blocks(seed, blocks, Q4_K_BLOCK_BYTES)
    draws = splitmix64(seed ^ 0x5EED, 4 * blocks).reshape(blocks, 4) if blocks else np.zeros((0, 4), np.uint64)
    u = uniform01(draws)
    d = np.abs(std * _box_muller(u[:, 0], u[:, 1])).astype(np.float16).view(np.uint16)
    dmin = np.abs(std * _box_muller(u[:, 2], u[:, 3])).astype(np.float16).view(np.uint16)
    out[:, 0:2] = d.astype("<u2").view(np.uint8).reshape(blocks, 2)
    out[:, 2:4] = dmin.astype("<u2").view(np.uint8).reshape(blocks, 2)
    return out.reshape(-1)


def q6_k_weights(seed: int, rows: int, cols: int, std: float = 0.0005) -> np.ndarray:
    """GGML Q6_K bytes for a ``[rows, cols]`` matrix (210-byte blocks of 256
    elements): 128 + 64 quant bytes and 16 int8 scales uniform, d
    ``|N(0, std)|`` in f16 in the last two bytes."""
    if cols % K_SUPER:
        raise ValueError("cols must be a multiple of 256")
    blocks = rows * (cols // K_SUPER)
    out = _random_blocks(seed, blocks, Q6_K_BLOCK_BYTES)
    draws = splitmix64(seed ^ 0x5EED, 2 * blocks).reshape(blocks, 2) if blocks else np.zeros((0, 2), np.uint64)
    u = uniform01(draws)
    d = np.abs(std * _box_muller(u[:, 0], u[:, 1])).astype(np.float16).view(np.uint16)
    out[:, 208:210] = d.astype("<u2").view(np.uint8).reshape(blocks, 2)
    return out.reshape(-1)


def reference_bench_q4_0_weights(rows: int, cols: int) -> np.ndarray:
    """The closed-form Q4_0 matrix of the reference's own benchmark
    (crates/mote-backend-hip/benches/quantized_linear.rs:134-152): block b of
    row o has scale f16(2^-6 ((3 o + b) % 4 + 1)), and byte j of it the low
    nibble (5 o + 3 b + j) % 16 and the high nibble (7 o + b + 3 j + 1) % 16."""
    blocks = cols // Q4_0_BLOCK_ELEMENTS
    o = np.arange(rows)[:, None]
    b = np.arange(blocks)[None, :]
    scale = (0.015625 * (((o * 3 + b) % 4) + 1)).astype(np.float16).view(np.uint16)
    out = np.empty((rows, blocks, Q4_0_BLOCK_BYTES), dtype=np.uint8)
    out[:, :, 0:2] = scale.astype("<u2").view(np.uint8).reshape(rows, blocks, 2)
    j = np.arange(16)[None, None, :]
    low = (o[:, :, None] * 5 + b[:, :, None] * 3 + j) % 16
    high = (o[:, :, None] * 7 + b[:, :, None] + j * 3 + 1) % 16
    out[:, :, 2:] = (low | (high << 4)).astype(np.uint8)
    return out.reshape(-1)


def reference_bench_inputs(rows: int, cols: int) -> np.ndarray:
    """The reference benchmark's f16 activations, element i = f16((i % 29) /
    14 - 1) (crates/mote-backend-hip/benches/quantized_linear.rs:128-132)."""
    i = np.arange(rows * cols)
    return ((i % 29).astype(np.float32) / 14.0 - 1.0).astype(np.float16).view(np.uint16)


def positions(seed: int, count: int, high: int = 8191) -> np.ndarray:
    """Uniform integers in ``[0, high]`` by rejection sampling on 13-bit draws."""
    bits = int(high).bit_length()
    out = []
    offset = 0
    while len(out) < count:
        draws = splitmix64(seed, 4 * count, offset)
        offset += 4 * count
        for z in (draws >> np.uint64(64 - bits)).tolist():
            if z <= high:
                out.append(z)
                if len(out) == count:
                    break
    return np.asarray(out, dtype=np.int64)


def rope_tables(positions_: np.ndarray, rotary_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """f32 ``cos``/``sin`` tables ``[tokens, rotary_dim / 2]`` for the
    rotate-half RoPE: ``inv_i = theta^(-2i / rotary_dim)``, angle ``pos * inv_i``,
    everything in float64 and rounded to float32 once.  The reference takes
    caller-built tables (``crates/mote-reference/src/lib.rs:158-163``)."""
    i = np.arange(rotary_dim // 2, dtype=np.float64)
    inv = np.power(float(theta), -(2.0 * i) / float(rotary_dim))
    angle = positions_.astype(np.float64)[:, None] * inv[None, :]
    return np.cos(angle).astype(np.float32), np.sin(angle).astype(np.float32)


def q8_0_row_bytes(cols: int) -> int:
    return (cols // Q4_0_BLOCK_ELEMENTS) * Q8_0_BLOCK_BYTES


def q4_0_row_bytes(cols: int) -> int:
    return (cols // Q4_0_BLOCK_ELEMENTS) * Q4_0_BLOCK_BYTES
