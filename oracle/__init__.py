"""CPU oracle for the Q4_0 quantized-linear path (TEST INFRASTRUCTURE ONLY).

Python bindings over ``oracle/libmote_oracle.so``, a plain-C restatement of the
pure-Rust reference oracle ``mote-reference`` (``crates/mote-reference/src/
quantized.rs`` and ``crates/mote-reference/src/lib.rs``).  Only the tests,
``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` use this
module, and only as the checker.  The product package ``mote_amd`` never
imports it.

Functions and the reference code they restate:

* ``f16_bits_to_f32`` / ``f32_to_f16_bits``: IEEE-754 binary16 conversion as used
  by ``half`` 2.7.1 at ``quantized.rs:181`` and in the HIP tests.
* ``dequantize_row``: ``dequantize_quantized_row``, ``quantized.rs:58-74`` plus
  ``decode_row_into``, ``quantized.rs:177-201``.
* ``quantized_linear_f32``: ``quantized_linear_f32``, ``quantized.rs:89-144``
  (bit-identical f32 restatement).
* ``quantized_linear_f64``: the same sum accumulated in binary64, the parity
  judge for the linear (products are exact, only the summation rounds).
* ``gate_up_silu_f64``: ``silu(x Wg^T) * (x Wu^T)`` in binary64.  This op has no
  counterpart in the reference.
* ``matmul_f32``: ``lib.rs:116-156``; ``rope_f32``: ``lib.rs:170-244``;
  ``rms_norm_f32``: ``lib.rs:262-301``; ``fused_add_rms_norm_f32``:
  ``lib.rs:333-384``.
* ``rope_tables``: theta/position cos-sin tables in binary64.  The reference has
  no table builder; this is pinned by the closed form.
* ``dequantize_kquant_row`` / ``kquant_linear_f64``: Q4_K and Q6_K super-blocks
  as GGML defines them (ggml-common.h ``block_q4_K`` / ``block_q6_K``,
  ggml-quants.c ``dequantize_row_q4_K`` / ``dequantize_row_q6_K``).  The
  reference has their geometry only (``crates/mote-types/src/lib.rs:39-74``)
  and its oracle rejects them (``quantized.rs:154-156``): parity against the
  reference is unpinned; the tests pin the layout with hand-derived
  known-answer blocks and an encoder-side packer, and the rounding with the
  exact-rational value of every element.

Errors raise :class:`OracleError` carrying the variant name and fields of the
Rust error enum.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libmote_oracle.so")

Q8_0, Q4_0, Q4_K, Q6_K = 0, 1, 2, 3
HALF_SPLIT, INTERLEAVED = 0, 1

_ERRORS = {
    1: ("UnsupportedFormat", ("format",)),
    2: ("RowMisaligned", ("format", "row_elements", "block_elements")),
    3: ("DimensionsOverflow", ("rows", "output_features", "input_features")),
    4: ("InputLengthMismatch", ("expected", "actual")),
    5: ("WeightLengthMismatch", ("expected", "actual")),
    6: ("RowByteLengthMismatch", ("expected", "actual")),
    20: ("ZeroHiddenSize", ()),
    21: ("WeightLengthMismatch", ("weight_len", "hidden_size")),
    22: ("InputNotMultiple", ("input_len", "hidden_size")),
    23: ("ResidualLengthMismatch", ("residual_len", "input_len")),
    24: ("InvalidEpsilon", ()),
    30: ("OddRotaryDimension", ("rotary_dim",)),
    31: ("RotaryDimensionTooLarge", ("rotary_dim", "head_dim")),
    32: ("DimensionsOverflow", ("tokens", "heads", "head_dim")),
    33: ("InputLengthMismatch", ("expected", "actual")),
    34: ("CosLengthMismatch", ("expected", "actual")),
    35: ("SinLengthMismatch", ("expected", "actual")),
    40: ("DimensionsOverflow", ("m", "n", "k")),
    41: ("LhsLengthMismatch", ("expected", "actual")),
    42: ("RhsLengthMismatch", ("expected", "actual")),
}


class OracleError(Exception):
    """A reference error variant: ``kind`` is its name, ``fields`` its payload."""

    def __init__(self, code: int, detail):
        name, keys = _ERRORS.get(code, (f"Unknown({code})", ()))
        self.code = code
        self.kind = name
        self.fields = {key: int(detail[i]) for i, key in enumerate(keys)}
        super().__init__(f"{name} {self.fields}")


def build() -> str:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_S = ctypes.c_size_t


def _declare(h: ctypes.CDLL) -> None:
    h.mote_oracle_f16_to_f32.restype = ctypes.c_float
    h.mote_oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    h.mote_oracle_f32_to_f16.restype = ctypes.c_uint16
    h.mote_oracle_f32_to_f16.argtypes = [ctypes.c_float]
    h.mote_oracle_f16_to_f32_array.argtypes = [_P, _P, _S]
    h.mote_oracle_f32_to_f16_array.argtypes = [_P, _P, _S]
    for name in ("block_elements", "block_bytes", "alignment_bytes"):
        fn = getattr(h, f"mote_oracle_{name}")
        fn.restype = _S
        fn.argtypes = [ctypes.c_int]
    h.mote_oracle_dequantize_row.argtypes = [_P, _S, ctypes.c_int, _S, _P, _P]
    h.mote_oracle_quantized_linear_f32.argtypes = [_P, _S, _P, _S, ctypes.c_int, _S, _S, _S, _P, _P]
    h.mote_oracle_quantized_linear_f64.argtypes = [_P, _P, ctypes.c_int, _S, _S, _S, _P, _S, _P]
    h.mote_oracle_gate_up_silu_f64.argtypes = [_P, _P, _P, _S, _S, _S, _P, _S, _P]
    h.mote_oracle_matmul_f32.argtypes = [_P, _S, _P, _S, _S, _S, _S, _P, _P]
    h.mote_oracle_rope_f32.argtypes = [_P, _S, _P, _S, _P, _S, _S, _S, _S, _S, ctypes.c_int, _P, _P]
    h.mote_oracle_rope_tables.argtypes = [_P, _S, _S, ctypes.c_double, _P, _P]
    h.mote_oracle_rms_norm_f32.argtypes = [_P, _S, _P, _S, _S, ctypes.c_float, _P, _P]
    h.mote_oracle_fused_add_rms_norm_f32.argtypes = [_P, _S, _P, _S, _P, _S, _S, ctypes.c_float, _P, _P, _P]
    h.mote_oracle_time_quantized_linear_f32.restype = ctypes.c_double
    h.mote_oracle_time_quantized_linear_f32.argtypes = [_P, _P, _S, _S, _S, _P, ctypes.c_int]
    h.mote_oracle_dequantize_kquant_row.argtypes = [_P, _S, ctypes.c_int, _S, _P]
    h.mote_oracle_kquant_linear_f64.argtypes = [_P, _P, ctypes.c_int, _S, _S, _S, _P]


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(np.frombuffer(bytes(a), dtype=np.uint8)) if isinstance(
        a, (bytes, bytearray)
    ) else np.ascontiguousarray(np.asarray(a, dtype=np.uint8))


def _check(code: int, detail: np.ndarray) -> None:
    if code != 0:
        raise OracleError(code, detail)


# --- binary16 -------------------------------------------------------------

def f16_bits_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16))
    out = np.empty(b.shape, dtype=np.float32)
    lib().mote_oracle_f16_to_f32_array(_ptr(b), _ptr(out), b.size)
    return out


def f32_to_f16_bits(values) -> np.ndarray:
    v = _f32(values)
    out = np.empty(v.shape, dtype=np.uint16)
    lib().mote_oracle_f32_to_f16_array(_ptr(v), _ptr(out), v.size)
    return out


def block_geometry(fmt: int) -> tuple[int, int, int]:
    h = lib()
    return (
        h.mote_oracle_block_elements(fmt),
        h.mote_oracle_block_bytes(fmt),
        h.mote_oracle_alignment_bytes(fmt),
    )


# --- quantized rows and linear ---------------------------------------------

def dequantize_row(data, fmt: int, row_elements: int) -> np.ndarray:
    w = _u8(data)
    # Overflowing geometries are rejected before anything is written, so they
    # get a one-element buffer.
    out = np.zeros(row_elements if 0 < row_elements < (1 << 40) else 1, dtype=np.float32)
    detail = np.zeros(3, dtype=np.uint64)
    _check(lib().mote_oracle_dequantize_row(_ptr(w), w.size, fmt, row_elements, _ptr(out), _ptr(detail)), detail)
    return out[:row_elements]


def quantized_linear_f32(x, weights, fmt: int, rows: int, n: int, k: int) -> np.ndarray:
    xv = _f32(x).reshape(-1)
    w = _u8(weights)
    size = rows * n if rows * n < (1 << 40) else 0
    out = np.zeros(max(size, 1), dtype=np.float32)
    detail = np.zeros(3, dtype=np.uint64)
    _check(
        lib().mote_oracle_quantized_linear_f32(
            _ptr(xv), xv.size, _ptr(w), w.size, fmt, rows, n, k, _ptr(out), _ptr(detail)
        ),
        detail,
    )
    return out[:size]


def quantized_linear_f64(x, weights, rows: int, n: int, k: int, columns=None, fmt: int = Q4_0) -> np.ndarray:
    """f64-accumulated ``x @ W^T``; returns ``[rows, len(columns) or n]``."""
    xv = _f32(x).reshape(-1)
    w = _u8(weights)
    cols = None if columns is None else np.ascontiguousarray(np.asarray(columns, dtype=np.uint64))
    count = n if cols is None else cols.size
    out = np.zeros((rows, count), dtype=np.float64)
    code = lib().mote_oracle_quantized_linear_f64(_ptr(xv), _ptr(w), fmt, rows, n, k, _ptr(cols), count, _ptr(out))
    if code != 0:
        raise OracleError(code, np.zeros(3))
    return out


def gate_up_silu_f64(x, gate, up, rows: int, n: int, k: int, columns=None) -> np.ndarray:
    xv = _f32(x).reshape(-1)
    g = _u8(gate)
    u = _u8(up)
    cols = None if columns is None else np.ascontiguousarray(np.asarray(columns, dtype=np.uint64))
    count = n if cols is None else cols.size
    out = np.zeros((rows, count), dtype=np.float64)
    code = lib().mote_oracle_gate_up_silu_f64(_ptr(xv), _ptr(g), _ptr(u), rows, n, k, _ptr(cols), count, _ptr(out))
    if code != 0:
        raise OracleError(code, np.zeros(3))
    return out


def dequantize_kquant_row(data, fmt: int, row_elements: int) -> np.ndarray:
    """Q4_K / Q6_K bytes of ``row_elements`` (a multiple of 256) elements to f32."""
    w = _u8(data)
    out = np.zeros(max(row_elements, 1), dtype=np.float32)
    code = lib().mote_oracle_dequantize_kquant_row(_ptr(w), w.size, fmt, row_elements, _ptr(out))
    if code != 0:
        raise OracleError(code, np.zeros(3))
    return out[:row_elements]


def kquant_linear_f64(x, weights, fmt: int, rows: int, n: int, k: int) -> np.ndarray:
    """f64-accumulated ``x @ W^T`` for Q4_K / Q6_K weights ``[n, k]``; ``[rows, n]``."""
    xv = _f32(x).reshape(-1)
    w = _u8(weights)
    out = np.zeros((rows, n), dtype=np.float64)
    code = lib().mote_oracle_kquant_linear_f64(_ptr(xv), _ptr(w), fmt, rows, n, k, _ptr(out))
    if code != 0:
        raise OracleError(code, np.zeros(3))
    return out


def matmul_f32(lhs, rhs, m: int, n: int, k: int) -> np.ndarray:
    a, b = _f32(lhs).reshape(-1), _f32(rhs).reshape(-1)
    size = m * n if m * n < (1 << 40) else 0
    out = np.zeros(max(size, 1), dtype=np.float32)
    detail = np.zeros(3, dtype=np.uint64)
    _check(lib().mote_oracle_matmul_f32(_ptr(a), a.size, _ptr(b), b.size, m, n, k, _ptr(out), _ptr(detail)), detail)
    return out[:size]


# --- RoPE and norms --------------------------------------------------------

def rope_f32(x, cos, sin, tokens: int, heads: int, head_dim: int, rotary_dim: int, layout: int) -> np.ndarray:
    xv, c, s = _f32(x).reshape(-1), _f32(cos).reshape(-1), _f32(sin).reshape(-1)
    out = np.zeros(max(xv.size, 1), dtype=np.float32)
    detail = np.zeros(3, dtype=np.uint64)
    _check(
        lib().mote_oracle_rope_f32(
            _ptr(xv), xv.size, _ptr(c), c.size, _ptr(s), s.size,
            tokens, heads, head_dim, rotary_dim, layout, _ptr(out), _ptr(detail),
        ),
        detail,
    )
    return out[: xv.size]


def rope_tables(positions, rotary_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    pos = np.ascontiguousarray(np.asarray(positions, dtype=np.int64))
    half = rotary_dim // 2
    c = np.zeros((pos.size, half), dtype=np.float32)
    s = np.zeros((pos.size, half), dtype=np.float32)
    lib().mote_oracle_rope_tables(_ptr(pos), pos.size, rotary_dim, float(theta), _ptr(c), _ptr(s))
    return c, s


def rms_norm_f32(x, weight, hidden: int, eps: float) -> np.ndarray:
    xv, w = _f32(x).reshape(-1), _f32(weight).reshape(-1)
    out = np.zeros(max(xv.size, 1), dtype=np.float32)
    detail = np.zeros(3, dtype=np.uint64)
    _check(lib().mote_oracle_rms_norm_f32(_ptr(xv), xv.size, _ptr(w), w.size, hidden, eps, _ptr(out), _ptr(detail)), detail)
    return out[: xv.size]


def fused_add_rms_norm_f32(x, residual, weight, hidden: int, eps: float) -> tuple[np.ndarray, np.ndarray]:
    xv, r, w = _f32(x).reshape(-1), _f32(residual).reshape(-1), _f32(weight).reshape(-1)
    normalized = np.zeros(max(xv.size, 1), dtype=np.float32)
    res = np.zeros(max(xv.size, 1), dtype=np.float32)
    detail = np.zeros(3, dtype=np.uint64)
    _check(
        lib().mote_oracle_fused_add_rms_norm_f32(
            _ptr(xv), xv.size, _ptr(r), r.size, _ptr(w), w.size, hidden, eps,
            _ptr(normalized), _ptr(res), _ptr(detail),
        ),
        detail,
    )
    return normalized[: xv.size], res[: xv.size]


def time_quantized_linear_f32(x, weights, rows: int, n: int, k: int, iterations: int = 1) -> float:
    """Seconds for ``iterations`` single-threaded runs of the f32 oracle."""
    xv, w = _f32(x).reshape(-1), _u8(weights)
    out = np.zeros(rows * n, dtype=np.float32)
    return lib().mote_oracle_time_quantized_linear_f32(_ptr(xv), _ptr(w), rows, n, k, _ptr(out), iterations)
