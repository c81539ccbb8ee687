"""GPU parity of the Q8_0 quantized linear against the oracle.

Q8_0 is the format the reference's oracle decodes beside Q4_0
(crates/mote-reference/src/quantized.rs:191-195: 34-byte blocks, an f16 scale
and 32 two's-complement bytes, value v * d) without a HIP kernel; this build
adds the linear.  Tolerance as for Q4_0: an element passes if
|y - y64| <= 1e-3 |y64| or |y - y64| <= 2e-3 sqrt(K) max|d| max|x| against the
f64-accumulated oracle (+2^-11 |y64| for f16 outputs).  Every call goes
through the C ABI of libmote_hip.so.
"""

from __future__ import annotations

import functools
import re

import numpy as np
import pytest

from helpers import assert_linear_close, bits_to_f32, f16_bits
from mote_amd import _ffi, ops, workloads as wl
from mote_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu

F16_REL = 2.0 ** -11
BLOCK = 34


@functools.lru_cache(maxsize=None)
def weights(seed: int, n: int, k: int) -> np.ndarray:
    return wl.q8_0_weights(seed, n, k)


@functools.lru_cache(maxsize=None)
def normal_x(seed: int, m: int, k: int) -> np.ndarray:
    return wl.normal_f16(seed, m * k)


def q8_block(scale_bits: int, quants) -> np.ndarray:
    out = np.zeros(BLOCK, dtype=np.uint8)
    out[0:2] = np.array([scale_bits], dtype="<u2").view(np.uint8)
    out[2:] = np.asarray(quants, dtype=np.int8).view(np.uint8)
    return out


def scales(w: np.ndarray) -> np.ndarray:
    return w.reshape(-1, BLOCK)[:, 0:2].copy().view("<u2")[:, 0].view(np.float16).astype(np.float32)


def run(stream, x_bits, w, m, n, k, f16_out=False, dispatch=None, w_offset=0):
    xb = DeviceBuffer.from_array(x_bits) if x_bits.size else DeviceBuffer(0)
    wb = DeviceBuffer(w.nbytes + w_offset)
    wb.upload(w, offset=w_offset)
    out_bytes = m * n * (2 if f16_out else 4)
    yb = DeviceBuffer(out_bytes)
    yb.upload(np.full(out_bytes, 0xA5, dtype=np.uint8))  # sentinel: every element must be written
    args = (xb.ptr, wb.ptr + w_offset, yb.ptr, m, n, k)
    if dispatch is not None:
        dispatch.linear_q8_0(*args, stream, f16_out=f16_out)
    elif f16_out:
        ops.quantized_linear_q8_0_f16(*args, stream)
    else:
        ops.quantized_linear_q8_0_f32(*args, stream)
    stream.synchronize()
    y = yb.download(np.uint16 if f16_out else np.float32)
    if f16_out:
        y = bits_to_f32(y)
    return y.reshape(m, n)


def check(oracle, y, x_bits, w, m, n, k, columns=None, f16_out=False, what="output"):
    y64 = oracle.quantized_linear_f64(bits_to_f32(x_bits), w, m, n, k, columns, fmt=oracle.Q8_0)
    got = y if columns is None else y[:, columns]
    max_d = float(np.max(np.abs(scales(w)))) if k else 0.0
    max_x = float(np.max(np.abs(bits_to_f32(x_bits)))) if x_bits.size else 0.0
    assert_linear_close(got, y64, k, max_d, max_x, extra_rel=F16_REL if f16_out else 0.0, what=what)


def sample_columns(n: int, count: int = 256, seed: int = 7) -> np.ndarray:
    rng = np.random.default_rng(seed)
    cols = np.unique(np.concatenate([[0, n - 1], rng.choice(n, size=min(count, n), replace=False)]))
    return cols.astype(np.uint64)


def _variants(prefix):
    return [v for v in ops.variant_names() if v.startswith(prefix)]


# --- the reference's known answers ---------------------------------------------------

def test_reference_kat_rows_without_crossing_row_boundaries(stream, oracle):
    """crates/mote-reference/tests/quantized_rows.rs:68-83: two Q8_0 rows, x
    with 3.0 at 0 and 2.0 at 31, expected [-1, 1] exactly."""
    first = np.zeros(32, np.int8)
    first[0], first[31] = 2, -4
    second = np.zeros(32, np.int8)
    second[0], second[31] = -3, 5
    w = np.concatenate([q8_block(0x3800, first), q8_block(0x3C00, second)])
    x = np.zeros(32, np.float32)
    x[0], x[31] = 3.0, 2.0
    y = run(stream, f16_bits(x), w, 1, 2, 32)
    assert y.tolist() == [[-1.0, 1.0]]
    assert oracle.quantized_linear_f32(x, w, oracle.Q8_0, 1, 2, 32).tolist() == [-1.0, 1.0]


def test_reference_kat_signed_values_and_scale(stream):
    """crates/mote-reference/tests/quantized_rows.rs:43-52: quants [-128, -1,
    0, 1, 127] at scale 0.5 decode to [-64, -0.5, 0, 0.5, 63.5]; one-hot
    activations read them back through the linear, exactly."""
    q = np.zeros(32, np.int8)
    q[:5] = [-128, -1, 0, 1, 127]
    w = q8_block(0x3800, q)
    x = np.eye(5, 32, dtype=np.float32)
    y = run(stream, f16_bits(x.reshape(-1)), w, 5, 1, 32)
    assert y.reshape(-1).tolist() == [-64.0, -0.5, 0.0, 0.5, 63.5]


# --- every kernel, bit-exact where the arithmetic is exact ------------------------------

STREAM_AND_GENERIC = [v for v in _variants("q8_") if not v.startswith(("q8_skinny_", "q8_mfma_")) and "_m4x_" not in v]


@pytest.mark.parametrize("variant", STREAM_AND_GENERIC)
def test_one_hot_activations_read_back_the_decode_exactly(stream, oracle, variant):
    """x = e_j per token: y = v_j d of each row with no rounding (one product,
    exact in f32, and zeros elsewhere), so the output equals the oracle's
    decode bit for bit.  Positions cover both blocks of a pair, both halves of
    a dword, block 0's re-aligned bytes and the last element."""
    d = ops.Q4_0Dispatch()
    d.force(variant)
    tokens = int(variant.split("_m")[1].split("_")[0]) if "_m" in variant else 1
    slots = int(variant.split("_s")[2].split("_")[0]) if variant.count("_s") > 1 else 1
    k = 4096 * slots if variant != "q8_generic" else 4096
    n = 37
    w = weights(wl.seed_for(20, n), n, k)
    rb = wl.q8_0_row_bytes(k)
    decoded = np.stack([oracle.dequantize_row(w[r * rb:(r + 1) * rb], oracle.Q8_0, k) for r in range(n)])
    positions = [0, 1, 2, 3, 30, 31, 32, 33, 63, 64, 2047, k - 1]
    for start in range(0, len(positions), tokens):
        chunk = positions[start:start + tokens]
        chunk += [chunk[-1]] * (tokens - len(chunk))
        x = np.zeros((tokens, k), np.float32)
        for t, j in enumerate(chunk):
            x[t, j] = 1.0
        y = run(stream, f16_bits(x.reshape(-1)), w, tokens, n, k, dispatch=d)
        for t, j in enumerate(chunk):
            assert np.array_equal(y[t].view(np.uint32), decoded[:, j].view(np.uint32)), (variant, j)


@pytest.mark.parametrize("variant", [v for v in STREAM_AND_GENERIC if not v.startswith("q8_rowlds_")])
def test_every_q8_variant(stream, oracle, variant):
    """Ragged N, idle lanes (K below a slot's 4096), K filling every slot and
    one pair past a slot boundary, N = 140001 at K = 64 (register flush past 64
    rows per wave), the 14336 -> 4096 down projection where it fits; the
    generic kernel also on K = 32 (unpaired blocks) and 3 tokens."""
    d = ops.Q4_0Dispatch()
    d.force(variant)
    if variant == "q8_generic":
        shapes = [(3, 61, 96), (1, 130, 32), (5, 257, 4160), (2, 14336, 4096)]
    else:
        tokens = int(variant.split("_m")[1].split("_")[0]) if "_m" in variant else 1
        slots = int(variant.split("_s")[2].split("_")[0]) if variant.count("_s") > 1 else 1
        shapes = [(1, 64), (7, 4096), (257, 1024), (130, 64), (140001, 64)]
        if slots > 1:
            shapes += [(61, 4096 * slots), (1000, 4096 * (slots - 1) + 64)]
            if 14336 <= 4096 * slots:
                shapes.append((4096, 14336))
        shapes.append((14336, 4096))
        shapes = [(tokens, n, k) for n, k in shapes]
    for m, n, k in shapes:
        x = normal_x(wl.seed_for(21, k), m, k)
        w = weights(wl.seed_for(21, 100 + n), n, k)
        y = run(stream, x, w, m, n, k, dispatch=d)
        cols = None if n < 2000 else sample_columns(n, 512)
        check(oracle, y, x, w, m, n, k, columns=cols, what=f"{variant} {m}x{n}x{k}")
    y16 = run(stream, x, w, m, n, k, dispatch=d, f16_out=True)
    check(oracle, y16, x, w, m, n, k, columns=cols, f16_out=True, what=f"{variant} f16")


@pytest.mark.parametrize("variant", [v for v in _variants("q8_skinny_") if not v.endswith("_sk")])
def test_every_q8_skinny_variant(stream, oracle, variant):
    """Matrix-core Q8_0 skinny GEMM (K = 4096): one token, tokens padded inside
    a 16-token tile, one over a tile, the 64-token maximum, N ragged against
    the 16-row tiles, several items per workgroup (20 x 14336), f32 and f16
    outputs.  The products are rounded once to binary16 before the MFMA, so
    the check is the tolerance, not bit equality."""
    d = ops.Q4_0Dispatch()
    d.force(variant)
    k = 4096
    for m, n in [(1, 100), (3, 33), (5, 37), (16, 16), (17, 130), (32, 61), (33, 7), (64, 80), (20, 14336)]:
        x = normal_x(wl.seed_for(24, m), m, k)
        w = weights(wl.seed_for(24, 100 + n), n, k)
        y = run(stream, x, w, m, n, k, dispatch=d)
        cols = None if n < 2000 else sample_columns(n, 256)
        check(oracle, y, x, w, m, n, k, columns=cols, what=f"{variant} {m}x{n}x{k}")
    y16 = run(stream, x, w, m, n, k, dispatch=d, f16_out=True)
    check(oracle, y16, x, w, m, n, k, columns=cols, f16_out=True, what=f"{variant} f16")


@pytest.mark.parametrize("variant", _variants("q8_mfma_"))
def test_every_q8_prefill_variant(stream, oracle, variant):
    """Prefill tiles over Q8_0 pairs (64 or more tokens): M and N ragged
    against the tiles, K of one pair and K = 4160 (65 pairs), f32 and f16;
    `_k<P>` tiles (P pairs per step) the shapes whose K they divide, plus
    K = 768 (12 pairs)."""
    d = ops.Q4_0Dispatch()
    d.force(variant)
    kp = int(re.search(r"_k(\d+)$", variant).group(1)) if re.search(r"_k(\d+)$", variant) else 1
    shapes = [(70, 200, 512), (130, 67, 1024), (64, 128, 64), (65, 33, 4160), (96, 160, 768)]
    for m, n, k in [sh for sh in shapes if sh[2] % (64 * kp) == 0]:
        x = normal_x(wl.seed_for(25, m), m, k)
        w = weights(wl.seed_for(25, 100 + n), n, k)
        y = run(stream, x, w, m, n, k, dispatch=d)
        check(oracle, y, x, w, m, n, k, what=f"{variant} {m}x{n}x{k}")
    y16 = run(stream, x, w, m, n, k, dispatch=d, f16_out=True)
    check(oracle, y16, x, w, m, n, k, f16_out=True, what=f"{variant} f16")


# --- default entry points at full size ------------------------------------------------

@pytest.mark.parametrize("m,k,n", [(1, 4096, 14336), (1, 14336, 4096), (2, 4096, 4096), (4, 4096, 6144),
                                   (3, 4096, 4096), (8, 4096, 4096), (16, 4096, 14336), (32, 4096, 14336),
                                   (64, 4096, 14336), (128, 4096, 14336), (512, 4096, 14336),
                                   (3, 8192, 8192), (3, 14336, 4096)])
def test_llama_shapes_through_the_default_entry_points(stream, oracle, m, k, n):
    x = normal_x(wl.seed_for(22, m), m, k)
    w = weights(wl.seed_for(22, n), n, k)
    cols = sample_columns(n)
    check(oracle, run(stream, x, w, m, n, k), x, w, m, n, k, columns=cols)
    check(oracle, run(stream, x, w, m, n, k, f16_out=True), x, w, m, n, k, columns=cols, f16_out=True,
          what="f16 output")


def test_misaligned_weights_take_the_generic_kernel(stream, oracle):
    """2-byte-aligned storage (the Q8_0 alignment of crates/mote-types/src/
    lib.rs:67-73) is accepted and computed by the generic kernel."""
    m, n, k = 1, 300, 4096
    x = normal_x(wl.seed_for(23, 0), m, k)
    w = weights(wl.seed_for(23, 1), n, k)
    d = ops.Q4_0Dispatch()
    y = run(stream, x, w, m, n, k, dispatch=d, w_offset=2)
    check(oracle, y, x, w, m, n, k)
    assert d.plan(m, n, k, q8_0=True) == "q8_generic"


@pytest.mark.parametrize("m,k,n", [(1, 4096, 14336), (1, 14336, 4096), (4, 4096, 4096)])
def test_exact_properties_at_full_size(stream, m, k, n):
    """Doubling x doubles y and negating every scale negates y, bit for bit
    (power-of-two and sign changes are exact through the subnormal products,
    the f32 sums and the final rescale); repeated runs are identical."""
    x = normal_x(wl.seed_for(24, m), m, k)
    w = weights(wl.seed_for(24, n), n, k)
    d = ops.Q4_0Dispatch()
    y = run(stream, x, w, m, n, k, dispatch=d)
    assert d.plan(m, n, k, q8_0=True).startswith(("q8_stream", "q8_rowlds"))  # the vector-ALU GEMVs
    assert np.array_equal(y, run(stream, x, w, m, n, k, dispatch=d)), "non-deterministic"
    x2 = f16_bits(bits_to_f32(x) * 2.0)
    assert np.array_equal(run(stream, x2, w, m, n, k, dispatch=d), 2.0 * y)
    wneg = w.copy().reshape(-1, BLOCK)
    wneg[:, 1] ^= 0x80
    assert np.array_equal(run(stream, x, wneg.reshape(-1), m, n, k, dispatch=d), -y)


# --- argument handling (same statuses as the Q4_0 entry points) -----------------------

def test_argument_errors_and_empty_problems(stream):
    w = weights(wl.seed_for(25, 0), 2, 64)
    wb = DeviceBuffer.from_array(w)
    xb = DeviceBuffer(2 * 64 * 2)
    yb = DeviceBuffer(2 * 2 * 4)
    lib = _ffi.lib()
    s = stream.handle
    assert lib.mote_hip_quantized_linear_q8_0_f32(None, wb.ptr, yb.ptr, 2, 2, 64, s) == 1
    assert lib.mote_hip_quantized_linear_q8_0_f32(xb.ptr, wb.ptr, yb.ptr, 2, 2, 48, s) == 1
    assert lib.mote_hip_quantized_linear_q8_0_f32(xb.ptr, wb.ptr, yb.ptr, 0, 2, 64, s) == 0
    assert lib.mote_hip_quantized_linear_q8_0_f16(xb.ptr, wb.ptr, yb.ptr, 2, 0, 64, s) == 0
    assert lib.mote_hip_quantized_linear_q8_0_f32(xb.ptr, wb.ptr, yb.ptr, 1 << 32, 2, 64, s) == 9
    y = run(stream, np.zeros(0, np.uint16), np.zeros(0, np.uint8), 3, 2, 0)
    assert np.array_equal(y, np.zeros((3, 2), np.float32)) and not np.signbit(y).any()
