"""GPU parity of RMSNorm, fused add + RMSNorm and RoPE against the oracle.

Mirrors crates/mote-backend-hip/tests/rms_norm.rs, fused_add_rms_norm.rs and
rope.rs: inputs are rounded to f16 first and widened to f32 for the oracle, the
oracle output is rounded to f16, and an element passes if
|actual - expected| <= max(3e-3, 3e-3 |expected|) (rms_norm.rs:57,
rope.rs:416); the RoPE tail past rotary_dim must be bit-exact (rope.rs:423-429).
Adds the seeded workload (hidden 4096, eps 1e-5, 32 tokens, RoPE on 32 query
and 8 key heads of head_dim 128 with theta 500000) and the fused q/k RoPE and
cos/sin table entry points.  Every call goes through the C ABI.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import (
    bits_to_f32,
    f16_bits,
    ref_norm_input,
    ref_norm_weight,
    ref_residual,
    ref_rope_cos,
    ref_rope_sin,
)
from mote_amd import _ffi, ops, workloads as wl
from mote_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu


def assert_f16_close(actual_bits, expected_f32, what):
    actual = bits_to_f32(actual_bits)
    expected = bits_to_f32(f16_bits(expected_f32))
    tol = np.maximum(3e-3, 3e-3 * np.abs(expected))
    bad = ~(np.abs(actual - expected) <= tol)
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} mismatches, first at {int(np.argmax(bad))}: "
        f"got {actual[bad][:4]}, want {expected[bad][:4]}"
    )


def status(fn, *args) -> int:
    return int(getattr(_ffi.lib(), fn)(*args))


# --- RMSNorm -------------------------------------------------------------------------

@pytest.mark.parametrize("rows,hidden,eps,in_place", [(3, 513, 1e-6, False), (3, 513, 1e-6, True),
                                                      (2, 4096, 1e-6, True), (5, 8200, 1e-6, False)])
def test_rms_norm_reference_fixture(stream, oracle, rows, hidden, eps, in_place):
    """crates/mote-backend-hip/tests/rms_norm.rs:20-62 (hidden 513, 3 rows),
    plus the vectorised row sizes and in-place operation."""
    x = ref_norm_input(rows * hidden)
    w = ref_norm_weight(hidden)
    expected = oracle.rms_norm_f32(bits_to_f32(x), bits_to_f32(w), hidden, eps)
    xb, wb = DeviceBuffer.from_array(x), DeviceBuffer.from_array(w)
    yb = xb if in_place else DeviceBuffer(x.nbytes)
    ops.rms_norm_f16(xb.ptr, wb.ptr, yb.ptr, rows, hidden, eps, stream)
    stream.synchronize()
    assert_f16_close(yb.download(np.uint16), expected, f"rms_norm {rows}x{hidden}")


def test_rms_norm_seeded_workload(stream, oracle):
    """32 tokens x hidden 4096, eps 1e-5, w = f16(N(1, 0.1)), x = f16(N(0, 1))."""
    rows, hidden, eps = 32, 4096, 1e-5
    x = wl.normal_f16(wl.seed_for(3, 0), rows * hidden)
    w = wl.normal_f16(wl.seed_for(3, 1), hidden, mean=1.0, std=0.1)
    expected = oracle.rms_norm_f32(bits_to_f32(x), bits_to_f32(w), hidden, eps)
    xb, wb, yb = DeviceBuffer.from_array(x), DeviceBuffer.from_array(w), DeviceBuffer(x.nbytes)
    ops.rms_norm_f16(xb.ptr, wb.ptr, yb.ptr, rows, hidden, eps, stream)
    stream.synchronize()
    assert_f16_close(yb.download(np.uint16), expected, "rms_norm 32x4096")


def test_rms_norm_empty_and_invalid(stream):
    """rms_norm.rs:65-98 and the shim's checks (rms_norm.hip:75-83)."""
    w = DeviceBuffer.from_array(ref_norm_weight(8))
    x = DeviceBuffer(16)
    assert status("mote_hip_rms_norm_f16", x.ptr, w.ptr, x.ptr, 0, 8, 1e-6, stream.handle) == 0
    assert status("mote_hip_rms_norm_f16", x.ptr, w.ptr, x.ptr, 2, 0, 1e-6, stream.handle) == 0
    assert status("mote_hip_rms_norm_f16", None, w.ptr, x.ptr, 1, 8, 1e-6, stream.handle) == -1
    assert status("mote_hip_rms_norm_f16", x.ptr, w.ptr, x.ptr, 1, 8, 1e-6, None) == -1
    assert status("mote_hip_rms_norm_f16", x.ptr, w.ptr, x.ptr, 1 << 33, 8, 1e-6, stream.handle) == -1
    stream.synchronize()


# --- fused add + RMSNorm --------------------------------------------------------------

@pytest.mark.parametrize("hidden", [513, 4096])
@pytest.mark.parametrize("alias", ["none", "output_is_input", "residual_is_input"])
def test_fused_add_rms_norm_reference_fixture(stream, oracle, hidden, alias):
    """crates/mote-backend-hip/tests/fused_add_rms_norm.rs:23-152: hidden 513,
    3 rows, eps 1e-6, both outputs compared; output may alias input and the
    residual may alias the input."""
    rows, eps = 3, 1e-6
    x = ref_norm_input(rows * hidden)
    r = x if alias == "residual_is_input" else ref_residual(rows * hidden)
    w = ref_norm_weight(hidden)
    want_norm, want_res = oracle.fused_add_rms_norm_f32(bits_to_f32(x), bits_to_f32(r), bits_to_f32(w), hidden, eps)
    xb, wb = DeviceBuffer.from_array(x), DeviceBuffer.from_array(w)
    rb = xb if alias == "residual_is_input" else DeviceBuffer.from_array(r)
    yb = xb if alias == "output_is_input" else DeviceBuffer(x.nbytes)
    ops.fused_add_rms_norm_f16(xb.ptr, rb.ptr, wb.ptr, yb.ptr, rows, hidden, eps, stream)
    stream.synchronize()
    assert_f16_close(yb.download(np.uint16), want_norm, f"normalized ({alias})")
    assert_f16_close(rb.download(np.uint16), want_res, f"residual ({alias})")


def test_fused_add_rms_norm_rejections(stream):
    """fused_add_rms_norm.rs:154-258 / fused_add_rms_norm.hip:107-122:
    output == residual and bad epsilons are rejected before any launch."""
    x, r, w, y = DeviceBuffer(64), DeviceBuffer(64), DeviceBuffer(64), DeviceBuffer(64)
    s = stream.handle
    f = "mote_hip_fused_add_rms_norm_f16"
    assert status(f, x.ptr, r.ptr, w.ptr, r.ptr, 2, 16, 1e-6, s) == -1
    for eps in (-1e-6, float("nan"), float("inf"), float("-inf")):
        assert status(f, x.ptr, r.ptr, w.ptr, y.ptr, 2, 16, eps, s) == -1
    assert status(f, x.ptr, None, w.ptr, y.ptr, 2, 16, 1e-6, s) == -1
    assert status(f, x.ptr, r.ptr, w.ptr, y.ptr, 0, 16, 1e-6, s) == 0
    assert status(f, x.ptr, r.ptr, w.ptr, y.ptr, 2, 0, 1e-6, s) == 0
    stream.synchronize()


# --- RoPE ------------------------------------------------------------------------------

def _rope_case(stream, oracle, tokens, heads, head_dim, rotary_dim, layout, in_place):
    n = tokens * heads * head_dim
    x = ref_norm_input(n)
    half = rotary_dim // 2
    cos, sin = ref_rope_cos(tokens * half), ref_rope_sin(tokens * half)
    expected = oracle.rope_f32(bits_to_f32(x), cos, sin, tokens, heads, head_dim, rotary_dim, layout)
    xb = DeviceBuffer.from_array(x)
    cb, sb = DeviceBuffer.from_array(cos), DeviceBuffer.from_array(sin)
    yb = xb if in_place else DeviceBuffer(x.nbytes)
    ops.rope_f16(xb.ptr, cb.ptr, sb.ptr, yb.ptr, tokens, heads, head_dim, rotary_dim, layout, stream)
    stream.synchronize()
    got = yb.download(np.uint16)
    assert_f16_close(got, expected, f"rope layout {layout}")
    tail = (np.arange(n) % head_dim) >= rotary_dim
    assert np.array_equal(got[tail], x[tail]), "tail changed"


@pytest.mark.parametrize("layout", [ops.HALF_SPLIT, ops.INTERLEAVED], ids=["half_split", "interleaved"])
@pytest.mark.parametrize("tokens,in_place", [(2, False), (1, False), (4, False), (2, True)],
                         ids=["tokens2", "rank2", "flattened", "in_place"])
def test_rope_reference_fixture(stream, oracle, layout, tokens, in_place):
    """crates/mote-backend-hip/tests/rope.rs:25-51, 343-432: heads 3,
    head_dim 70, rotary_dim 66 (rotated prefix plus a copied tail)."""
    _rope_case(stream, oracle, tokens, 3, 70, 66, layout, in_place)


@pytest.mark.parametrize("layout", [ops.HALF_SPLIT, ops.INTERLEAVED], ids=["half_split", "interleaved"])
@pytest.mark.parametrize("head_dim,rotary_dim", [(128, 128), (128, 64), (96, 0)])
def test_rope_vector_path(stream, oracle, layout, head_dim, rotary_dim):
    _rope_case(stream, oracle, 5, 4, head_dim, rotary_dim, layout, False)
    _rope_case(stream, oracle, 5, 4, head_dim, rotary_dim, layout, True)


def test_rope_tables_match_oracle(stream, oracle):
    """Device cos/sin tables (binary64, rounded once) against the oracle's:
    equal except where the two libms' binary64 results straddle a binary32
    rounding boundary, which leaves at most one ulp."""
    pos = wl.positions(wl.seed_for(3, 2), 32)
    pos = np.concatenate([pos, np.array([0, 1, 8191], np.int64)])
    want_c, want_s = oracle.rope_tables(pos, 128, 500000.0)
    pb = DeviceBuffer.from_array(pos)
    cb, sb = DeviceBuffer(want_c.nbytes), DeviceBuffer(want_s.nbytes)
    ops.rope_tables_f32(pb.ptr, cb.ptr, sb.ptr, pos.size, 128, 500000.0, stream)
    stream.synchronize()
    for got, want in ((cb.download(np.float32), want_c.ravel()), (sb.download(np.float32), want_s.ravel())):
        ulps = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
        assert ulps.max() <= 1
        assert np.mean(ulps == 0) > 0.99


def test_rope_seeded_workload_fused_qk(stream, oracle):
    """32 tokens, q 32 heads and k 8 heads of head_dim 128, rotate-half,
    theta 500000, positions uniform in [0, 8191]; the fused q/k launch must
    equal two single-tensor launches bit for bit and match the oracle."""
    tokens, qh, kh, d = 32, 32, 8, 128
    pos = wl.positions(wl.seed_for(3, 2), tokens)
    cos, sin = oracle.rope_tables(pos, d, 500000.0)
    q = wl.normal_f16(wl.seed_for(3, 3), tokens * qh * d)
    k = wl.normal_f16(wl.seed_for(3, 4), tokens * kh * d)
    want_q = oracle.rope_f32(bits_to_f32(q), cos, sin, tokens, qh, d, d, oracle.HALF_SPLIT)
    want_k = oracle.rope_f32(bits_to_f32(k), cos, sin, tokens, kh, d, d, oracle.HALF_SPLIT)
    qb, kb = DeviceBuffer.from_array(q), DeviceBuffer.from_array(k)
    cb, sb = DeviceBuffer.from_array(cos), DeviceBuffer.from_array(sin)
    qo, ko = DeviceBuffer(q.nbytes), DeviceBuffer(k.nbytes)
    ops.rope_qk_f16(qb.ptr, kb.ptr, cb.ptr, sb.ptr, qo.ptr, ko.ptr, tokens, qh, kh, d, d, ops.HALF_SPLIT, stream)
    q1, k1 = DeviceBuffer(q.nbytes), DeviceBuffer(k.nbytes)
    ops.rope_f16(qb.ptr, cb.ptr, sb.ptr, q1.ptr, tokens, qh, d, d, ops.HALF_SPLIT, stream)
    ops.rope_f16(kb.ptr, cb.ptr, sb.ptr, k1.ptr, tokens, kh, d, d, ops.HALF_SPLIT, stream)
    stream.synchronize()
    gq, gk = qo.download(np.uint16), ko.download(np.uint16)
    assert np.array_equal(gq, q1.download(np.uint16))
    assert np.array_equal(gk, k1.download(np.uint16))
    assert_f16_close(gq, want_q, "q")
    assert_f16_close(gk, want_k, "k")


def test_rope_rejections_and_empty(stream):
    """rope.rs:53-160 and the shim's checks (rope.hip:109-130)."""
    x, c, s = DeviceBuffer(1024), DeviceBuffer(256), DeviceBuffer(256)
    h = stream.handle
    f = "mote_hip_rope_f16"
    assert status(f, x.ptr, c.ptr, s.ptr, x.ptr, 2, 3, 8, 7, 0, h) == -1   # odd rotary_dim
    assert status(f, x.ptr, c.ptr, s.ptr, x.ptr, 2, 3, 8, 10, 0, h) == -1  # rotary_dim > head_dim
    assert status(f, x.ptr, c.ptr, s.ptr, x.ptr, 2, 3, 8, 8, 2, h) == -1   # unknown layout
    assert status(f, x.ptr, None, s.ptr, x.ptr, 2, 3, 8, 8, 0, h) == -1    # null cos with R > 0
    assert status(f, x.ptr, None, None, x.ptr, 2, 3, 8, 0, 0, h) == 0      # R == 0: tables unused
    assert status(f, x.ptr, c.ptr, s.ptr, x.ptr, 0, 3, 8, 8, 0, h) == 0
    assert status(f, x.ptr, c.ptr, s.ptr, x.ptr, 2, 0, 8, 8, 0, h) == 0
    assert status(f, x.ptr, c.ptr, s.ptr, x.ptr, 2, 3, 0, 0, 0, h) == 0
    assert status(f, x.ptr, c.ptr, s.ptr, x.ptr, 1 << 31, 1 << 31, 8, 8, 0, h) == -1
    stream.synchronize()
