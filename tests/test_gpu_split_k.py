"""GPU parity of the split-K skinny GEMM (1-64 tokens, K a multiple of the
K slice: the MLP down projection, K = 14336, among others; the fused gate/up at
K = 8192) against the oracle.

The split-K tiles cut K into parts and write each part's partial tile to a
per-stream scratch buffer; a second kernel adds the parts in part order, or,
with the fold turned on on a dispatch handle, the last workgroup of a tile to
finish (counted by a per-tile arrival counter) does, in the same order.  The
products are rounded once to binary16 before the MFMA, so the check is the
path's tolerance (|y - y64| <= 1e-3 |y64| or <= 2e-3 sqrt(K) max|d| max|x|,
y64 the f64-accumulated oracle); two runs, and the two epilogues, must agree
bit for bit.
"""

from __future__ import annotations

import functools

import numpy as np
import pytest

from mote_amd import ops, workloads as wl
from test_gpu_q4_0 import check_against_oracle, check_gate_up, run_gate_up, run_linear, sample_columns
import test_gpu_q8_0 as q8

pytestmark = pytest.mark.gpu


@functools.lru_cache(maxsize=None)
def q4_weights(seed: int, n: int, k: int) -> np.ndarray:
    return wl.q4_0_weights(seed, n, k)


@functools.lru_cache(maxsize=None)
def normal_x(seed: int, m: int, k: int) -> np.ndarray:
    return wl.normal_f16(seed, m * k)


def _slice(variant: str) -> int:
    ks, rest = variant.split("_k", 1)[1].split("_s", 1)
    return int(ks) * int(rest.split("_t")[0]) * 256


SPLIT_K = [v for v in ops.variant_names() if v.startswith("skinny_mfma_") and v.endswith("_sk")]
GATE_UP_SPLIT_K = [v for v in ops.variant_names() if v.startswith("gateup_skinny_") and v.endswith("_sk")]
Q8_SPLIT_K = [v for v in ops.variant_names() if v.startswith("q8_skinny_") and v.endswith("_sk")]


@pytest.mark.parametrize("variant", SPLIT_K)
def test_every_split_k_variant(stream, oracle, variant):
    """Two, three and seven K parts; tokens padded inside a tile, exactly one
    and two tiles, one over, the 64-token maximum; N ragged against the
    16-row tiles; f32 and f16 outputs; a repeat is bitwise equal."""
    d = ops.Q4_0Dispatch()
    d.force(variant)
    span = _slice(variant)
    for m, n, parts in [(3, 100, 2), (16, 48, 3), (17, 130, 2), (33, 7, 7), (64, 80, 2), (20, 1000, 3)]:
        k = span * parts
        x = normal_x(wl.seed_for(40, m), m, k)
        w = q4_weights(wl.seed_for(40, 100 + n), n, k)
        y = run_linear(stream, x, w, m, n, k, dispatch=d)
        check_against_oracle(oracle, y, x, w, m, n, k, what=f"{variant} {m}x{n}x{k}")
    assert np.array_equal(y, run_linear(stream, x, w, m, n, k, dispatch=d)), "split-K result differs between runs"
    y16 = run_linear(stream, x, w, m, n, k, dispatch=d, f16_out=True)
    check_against_oracle(oracle, y16, x, w, m, n, k, f16_out=True, what=f"{variant} f16")


@pytest.mark.parametrize("variant", SPLIT_K + Q8_SPLIT_K + GATE_UP_SPLIT_K)
def test_fold_matches_the_second_kernel(stream, variant):
    """The folded epilogue and the second kernel add the same parts in the
    same order: bitwise equal outputs, over consecutive calls of different
    shapes on one stream (each call must leave every tile counter at zero for
    the next; the last call repeats the first)."""
    fold, kernel = ops.Q4_0Dispatch(), ops.Q4_0Dispatch()
    fold.force(variant)
    fold.set_splitk_fold(True)
    kernel.force(variant)
    span = _slice(variant)
    for i, (m, n, parts) in enumerate([(3, 100, 2), (17, 130, 3), (64, 80, 7), (33, 1000, 2), (3, 100, 2)]):
        k = span * parts
        x = normal_x(wl.seed_for(46, m), m, k)
        f16_out = i == 1
        if variant.startswith("gateup_"):
            wg, wu = q4_weights(wl.seed_for(46, 100 + n), n, k), q4_weights(wl.seed_for(46, 200 + n), n, k)
            a = run_gate_up(stream, x, wg, wu, m, n, k, dispatch=fold, f16_out=f16_out)
            b = run_gate_up(stream, x, wg, wu, m, n, k, dispatch=kernel, f16_out=f16_out)
        elif variant.startswith("q8_"):
            w = q8.weights(wl.seed_for(46, 300 + n), n, k)
            a = q8.run(stream, x, w, m, n, k, dispatch=fold, f16_out=f16_out)
            b = q8.run(stream, x, w, m, n, k, dispatch=kernel, f16_out=f16_out)
        else:
            w = q4_weights(wl.seed_for(46, 400 + n), n, k)
            a = run_linear(stream, x, w, m, n, k, dispatch=fold, f16_out=f16_out)
            b = run_linear(stream, x, w, m, n, k, dispatch=kernel, f16_out=f16_out)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{variant} {m}x{n}x{k}: the epilogues differ"


@pytest.mark.parametrize("m", [2, 3, 8, 16, 32, 64])
def test_llama_down_projection_through_the_default_entry_point(stream, oracle, m):
    """The Llama-3-8B MLP down projection (K = 14336, N = 4096) at several
    token counts, through mote_hip_quantized_linear_q4_0_f32 (the library's
    own choice of kernel: the two-token streaming GEMV with rows split over
    4 waves, then the split-K tiles), checked on sampled columns."""
    k, n = 14336, 4096
    x = normal_x(wl.seed_for(41, m), m, k)
    w = q4_weights(wl.seed_for(41, 1), n, k)
    y = run_linear(stream, x, w, m, n, k)
    check_against_oracle(oracle, y, x, w, m, n, k, columns=sample_columns(n, 128), what=f"down {m}")


@pytest.mark.parametrize("variant", Q8_SPLIT_K)
def test_every_q8_split_k_variant(stream, oracle, variant):
    d = ops.Q4_0Dispatch()
    d.force(variant)
    span = _slice(variant)
    for m, n, parts in [(3, 100, 2), (16, 48, 3), (33, 7, 7), (64, 80, 2)]:
        k = span * parts
        x = q8.normal_x(wl.seed_for(42, m), m, k)
        w = q8.weights(wl.seed_for(42, 100 + n), n, k)
        y = q8.run(stream, x, w, m, n, k, dispatch=d)
        q8.check(oracle, y, x, w, m, n, k, what=f"{variant} {m}x{n}x{k}")
    y16 = q8.run(stream, x, w, m, n, k, dispatch=d, f16_out=True)
    q8.check(oracle, y16, x, w, m, n, k, f16_out=True, what=f"{variant} f16")


@pytest.mark.parametrize("variant", GATE_UP_SPLIT_K)
def test_every_gate_up_split_k_variant(stream, oracle, variant):
    """silu(gate) * up applied after the K parts are added: ragged tokens and
    rows, two, three and seven parts, f32 and f16 outputs, a repeat bitwise
    equal, separate and concatenated weight buffers identical."""
    d = ops.Q4_0Dispatch()
    d.force(variant)
    span = _slice(variant)
    for m, n, parts in [(1, 40, 2), (5, 33, 3), (17, 130, 2), (33, 7, 7), (64, 80, 2)]:
        k = span * parts
        x = normal_x(wl.seed_for(43, m), m, k)
        wg, wu = q4_weights(wl.seed_for(43, 100 + n), n, k), q4_weights(wl.seed_for(43, 200 + n), n, k)
        y = run_gate_up(stream, x, wg, wu, m, n, k, dispatch=d)
        check_gate_up(oracle, y, x, wg, wu, m, n, k, what=f"{variant} {m}x{n}x{k}")
    assert np.array_equal(y, run_gate_up(stream, x, wg, wu, m, n, k, dispatch=d)), "split-K result differs between runs"
    assert np.array_equal(y, run_gate_up(stream, x, wg, wu, m, n, k, dispatch=d, concatenated=True))
    y16 = run_gate_up(stream, x, wg, wu, m, n, k, dispatch=d, f16_out=True)
    check_gate_up(oracle, y16, x, wg, wu, m, n, k, f16_out=True, what=f"{variant} f16")


@pytest.mark.parametrize("m", [1, 2, 3, 4, 32])
def test_llama_70b_gate_up_through_the_default_entry_point(stream, oracle, m):
    """The Llama-3-70B fused gate/up (K = 8192, N = 28672) through
    mote_hip_quantized_gate_up_silu_q4_0_f32 (1-3 tokens on the streaming
    GEMV with rows split over 2 waves, then the split-K tiles), checked on
    sampled columns."""
    k, n = 8192, 28672
    x = normal_x(wl.seed_for(44, m), m, k)
    wg, wu = q4_weights(wl.seed_for(44, 1), n, k), q4_weights(wl.seed_for(44, 2), n, k)
    y = run_gate_up(stream, x, wg, wu, m, n, k)
    check_gate_up(oracle, y, x, wg, wu, m, n, k, cols=sample_columns(n, 96), what=f"70b gate/up {m}")


def test_scratch_growth_with_launches_in_flight(oracle):
    """Split-K calls on a new stream at growing sizes (then a small one),
    issued back to back with no synchronisation between them: the partial-tile
    buffer grows from 1 MiB to 32 MiB while earlier launches may still read
    the buffer they were given, and every output must match the oracle.  The
    stream is the caller's own (hipStreamCreate), so the library reserved no
    scratch for it."""
    from mote_amd.device import DeviceBuffer
    from mote_amd.hip_runtime import HipRuntime

    s = HipRuntime().foreign_stream()
    d = ops.Q4_0Dispatch()
    d.force("skinny_mfma_k8_s1_t2_d1_g1_r1_tr_l8_c_w_sk")  # 14 parts of 2048 at K = 28672
    k, n_max = 28672, 8192
    w = q4_weights(wl.seed_for(45, 1), n_max, k)
    wb = DeviceBuffer.from_array(w)
    cases = []
    for m, n in [(2, 1024), (16, 4096), (64, 8192), (3, 2048)]:
        x = normal_x(wl.seed_for(45, m), m, k)
        cases.append((m, n, x, DeviceBuffer.from_array(x), DeviceBuffer(m * n * 4)))
    for m, n, _, xb, yb in cases:  # uploads done: the launches queue up behind each other
        d.linear(xb.ptr, wb.ptr, yb.ptr, m, n, k, s)
    s.synchronize()
    row_bytes = wl.q4_0_row_bytes(k)
    for m, n, x, _, yb in cases:
        y = yb.download(np.float32).reshape(m, n)
        check_against_oracle(oracle, y, x, w[: n * row_bytes], m, n, k, columns=sample_columns(n, 64),
                             what=f"growth {m}x{n}x{k}")
    d.close()
    s.close()


def test_stream_destroyed_with_split_k_work_queued(oracle):
    """mote_hip_stream_destroy does not wait for the stream's work, as in the
    reference: split-K calls (a small one, then one that grows the scratch)
    are queued on a new stream that is destroyed at once, three times over,
    so later streams may reuse the address while the parked scratch of the
    earlier ones is still in use.  Every output must match the oracle, and
    once the device is idle the next stream destroy frees every parked
    buffer."""
    from mote_amd._ffi import check, lib
    from mote_amd.device import DeviceBuffer, Stream, memory_info
    from mote_amd.hip_runtime import HipRuntime

    hip = HipRuntime()
    d = ops.Q4_0Dispatch()
    d.force("skinny_mfma_k8_s1_t2_d1_g1_r1_tr_l8_c_w_sk")  # 14 parts of 2048 at K = 28672
    k, n_max = 28672, 8192
    w = q4_weights(wl.seed_for(46, 1), n_max, k)
    wb = DeviceBuffer.from_array(w)
    rounds = []
    for r in range(3):
        calls = []
        for m, n in [(16, 4096), (64, 8192)]:  # 4 MB of partial tiles, then 32 MB
            x = normal_x(wl.seed_for(46, 10 * r + m), m, k)
            calls.append((m, n, x, DeviceBuffer.from_array(x), DeviceBuffer(m * n * 4)))
        rounds.append(calls)
    idle = Stream()
    hip.device_synchronize()
    free_before = memory_info()[0]
    for calls in rounds:
        s = Stream()  # 64 MiB of scratch reserved, 3 x 64 MiB parked by the three destroys
        for m, n, _, xb, yb in calls:
            d.linear(xb.ptr, wb.ptr, yb.ptr, m, n, k, s)
        check(lib().mote_hip_stream_destroy(s.handle), "destroy stream")
        s.handle = 0
    hip.device_synchronize()
    idle.synchronize()  # frees the parked scratch whose work has completed
    free_after = memory_info()[0]
    idle.close()
    assert free_after >= free_before - (8 << 20), f"parked scratch not freed: {free_before - free_after} bytes held"
    row_bytes = wl.q4_0_row_bytes(k)
    for r, calls in enumerate(rounds):
        for m, n, x, _, yb in calls:
            y = yb.download(np.float32).reshape(m, n)
            check_against_oracle(oracle, y, x, w[: n * row_bytes], m, n, k, columns=sample_columns(n, 48),
                                 what=f"destroyed stream {r}: {m}x{n}x{k}")
    d.close()


@pytest.mark.parametrize("m,k,n,kind", [(4, 5120, 5120, "linear"), (32, 3072, 8192, "linear"), (64, 5120, 1024, "linear"),
                                        (8, 3072, 8192, "gate_up"), (24, 2048, 5632, "gate_up"),
                                        (4, 5120, 5120, "q8"), (40, 3072, 3072, "q8")])
def test_k_multiple_of_1024_through_the_default_entry_points(stream, oracle, m, k, n, kind):
    """Hidden sizes that no 2048-wide K slice divides (3072, 5120) and the
    gate/up at K = 2048: the default entry points use split-K parts of 1024;
    checked on sampled columns."""
    cols = sample_columns(n, 96)
    if kind == "q8":
        x = q8.normal_x(wl.seed_for(46, m), m, k)
        w = q8.weights(wl.seed_for(46, n), n, k)
        y = q8.run(stream, x, w, m, n, k)
        q8.check(oracle, y, x, w, m, n, k, columns=cols, what=f"q8 {m}x{n}x{k}")
        return
    x = normal_x(wl.seed_for(46, m), m, k)
    w = q4_weights(wl.seed_for(46, n), n, k)
    if kind == "linear":
        y = run_linear(stream, x, w, m, n, k)
        check_against_oracle(oracle, y, x, w, m, n, k, columns=cols, what=f"linear {m}x{n}x{k}")
    else:
        wu = q4_weights(wl.seed_for(47, n), n, k)
        y = run_gate_up(stream, x, w, wu, m, n, k)
        check_gate_up(oracle, y, x, w, wu, m, n, k, cols=cols, what=f"gate/up {m}x{n}x{k}")
