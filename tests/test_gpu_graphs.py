"""The entry points captured in a HIP graph and replayed.

A serving loop captures a decoder step once and replays it; every kernel here
must then behave exactly as when issued eagerly.  The test issues a step's
worth of calls eagerly (fused add + RMSNorm, Q4_0 linears at 1, 16 and 512
tokens, the 16-token down projection on the split-K tiles, whose scratch the
eager call sizes, the fused gate/up at 1 and 16 tokens, a Q8_0 linear, q/k
RoPE),
captures the same calls into a graph, and replays it three times.  Before
every replay the outputs are overwritten with a sentinel and the residual
(updated in place by the fused norm) is restored, eagerly, on the same stream;
each replay must reproduce the eager outputs bit for bit.  No entry point
records a memset or synchronises, so capture needs nothing special once a
shape's plan is cached (the default entry points choose plans on the host).
"""

from __future__ import annotations

import numpy as np
import pytest

from mote_amd import ops, workloads as wl
from mote_amd.device import DeviceBuffer
from mote_amd.hip_runtime import HipRuntime

pytestmark = pytest.mark.gpu

H, FF, HEADS, KV, HD = 4096, 14336, 32, 8, 128


def test_decoder_step_graph_replays_match_eager(stream):
    hip = HipRuntime()
    bufs = {}

    def buf(name, array):
        bufs[name] = DeviceBuffer.from_array(array)
        return bufs[name]

    def out(name, nbytes):
        bufs[name] = DeviceBuffer(nbytes)
        return bufs[name]

    x1 = buf("x1", wl.normal_f16(40, H))
    x16 = buf("x16", wl.normal_f16(41, 16 * H))
    x512 = buf("x512", wl.normal_f16(42, 512 * H))
    x16ff = buf("x16ff", wl.normal_f16(51, 16 * FF))
    res = wl.normal_f16(43, 16 * H)
    r16 = buf("res", res)
    nw = buf("nw", wl.normal_f16(44, H, mean=1.0, std=0.1))
    wq4 = buf("wq4", wl.q4_0_weights(45, FF, H))
    wup = buf("wup", wl.q4_0_weights(46, FF, H))
    wq8 = buf("wq8", wl.q8_0_weights(47, 1024, H))
    pos = wl.positions(48, 16)
    cos, sin = wl.rope_tables(pos, HD, 500000.0)
    c, s = buf("cos", cos), buf("sin", sin)
    q = buf("q", wl.normal_f16(49, 16 * HEADS * HD))
    k = buf("k", wl.normal_f16(50, 16 * KV * HD))
    outs = {
        "norm": out("norm", 16 * H * 2),
        "y1": out("y1", FF * 4),
        "y16": out("y16", 16 * FF * 4),
        "y512": out("y512", 512 * FF * 4),
        "down16": out("down16", 16 * H * 4),
        "gu1": out("gu1", FF * 4),
        "gu16": out("gu16", 16 * FF * 4),
        "q8": out("q8", 1024 * 4),
        "qo": out("qo", 16 * HEADS * HD * 2),
        "ko": out("ko", 16 * KV * HD * 2),
    }

    def step():
        ops.fused_add_rms_norm_f16(x16.ptr, r16.ptr, nw.ptr, outs["norm"].ptr, 16, H, 1e-5, stream)
        ops.quantized_linear_q4_0_f32(x1.ptr, wq4.ptr, outs["y1"].ptr, 1, FF, H, stream)
        ops.quantized_linear_q4_0_f32(x16.ptr, wq4.ptr, outs["y16"].ptr, 16, FF, H, stream)
        ops.quantized_linear_q4_0_f32(x512.ptr, wq4.ptr, outs["y512"].ptr, 512, FF, H, stream)
        # the gate bytes read as [H, FF]: the same 18-byte blocks, regrouped into rows
        ops.quantized_linear_q4_0_f32(x16ff.ptr, wq4.ptr, outs["down16"].ptr, 16, H, FF, stream)
        ops.q4_0_gate_up_silu_f32(x1.ptr, wq4.ptr, wup.ptr, outs["gu1"].ptr, 1, FF, H, stream)
        ops.q4_0_gate_up_silu_f32(x16.ptr, wq4.ptr, wup.ptr, outs["gu16"].ptr, 16, FF, H, stream)
        ops.quantized_linear_q8_0_f32(x1.ptr, wq8.ptr, outs["q8"].ptr, 1, 1024, H, stream)
        ops.rope_qk_f16(q.ptr, k.ptr, c.ptr, s.ptr, outs["qo"].ptr, outs["ko"].ptr, 16, HEADS, KV, HD, HD,
                        ops.HALF_SPLIT, stream)

    def reset():
        for b in outs.values():
            b.upload(np.full(b.nbytes, 0xA5, dtype=np.uint8))
        r16.upload(res)

    def snapshot():
        stream.synchronize()
        return {name: b.download(np.uint8) for name, b in outs.items()} | {"res": r16.download(np.uint8)}

    reset()
    step()
    eager = snapshot()
    assert not np.array_equal(eager["res"], res.view(np.uint8))  # the norm updated the residual

    exe = hip.capture(stream, step)
    try:
        for replay in range(3):
            reset()
            hip.launch_graph(exe, stream)
            got = snapshot()
            for name, want in eager.items():
                assert np.array_equal(got[name], want), f"replay {replay}: {name} differs from the eager run"
    finally:
        hip.destroy_graph(exe)
        for b in bufs.values():
            b.free()


def test_first_split_k_call_under_capture(oracle):
    """A split-K call (16 tokens of the Llama-3-8B down projection, K = 14336)
    captured before any eager call on its stream.  On a stream the library
    created, the scratch reserved at creation holds the partial tiles, so the
    graph runs the split-K tiles: bit for bit the eager result.  On the
    caller's own stream the library has no scratch yet and a capture may not
    allocate, so the captured call runs the best plan without split K (to the
    oracle's tolerance); the next eager call sizes the scratch and runs the
    split-K tiles again."""
    from mote_amd.device import Stream
    from test_gpu_q4_0 import check_against_oracle, sample_columns

    m, n, k = 16, 4096, 14336
    assert ops.Q4_0Dispatch().select(m, n, k).endswith("_sk")  # the shape plans the split-K tiles
    hip = HipRuntime()
    x, w = wl.normal_f16(52, m * k), wl.q4_0_weights(53, n, k)
    xb, wb = DeviceBuffer.from_array(x), DeviceBuffer.from_array(w)
    ys = {name: DeviceBuffer(m * n * 4) for name in ("eager", "graph", "foreign_graph", "foreign_eager")}
    cols = sample_columns(n, 96)

    def call(out, s):
        return lambda: ops.quantized_linear_q4_0_f32(xb.ptr, wb.ptr, ys[out].ptr, m, n, k, s)

    def result(out, s):
        s.synchronize()
        return ys[out].download(np.float32).reshape(m, n)

    own, foreign = Stream(), hip.foreign_stream()
    try:
        for out in ys:
            ys[out].upload(np.full(m * n * 4, 0xA5, dtype=np.uint8))
        exe = hip.capture(own, call("graph", own))
        try:
            hip.launch_graph(exe, own)
            graph = result("graph", own)
        finally:
            hip.destroy_graph(exe)
        call("eager", own)()
        eager = result("eager", own)
        check_against_oracle(oracle, eager, x, w, m, n, k, columns=cols, what="eager split K")
        assert np.array_equal(graph, eager), "the captured call on the library's stream is not the split-K result"

        exe = hip.capture(foreign, call("foreign_graph", foreign))
        try:
            hip.launch_graph(exe, foreign)
            captured = result("foreign_graph", foreign)
        finally:
            hip.destroy_graph(exe)
        check_against_oracle(oracle, captured, x, w, m, n, k, columns=cols, what="captured without split K")
        call("foreign_eager", foreign)()
        assert np.array_equal(result("foreign_eager", foreign), eager), "the eager call after capture is not split K"
    finally:
        foreign.close()
        own.close()
        for b in [xb, wb, *ys.values()]:
            b.free()


@pytest.mark.parametrize("name", ["q4_k", "q6_k"])
def test_k_quant_split_k_under_capture(oracle, name):
    """The K-quant split-K tiles (16 tokens, K = 14336: four K parts) under
    capture.  On a stream the library created, its reserved scratch holds the
    partial planes: the graph, replayed three times with the output reset to
    a sentinel between replays, gives the eager result bit for bit.  On the
    caller's own stream the library has no scratch yet and a capture may not
    allocate, so the captured call runs the ring GEMV (to the oracle's
    tolerance); the next eager call sizes the scratch and gives the split-K
    result again."""
    from mote_amd.device import Stream
    from test_gpu_kquant import FORMATS, _check, _judge

    m, n, k = 16, 1024, 14336
    hip = HipRuntime()
    w = (wl.q4_k_weights if name == "q4_k" else wl.q6_k_weights)(54, n, k)
    x = wl.normal_f16(55, m * k)
    y64, max_w, max_x = _judge(oracle, name, x, w, m, n, k)
    xb, wb = DeviceBuffer.from_array(x), DeviceBuffer.from_array(w)
    ys = {out: DeviceBuffer(m * n * 4) for out in ("eager", "graph", "foreign_graph", "foreign_eager")}
    linear = FORMATS[name][2]

    def call(out, s):
        return lambda: linear(xb.ptr, wb.ptr, ys[out].ptr, m, n, k, s)

    def result(out, s):
        s.synchronize()
        return ys[out].download(np.float32).reshape(m, n).astype(np.float64)

    own, foreign = Stream(), hip.foreign_stream()
    try:
        for out in ys:
            ys[out].upload(np.full(m * n * 4, 0xA5, dtype=np.uint8))
        exe = hip.capture(own, call("graph", own))
        try:
            graphs = []
            for _ in range(3):
                ys["graph"].upload(np.full(m * n * 4, 0xA5, dtype=np.uint8))
                own.synchronize()
                hip.launch_graph(exe, own)
                graphs.append(result("graph", own))
        finally:
            hip.destroy_graph(exe)
        call("eager", own)()
        eager = result("eager", own)
        _check(eager, y64, k, max_w, max_x, what=f"{name} eager split K")
        for i, g in enumerate(graphs):
            assert np.array_equal(g, eager), f"{name}: replay {i} on the library's stream is not the split-K result"

        exe = hip.capture(foreign, call("foreign_graph", foreign))
        try:
            hip.launch_graph(exe, foreign)
            captured = result("foreign_graph", foreign)
        finally:
            hip.destroy_graph(exe)
        _check(captured, y64, k, max_w, max_x, what=f"{name} captured without scratch (ring)")
        call("foreign_eager", foreign)()
        assert np.array_equal(result("foreign_eager", foreign), eager), f"{name}: the eager call after capture is not split K"
    finally:
        foreign.close()
        own.close()
        for b in [xb, wb, *ys.values()]:
            b.free()
