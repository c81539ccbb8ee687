"""Benchmark of the Q4_0 quantized-linear hot path on one MI355X.

Workload (the headline case): the Llama-3-8B MLP up/gate decode linear,
M = 1 token, K = 4096 input features, N = 14336 output features, GGML Q4_0
weights (18-byte blocks of 32), f16 activations, f32 output, through the C ABI
entry point ``mote_hip_quantized_linear_q4_0_f32`` of ``libmote_hip.so``.

* A "step" is one call of the linear.  ``--warmup`` untimed calls, then
  ``--steps`` calls captured once into a HIP graph (stream capture of the C-ABI
  calls) and replayed three times, bracketed by HIP events recorded on the
  launch stream and by the host clock (stream synchronised on both sides).
  The graph issues the kernels back to back with no host work in between, as
  a decode loop captured in a graph does; the eager rate (one Python ctypes
  call per step, bounded by the host for kernels this short) is reported
  beside it.
* The weights rotate over enough distinct device copies (>= 384 MB) that no
  call finds its matrix in the 256 MB last-level cache (MALL): every call
  reads its weights from HBM, as a decode step over a real model does.
* Algorithmic bytes per call: |W| = N (K/32) 18, |x| = 2 M K, |y| = 4 M N,
  each counted once (33 095 680 B for the headline case).
* ``value`` is the whole-job rate, bytes x calls / host time of the replays;
  ``roofline.achieved`` divides the same bytes by the average launch duration
  from the events (the kernels run back to back, so this agrees with the
  kernel durations of a rocprofv3 kernel trace).
* ``roofline.traffic`` is the HBM traffic per launch measured by rocprofv3
  counters, read from the committed summary under ``profiles/`` (null when
  absent); the line says so in ``roofline.traffic_source``.
* ``reference_statistics`` (and ``kernel_us_median`` / ``kernel_us_spread_pct``)
  are the reference benchmark's statistics: 5 warm-ups, 9 samples of 20
  calls, median and spread (max - min) / median, each sample one replay of a
  graph of 20 captured calls timed by events on the launch stream.
* ``cpu_baseline`` times the single-threaded C restatement of the reference's
  CPU oracle (``quantized_linear_f32``, crates/mote-reference/src/
  quantized.rs:89-144) on the same inputs for a bounded number of calls, and
  uses its output to check the GPU result.

Usage: ``python bench.py [--gpus 1] [--steps K] [--warmup W] [--sweep]``.
``--sweep`` also prints one line per parity-test configuration to stderr.
"""

from __future__ import annotations

import argparse
import ctypes
import faulthandler
import json
import math
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from mote_amd import _ffi, ops, workloads as wl  # noqa: E402
from mote_amd.device import DeviceBuffer, Stream, device_count  # noqa: E402
from mote_amd.hip_runtime import HipRuntime  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 << 20
ROTATION_BYTES = 384 << 20
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "q4_0_gemv_m1_k4096_n14336_traffic.md")


def linear_bytes(m: int, n: int, k: int, out_bytes: int = 4) -> int:
    return n * (k // 32) * 18 + 2 * m * k + out_bytes * m * n


def read_traffic() -> dict | None:
    """Per-launch HBM bytes from the committed rocprofv3 counter summary: the
    line ``traffic_bytes_per_launch: <int>`` (FETCH_SIZE + WRITE_SIZE, scaled by
    the copy-kernel calibration stated in the summary)."""
    try:
        with open(TRAFFIC_SUMMARY, encoding="utf-8") as f:
            text = f.read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", text)
    return int(m.group(1)) if m else None


class LinearCase:
    """Device buffers for one Q4_0 (or Q8_0) linear problem with rotating weight copies."""

    def __init__(self, m: int, n: int, k: int, workload: int, x_uniform: bool = False,
                 gate_up: bool = False, q8_0: bool = False, reference_inputs: bool = False,
                 kquant: str | None = None) -> None:
        """`reference_inputs`: the reference benchmark's closed-form inputs
        and weights, through the F16-output entry point it times
        (crates/mote-backend-hip/benches/quantized_linear.rs:8-13,128-152).
        `kquant`: "q4_k" or "q6_k" weights through their f32 entry points."""
        self.m, self.n, self.k, self.gate_up, self.q8_0 = m, n, k, gate_up, q8_0
        self.f16_out = reference_inputs
        self.kquant = kquant
        if reference_inputs:
            self.x = wl.reference_bench_inputs(m, k)
            self.w = wl.reference_bench_q4_0_weights(n, k)
        elif kquant is not None:
            self.x = wl.normal_f16(wl.seed_for(workload, 0), m * k)
            self.w = (wl.q4_k_weights if kquant == "q4_k" else wl.q6_k_weights)(wl.seed_for(workload, 1), n, k)
        else:
            self.x = (wl.uniform_f16 if x_uniform else wl.normal_f16)(wl.seed_for(workload, 0), m * k)
            self.w = (wl.q8_0_weights if q8_0 else wl.q4_0_weights)(wl.seed_for(workload, 1), n, k)
        self.w_up = wl.q4_0_weights(wl.seed_for(workload, 2), n, k) if gate_up else None
        per_copy = self.w.nbytes * (2 if gate_up else 1)
        self.copies = max(2, math.ceil(ROTATION_BYTES / per_copy))
        self.xb = DeviceBuffer.from_array(self.x)
        self.wb = []
        for _ in range(self.copies):
            mats = [self.w] if not gate_up else [self.w, self.w_up]
            self.wb.append([DeviceBuffer.from_array(a) for a in mats])
        self.yb = DeviceBuffer(m * n * 4)

    def launch(self, i: int, stream: Stream) -> None:
        bufs = self.wb[i % self.copies]
        if self.gate_up:
            ops.q4_0_gate_up_silu_f32(self.xb.ptr, bufs[0].ptr, bufs[1].ptr, self.yb.ptr,
                                      self.m, self.n, self.k, stream)
        elif self.q8_0:
            ops.quantized_linear_q8_0_f32(self.xb.ptr, bufs[0].ptr, self.yb.ptr,
                                          self.m, self.n, self.k, stream)
        elif self.kquant is not None:
            fn = ops.quantized_linear_q4_k_f32 if self.kquant == "q4_k" else ops.quantized_linear_q6_k_f32
            fn(self.xb.ptr, bufs[0].ptr, self.yb.ptr, self.m, self.n, self.k, stream)
        elif self.f16_out:
            ops.quantized_linear_q4_0_f16(self.xb.ptr, bufs[0].ptr, self.yb.ptr,
                                          self.m, self.n, self.k, stream)
        else:
            ops.quantized_linear_q4_0_f32(self.xb.ptr, bufs[0].ptr, self.yb.ptr,
                                          self.m, self.n, self.k, stream)

    def algorithmic_bytes(self) -> int:
        if self.q8_0 or self.kquant is not None:
            return self.w.nbytes + 2 * self.m * self.k + 4 * self.m * self.n
        b = linear_bytes(self.m, self.n, self.k, 2 if self.f16_out else 4)
        return b + (self.w_up.nbytes if self.gate_up else 0)

    def flops(self) -> int:
        return 2 * self.m * self.n * self.k * (2 if self.gate_up else 1)

    def output(self) -> np.ndarray:
        return self.yb.download(np.float32).reshape(self.m, self.n)

    def free(self) -> None:
        self.xb.free()
        self.yb.free()
        for bufs in self.wb:
            for b in bufs:
                b.free()


SETTLE_S = 0.02  # untimed graph replays before the timed ones


def time_case(case: LinearCase, stream: Stream, hip: HipRuntime, steps: int, warmup: int,
              replays: int = 3) -> dict:
    """`steps` calls back to back, issued two ways.

    * graph: the `steps` C-ABI calls are captured once into a HIP graph, which
      is then replayed; the kernels run back to back with no host work between
      them.  An event pair on the launch stream around the replays gives the
      average kernel launch duration (it agrees with rocprofv3's kernel trace),
      and the host clock around the same replays the whole-job rate.
    * eager: each call enqueued from Python through ctypes; for kernels of a
      few microseconds this rate is bounded by the host, and is reported for
      reference only.
    """
    for i in range(warmup):
        case.launch(i, stream)
    stream.synchronize()

    start, stop = hip.create(), hip.create()
    hip.record(start, stream)
    t0 = time.perf_counter()
    for i in range(steps):
        case.launch(i, stream)
    hip.record(stop, stream)
    stream.synchronize()
    eager_wall_s = time.perf_counter() - t0
    eager_gpu_ms = hip.elapsed_ms(start, stop)

    exe = hip.capture(stream, lambda: [case.launch(i, stream) for i in range(steps)])
    try:
        # Untimed replays for at least SETTLE_S first: after a short warm-up
        # the device still runs below its steady clocks (measured on MI355X
        # at the headline shape: 7.96 us per call after 20 warm-up calls,
        # 7.57-7.58 us after 2000 or 20000).
        t0 = time.perf_counter()
        while True:
            hip.launch_graph(exe, stream)
            stream.synchronize()
            if time.perf_counter() - t0 >= SETTLE_S:
                break
        t0 = time.perf_counter()
        hip.record(start, stream)
        for _ in range(replays):
            hip.launch_graph(exe, stream)
        hip.record(stop, stream)
        stream.synchronize()
        wall_s = time.perf_counter() - t0
        gpu_ms = hip.elapsed_ms(start, stop)
    finally:
        hip.destroy_graph(exe)
        hip.destroy(start)
        hip.destroy(stop)
    calls = steps * replays
    return {
        "ms_per_step": wall_s * 1e3 / calls,
        "kernel_ms_mean": gpu_ms / calls,
        "eager_ms_per_step": eager_wall_s * 1e3 / steps,
        "eager_gpu_ms_per_step": eager_gpu_ms / steps,
    }


REF_WARMUPS, REF_SAMPLES, REF_BATCH = 5, 9, 20


def reference_statistics(case: LinearCase, stream: Stream, hip: HipRuntime) -> dict:
    """The reference benchmark's statistics (crates/mote-backend-hip/benches/
    quantized_linear.rs:14-16,51-62): 5 warm-ups, then 9 samples of 20 calls,
    the median µs per call and the spread (max - min) / median.  Here the 20
    calls of a sample are one replay of a captured graph (rotating weight
    copies, as every call of this benchmark), timed by HIP events on the launch
    stream; the host clock around the same replay (synchronised, as the
    reference's Instant pair) is reported beside it."""
    exe = hip.capture(stream, lambda: [case.launch(i, stream) for i in range(REF_BATCH)])
    start, stop = hip.create(), hip.create()
    try:
        t0 = time.perf_counter()
        while True:  # the same settling as the timed replays of time_case
            hip.launch_graph(exe, stream)
            stream.synchronize()
            if time.perf_counter() - t0 >= SETTLE_S:
                break
        for _ in range(REF_WARMUPS):
            hip.launch_graph(exe, stream)
        stream.synchronize()
        dev, host = [], []
        for _ in range(REF_SAMPLES):
            t0 = time.perf_counter()
            hip.record(start, stream)
            hip.launch_graph(exe, stream)
            hip.record(stop, stream)
            stream.synchronize()
            host.append((time.perf_counter() - t0) * 1e6 / REF_BATCH)
            dev.append(hip.elapsed_ms(start, stop) * 1e3 / REF_BATCH)
    finally:
        hip.destroy_graph(exe)
        hip.destroy(start)
        hip.destroy(stop)
    dev.sort()
    host.sort()
    med, hmed = dev[REF_SAMPLES // 2], host[REF_SAMPLES // 2]
    return {
        "warmups": REF_WARMUPS, "samples": REF_SAMPLES, "calls_per_sample": REF_BATCH,
        "kernel_us_median": round(med, 3),
        "kernel_us_min": round(dev[0], 3),
        "kernel_us_max": round(dev[-1], 3),
        "spread_pct": round((dev[-1] - dev[0]) / med * 100.0, 2),
        "host_us_median": round(hmed, 3),
        "host_spread_pct": round((host[-1] - host[0]) / hmed * 100.0, 2),
        "clock": "HIP events on the launch stream around one graph replay of 20 captured calls per sample",
    }


def cpu_baseline(case: LinearCase, budget_s: float) -> tuple[dict, np.ndarray]:
    """The single-threaded C oracle on the same inputs: calls until `budget_s`
    of CPU time (at least one).  Returns the report and one f32 output."""
    import oracle  # the CPU restatement of the reference oracle (checker only)

    x32 = case.x.view(np.float16).astype(np.float32)
    first = oracle.time_quantized_linear_f32(x32, case.w, case.m, case.n, case.k, 1)
    calls = max(1, min(200, int(budget_s / max(first, 1e-6))))
    seconds = oracle.time_quantized_linear_f32(x32, case.w, case.m, case.n, case.k, calls)
    y_cpu = oracle.quantized_linear_f32(x32, case.w, oracle.Q4_0, case.m, case.n, case.k)
    per_call = seconds / calls
    report = {
        "value": round(case.algorithmic_bytes() / per_call / 1e9, 4),
        "unit": "GB/s",
        "us_per_call": round(per_call * 1e6, 1),
        "cores": 1,
        "kind": "port",
        "sample": (f"{calls} calls of the f32 oracle (gcc -O2, -ffp-contract=off) at "
                   f"M={case.m} K={case.k} N={case.n}, {seconds:.1f} s, host has "
                   f"{os.cpu_count()} cores"),
    }
    return report, y_cpu.reshape(case.m, case.n)


def check_output(case: LinearCase, y_cpu: np.ndarray) -> None:
    """Parity with the oracle's f32 output: |y - y_cpu| <= 1e-3 |y_cpu| +
    2e-3 sqrt(K) max|d| max|x| (the f32 oracle itself is within a few ulps of
    the f64 sum at these sizes)."""
    y = case.output()
    scales = case.w.reshape(case.n, case.k // 32, 18)[:, :, 0:2].copy().view("<u2")[..., 0]
    max_d = float(np.abs(scales.view(np.float16).astype(np.float32)).max())
    max_x = float(np.abs(case.x.view(np.float16).astype(np.float32)).max())
    tol = np.maximum(1e-3 * np.abs(y_cpu), 2e-3 * math.sqrt(case.k) * max_d * max_x)
    bad = np.abs(y.astype(np.float64) - y_cpu) > tol
    if bad.any():
        raise SystemExit(f"bench: GPU output differs from the oracle in {int(bad.sum())} elements")


def profile_run(case: LinearCase, stream: Stream, hip: HipRuntime) -> int:
    """Copy one weight matrix device to device (reads and writes |W| bytes:
    the runtime's copy kernel calibrates the HBM byte counters), then run the
    headline linear 20 times on rotating weight copies."""
    dst = DeviceBuffer(case.w.nbytes)
    hip.copy_device_to_device(dst.ptr, case.wb[0][0].ptr, case.w.nbytes)
    for i in range(20):
        case.launch(i + 1, stream)
    stream.synchronize()
    print(f"profile run: copied {case.w.nbytes} bytes, 20 calls of M={case.m} K={case.k} N={case.n}"
          f"{' gate/up' if case.gate_up else ''}", file=sys.stderr)
    dst.free()
    case.free()
    stream.close()
    return 0


SWEEP = (
    [("decode", 1, 4096, 4096, 0, True, False), ("mlp up/gate", 1, 4096, 14336, 1, False, False),
     ("mlp down", 1, 14336, 4096, 1, False, False)]
    + [("skinny", m, 4096, n, 2, False, False) for n in (4096, 6144, 14336) for m in (2, 4, 8, 16, 32)]
    + [("prefill", m, 4096, 14336, 4, False, False) for m in (64, 256, 512)]
    # prefill beyond one dispatch wave of tiles, and the q/o projection's N = 4096
    + [("prefill", m, 4096, 14336, 4, False, False) for m in (384, 1024)]
    + [("prefill o proj", m, 4096, 4096, 4, False, False) for m in (128, 256, 512)]
    + [("down split-K", m, 14336, 4096, 2, False, False) for m in (2, 4, 16, 32, 64)]
    + [("70b o split-K", m, 8192, 8192, 2, False, False) for m in (16, 64)]
    + [("70b down", m, 28672, 8192, 2, False, False) for m in (1, 2, 16, 64)]
    + [("13b linear", m, 5120, 5120, 2, False, False) for m in (4, 32)]
    + [("fused gate/up", m, 4096, 14336, 4, False, True) for m in (1, 2, 4, 16, 32, 64, 256, 512)]
    + [("70b gate/up", m, 8192, 28672, 4, False, True) for m in (1, 4, 16, 32, 64)]
    + [("q8_0 decode", 1, 4096, 4096, 5, False, "q8"), ("q8_0 up/gate", 1, 4096, 14336, 5, False, "q8"),
       ("q8_0 down", 1, 14336, 4096, 5, False, "q8"), ("q8_0 2 tok", 2, 4096, 14336, 5, False, "q8"),
       ("q8_0 4 tok", 4, 4096, 14336, 5, False, "q8")]
    + [("q8_0 skinny", m, 4096, 14336, 5, False, "q8") for m in (8, 16, 32, 64)]
    + [("q8_0 prefill", m, 4096, 14336, 5, False, "q8") for m in (256, 512)]
    + [("q8_0 prefill o proj", 256, 4096, 4096, 5, False, "q8")]
    + [("3 tok o proj", 3, 8192, 8192, 2, False, False), ("3 tok down", 3, 14336, 4096, 2, False, False),
       ("q8_0 3 tok", 3, 8192, 8192, 5, False, "q8"), ("3 tok gate/up", 3, 8192, 28672, 4, False, True)]
    # the reference benchmark's cases (rows, N, K), its inputs, the F16-output entry point
    + [("ref bench f16", m, k, n, 0, False, "ref") for m, n, k in
       ((1, 4096, 4096), (1, 11008, 4096), (1, 4096, 11008), (16, 4096, 4096))]
    # K-quant GEMV (Q4_K, Q6_K): the decode-shaped linears
    + [(f"{f} {what}", m, k, n, 6, False, f) for f in ("q4_k", "q6_k")
       for what, m, k, n in (("decode", 1, 4096, 4096), ("up/gate", 1, 4096, 14336), ("down", 1, 14336, 4096),
                             ("2 tok", 2, 4096, 14336), ("3 tok", 3, 4096, 14336), ("4 tok", 4, 4096, 14336), ("8 tok", 8, 4096, 14336), ("16 tok", 16, 4096, 14336),
                             ("32 tok", 32, 4096, 14336), ("64 tok", 64, 4096, 14336))]
)


# The plan table's workloads (op: 0 linear, 1 fused gate/up; M, K, N): the
# decode linears (1 x 4096 x 4096, the Llama-3-8B up/gate and down), the
# reference benchmark's 11 008 shapes, the skinny sweep (2-32 tokens, K =
# 4096, N = 4096 / 6144 / 14 336) and the prefill linears and gate/up (64,
# 256, 512 tokens, 4096 x 14 336).
PLAN_SHAPES = (
    [(0, 1, 4096, 4096), (0, 1, 4096, 14336), (0, 1, 14336, 4096), (0, 1, 4096, 11008), (0, 1, 11008, 4096)]
    + [(0, m, 4096, n) for n in (4096, 6144, 14336) for m in (2, 4, 8, 16, 32)]
    + [(op, m, 4096, 14336) for op in (0, 1) for m in (64, 256, 512)]
)


class ForcedCase:
    """A LinearCase run through a dispatch context with one variant forced."""

    def __init__(self, case: LinearCase, dispatch: "ops.Q4_0Dispatch") -> None:
        self.case, self.dispatch = case, dispatch

    def launch(self, i: int, stream: Stream) -> None:
        c, bufs = self.case, self.case.wb[i % self.case.copies]
        if c.gate_up:
            self.dispatch.gate_up_silu(c.xb.ptr, bufs[0].ptr, bufs[1].ptr, c.yb.ptr, c.m, c.n, c.k, stream)
        else:
            self.dispatch.linear(c.xb.ptr, bufs[0].ptr, c.yb.ptr, c.m, c.n, c.k, stream)

    def algorithmic_bytes(self) -> int:
        return self.case.algorithmic_bytes()


def run_plan_table(stream: Stream, hip: HipRuntime, path: str, steps: int = 50, warmup: int = 5,
                   samples: int = 3) -> None:
    """Times every candidate variant of every PLAN_SHAPES workload (the median
    of `samples` kernel means over `steps` graph-replayed calls, weights
    rotated past the MALL) and writes the entries as the C++ initialiser list
    that q4_0_api.hip compiles in as its plan table."""
    d = ops.Q4_0Dispatch()
    lines = []
    print(f"{'op':<8}{'M':>5}{'K':>7}{'N':>7}  {'fastest':<48}{'us':>8}  this build's plan (us)", file=sys.stderr)
    for op, m, k, n in PLAN_SHAPES:
        case = LinearCase(m, n, k, workload=4 if m >= 64 else (2 if m > 1 else 1), gate_up=op == 1)
        d.force(None)
        names = d.candidates(m, n, k, gate_up=op == 1)
        timed = []
        for name in names:
            d.force(name)
            fc = ForcedCase(case, d)
            us = sorted(time_case(fc, stream, hip, steps, warmup)["kernel_ms_mean"] * 1e3
                        for _ in range(samples))[samples // 2]
            timed.append((us, name))
            lines.append(f"    {{{op}, {m}, {k}, {n}, \"{name}\", {us:.3f}}},")
        d.force(None)
        timed.sort()
        by_name = {v: u for u, v in timed}
        sel = d.select(m, n, k, gate_up=op == 1)  # the table compiled into this build, then the rules
        print(f"{('gate/up' if op else 'linear'):<8}{m:>5}{k:>7}{n:>7}  {timed[0][1]:<48}{timed[0][0]:>8.2f}  "
              f"{sel} ({by_name.get(sel, float('nan')):.2f})", file=sys.stderr, flush=True)
        case.free()
    d.close()
    with open(path, "w") as f:
        f.write("// The plan table: {op (0 linear, 1 gate/up), M, K, N, variant, kernel us}, every candidate of\n"
                "// each workload, median of %d samples of %d graph-replayed calls (weights rotated past the\n"
                "// MALL).  Generated on MI355X by: python bench.py --plan-table <this file>\n" % (samples, steps))
        f.write("\n".join(lines) + "\n")
    print(f"plan table: {len(lines)} entries -> {path}", file=sys.stderr, flush=True)


class CopyRowsCase:
    """The probe library's row copy (one 256-thread workgroup per row), the
    smallest kernel of the norm's launch shape."""

    def __init__(self, probe, rows: int, row_bytes: int) -> None:
        self.probe, self.rows, self.row_bytes = probe, rows, row_bytes
        self.src = DeviceBuffer(rows * row_bytes)
        self.src.upload(np.arange(rows * row_bytes, dtype=np.uint32).astype(np.uint8))
        self.dst = DeviceBuffer(rows * row_bytes)

    def launch(self, i: int, stream: Stream) -> None:
        _ffi.check(self.probe.mote_probe_copy_rows(self.src.ptr, self.dst.ptr, self.rows, self.row_bytes,
                                                   stream.handle), "copy probe")

    def algorithmic_bytes(self) -> int:
        return 2 * self.rows * self.row_bytes

    def free(self) -> None:
        self.src.free()
        self.dst.free()


class NormRopeCase:
    """RMSNorm, fused add + RMSNorm or q/k RoPE on the decoder-step shape: 32
    tokens, hidden 4096 (f16, eps 1e-5, weight f16(1 + 0.1 N(0,1))); RoPE on 32
    query and 8 KV heads of head_dim 128, theta 500000, rotate-half layout,
    positions uniform in [0, 8191].  Algorithmic bytes: every input and output
    element once (RMSNorm 532 480 B, fused add + RMSNorm 1 056 768 B with the
    residual read and written back, RoPE 671 744 B)."""

    TOKENS, HIDDEN, QH, KH, HD = 32, 4096, 32, 8, 128

    def __init__(self, kind: str) -> None:
        self.kind = kind
        t, h = self.TOKENS, self.HIDDEN
        self.bufs = []
        def buf(arr):
            b = DeviceBuffer.from_array(arr)
            self.bufs.append(b)
            return b
        if kind in ("rmsnorm", "fused add+rmsnorm"):
            self.x = buf(wl.normal_f16(wl.seed_for(3, 0), t * h))
            self.res = buf(wl.normal_f16(wl.seed_for(3, 2), t * h))
            self.w = buf(wl.normal_f16(wl.seed_for(3, 1), h, mean=1.0, std=0.1))
            self.y = buf(np.zeros(t * h, np.uint16))
            self.nbytes = (2 * t * h + h) * 2 + (2 * t * h * 2 if kind != "rmsnorm" else 0)
        else:
            pos = wl.positions(wl.seed_for(3, 3), t)
            cos, sin = wl.rope_tables(pos, self.HD, 500000.0)
            self.q = buf(wl.normal_f16(wl.seed_for(3, 4), t * self.QH * self.HD))
            self.k = buf(wl.normal_f16(wl.seed_for(3, 5), t * self.KH * self.HD))
            self.cos, self.sin = buf(cos), buf(sin)
            self.qo = buf(np.zeros(t * self.QH * self.HD, np.uint16))
            self.ko = buf(np.zeros(t * self.KH * self.HD, np.uint16))
            self.nbytes = 2 * t * (self.QH + self.KH) * self.HD * 2 + 2 * cos.nbytes
        self.m, self.n, self.k_dim = t, h, 0

    def launch(self, i: int, stream: Stream) -> None:
        t, h = self.TOKENS, self.HIDDEN
        if self.kind == "rmsnorm":
            ops.rms_norm_f16(self.x.ptr, self.w.ptr, self.y.ptr, t, h, 1e-5, stream)
        elif self.kind == "fused add+rmsnorm":
            ops.fused_add_rms_norm_f16(self.x.ptr, self.res.ptr, self.w.ptr, self.y.ptr, t, h, 1e-5, stream)
        else:
            ops.rope_qk_f16(self.q.ptr, self.k.ptr, self.cos.ptr, self.sin.ptr, self.qo.ptr, self.ko.ptr,
                            t, self.QH, self.KH, self.HD, self.HD, 0, stream)

    def algorithmic_bytes(self) -> int:
        return self.nbytes

    def free(self) -> None:
        for b in self.bufs:
            b.free()


class DenseCase:
    """The dense f16 x f16 -> f32 matmul of the hipBLASLt boundary on the
    prefill shape M x K x N with the weights as a row-major f16 [K, N]
    operand, rotated over copies of >= 384 MB so every call reads HBM; the
    first (warm-up) call tunes and caches the plan.  Algorithmic bytes
    |A| + |B| + |C| once, flops 2 M N K."""

    def __init__(self, m: int, n: int, k: int) -> None:
        self.m, self.n, self.k = m, n, k
        self.ctx = ops.DenseMatmul()
        self.ws = DeviceBuffer(ops.DenseMatmul.WORKSPACE_BYTES)
        self.a = DeviceBuffer.from_array(wl.normal_f16(wl.seed_for(6, 0), m * k))
        b = wl.normal_f16(wl.seed_for(6, 1), k * n, std=0.05)
        self.copies = max(2, -(-384_000_000 // b.nbytes))
        self.b = [DeviceBuffer.from_array(b) for _ in range(self.copies)]
        self.c = DeviceBuffer(m * n * 4)

    def launch(self, i: int, stream: Stream) -> None:
        self.ctx.matmul_f16_f32(self.m, self.n, self.k, self.a.ptr, self.b[i % self.copies].ptr, self.c.ptr,
                                self.ws.ptr, ops.DenseMatmul.WORKSPACE_BYTES, stream)

    def algorithmic_bytes(self) -> int:
        return (self.m * self.k + self.k * self.n) * 2 + self.m * self.n * 4

    def flops(self) -> int:
        return 2 * self.m * self.n * self.k

    def free(self) -> None:
        for buf in [self.a, self.c, self.ws, *self.b]:
            buf.free()
        self.ctx.close()


def run_sweep(stream: Stream, hip: HipRuntime, steps: int, warmup: int, only: str | None = None,
              marker=None) -> None:
    """One line per configuration; the last column is the kernel variant the
    library's shape heuristic plans for it (the one the default entry points
    launch).  `only`: just the linear configurations whose name contains it.
    `marker`: called (and the stream synchronised) before every row and after
    the last, so that a kernel trace can be cut into rows (--trace-markers)."""
    mark = marker if marker is not None else (lambda: None)
    print(f"{'case':<15}{'M':>5}{'K':>7}{'N':>7}{'kernel us':>11}{'eager us':>10}{'GB/s':>9}"
          f"{'%HBM':>7}{'TFLOP/s':>9}{'%MFMA':>7}  kernel", file=sys.stderr)
    planner = ops.Q4_0Dispatch()  # no autotuning: the default entry points' heuristic
    for name, m, k, n, workload, uni, kind in SWEEP:
        if only is not None and only not in name:
            continue
        kq = kind if kind in ("q4_k", "q6_k") else None
        case = LinearCase(m, n, k, workload, x_uniform=uni, gate_up=kind is True, q8_0=kind == "q8",
                          reference_inputs=kind == "ref", kquant=kq)
        mark()
        t = time_case(case, stream, hip, steps, warmup)
        us = t["kernel_ms_mean"] * 1e3
        w = case.wb[0]
        if kq is not None:
            pass
        elif kind is True:
            planner.gate_up_silu(case.xb.ptr, w[0].ptr, w[1].ptr, case.yb.ptr, m, n, k, stream)
        elif kind == "q8":
            planner.linear_q8_0(case.xb.ptr, w[0].ptr, case.yb.ptr, m, n, k, stream)
        else:
            planner.linear(case.xb.ptr, w[0].ptr, case.yb.ptr, m, n, k, stream, f16_out=kind == "ref")
        stream.synchronize()
        variant = (f"kq_gemv_{kq}" if kq is not None else
                   planner.plan(m, n, k, gate_up=kind is True, q8_0=kind == "q8", f16_out=kind == "ref"))
        gbs = case.algorithmic_bytes() / (us * 1e-6) / 1e9
        tf = case.flops() / (us * 1e-6) / 1e12
        print(f"{name:<15}{m:>5}{k:>7}{n:>7}{us:>11.2f}{t['eager_ms_per_step'] * 1e3:>10.2f}{gbs:>9.0f}"
              f"{100 * gbs / HBM_PEAK_GBS:>6.1f}%{tf:>9.1f}{100 * tf / MFMA_F16_PEAK_TFLOPS:>6.1f}%  {variant}",
              file=sys.stderr, flush=True)
        case.free()
    planner.close()
    if only is not None:
        mark()
        return
    for m in (64, 512):
        case = DenseCase(m, 14336, 4096)
        mark()
        t = time_case(case, stream, hip, steps, max(warmup, 1))
        us = t["kernel_ms_mean"] * 1e3
        gbs = case.algorithmic_bytes() / (us * 1e-6) / 1e9
        tf = case.flops() / (us * 1e-6) / 1e12
        print(f"{'dense f16 mm':<15}{m:>5}{case.k:>7}{case.n:>7}{us:>11.2f}{t['eager_ms_per_step'] * 1e3:>10.2f}"
              f"{gbs:>9.0f}{100 * gbs / HBM_PEAK_GBS:>6.1f}%{tf:>9.1f}{100 * tf / MFMA_F16_PEAK_TFLOPS:>6.1f}%  "
              f"mote_hipblaslt_matmul_f16_f32", file=sys.stderr, flush=True)
        case.free()
    # The floor under these launch-bound kernels: a plain copy of RMSNorm's
    # bytes (32 rows of 8 KiB in and out) by one 256-thread workgroup per row.
    probe = load_probe()
    floor = CopyRowsCase(probe, NormRopeCase.TOKENS, NormRopeCase.HIDDEN * 2)
    mark()
    t = time_case(floor, stream, hip, steps, warmup)
    us = t["kernel_ms_mean"] * 1e3
    gbs = floor.algorithmic_bytes() / (us * 1e-6) / 1e9
    print(f"{'copy floor':<15}{floor.rows:>5}{0:>7}{NormRopeCase.HIDDEN:>7}{us:>11.2f}{t['eager_ms_per_step'] * 1e3:>10.2f}"
          f"{gbs:>9.0f}{100 * gbs / HBM_PEAK_GBS:>6.1f}%{0.0:>9.1f}{0.0:>6.1f}%  mote_probe_copy_rows",
          file=sys.stderr, flush=True)
    floor.free()
    entry = {"rmsnorm": "mote_hip_rms_norm_f16", "fused add+rmsnorm": "mote_hip_fused_add_rms_norm_f16",
             "rope q+k": "mote_hip_rope_qk_f16"}
    for kind in ("rmsnorm", "fused add+rmsnorm", "rope q+k"):
        case = NormRopeCase(kind)
        mark()
        t = time_case(case, stream, hip, steps, warmup)
        us = t["kernel_ms_mean"] * 1e3
        gbs = case.algorithmic_bytes() / (us * 1e-6) / 1e9
        print(f"{kind:<15}{case.TOKENS:>5}{0:>7}{case.HIDDEN:>7}{us:>11.2f}{t['eager_ms_per_step'] * 1e3:>10.2f}"
              f"{gbs:>9.0f}{100 * gbs / HBM_PEAK_GBS:>6.1f}%{0.0:>9.1f}{0.0:>6.1f}%  {entry[kind]}",
              file=sys.stderr, flush=True)
        case.free()
    mark()


def sweep_marker(stream: Stream):
    """A row delimiter for kernel traces of the sweep: the probe library's row
    copy with one 16-byte row (one workgroup; the copy-floor row copies 32 rows
    of 8 KiB, so the two never look alike), then a synchronisation."""
    probe = load_probe()
    src, dst = DeviceBuffer(16), DeviceBuffer(16)
    src.upload(np.zeros(16, dtype=np.uint8))

    def mark() -> None:
        _ffi.check(probe.mote_probe_copy_rows(src.ptr, dst.ptr, 1, 16, stream.handle), "sweep marker")
        stream.synchronize()
    return mark


def trace_table(trace_csv: str, sweep_log: str) -> int:
    """The sweep's kernel-trace table: cuts rocprofv3's kernel_trace.csv of a
    `--sweep --trace-markers` run at the marker dispatches (one-workgroup row
    copies), pairs each segment with the sweep row printed in the same order in
    `sweep_log` (the run's stderr; the segment before the first marker is the
    headline measurement), and prints per row every kernel with its grid in
    workgroups and its average and minimum traced duration.  Runs on the CPU."""
    import csv
    with open(trace_csv, newline="") as f:
        recs = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    rows, in_table = [], False
    with open(sweep_log) as f:
        for line in f:
            if line.startswith("case ") and "kernel us" in line:
                in_table = True
                continue
            if in_table and len(line) > 60 and line[15:].split() and line[15:].split()[0].isdigit():
                name, rest = line[:15].strip(), line[15:].split()
                rows.append((name, int(rest[0]), int(rest[1]), int(rest[2]), rest[-1]))
    segments, cur = [], []
    for r in recs:
        groups = int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"]))
        if "copy_rows_kernel" in r["Kernel_Name"] and groups == 1:
            segments.append(cur)
            cur = []
        else:
            cur.append(r)
    segments.append(cur)
    if len(segments) != len(rows) + 2:
        print(f"trace_table: {len(segments)} segments for {len(rows)} sweep rows (+ headline, + tail)",
              file=sys.stderr)
        return 1

    def short(name: str) -> str:
        name = re.sub(r"^void ", "", name)
        name = re.sub(r"^(mote::)?(q4_0::|kquant::|rope::)?(\(anonymous namespace\)::)?", "", name)
        return re.sub(r"\(.*$", "", name)  # the parameter list

    def describe(seg):
        kernels = {}
        for r in seg:
            dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            groups = int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"]))
            k = kernels.setdefault(short(r["Kernel_Name"]), {"n": 0, "sum": 0.0, "min": 1e30, "grid": groups})
            k["n"] += 1
            k["sum"] += dur
            k["min"] = min(k["min"], dur)
        main = [(k, v) for k, v in kernels.items() if "copyBuffer" not in k and "fillBuffer" not in k]
        return (" + ".join(f"`{k}`" for k, _ in main), " + ".join(str(v["grid"]) for _, v in main),
                " + ".join(f"{v['sum'] / v['n']:.2f}" for _, v in main),
                " + ".join(f"{v['min']:.2f}" for _, v in main))

    print("| workload | variant | kernel | grid (workgroups) | average µs | min µs |")
    print("|---|---|---|---|---|---|")
    k, g, a, mn = describe(segments[0])
    print(f"| headline (bench.py default): M=1 K=4096 N=14336 | | {k} | {g} | {a} | {mn} |")
    for (name, m, kk, n, variant), seg in zip(rows, segments[1:]):
        k, g, a, mn = describe(seg)
        print(f"| {name}: M={m} K={kk} N={n} | `{variant}` | {k} | {g} | {a} | {mn} |")
    return 0


READ_FLOOR_BYTES = (9_461_760, 14_188_544, 33_095_680)  # 1 x 4096 x {4096, 6144, 14336} linears


class ReadCase:
    """One pure-read pattern of the probe library's mote_probe_read_u128 over
    `nbytes`, rotated over copies of >= 384 MB in all (past the MALL)."""

    def __init__(self, probe, bufs, nbytes, sink, grid, threads, in_flight, nt) -> None:
        self.probe, self.bufs, self.nbytes, self.sink = probe, bufs, nbytes, sink
        self.args = (grid, threads, in_flight, nt)

    def launch(self, i: int, stream: Stream) -> None:
        grid, threads, in_flight, nt = self.args
        _ffi.check(self.probe.mote_probe_read_u128(self.bufs[i % len(self.bufs)].ptr, self.nbytes, grid,
                                                   threads, in_flight, nt, self.sink.ptr, stream.handle),
                   "read probe")


def install_fault_report() -> None:
    """The probe library's fatal-signal report (signal, faulting address,
    program counter, /proc/self/maps on stderr, then the previous handler);
    skipped when the probe library is not built."""
    path = os.path.join(ROOT, "mote_amd", "libmote_probe.so")
    if not os.path.exists(path):
        return
    probe = ctypes.CDLL(path)
    probe.mote_probe_install_fault_report.restype = ctypes.c_int
    probe.mote_probe_install_fault_report.argtypes = [ctypes.c_int]
    if probe.mote_probe_install_fault_report(2) != 0:
        print("bench.py: could not install the fault report", file=sys.stderr)


def load_probe():
    """libmote_probe.so, the measuring kernels built beside the library."""
    path = os.path.join(ROOT, "mote_amd", "libmote_probe.so")
    if not os.path.exists(path):
        raise SystemExit(f"bench.py: {path} is missing: build with `python -m mote_amd.build`")
    _ffi.lib()  # the HIP runtime first
    probe = ctypes.CDLL(path)
    P, U32 = ctypes.c_void_p, ctypes.c_uint32
    probe.mote_probe_read_u128.restype = ctypes.c_int
    probe.mote_probe_read_u128.argtypes = [P, ctypes.c_size_t, U32, U32, U32, ctypes.c_int, P, P]
    probe.mote_probe_copy_rows.restype = ctypes.c_int
    probe.mote_probe_copy_rows.argtypes = [P, P, U32, U32, P]
    probe.mote_probe_ring_record_words.restype = U32
    probe.mote_probe_ring_record_words.argtypes = []
    probe.mote_probe_ring_waves.restype = U32
    probe.mote_probe_ring_waves.argtypes = [U32]
    probe.mote_probe_ring_timeline.restype = ctypes.c_int
    probe.mote_probe_ring_timeline.argtypes = [P, P, P, U32, U32, P, ctypes.c_size_t, P]
    probe.mote_probe_ring_read.restype = ctypes.c_int
    probe.mote_probe_ring_read.argtypes = [P, U32, U32, P, ctypes.c_size_t, P]
    probe.mote_probe_skinny_record_words.restype = U32
    probe.mote_probe_skinny_record_words.argtypes = []
    probe.mote_probe_skinny_waves.restype = U32
    probe.mote_probe_skinny_waves.argtypes = [U32, U32]
    probe.mote_probe_skinny_timeline.restype = ctypes.c_int
    probe.mote_probe_skinny_timeline.argtypes = [P, P, P, U32, U32, U32, P, ctypes.c_size_t, P]
    return probe


class RingTimelineCase:
    """The shipped decode ring kernel with per-wave timestamps
    (mote_probe_ring_timeline), or with `loads_only` the ring kernel's own
    loads and nothing else (mote_probe_ring_read: grid, row order,
    non-temporal 16-byte direct-to-LDS loads, 2 slots, 1 row in flight, its
    waits), over the rotated weight copies of a LinearCase.  With `regions`
    launch i writes its per-wave records to region i % regions of one stamp
    buffer; with regions = 0 nothing is recorded."""

    def __init__(self, probe, case: "LinearCase", regions: int, loads_only: bool = False) -> None:
        self.probe, self.case, self.regions, self.loads_only = probe, case, regions, loads_only
        self.waves = probe.mote_probe_ring_waves(case.n)
        self.words = probe.mote_probe_ring_record_words()
        self.region_bytes = self.waves * self.words * 4
        self.stamps = DeviceBuffer(self.region_bytes * regions) if regions else None

    def launch(self, i: int, stream: Stream) -> None:
        c = self.case
        st = self.stamps.ptr + (i % self.regions) * self.region_bytes if self.stamps else None
        if self.loads_only:
            _ffi.check(self.probe.mote_probe_ring_read(c.wb[i % c.copies][0].ptr, c.n, c.k, st,
                                                       self.region_bytes if st else 0, stream.handle),
                       "ring read probe")
        else:
            _ffi.check(self.probe.mote_probe_ring_timeline(
                c.xb.ptr, c.wb[i % c.copies][0].ptr, c.yb.ptr, c.n, c.k, st, self.region_bytes, stream.handle),
                "ring timeline probe")

    def algorithmic_bytes(self) -> int:
        return self.case.w.nbytes if self.loads_only else self.case.algorithmic_bytes()

    def records(self) -> np.ndarray:
        return self.stamps.download(np.uint32).reshape(self.regions, self.waves, self.words)

    def free(self) -> None:
        if self.stamps:
            self.stamps.free()


def RingReadCase(probe, case: "LinearCase") -> RingTimelineCase:
    """The ring kernel's loads alone, unrecorded (read-floor rows)."""
    return RingTimelineCase(probe, case, 0, loads_only=True)


def _pct(values, q) -> float:
    return float(np.percentile(values, q)) if len(values) else float("nan")


def _timeline_summary(rec: np.ndarray, row_bytes: int, has_compute: bool) -> list[dict]:
    """Per launch: phase times in µs from the launch's first wave start (the
    100 MHz real-time clock, 10 ns ticks)."""
    tick_us = 0.01
    out = []
    launches = len(rec)
    for L in range(launches):
        r = rec[L]
        base = r[:, 0].min()
        rel = lambda a: ((a - base) & 0xFFFFFFFF) * tick_us  # noqa: E731
        begin, ready, end, nrows = rel(r[:, 0]), rel(r[:, 1]), rel(r[:, 2]), r[:, 3]
        active = nrows > 0
        arr = [rel(r[w, 4:4 + int(nrows[w])]) for w in range(len(r)) if nrows[w] > 0]
        done = [rel(r[w, 68:68 + int(nrows[w])]) for w in range(len(r)) if nrows[w] > 0]
        landed = np.sort(np.concatenate(arr))
        frac = lambda q: landed[min(len(landed) - 1, int(q * len(landed)))]  # noqa: E731
        comp = np.concatenate([d - a for d, a in zip(done, arr)])
        maxrows = int(nrows.max())
        per_row = [(np.median([a[j] for a in arr if len(a) > j]), np.median([d[j] for d in done if len(d) > j]))
                   for j in range(maxrows)]
        mid = frac(0.75) - frac(0.25)
        steady = 0.5 * len(landed) * row_bytes / (mid * 1e-6) / 1e12 if mid > 0 else float("nan")
        gap = None
        if L + 1 < launches:
            gap = ((rec[L + 1][:, 0].min() - base) & 0xFFFFFFFF) * tick_us - end[active].max()
        out.append(dict(L=L, begin_max=begin.max(),
                        ready=(f"{_pct(ready[active], 50):.2f} / {ready[active].max():.2f}" if has_compute else "—"),
                        first_p50=_pct([a[0] for a in arr], 50), l10=frac(0.10), l50=frac(0.50), l90=frac(0.90),
                        l100=landed[-1], end_p50=_pct(end[active], 50), end_max=end[active].max(),
                        comp=(f"{_pct(comp, 50):.3f}" if has_compute else "—"), steady=steady, gap=gap,
                        per_row=per_row))
    return out


def run_timeline(launches: int = 8) -> int:
    """Per-phase timeline of the shipped decode ring kernel at the headline
    shape (M = 1, K = 4096, N = 14336) beside the same timeline of the ring's
    loads alone: `launches` back-to-back launches of each, captured in one
    graph (rotating weights), replayed until the device has settled, then once
    more; the records of the last replay are summarised as markdown on
    stdout.  Times are the 100 MHz real-time clock (10 ns ticks) relative to
    the first wave start of each launch.  Event timings of the shipped kernel
    and of the two stamped kernels, stamped and not (graph replays of 200
    launches), come first."""
    probe = load_probe()
    stream, hip = Stream(), HipRuntime()
    m, k, n = 1, 4096, 14336
    case = LinearCase(m, n, k, workload=1)
    cases = {"shipped kernel (rowlds_r2d1)": case,
             "shipped kernel body, stamped": RingTimelineCase(probe, case, launches),
             "ring loads only": RingTimelineCase(probe, case, 0, loads_only=True),
             "ring loads only, stamped": RingTimelineCase(probe, case, launches, loads_only=True)}
    timed = {}
    for name, c in cases.items():
        timed[name] = time_case(c, stream, hip, 200, 20)["kernel_ms_mean"] * 1e3
        print(f"timeline: {name}: {timed[name]:.3f} us", file=sys.stderr, flush=True)
    print("## Event timings (graph replays of 200 launches, rotated weights)\n")
    print("| kernel | µs / launch | GB/s of its bytes |")
    print("|---|---|---|")
    for name, us in timed.items():
        print(f"| {name} | {us:.3f} | {cases[name].algorithmic_bytes() / (us * 1e-6) / 1e9:.0f} |")
    row_bytes = case.w.nbytes // n
    for name in ("shipped kernel body, stamped", "ring loads only, stamped"):
        tl = cases[name]
        exe = hip.capture(stream, lambda: [tl.launch(i, stream) for i in range(launches)])
        try:
            t0 = time.perf_counter()
            while time.perf_counter() - t0 < max(SETTLE_S, 0.02):
                hip.launch_graph(exe, stream)
                stream.synchronize()
            hip.launch_graph(exe, stream)
            stream.synchronize()
        finally:
            hip.destroy_graph(exe)
        rows = _timeline_summary(tl.records().astype(np.int64), row_bytes, not tl.loads_only)
        print(f"\n## {name}: phases of each launch (µs from the launch's first wave start; {tl.waves} waves, "
              f"{n // tl.waves} rows per wave)\n")
        print("| launch | last wave start | x staged (p50 / max) | first row landed (p50) | rows landed 10 % / 50 % / "
              "90 % / all | last wave end (p50 / max) | row compute (p50) | TB/s landed 25-75 % | gap to next launch |")
        print("|---|---|---|---|---|---|---|---|---|")
        for o in rows:
            gap = f"{o['gap']:.2f}" if o["gap"] is not None else "—"
            print(f"| {o['L']} | {o['begin_max']:.2f} | {o['ready']} | {o['first_p50']:.2f} | {o['l10']:.2f} / "
                  f"{o['l50']:.2f} / {o['l90']:.2f} / {o['l100']:.2f} | {o['end_p50']:.2f} / {o['end_max']:.2f} "
                  f"| {o['comp']} | {o['steady']:.2f} | {gap} |")
        o = rows[launches // 2]
        print(f"\n{name}, rows of launch {o['L']} (median over waves, µs)\n")
        print("| row j | landed | sum formed |" if not tl.loads_only else "| row j | landed |")
        print("|---|---|---|" if not tl.loads_only else "|---|---|")
        for j, (a, d) in enumerate(o["per_row"]):
            print(f"| {j} | {a:.2f} | {d:.2f} |" if not tl.loads_only else f"| {j} | {a:.2f} |")
    for c in cases.values():
        if c is not case:
            c.free()
    case.free()
    stream.close()
    return 0


class SkinnyTimelineCase:
    """The shipped skinny matrix-core kernel of 4-32 tokens at K = 4096
    (skinny_mfma_k16_s1_t1_d1_g1_r1_tr_l4_c_w) with per-wave timestamps
    (mote_probe_skinny_timeline), over the rotated weight copies of a
    LinearCase; launch i writes its records to region i % regions."""

    def __init__(self, probe, case: "LinearCase", regions: int) -> None:
        self.probe, self.case, self.regions = probe, case, regions
        self.waves = probe.mote_probe_skinny_waves(case.m, case.n)
        self.words = probe.mote_probe_skinny_record_words()
        self.region_bytes = self.waves * self.words * 4
        self.stamps = DeviceBuffer(self.region_bytes * regions)

    def launch(self, i: int, stream: Stream) -> None:
        c = self.case
        _ffi.check(self.probe.mote_probe_skinny_timeline(
            c.xb.ptr, c.wb[i % c.copies][0].ptr, c.yb.ptr, c.m, c.n, c.k,
            self.stamps.ptr + (i % self.regions) * self.region_bytes, self.region_bytes, stream.handle),
            "skinny timeline probe")

    def algorithmic_bytes(self) -> int:
        return self.case.algorithmic_bytes()

    def records(self) -> np.ndarray:
        return self.stamps.download(np.uint32).reshape(self.regions, self.waves, self.words)

    def free(self) -> None:
        self.stamps.free()


SKINNY_TIMELINE_VARIANT = "skinny_mfma_k16_s1_t1_d1_g1_r1_tr_l4_c_w"


def run_skinny_timeline(launches: int = 8, shapes=((4, 4096, 4096), (16, 4096, 4096), (32, 4096, 4096),
                                                    (16, 4096, 6144), (16, 4096, 14336))) -> int:
    """Per-phase timeline of the skinny matrix-core kernel the library plans
    for the skinny sweep (M x 4096 x N): for each shape, event timings of the
    library's planned call, of the variant forced, and of the probe's stamped
    instantiation (graph replays of 200 launches), then the records of
    `launches` back-to-back stamped launches (one graph, rotating weights,
    replayed until the device has settled, then once more), summarised per
    launch as markdown on stdout.  Times are the 100 MHz real-time clock (10 ns
    ticks) relative to the first wave start of each launch; each workgroup's
    16 waves share its items."""
    probe = load_probe()
    stream, hip = Stream(), HipRuntime()
    d = ops.Q4_0Dispatch()
    tick_us = 0.01
    for m, k, n in shapes:
        case = LinearCase(m, n, k, workload=2)
        plan = d.select(m, n, k)
        d.force(SKINNY_TIMELINE_VARIANT)
        forced = ForcedCase(case, d)
        tl = SkinnyTimelineCase(probe, case, launches)
        timed = {f"planned call (`{plan}`)": time_case(case, stream, hip, 200, 20)["kernel_ms_mean"] * 1e3,
                 f"`{SKINNY_TIMELINE_VARIANT}` forced": time_case(forced, stream, hip, 200, 20)["kernel_ms_mean"] * 1e3,
                 "the same kernel, stamped (probe)": time_case(tl, stream, hip, 200, 20)["kernel_ms_mean"] * 1e3}
        d.force(None)
        exe = hip.capture(stream, lambda: [tl.launch(i, stream) for i in range(launches)])
        try:
            t0 = time.perf_counter()
            while time.perf_counter() - t0 < max(SETTLE_S, 0.02):
                hip.launch_graph(exe, stream)
                stream.synchronize()
            hip.launch_graph(exe, stream)
            stream.synchronize()
        finally:
            hip.destroy_graph(exe)
        rec = tl.records().astype(np.int64)
        items = rec[0][:, 4]
        groups = tl.waves // 16
        print(f"\n## {m} × {k} × {n} ({groups} workgroups of 16 waves, {int(items.max())} item(s) of 16 rows "
              f"per workgroup at most)\n")
        print("| kernel | µs / launch | GB/s of the call's bytes |")
        print("|---|---|---|")
        for name, us in timed.items():
            print(f"| {name} | {us:.3f} | {case.algorithmic_bytes() / (us * 1e-6) / 1e9:.0f} |")
            print(f"timeline-skinny {m}x{k}x{n}: {name}: {us:.3f} us", file=sys.stderr, flush=True)
        print("\nPhases of each launch (µs from the launch's first wave start; p10 / p50 / p90 / max over the "
              "waves that own an item):\n")
        print("| launch | last wave start | x converted | item 1 weights landed | item 1 MFMAs issued | "
              "last item MFMAs issued | reduced and stored | wave end | gap to next launch |")
        print("|---|---|---|---|---|---|---|---|---|")
        for L in range(launches):
            r = rec[L]
            live = r[:, 4] > 0
            base = r[:, 0].min()
            rel = lambda a: ((a - base) & 0xFFFFFFFF) * tick_us  # noqa: E731
            q = lambda a: " / ".join(f"{_pct(a, p):.2f}" for p in (10, 50, 90)) + f" / {a.max():.2f}"  # noqa: E731
            last_issue = np.array([rel(r[w, 5 + 4 + int(r[w, 4]) - 1]) for w in np.nonzero(live)[0]])
            end = rel(r[:, 3])
            gap = "—"
            if L + 1 < launches:
                gap = f"{((rec[L + 1][:, 0].min() - base) & 0xFFFFFFFF) * tick_us - end.max():.2f}"
            print(f"| {L} | {rel(r[:, 0]).max():.2f} | {q(rel(r[live, 1]))} | {q(rel(r[live, 5]))} | "
                  f"{q(rel(r[live, 9]))} | {q(last_issue)} | {q(rel(r[live, 2]))} | {q(end[live])} | {gap} |")
        tl.free()
        case.free()
    d.close()
    stream.close()
    return 0


def run_read_floor(sizes=READ_FLOOR_BYTES) -> int:
    """Times grid-stride pure reads (threads x loads in flight x non-temporal
    x grid) of each byte count with graph replays, as one markdown table per
    size, fastest first: the HBM floor of the linears that stream as many
    bytes."""
    probe = load_probe()
    stream, hip = Stream(), HipRuntime()
    sink = DeviceBuffer(16)
    for nbytes in sizes:
        copies = max(2, math.ceil(ROTATION_BYTES / nbytes))
        bufs = [DeviceBuffer(nbytes) for _ in range(copies)]
        for i, b in enumerate(bufs):
            b.upload(np.full(nbytes, (i * 7 + 1) % 256, dtype=np.uint8))
        rows = []
        for threads, in_flight in ((256, 2), (256, 4), (256, 8), (512, 2), (512, 4), (1024, 2)):
            for nt in (1, 0):
                for grid in (256, 512, 768, 1024, 2048):
                    case = ReadCase(probe, bufs, nbytes, sink, grid, threads, in_flight, nt)
                    us = time_case(case, stream, hip, 100, 26)["kernel_ms_mean"] * 1e3
                    rows.append((us, f"t{threads} u{in_flight} {'nt' if nt else '--'} grid {grid}"))
                    print(f"read floor {nbytes} B: {rows[-1][1]}: {us:.2f} us", file=sys.stderr, flush=True)
        rows.sort()
        print(f"\n{nbytes} bytes, {copies} copies\n")
        print("| pattern (threads, loads in flight, non-temporal, grid) | µs / launch | GB/s | % of 8 TB/s |")
        print("|---|---|---|---|")
        for us, name in rows:
            gbs = nbytes / (us * 1e-6) / 1e9
            print(f"| {name} | {us:.2f} | {gbs:.0f} | {100 * gbs / HBM_PEAK_GBS:.1f} % |")
        for b in bufs:
            b.free()
    sink.free()
    # The decode ring kernel's own access pattern (mote_probe_ring_read): its
    # grid, row order, non-temporal direct-to-LDS 16-byte loads, 2 slots and 1
    # row in flight, and nothing else, over the weights of the M = 1, K =
    # 4096 linears.
    print("\nThe decode ring kernel's own loads (weights only, K = 4096)\n")
    print("| N | weight bytes | copies | µs / launch | GB/s | % of 8 TB/s |")
    print("|---|---|---|---|---|---|")
    for n in (4096, 6144, 14336):
        case = LinearCase(1, n, 4096, workload=1)
        ring = RingReadCase(probe, case)
        us = time_case(ring, stream, hip, 100, 26)["kernel_ms_mean"] * 1e3
        gbs = case.w.nbytes / (us * 1e-6) / 1e9
        print(f"read floor ring pattern N={n}: {us:.2f} us", file=sys.stderr, flush=True)
        print(f"| {n} | {case.w.nbytes} | {case.copies} | {us:.2f} | {gbs:.0f} | {100 * gbs / HBM_PEAK_GBS:.1f} % |")
        case.free()
    stream.close()
    return 0


def run_comparator(steps: int = 40) -> int:
    """Comparators from the vendor libraries, through torch.  Prefill: the
    dense f16 GEMM (torch.matmul, i.e. hipBLASLt on ROCm) at M in {64, 256,
    512}, K = 4096, N = 14336, with the weights already in f16 (117 MB per
    matrix, rotated over 4 copies so every call reads HBM), captured in a
    graph; plus the time to write and re-read one f16 weight matrix, the extra
    cost a dequantise-then-GEMM path pays per call.  Decode: a plain read of
    the headline's 33 095 680 bytes by the library's reduction kernel.  Runs
    in its own process: it loads torch's HIP runtime and never this library."""
    import torch

    dev = torch.device("cuda:0")
    k, n = 4096, 14336
    print(f"{'comparator':<22}{'M':>5}{'K':>7}{'N':>7}{'kernel us':>11}{'TFLOP/s':>9}{'%MFMA':>7}",
          file=sys.stderr)
    for m in (64, 256, 512):
        x = torch.randn(m, k, device=dev, dtype=torch.float16)
        ws = [torch.randn(n, k, device=dev, dtype=torch.float16) for _ in range(4)]
        side = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            for _ in range(3):
                y = x @ ws[0].t()
            side.synchronize()
            with torch.cuda.graph(graph, stream=side):
                for i in range(steps):
                    y = x @ ws[i % 4].t()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / steps
        tf = 2 * m * n * k / (us * 1e-6) / 1e12
        print(f"{'f16 GEMM (library)':<22}{m:>5}{k:>7}{n:>7}{us:>11.2f}{tf:>9.1f}"
              f"{100 * tf / MFMA_F16_PEAK_TFLOPS:>6.1f}%", file=sys.stderr, flush=True)
        del graph, y
    e0.record()
    for i in range(10):
        ws[(i + 1) % 4].copy_(ws[i % 4])
    e1.record()
    torch.cuda.synchronize()
    print(f"f16 weight matrix write + read ({2 * n * k * 2 / 1e6:.0f} MB): "
          f"{e0.elapsed_time(e1) * 1e3 / 10:.2f} us", file=sys.stderr, flush=True)
    del ws
    # The decode headline's byte count read by the library's own reduction
    # (amax over int32 words), 13 rotated copies, graph-captured.
    words = linear_bytes(1, n, k) // 4
    bufs = [torch.randint(0, 1 << 30, (words,), device=dev, dtype=torch.int32) for _ in range(13)]
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        for b in bufs:
            r = b.amax()
        side.synchronize()
        with torch.cuda.graph(graph, stream=side):
            for i in range(steps * 5):
                r = bufs[i % 13].amax()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (steps * 5)
    gbs = words * 4 / (us * 1e-6) / 1e9
    print(f"read of {words * 4} B (library amax reduction): {us:.2f} us, {gbs:.0f} GB/s, "
          f"{100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak", file=sys.stderr, flush=True)
    return 0


def main() -> int:
    global SETTLE_S
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--settle-ms", type=float, default=SETTLE_S * 1e3,
                    help="untimed graph replays before the timed ones, in ms of wall time (at least one)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="CPU time budget of the oracle baseline (0 skips it)")
    ap.add_argument("--sweep", action="store_true", help="also time every configuration (stderr)")
    ap.add_argument("--sweep-only", default=None, metavar="TEXT",
                    help="time only the sweep configurations whose name contains TEXT, and nothing "
                         "else (stderr table, no result line)")
    ap.add_argument("--profile-run", action="store_true",
                    help="for rocprofv3 counter passes: one device-to-device copy of one weight "
                         "matrix (the calibration kernel of known size), then 20 calls of the "
                         "headline linear; prints no result line")
    ap.add_argument("--profile-shape", default=None, metavar="M,K,N",
                    help="with --profile-run: profile this linear shape instead of the headline")
    ap.add_argument("--profile-gate-up", action="store_true",
                    help="with --profile-run: profile the fused gate/up SiLU-mul of the shape")
    ap.add_argument("--comparator", action="store_true",
                    help="time the vendor library's dense f16 GEMM at the prefill shapes (needs torch; "
                         "stderr table, no result line)")
    ap.add_argument("--read-floor", action="store_true",
                    help="time pure 16-byte reads of 9.46, 14.2 and 33.1 MB (the bytes of the 1 x 4096 x "
                         "{4096, 6144, 14336} linears) in many grid shapes: the HBM floor of the GEMVs "
                         "(probe library; stdout tables, no result line)")
    ap.add_argument("--plan-table", default=None, metavar="PATH",
                    help="time every candidate variant of the plan table's workloads, write the table "
                         "(q4_0_api.hip's plan_table.inc) to PATH, and nothing else")
    ap.add_argument("--timeline-skinny", action="store_true",
                    help="per-wave timeline of the skinny matrix-core kernel at the skinny sweep's K = 4096 shapes "
                         "(probe library: the shipped kernel with timestamps), as markdown on stdout, and nothing else")
    ap.add_argument("--timeline", action="store_true",
                    help="per-wave timeline of the headline's decode ring kernel (probe library: the shipped "
                         "kernel body with real-time stamps; stdout tables, no result line)")
    ap.add_argument("--read-bytes", default=None, metavar="B1,B2,...",
                    help="with --read-floor: these byte counts (multiples of 16) instead")
    ap.add_argument("--trace-markers", action="store_true",
                    help="with --sweep: a one-workgroup marker kernel between rows, to cut a kernel trace "
                         "of the run into rows (--trace-table)")
    ap.add_argument("--trace-table", nargs=2, default=None, metavar=("KERNEL_TRACE_CSV", "SWEEP_LOG"),
                    help="print the sweep's kernel-trace table from rocprofv3's kernel_trace.csv of a "
                         "--sweep --trace-markers run and that run's stderr (CPU only)")
    args = ap.parse_args()
    # A crash inside a runtime or profiler call then names the Python line
    # (and so the C-ABI call) it happened in, and the probe library's report
    # (installed in front of it) prints the faulting address, the program
    # counter and /proc/self/maps, which names the library the fault was in.
    faulthandler.enable()
    install_fault_report()
    SETTLE_S = max(args.settle_ms, 0.0) / 1e3
    if args.trace_table:
        return trace_table(*args.trace_table)
    if args.comparator:
        return run_comparator()
    if args.timeline:
        return run_timeline()
    if args.timeline_skinny:
        return run_skinny_timeline()
    if args.read_floor:
        sizes = tuple(int(v) for v in args.read_bytes.split(",")) if args.read_bytes else READ_FLOOR_BYTES
        return run_read_floor(sizes)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the Q4_0 linear shards by output rows with no exchange; see the design notes)",
              file=sys.stderr)
        return 2
    if args.steps < 1:
        print("bench.py: --steps must be >= 1", file=sys.stderr)
        return 2
    if device_count() < 1:
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1

    stream = Stream()
    hip = HipRuntime()
    if args.plan_table:
        run_plan_table(stream, hip, args.plan_table)
        return 0
    m, k, n = 1, 4096, 14336
    if args.profile_run:
        if args.profile_shape:
            pm, pk, pn = (int(v) for v in args.profile_shape.split(","))
            case = LinearCase(pm, pn, pk, workload=4 if pm >= 64 else (2 if pm > 1 else 1),
                              gate_up=args.profile_gate_up)
        else:
            case = LinearCase(m, n, k, workload=1)
        return profile_run(case, stream, hip)
    if args.sweep_only is not None:
        run_sweep(stream, hip, min(args.steps, 50), min(args.warmup, 5), only=args.sweep_only)
        stream.close()
        return 0
    case = LinearCase(m, n, k, workload=1)
    print(f"bench: Q4_0 linear M={m} K={k} N={n}, {case.copies} weight copies "
          f"({case.copies * case.w.nbytes / 1e6:.0f} MB), warmup {args.warmup}, steps {args.steps}",
          file=sys.stderr, flush=True)
    t = time_case(case, stream, hip, args.steps, args.warmup)
    stats = reference_statistics(case, stream, hip)
    nbytes = case.algorithmic_bytes()
    value = nbytes / (t["ms_per_step"] * 1e-3) / 1e9
    achieved = nbytes / (t["kernel_ms_mean"] * 1e-3) / 1e9

    cpu = None
    if args.cpu_seconds > 0:
        cpu, y_cpu = cpu_baseline(case, args.cpu_seconds)
        check_output(case, y_cpu)

    line = {
        "metric": "Q4_0 linear µs/call + achieved HBM GB/s (% peak), M=1 K=4096 N=14336",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t["ms_per_step"], 6),
        "us_per_call": round(t["ms_per_step"] * 1e3, 3),
        "kernel_us": round(t["kernel_ms_mean"] * 1e3, 3),
        "kernel_us_median": stats["kernel_us_median"],
        "kernel_us_spread_pct": stats["spread_pct"],
        "reference_statistics": stats,
        "eager_us_per_call": round(t["eager_ms_per_step"] * 1e3, 3),
        "issue": "HIP graph of `steps` captured C-ABI calls, replayed 3 times",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "Q4_0 decode linear, Llama-3-8B MLP up/gate: M=1, K=4096, N=14336",
            "M": m, "K": k, "N": n,
            "weights": "GGML Q4_0, d=f16(|N(0,0.02)|), uniform nibbles, SplitMix64 seeded",
            "activations": "f16 N(0,1)", "output": "f32",
            "entry_point": "mote_hip_quantized_linear_q4_0_f32",
            "weight_copies": case.copies,
            "algorithmic_bytes_per_call": nbytes,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": read_traffic(),
            "traffic_source": ("rocprofv3 FETCH_SIZE + WRITE_SIZE passes of this workload, copy-calibrated, "
                               "read from profiles/q4_0_gemv_m1_k4096_n14336_traffic.md (not measured in "
                               "this run)"),
        },
        "cpu_baseline": cpu,
    }
    if args.sweep:
        run_sweep(stream, hip, min(args.steps, 50), min(args.warmup, 5),
                  marker=sweep_marker(stream) if args.trace_markers else None)
    case.free()
    stream.close()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
