"""CPU tests of the dispatch heuristic (host logic, no device): the variant
each configuration of the path plans, through mote_q4_0_dispatch_select,
which runs the same heuristic as a call without launching.

Every selected name must be a compiled variant.  The benchmark workloads
(decode, skinny sweep, prefill, fused gate/up) run the fastest entry of the
measured plan table compiled into the library (mote_amd/csrc/plan_table.inc,
written by bench.py --plan-table); every other decode, skinny, split-K,
prefill, Q8_0 and fused gate/up shape lands on the kernel the rules chose,
including three tokens past K = 4096 (rows split over 2 or 4 waves up to K =
16384, the split-K tiles beyond)."""

from __future__ import annotations

import os
import re

import pytest

from mote_amd import HipError, ops

PLAN_TABLE = os.path.join(os.path.dirname(__file__), "..", "mote_amd", "csrc", "plan_table.inc")

# The benchmark workloads the plan table must list (op 0 linear, 1 gate/up;
# M, K, N): configs 0-2 (decode, Llama-3-8B up/gate and down, the skinny
# sweep), the reference benchmark's 11 008 shapes, and config 4's prefill
# linear and fused gate/up.
TABLE_SHAPES = (
    [(0, 1, 4096, 4096), (0, 1, 4096, 14336), (0, 1, 14336, 4096), (0, 1, 4096, 11008), (0, 1, 11008, 4096)]
    + [(0, m, 4096, n) for n in (4096, 6144, 14336) for m in (2, 4, 8, 16, 32)]
    + [(op, m, 4096, 14336) for op in (0, 1) for m in (64, 256, 512)]
)


def plan_table() -> dict:
    """{(op, M, K, N): [(us, variant), ...]} from the compiled-in table."""
    rx = re.compile(r'\{(\d+), (\d+), (\d+), (\d+), "([^"]+)", ([0-9.]+)\}')
    table: dict = {}
    with open(PLAN_TABLE) as f:
        for line in f:
            m = rx.search(line)
            if m:
                op, mm, k, n = (int(v) for v in m.groups()[:4])
                table.setdefault((op, mm, k, n), []).append((float(m.group(6)), m.group(5)))
    return table


@pytest.fixture(scope="module")
def d():
    ctx = ops.Q4_0Dispatch()
    yield ctx
    ctx.close()


LINEAR = [
    # (M, K, N) -> variant
    ((1, 4096, 14336), "rowlds_r2d1"),
    ((1, 4096, 4096), "rowlds_r2d1"),
    ((1, 4096, 6144), "rowlds_r2d1"),
    ((1, 1024, 4096), "rowlds_r2d1"),
    ((1, 4160, 4096), "stream_s2_d1_g2"),
    ((1, 14336, 4096), "rowlds_s4_r3d2_g1"),
    ((1, 13824, 5120), "rowlds_s4_r3d2_g1"),
    ((1, 5120, 13824), "rowlds_s2_r3d2_g1"),
    ((1, 8192, 28672), "rowlds_s2_r3d2_g1"),
    ((1, 14336, 1024), "stream_s4_d1q_g1"),
    ((1, 8192, 8192), "stream_s2_d1_g2"),
    ((1, 11008, 4096), "stream_s4_d1q_g2"),
    ((1, 4096, 11008), "rowlds_r2d1"),
    ((1, 28672, 8192), "rowlds_s8_r3d2_g1"),
    ((2, 4096, 14336), "rowlds_m2_r2d1"),
    ((2, 4096, 8192), "rowlds_m2_r2d1"),
    ((2, 1024, 4096), "rowlds_m2_r2d1"),
    ((2, 4032, 4096), "stream_m2_d1q_g1"),  # K % 256 != 0: no ring
    ((3, 4096, 4096), "rowlds_m3_r2d1"),
    ((3, 4096, 6144), "rowlds_m3_r2d1"),
    ((3, 4096, 8192), "skinny_mfma_k16_s1_t1_d1_g1_r1_tr_l4_c_w"),
    ((4, 4096, 2048), "rowlds_m4_r2d1"),
    ((2, 14336, 4096), "stream_s4_m2_d1q_g1"),
    ((3, 8192, 8192), "stream_s2_m3_d1q_g1"),
    ((3, 14336, 4096), "stream_s4_m3_d1q_g1"),
    ((4, 4096, 4096), "skinny_mfma_k16_s1_t1_d1_g1_r1_tr_l4_c_w"),
    ((16, 4096, 14336), "skinny_mfma_k16_s1_t1_d1_g1_r1_tr_l4_c_w"),
    ((24, 4096, 14336), "skinny_mfma_k8_s2_t2_d1_g1_r1_tr_l4_c_w"),
    ((32, 4096, 14336), "skinny_mfma_k8_s2_t2_d1_g1_r1_tr_l4_c_w"),
    ((64, 4096, 14336), "mfma_x32s_m64_n64_w2_k4"),
    ((40, 4096, 14336), "skinny_mfma_k8_s2_t2_d1_g1_r1_tr_l8_c_w"),
    ((40, 5120, 13824), "mfma_x32s_m64_n64_w2_k4"),
    ((48, 5120, 5120), "skinny_mfma_k4_s1_t1_d1_g1_r1_tr_l8_c_w_sk"),
    ((4, 11008, 4096), "stream_s4_m4_d1q_g1"),
    ((4, 13824, 5120), "stream_s4_m4_d1q_g1"),
    ((4, 14336, 4096), "skinny_mfma_k8_s1_t1_d1_g1_r1_tr_l4_c_w_sk"),
    ((16, 11008, 4096), "mfma_x32s_m64_n64_w2_k4"),
    ((8, 11008, 4096), "stream_s4_m4x_d1q_g1"),
    ((5, 5376, 4096), "stream_s2_m4x_d1q_g1"),
    ((12, 11008, 4096), "mfma_x32s_m64_n64_w2_k4"),
    ((48, 4096, 4096), "skinny_mfma_k8_s2_t2_d1_g1_r1_tr_l4_c_w"),
    ((40, 8192, 28672), "mfma_x32s_m64_n128_w1_k4"),
    ((64, 8192, 28672), "mfma_x32s_m64_n128_w1_k4"),
    ((32, 8192, 28672), "skinny_mfma_k8_s2_t2_d1_g1_r1_tr_l8_c_w_sk"),
    ((64, 8192, 8192), "skinny_mfma_k8_s2_t2_d1_g1_r1_tr_l8_c_w_sk"),
    ((48, 4096, 2048), "skinny_mfma_k16_s1_t1_d1_g1_r1_tr_l4_c_w"),
    ((56, 4096, 4096), "skinny_mfma_k16_s1_t1_d1_g1_r1_tr_l4_c_w"),
    ((128, 4096, 14336), "mfma_x32s_m64_n128_w1_k4"),
    ((256, 4096, 14336), "mfma_x32s_m128_n128_w1_k2"),
    ((384, 4096, 14336), "mfma_x32s_m128_n256_w1_k2"),
    ((1024, 4096, 14336), "mfma_x32s_m128_n256_w1_k2"),
    ((128, 4096, 4096), "mfma_x32s_m64_n64_w2_k4"),
    ((256, 4096, 4096), "mfma_x32s_m64_n64_w2_k4"),
    ((512, 4096, 4096), "mfma_x32s_m64_n128_w1_k4"),
    ((512, 4096, 6144), "mfma_x32s_m128_n128_w1_k2"),
    ((256, 14336, 4096), "mfma_x32s_m64_n64_w2_k4"),
    ((512, 4096, 14336), "mfma_x32s_m128_n256_w1_k2"),
    ((256, 4160, 14336), "mfma_x32s_m128_n128_w1"),  # 65 block pairs: one pair per step
    # 3-4 tokens at 2048 < K < 4096: each row read once for all tokens, through
    # the LDS ring up to five rows per wave
    ((3, 3072, 8192), "rowlds_m3_r2d1"),
    ((4, 2560, 10240), "rowlds_m4_r2d1"),
    ((3, 3584, 18944), "stream_m3_d1_g1"),
    ((4, 3584, 18944), "stream_m4_d1_g1"),
    # 5-11 tokens at K = 3584 (no K slicing): passes of four tokens on wide N,
    # the one-token-per-pass vector-ALU GEMV on narrow N and past K = 16384
    ((6, 3584, 18944), "stream_m4x_d1q_g1"),
    ((11, 3584, 18944), "stream_m4x_d1q_g1"),
    ((6, 3584, 4608), "gemv_r4_t1_k1"),
    ((3, 18944, 3584), "gemv_r4_t1_k1"),
    ((5, 18944, 3584), "gemv_r4_t1_k1"),
    # K = 8192 on narrow N: parts of 2048, 4 items per workgroup
    ((4, 8192, 3072), "skinny_mfma_k8_s1_t1_d1_g1_r1_tr_l4_c_w_sk"),
    ((16, 8192, 8192), "skinny_mfma_k16_s1_t1_d1_g1_r1_tr_l4_c_w_sk"),
    ((32, 8192, 2048), "skinny_mfma_k8_s1_t1_d1_g1_r1_tr_l4_c_w_sk"),
    ((48, 8192, 2048), "skinny_mfma_k8_s1_t2_d1_g1_r1_tr_l4_c_w_sk"),
    ((64, 8192, 3072), "skinny_mfma_k8_s1_t2_d1_g1_r1_tr_l8_c_w_sk"),
    # 160 64 x 64 tiles past K = 4096 (the 70B fused q/k/v)
    ((48, 8192, 10240), "mfma_x32s_m64_n64_w2_k4"),
    ((64, 4096, 11008), "skinny_mfma_k8_s2_t2_d1_g1_r1_tr_l8_c_w"),
    ((64, 3072, 8192), "mfma_x32s_m64_n64_w2_k4"),
    # K = 14336 on 5120 / 3584 rows: 16-token items, 4 per workgroup
    ((4, 14336, 5120), "skinny_mfma_k8_s1_t1_d1_g1_r1_tr_l4_c_w_sk"),
    ((48, 14336, 3584), "skinny_mfma_k8_s1_t1_d1_g1_r1_tr_l4_c_w_sk"),
]


# shapes the plan table lists are decided by it (tested below), the rest by the rules
LINEAR_RULES = [(s, v) for s, v in LINEAR if (0, *s) not in plan_table()]


@pytest.mark.parametrize("shape,want", LINEAR_RULES, ids=[f"{m}x{k}x{n}" for (m, k, n), _ in LINEAR_RULES])
def test_linear_plans(d, shape, want):
    m, k, n = shape
    assert d.select(m, n, k) == want


def test_plan_table_lists_every_benchmark_workload():
    """Every benchmark workload has measured candidates in the table, each a
    compiled variant of the workload's kind, with positive times."""
    table, names = plan_table(), set(ops.variant_names())
    for shape in TABLE_SHAPES:
        entries = table.get(shape)
        assert entries and len(entries) >= 2, shape
        for us, v in entries:
            assert v in names and us > 0, (shape, v)
            assert v.startswith("gateup_") == (shape[0] == 1), (shape, v)


@pytest.mark.parametrize("shape", TABLE_SHAPES, ids=[f"{'gu' if o else 'lin'}-{m}x{k}x{n}" for o, m, k, n in TABLE_SHAPES])
def test_benchmark_workloads_run_the_table_fastest_entry(d, shape):
    """The plan of a listed workload (aligned operands) is its fastest
    measured candidate."""
    op, m, k, n = shape
    fastest = min(plan_table()[shape])[1]
    assert d.select(m, n, k, gate_up=op == 1) == fastest


def test_every_selection_is_a_compiled_variant(d):
    names = set(ops.variant_names())
    for m in (1, 2, 3, 4, 5, 8, 16, 17, 24, 32, 33, 48, 64, 65, 128, 256, 512):
        for k in (64, 1024, 2048, 3072, 4096, 5120, 8192, 11008, 14336, 28672):
            for n in (7, 4096, 14336):
                assert d.select(m, n, k) in names, (m, k, n)
                assert d.select(m, n, k, q8_0=True) in names, (m, k, n)
                assert d.select(m, n, k, gate_up=True) in names, (m, k, n)


def test_three_tokens_past_4096(d):
    """Linear, Q8_0 and gate/up: rows split over 2 / 4 waves for 4096 < K <=
    16384; beyond that the split-K tiles (no 8-way three-token form)."""
    assert d.select(3, 8192, 8192, q8_0=True) == "q8_stream_s2_m3_d1q_g1"
    assert d.select(3, 4096, 14336, q8_0=True) == "q8_stream_s4_m3_d1q_g1"
    assert d.select(3, 28672, 8192, gate_up=True) == "gateup_stream_s2_m3_d1q_g1"
    assert d.select(3, 4096, 14336, gate_up=True) == "gateup_stream_s4_m3_d1q_g1"
    assert d.select(3, 8192, 28672).endswith("_sk")
    assert d.select(3, 8192, 28672, q8_0=True).endswith("_sk")
    assert d.select(3, 8192, 28672, gate_up=True).endswith("_sk")


def test_gate_up_and_q8_plans(d):
    assert d.select(1, 14336, 4096, gate_up=True) == "gateup_stream_p1_d1_g1"
    assert d.select(2, 14336, 4096, gate_up=True) == "gateup_stream_p1_m2_d1q_g1"
    assert d.select(16, 14336, 4096, gate_up=True).startswith("gateup_skinny_")
    assert d.select(64, 28672, 8192, gate_up=True) == "gateup_mfma_x32s_m64_n128_w1_k4"
    assert d.select(32, 28672, 8192, gate_up=True) == "gateup_mfma_x32s_m64_n128_w1_k4"
    assert d.select(128, 14336, 4096, gate_up=True) == "gateup_mfma_x32s_m64_n128_w1_k4"
    assert d.select(192, 14336, 4096, gate_up=True) == "gateup_mfma_x32s_m128_n128_w1_k2"
    assert d.select(16, 28672, 8192, gate_up=True).startswith("gateup_skinny_")
    assert d.select(1, 14336, 4096, q8_0=True) == "q8_rowlds_r2d1"
    assert d.select(1, 4096, 4096, q8_0=True) == "q8_rowlds_r2d1"
    assert d.select(2, 14336, 4096, q8_0=True) == "q8_rowlds_m2_r2d1"
    assert d.select(3, 14336, 4096, q8_0=True) == "q8_rowlds_m3_r2d1"
    assert d.select(4, 14336, 4096, q8_0=True) == "q8_stream_m4_d1q_g1"
    assert d.select(1, 4096, 14336, q8_0=True) == "q8_rowlds_s4_r2d1"
    assert d.select(1, 8192, 28672, q8_0=True) == "q8_rowlds_s8_r2d1"
    assert d.select(1, 28672, 8192, q8_0=True) == "q8_rowlds_s2_r2d1"
    assert d.select(1, 4096, 4160, q8_0=True) == "q8_stream_s2_d1_g1"  # K % 256 != 0
    assert d.select(16, 14336, 4096, q8_0=True).startswith("q8_skinny_")
    assert d.select(512, 14336, 4096, q8_0=True) == "q8_mfma_x32s_m128_n256_w1_k2"
    assert d.select(256, 14336, 4096, q8_0=True) == "q8_mfma_x32s_m128_n128_w1_k2"
    assert d.select(128, 14336, 4096, q8_0=True) == "q8_mfma_x32s_m64_n128_w1_k4"
    assert d.select(128, 14336, 4160, q8_0=True) == "q8_mfma_r_m64_n64"
    assert d.select(48, 4096, 4096, gate_up=True) == "gateup_skinny_k8_s2_t2_d1_l4_c_w"
    assert d.select(48, 4096, 4096, q8_0=True) == "q8_skinny_k8_s2_t2_d1_l4_c_w"
    assert d.select(64, 14336, 4096, q8_0=True) == "q8_skinny_k16_s1_t2_d1_c"
    assert d.select(48, 28672, 8192, q8_0=True) == "q8_mfma_x32s_m64_n128_w1_k4"
    assert d.select(24, 28672, 8192, q8_0=True) == "q8_skinny_k8_s1_t2_d1_l8_c_w_sk"
    assert d.select(16, 4096, 14336, q8_0=True) == "q8_skinny_k4_s1_t1_d1_l8_c_w_sk"
    assert d.select(32, 4096, 14336, q8_0=True) == "q8_skinny_k8_s1_t1_d1_l8_c_w_sk"
    assert d.select(384, 14336, 4096, gate_up=True) == "gateup_mfma_x32s_m64_n128_w1_k2"
    assert d.select(4, 4096, 11008, q8_0=True) == "q8_stream_s4_m4_d1q_g1"
    assert d.select(8, 4096, 11008, q8_0=True) == "q8_stream_s4_m4x_d1q_g1"
    assert d.select(16, 5120, 13824, q8_0=True) == "q8_stream_s4_m4x_d1q_g1"
    assert d.select(32, 5120, 13824, q8_0=True) == "q8_mfma_x32s_m64_n128_w1_k4"
    assert d.select(4, 5120, 5120, q8_0=True) == "q8_stream_s2_m4_d1q_g1"
    assert d.select(64, 13824, 5120, q8_0=True) == "q8_mfma_x32s_m64_n128_w1_k4"
    assert d.select(48, 5120, 5120, gate_up=True) == "gateup_skinny_k4_s1_t2_d1_l8_c_w_sk"
    assert d.select(32, 5120, 5120, gate_up=True) == "gateup_skinny_k4_s1_t1_d1_l8_c_w_sk"
    assert d.select(32, 13824, 5120, gate_up=True) == "gateup_skinny_k4_s1_t2_d1_l8_c_w_sk"
    assert d.select(48, 13824, 5120, gate_up=True) == "gateup_mfma_x32s_m64_n64_w2_k4"
    assert d.select(64, 11008, 4096, gate_up=True) == "gateup_mfma_x32s_m64_n64_w2_k4"
    # prefill tiles by dispatch waves x wave time
    assert d.select(256, 4096, 4096, q8_0=True) == "q8_mfma_x32s_m64_n128_w1_k4"
    assert d.select(384, 14336, 4096, q8_0=True) == "q8_mfma_x32s_m128_n256_w1_k2"
    assert d.select(256, 4096, 4096, gate_up=True) == "gateup_mfma_x32s_m64_n64_w2_k4"
    assert d.select(512, 4096, 4096, gate_up=True) == "gateup_mfma_x32s_m64_n128_w1_k4"


def test_forced_variant_and_bad_shapes(d):
    d.force("stream_d1q_g1")
    try:
        assert d.select(7, 100, 64) == "stream_d1q_g1"
    finally:
        d.force(None)
    for shape in [(0, 1, 32), (1, 0, 32), (1, 1, 0), (1, 1, 33)]:
        with pytest.raises(HipError):
            d.select(*shape)


def test_k_past_the_tiled_kernels_plans_the_64_bit_path(d):
    """K above 2^31 - 1 (the reference takes 64-bit sizes) runs the 64-bit
    K-part path for every op; a forced variant cannot run it."""
    assert d.select(1, 4096, (1 << 31) - 32) != "wide_k"
    for k in (1 << 31, (1 << 31) + 32, 1 << 40):
        assert d.select(1, 3, k) == "wide_k"
        assert d.select(5, 7, k, gate_up=True) == "wide_k"
        assert d.select(2, 3, k, q8_0=True) == "wide_k"
    d.force("stream_d1q_g1")
    try:
        with pytest.raises(HipError):
            d.select(1, 3, 1 << 31)
    finally:
        d.force(None)


def test_plans_below_k_4096_and_past_16384(d):
    """Gate/up: three tokens at 2048 < K < 4096 on the stream with rows split
    2 ways (K = 4096 keeps the one-slice skinny tiles), 49-64 tokens below K =
    4096 on 64 x 64 tiles, 32-token items at K = 2048 above 16 tokens.  Q8_0:
    5-16 tokens at K = 3584 as four-token passes, and past K = 16384 with no K
    slicing the generic kernel rather than the tiles."""
    assert d.select(3, 18944, 3584, gate_up=True) == "gateup_stream_s2_m3_d1q_g1"
    assert d.select(3, 14336, 4096, gate_up=True).startswith("gateup_skinny_k16_")
    assert d.select(64, 8192, 3072, gate_up=True) == "gateup_mfma_x32s_m64_n64_w2_k4"
    assert d.select(32, 8192, 2048, gate_up=True) == "gateup_skinny_k4_s1_t2_d1_l8_c_w_sk"
    assert d.select(64, 18944, 3584, gate_up=True).startswith("gateup_mfma_x32s_m64_n128_w1")
    assert d.select(6, 4608, 3584, q8_0=True) == "q8_stream_s2_m4x_d1q_g1"
    assert d.select(4, 3584, 18944, q8_0=True) == "q8_generic"
    assert d.select(4, 4096, 14336, q8_0=True) == "q8_stream_s4_m4_d1q_g1"
