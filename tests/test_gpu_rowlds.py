"""GPU parity of the decode GEMV that streams rows through a per-wave LDS ring
(q4_0_gemv_lds.hip: coalesced non-temporal direct-to-LDS loads, M = 1 to 4,
K a multiple of 256 up to 4096, Q4_0 and Q8_0; one token past K = 4096 with
rows split over waves).

Every variant runs row lengths that need one, two and three load instructions
per row with the last one partly idle (K = 256 ... 4096), N below one
workgroup, ragged N, and N = 140001 at K = 256, where each wave owns more
than 64 rows and stores its register-held sums mid-loop; f32 and f16
outputs.  The arithmetic is the pair-load streaming GEMV's, so the outputs
must equal it bit for bit, and the oracle's tolerance holds too.

The variants with rows split over S waves (``rowlds_s<S>_...``, K a multiple
of 256 with at most 64 pairs per slice) run slices of one to three load
instructions, slices that start 4, 8 and 12 bytes into a 16-byte chunk
(K = 3328, 4352, 11008, 13824 ...), a last slice shorter than the others
(K = 6400 and 2304 at S = 8), N below one workgroup's row groups, ragged N
(row groups of one workgroup with different row counts), the down
projection's 14336 x 4096, and more than 64 rows per group (the slice sums
are added through LDS mid-loop); they must equal the split-row streaming
GEMV with the same S bit for bit."""

from __future__ import annotations

import re

import numpy as np
import pytest

from mote_amd import ops, workloads as wl
from test_gpu_q4_0 import check_against_oracle, normal_x, run_linear, sample_columns, weights

pytestmark = pytest.mark.gpu

SHAPES = [(1, 256), (7, 1024), (257, 1792), (130, 2048), (61, 3072), (1000, 3584), (33, 3840), (4099, 4096),
          (14336, 4096), (140001, 256)]


SPLIT_SHAPES = {
    2: [(1, 512), (7, 2048), (257, 4352), (61, 6144), (1000, 7424), (4099, 8192), (70001, 768)],
    4: [(1, 1024), (5, 3328), (257, 5376), (130, 8192), (61, 11008), (4099, 14336), (4096, 14336), (33, 16384),
        (70001, 1280)],
    8: [(1, 2048), (3, 6400), (257, 10240), (130, 13824), (4099, 28672), (1000, 32768), (40001, 2304)],
}
REFERENCE = {1: "stream_d1_g2", 2: "stream_s2_d1_g1", 4: "stream_s4_d1q_g1", 8: "stream_s8_d1_g1"}
# the streaming GEMV reading each row once for every token (Q4_0 rings of 2 tokens)
TOKENS_REFERENCE = {2: "stream_m2_d1q_g1", 3: "stream_m3_d1_g1", 4: "stream_m4_d1_g1"}
# the Q8_0 streaming GEMV reading each row once for every token, or with rows
# split over S waves
Q8_REFERENCE = {1: "q8_stream_d1_g1", 2: "q8_stream_m2_d1q_g1", 4: "q8_stream_m4_d1q_g1"}
Q8_SPLIT_REFERENCE = {2: "q8_stream_s2_d1_g1", 4: "q8_stream_s4_d1_g1", 8: "q8_stream_s8_d1_g1"}


def _split(variant: str) -> int:
    m = re.match(r"rowlds_s(\d+)_", variant)
    return int(m.group(1)) if m else 1


def _tokens(variant: str) -> int:
    m = re.search(r"rowlds_m(\d+)_", variant)
    return int(m.group(1)) if m else 1


@pytest.mark.parametrize("variant", [v for v in ops.variant_names() if v.startswith("rowlds_")])
def test_every_rowlds_variant(stream, oracle, variant):
    """Q4_0 rings of two tokens (rowlds_m2_*) read each row once for both and
    must equal the two-token streaming GEMV bit for bit."""
    split, tokens = _split(variant), _tokens(variant)
    d = ops.Q4_0Dispatch()
    d.force(variant)
    ref = ops.Q4_0Dispatch()
    ref.force(REFERENCE[split] if tokens == 1 else TOKENS_REFERENCE[tokens])
    for n, k in SHAPES if split == 1 else SPLIT_SHAPES[split]:
        print(f"{variant} {tokens}x{n}x{k}", flush=True)
        x = normal_x(wl.seed_for(17, k), tokens, k)
        w = weights(wl.seed_for(17, 100 + n), n, k)
        cols = None if n < 5000 else sample_columns(n, 512)
        for f16_out in (False, True):
            y = run_linear(stream, x, w, tokens, n, k, dispatch=d, f16_out=f16_out)
            want = run_linear(stream, x, w, tokens, n, k, dispatch=ref, f16_out=f16_out)
            assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), (variant, n, k, f16_out)
            check_against_oracle(oracle, y, x, w, tokens, n, k, columns=cols, f16_out=f16_out,
                                 what=f"{variant} {tokens}x{n}x{k}{' f16' if f16_out else ''}")


@pytest.mark.parametrize("variant", [v for v in ops.variant_names() if v.startswith("q8_rowlds_")])
def test_every_q8_rowlds_variant(stream, oracle, variant):
    """Q8_0 through the ring (68-byte pairs, up to five load instructions per
    row or slice), one token with rows whole or split over S waves, or 2-4
    tokens per row read: the shapes above, bit for bit the Q8_0 streaming GEMV
    of the same shape of work (three tokens, which no streaming variant reads
    at K <= 4096: each token bit for bit the one-token ring), and within the
    oracle's tolerance."""
    from test_gpu_q8_0 import check as check_q8, run as run_q8, weights as q8_weights

    split, tokens = _split(variant.removeprefix("q8_")), _tokens(variant)
    d = ops.Q4_0Dispatch()
    d.force(variant)
    ref = ops.Q4_0Dispatch()
    ref.force(Q8_SPLIT_REFERENCE[split] if split > 1 else Q8_REFERENCE.get(tokens, "q8_rowlds_r2d1"))
    per_token = split == 1 and tokens not in Q8_REFERENCE
    for n, k in SHAPES if split == 1 else SPLIT_SHAPES[split]:
        print(f"{variant} {tokens}x{n}x{k}", flush=True)
        x = normal_x(wl.seed_for(19, k), tokens, k)
        w = q8_weights(wl.seed_for(19, 100 + n), n, k)
        cols = None if n < 5000 else sample_columns(n, 512)
        for f16_out in (False, True):
            y = run_q8(stream, x, w, tokens, n, k, dispatch=d, f16_out=f16_out)
            if per_token:
                want = np.concatenate([run_q8(stream, x[t * k:(t + 1) * k], w, 1, n, k, dispatch=ref,
                                              f16_out=f16_out) for t in range(tokens)])
            else:
                want = run_q8(stream, x, w, tokens, n, k, dispatch=ref, f16_out=f16_out)
            assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), (variant, n, k, f16_out)
            check_q8(oracle, y, x, w, tokens, n, k, columns=cols, f16_out=f16_out,
                     what=f"{variant} {tokens}x{n}x{k}{' f16' if f16_out else ''}")


@pytest.mark.parametrize("variant,shapes", [
    ("rowlds_r2d1", [(1, 64, 192), (1, 64, 4352), (2, 64, 1024)]),
    ("rowlds_s4_r3d2_g1", [(1, 64, 3200), (1, 64, 17408), (2, 64, 14336)]),
    ("rowlds_s8_r3d2_g1", [(1, 64, 1792), (1, 64, 14592), (1, 64, 33024)]),
    ("q8_rowlds_m2_r2d1", [(1, 64, 1024), (3, 64, 1024), (2, 64, 4352), (2, 64, 192)]),
    ("q8_rowlds_s8_r2d1", [(1, 64, 7424), (1, 64, 33024), (2, 64, 28672)]),
])
def test_rowlds_rejects_what_it_cannot_run(stream, variant, shapes):
    """K not a multiple of 256, more than 64 pairs per slice, slices whose
    last load instruction would be idle (K = 1792 and 14592 at S = 8) and two
    tokens fall outside the variant: forcing it is an error, never a silent
    misread."""
    from mote_amd import HipError
    from test_gpu_q8_0 import run as run_q8, weights as q8_weights

    q8 = variant.startswith("q8_")
    d = ops.Q4_0Dispatch()
    d.force(variant)
    for m, n, k in shapes:
        x = normal_x(wl.seed_for(17, 1), m, k)
        w = (q8_weights if q8 else weights)(wl.seed_for(17, 2), n, k)
        with pytest.raises(HipError):
            (run_q8 if q8 else run_linear)(stream, x, w, m, n, k, dispatch=d)


@pytest.mark.parametrize("q8", [False, True], ids=["q4_0", "q8_0"])
def test_cached_ring_plan_is_not_reused_off_the_16_byte_grid(stream, oracle, q8):
    """The ring kernels load weights and activations in 16-byte chunks, so
    they run only on 16-byte-aligned operands.  One dispatch context plans
    1 x 4096 x 14336 with aligned weights (the ring), then runs the same shape
    with the weights 4, 8 and 12 bytes off the 16-byte grid, and aligned again:
    the plan key carries the alignment class, so the misaligned calls get a
    kernel of their own (dword weight loads), and every call meets the
    oracle's tolerance.  The same sequence runs through the default entry
    points (the library's own context)."""
    from test_gpu_q8_0 import check as check_q8, run as run_q8, weights as q8_weights

    m, n, k = 1, 14336, 4096
    x = normal_x(wl.seed_for(18, k), m, k)
    w = q8_weights(wl.seed_for(18, n), n, k) if q8 else weights(wl.seed_for(18, n), n, k)
    cols = sample_columns(n, 512)
    d = ops.Q4_0Dispatch()
    for dispatch in (d, None):
        for step, offset in enumerate((0, 4, 8, 12, 0)):
            print(f"{'q8_0' if q8 else 'q4_0'} w_offset {offset} {'context' if dispatch else 'default'}", flush=True)
            if q8:
                y = run_q8(stream, x, w, m, n, k, dispatch=dispatch, w_offset=offset)
                check_q8(oracle, y, x, w, m, n, k, columns=cols, what=f"q8_0 w+{offset}")
            else:
                y = run_linear(stream, x, w, m, n, k, dispatch=dispatch, w_offset=offset)
                check_against_oracle(oracle, y, x, w, m, n, k, columns=cols, what=f"q4_0 w+{offset}")
            if dispatch is not None and step < 2:
                # the context's first plan of the shape (the lower alignment
                # class sorts first): the ring when aligned, not after
                plan = d.plan(m, n, k, q8_0=q8)
                assert plan is not None and ("rowlds" in plan) == (offset == 0), (offset, plan)
