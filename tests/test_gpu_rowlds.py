"""GPU parity of the decode GEMV that streams rows through a per-wave LDS ring
(q4_0_gemv_lds.hip: coalesced non-temporal direct-to-LDS loads, M = 1, K a
multiple of 256 up to 4096).

Every variant runs row lengths that need one, two and three load instructions
per row with the last one partly idle (K = 256 ... 4096), N below one
workgroup, ragged N, and N = 140001 at K = 256, where each wave owns more
than 64 rows and stores its register-held sums mid-loop; f32 and f16
outputs.  The arithmetic is the pair-load streaming GEMV's, so the outputs
must equal it bit for bit, and the oracle's tolerance holds too."""

from __future__ import annotations

import numpy as np
import pytest

from mote_amd import ops, workloads as wl
from test_gpu_q4_0 import check_against_oracle, normal_x, run_linear, sample_columns, weights

pytestmark = pytest.mark.gpu

SHAPES = [(1, 256), (7, 1024), (257, 1792), (130, 2048), (61, 3072), (1000, 3584), (33, 3840), (4099, 4096),
          (14336, 4096), (140001, 256)]


@pytest.mark.parametrize("variant", [v for v in ops.variant_names() if v.startswith("rowlds_")])
def test_every_rowlds_variant(stream, oracle, variant):
    d = ops.Q4_0Dispatch()
    d.force(variant)
    ref = ops.Q4_0Dispatch()
    ref.force("stream_d1_g2")
    for n, k in SHAPES:
        x = normal_x(wl.seed_for(17, k), 1, k)
        w = weights(wl.seed_for(17, 100 + n), n, k)
        cols = None if n < 5000 else sample_columns(n, 512)
        for f16_out in (False, True):
            y = run_linear(stream, x, w, 1, n, k, dispatch=d, f16_out=f16_out)
            want = run_linear(stream, x, w, 1, n, k, dispatch=ref, f16_out=f16_out)
            assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), (variant, n, k, f16_out)
            check_against_oracle(oracle, y, x, w, 1, n, k, columns=cols, f16_out=f16_out,
                                 what=f"{variant} 1x{n}x{k}{' f16' if f16_out else ''}")


def test_rowlds_rejects_what_it_cannot_run(stream):
    """K not a multiple of 256, K past 4096 and two tokens fall outside the
    variant: forcing it is an error, never a silent misread."""
    d = ops.Q4_0Dispatch()
    d.force("rowlds_r2d1")
    from mote_amd import HipError
    for m, n, k in [(1, 64, 192), (1, 64, 4352), (2, 64, 1024)]:
        x = normal_x(wl.seed_for(17, 1), m, k)
        w = weights(wl.seed_for(17, 2), n, k)
        with pytest.raises(HipError):
            run_linear(stream, x, w, m, n, k, dispatch=d)
