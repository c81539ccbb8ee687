"""Writes the regression fixtures of tests/golden from the CPU oracle.

* q4_0_fixture_3x5x64.json: the reference GPU test's closed-form fixture
  (crates/mote-backend-hip/tests/quantized_linear.rs:16-18,160-177): weight
  bytes, f16 input bits and the oracle's f32 output.
* oracle_regression.json: small seeded linears (SplitMix64 workloads) with the
  f32 oracle's output bits and a SHA-256 of the weight bytes.

These pin later changes of the oracle and the generators; they are not ground
truth (reference_kats.json, transcribed from the reference's own tests, is).
Run from the repository root: ``python tests/golden/make_golden.py``.
"""

import hashlib
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import numpy as np  # noqa: E402

import oracle  # noqa: E402
from helpers import bits_to_f32, ref_test_q4_0_inputs, ref_test_q4_0_weights  # noqa: E402
from mote_amd import workloads as wl  # noqa: E402

LINEAR_CASES = [
    {"m": 1, "n": 64, "k": 4096, "x": "uniform", "x_seed": wl.seed_for(0, 0), "w_seed": wl.seed_for(0, 1)},
    {"m": 4, "n": 16, "k": 512, "x": "normal", "x_seed": wl.seed_for(2, 0), "w_seed": wl.seed_for(2, 1)},
    {"m": 2, "n": 8, "k": 1024, "x": "normal", "x_seed": wl.seed_for(1, 0), "w_seed": wl.seed_for(1, 1)},
]


def main() -> None:
    w = ref_test_q4_0_weights(5, 64)
    x = ref_test_q4_0_inputs(3, 64)
    y = oracle.quantized_linear_f32(bits_to_f32(x), w, oracle.Q4_0, 3, 5, 64)
    with open(os.path.join(HERE, "q4_0_fixture_3x5x64.json"), "w", encoding="utf-8") as f:
        json.dump({"weights": w.tolist(), "input_f16_bits": x.tolist(), "expected_f32": y.tolist()}, f)
        f.write("\n")
    cases = []
    for c in LINEAR_CASES:
        m, n, k = c["m"], c["n"], c["k"]
        xs = (wl.uniform_f16 if c["x"] == "uniform" else wl.normal_f16)(c["x_seed"], m * k)
        ws = wl.q4_0_weights(c["w_seed"], n, k)
        ys = oracle.quantized_linear_f32(bits_to_f32(xs), ws, oracle.Q4_0, m, n, k)
        cases.append({**c, "w_sha256": hashlib.sha256(ws.tobytes()).hexdigest(),
                      "y_f32_bits": ys.view(np.uint32).tolist()})
    with open(os.path.join(HERE, "oracle_regression.json"), "w", encoding="utf-8") as f:
        json.dump({"linear": cases}, f)
        f.write("\n")


if __name__ == "__main__":
    main()
