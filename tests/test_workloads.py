"""CPU tests of the seeded workload generators (mote_amd.workloads)."""

from __future__ import annotations

import numpy as np

from mote_amd import workloads as wl


def test_splitmix64_published_vectors():
    """SplitMix64 reference outputs (Steele, Lea and Flood 2014; the values of
    Vigna's splitmix64.c): seed 0 and seed 1234567."""
    assert [int(v) for v in wl.splitmix64(0, 3)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    assert [int(v) for v in wl.splitmix64(1234567, 3)] == [6457827717110365317, 3203168211198807973,
                                                           9817491932198370423]
    assert np.array_equal(wl.splitmix64(5, 4, offset=2), wl.splitmix64(5, 6)[2:])


def test_distributions():
    x = wl.normal_f16(wl.seed_for(1, 0), 200000).view(np.float16).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    u = wl.uniform_f16(wl.seed_for(0, 0), 100000).view(np.float16).astype(np.float64)
    assert u.min() >= -1.0 and u.max() <= 1.0 and abs(u.mean()) < 0.01
    w = wl.normal_f16(wl.seed_for(3, 1), 100000, mean=1.0, std=0.1).view(np.float16).astype(np.float64)
    assert abs(w.mean() - 1.0) < 0.002 and abs(w.std() - 0.1) < 0.002


def test_q4_0_weight_layout():
    n, k = 64, 256
    w = wl.q4_0_weights(wl.seed_for(0, 1), n, k)
    assert w.size == n * (k // 32) * 18 == n * wl.q4_0_row_bytes(k)
    blocks = w.reshape(-1, 18)
    d = blocks[:, 0:2].copy().view("<u2")[:, 0].view(np.float16).astype(np.float64)
    assert np.all(d >= 0) and 0.012 < d.mean() < 0.020  # E|N(0, 0.02)| = 0.016
    nib = np.concatenate([blocks[:, 2:] & 15, blocks[:, 2:] >> 4]).ravel()
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.8 * nib.size / 16
    assert np.array_equal(w, wl.q4_0_weights(wl.seed_for(0, 1), n, k))


def test_positions_and_tables():
    pos = wl.positions(wl.seed_for(3, 2), 4096)
    assert pos.min() >= 0 and pos.max() <= 8191 and len(np.unique(pos)) > 3000
    c, s = wl.rope_tables(np.array([0, 3]), 8, 500000.0)
    assert c.shape == (2, 4) and np.all(c[0] == 1) and np.all(s[0] == 0)
    assert c[1, 0] == np.float32(np.cos(3.0))


def test_reference_bench_generators_follow_the_reference_loops():
    """The vectorised generators equal a direct transcription of the reference
    benchmark's loops (crates/mote-backend-hip/benches/quantized_linear.rs:
    128-152) on a small matrix, including the first block's known bytes."""
    n, k = 7, 96
    want = bytearray()
    for o in range(n):
        for b in range(k // 32):
            scale = np.float16(0.015625 * ((o * 3 + b) % 4 + 1)).view(np.uint16)
            want += int(scale).to_bytes(2, "little")
            for j in range(16):
                want.append(((o * 5 + b * 3 + j) % 16) | (((o * 7 + b + j * 3 + 1) % 16) << 4))
    got = wl.reference_bench_q4_0_weights(n, k)
    assert bytes(got) == bytes(want)
    assert bytes(got[:3]) == b"\x00\x24\x10"  # f16(1/64) = 0x2400, byte 0: low 0, high 1
    x = wl.reference_bench_inputs(2, 40)
    assert np.array_equal(x, np.array([np.float16(i % 29 / 14.0 - 1.0) for i in range(80)]).view(np.uint16))
