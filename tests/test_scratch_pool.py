"""CPU test of the split-K scratch pool's locking: tests/cpp/
scratch_pool_test.cpp built with g++ against mote_amd/csrc/scratch_pool.hpp
(host code only) and run.  It checks that two host threads calling a split-K
entry point on one stream keep each call's tiles kernel and epilogue adjacent,
that different streams (and devices) never share a buffer or wait for each
other, that growth retires the old buffer and release frees each buffer once,
and that release waits for a lease still held; plain and under the host
sanitizers."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


SANITIZERS = {
    "plain": [],
    "address": ["-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-fno-sanitize-recover=all"],
    "thread": ["-fsanitize=thread"],
}


@pytest.mark.parametrize("sanitizer", list(SANITIZERS))
def test_scratch_pool_locking(tmp_path, sanitizer):
    """The host build of the pool, plain and under AddressSanitizer (with
    UndefinedBehaviorSanitizer and leak checks: every buffer freed once) and
    ThreadSanitizer (the lease lock and the map lock)."""
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.fail("g++ is needed to build the scratch pool test")
    exe = tmp_path / "scratch_pool_test"
    build = subprocess.run(
        [cxx, "-std=c++17", "-O1", "-g", "-pthread", "-Wall", "-Werror", *SANITIZERS[sanitizer],
         f"-I{ROOT}/mote_amd/csrc", os.path.join(ROOT, "tests", "cpp", "scratch_pool_test.cpp"), "-o", str(exe)],
        capture_output=True, text=True,
    )
    if build.returncode != 0 and sanitizer != "plain" and "cannot find" in build.stderr:
        pytest.skip(f"the host compiler has no {sanitizer} sanitizer runtime")
    assert build.returncode == 0, build.stderr
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
