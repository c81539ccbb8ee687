"""CPU test of the split-K scratch pool's locking: tests/cpp/
scratch_pool_test.cpp built with g++ against mote_amd/csrc/scratch_pool.hpp
(host code only) and run.  It checks that two host threads calling a split-K
entry point on one stream keep each call's tiles kernel and epilogue adjacent,
that different streams (and devices) never share a buffer or wait for each
other, that growth retires the old buffer and release frees each buffer once,
and that release waits for a lease still held."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_scratch_pool_locking(tmp_path):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.fail("g++ is needed to build the scratch pool test")
    exe = tmp_path / "scratch_pool_test"
    subprocess.run(
        [cxx, "-std=c++17", "-O1", "-pthread", "-Wall", "-Werror", f"-I{ROOT}/mote_amd/csrc",
         os.path.join(ROOT, "tests", "cpp", "scratch_pool_test.cpp"), "-o", str(exe)],
        check=True, capture_output=True, text=True,
    )
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 0, proc.stdout + proc.stderr
