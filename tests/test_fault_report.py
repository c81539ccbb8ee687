"""The benchmark's fatal-signal report (mote_amd/probes/fault_maps.hip, loaded
by bench.py): a child process on the CPU installs it, as bench.py does, and
reads address 8.  Its stderr must hold the report (signal 11, the faulting
address, the program counter), the whole of /proc/self/maps (so a fault inside
a library names it: the probe library's own mapping must appear), and then
Python's faulthandler traceback, i.e. the previous handler still runs."""

from __future__ import annotations

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROBE = os.path.join(ROOT, "mote_amd", "libmote_probe.so")

CHILD = """
import ctypes, faulthandler, sys
sys.path.insert(0, {root!r})
faulthandler.enable()
import bench
bench.install_fault_report()
ctypes.string_at(8)
"""


@pytest.mark.skipif(not os.path.exists(PROBE), reason="libmote_probe.so is not built")
def test_fault_report_prints_maps_then_the_previous_handler():
    proc = subprocess.run([sys.executable, "-c", CHILD.format(root=ROOT)], capture_output=True, text=True,
                          timeout=120, env={**os.environ, "HIP_VISIBLE_DEVICES": ""})
    assert proc.returncode != 0
    err = proc.stderr
    assert "mote_probe fault report: signal 11 address 0x0000000000000008 pc 0x" in err, err[:2000]
    maps = err.split("*** /proc/self/maps:\n", 1)[1].split("*** end of maps", 1)[0]
    assert "libmote_probe.so" in maps and "[stack]" in maps
    assert "Fatal Python error: Segmentation fault" in err.split("*** end of maps", 1)[1]
