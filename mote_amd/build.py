"""Builds ``mote_amd/libmote_hip.so`` for gfx950 with hipcc.

Every ``csrc/*.hip`` file is compiled to an object in ``mote_amd/_build`` and
the objects are linked into one shared library whose exported symbols are the
C ABI declared in ``include/mote_hip.h``.  The measuring probes under
``probes/`` (the HBM read-floor kernel of ``bench.py --read-floor``) go into a
second library, ``mote_amd/libmote_probe.so``, which only the benchmark loads.  Packed-FP32 instructions are
disabled for the device pass; hipcc's host pass warns that it does not know
that target feature, which is harmless and filtered from the log.

Usage: ``python -m mote_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
PROBES = os.path.join(HERE, "probes")
BUILD = os.path.join(HERE, "_build")
LIBRARY = os.path.join(HERE, "libmote_hip.so")
PROBE_LIBRARY = os.path.join(HERE, "libmote_probe.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _filter_log(text: str) -> str:
    return "\n".join(
        line for line in text.splitlines() if "not a recognized feature for this target" not in line
    )


def _compile(source: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(source) + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, f"-I{CSRC}", "-c", source, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    log = _filter_log(proc.stdout + proc.stderr)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source}:\n{log}")
    if log.strip():
        print(log, file=sys.stderr)
    return obj


def sources(directory: str = CSRC) -> list[str]:
    return sorted(
        os.path.join(directory, name) for name in os.listdir(directory) if name.endswith(".hip")
    )


def _link(objects: list[str], library: str) -> None:
    tmp = library + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objects]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("link failed:\n" + _filter_log(proc.stdout + proc.stderr))
    os.replace(tmp, library)


def build(jobs: int | None = None) -> str:
    """Compiles every source, links the library and the probe library;
    returns the library's path."""
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    probes = sources(PROBES)
    workers = jobs or min(8, os.cpu_count() or 4, len(srcs) + len(probes))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(_compile, srcs + probes))
    _link(objects[: len(srcs)], LIBRARY)
    _link(objects[len(srcs):], PROBE_LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build())
