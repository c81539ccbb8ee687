"""bench.py --trace-table on a synthetic kernel trace (CPU only): the trace of
a `--sweep --trace-markers` run is cut at the one-workgroup marker copies and
each segment is paired with the sweep row printed in the same order."""

import csv
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

FIELDS = ["Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X", "Workgroup_Size_X"]


def _dispatch(name, start_ns, dur_ns, groups, threads=256):
    return {"Kernel_Name": name, "Start_Timestamp": start_ns, "End_Timestamp": start_ns + dur_ns,
            "Grid_Size_X": groups * threads, "Workgroup_Size_X": threads}


def test_trace_table_cuts_rows_at_markers(tmp_path):
    marker = "void mote::(anonymous namespace)::copy_rows_kernel(unsigned char const*, unsigned char*)"
    t, recs = 1000, []

    def add(name, dur, groups):
        nonlocal t
        recs.append(_dispatch(name, t, dur, groups))
        t += dur + 100

    add("void mote::q4_0::(anonymous namespace)::gemv_lds_kernel<FmtQ4, 1, 3, 2, 3, float>(x)", 7000, 256)  # headline
    add(marker, 500, 1)
    for dur in (4000, 3800, 3900):  # row 1: one kernel
        add("void mote::q4_0::(anonymous namespace)::gemv_lds_kernel<FmtQ4, 1, 2, 1, 3, float>(x)", dur, 256)
    add(marker, 500, 1)
    for dur in (10000, 9000):  # row 2: split K, two kernels per call
        add("void mote::q4_0::(anonymous namespace)::skinny_mfma_kernel<8, 1>(x)", dur, 448)
        add("void mote::q4_0::(anonymous namespace)::splitk_reduce_kernel<float, false>(x)", dur // 4, 64)
    add("void mote::(anonymous namespace)::copy_rows_kernel(unsigned char const*, unsigned char*)", 1800, 32)  # not a marker
    add(marker, 500, 1)
    trace = tmp_path / "kt_kernel_trace.csv"
    with open(trace, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        w.writerows(recs)
    log = tmp_path / "sweep.err"
    log.write_text(
        "bench: Q4_0 linear M=1 K=4096 N=14336, 13 weight copies (429 MB), warmup 20, steps 200\n"
        "case               M      K      N  kernel us  eager us     GB/s   %HBM  TFLOP/s  %MFMA  kernel\n"
        "decode             1   4096   4096       4.04      4.68     2344  29.3%      8.3   0.3%  rowlds_r2d1\n"
        "down split-K       4  14336   4096      11.81     12.31     2812  35.2%     39.8   1.6%  skinny_sk\n")
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--trace-table", str(trace), str(log)],
                         capture_output=True, text=True, check=True).stdout.splitlines()
    assert out[0].startswith("| workload | variant | kernel |")
    assert "`gemv_lds_kernel<FmtQ4, 1, 3, 2, 3, float>` | 256 | 7.00 | 7.00" in out[2]
    assert out[3] == "| decode: M=1 K=4096 N=4096 | `rowlds_r2d1` | `gemv_lds_kernel<FmtQ4, 1, 2, 1, 3, float>` | 256 | 3.90 | 3.80 |"
    assert out[4].startswith("| down split-K: M=4 K=14336 N=4096 | `skinny_sk` | `skinny_mfma_kernel<8, 1>` + "
                             "`splitk_reduce_kernel<float, false>` + `copy_rows_kernel` | 448 + 64 + 32 | 9.50 + 2.38 + 1.80 |")
    assert len(out) == 5
