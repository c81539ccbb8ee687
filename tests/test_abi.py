"""CPU tests of the C ABI of libmote_hip.so (no GPU needed, nothing launched).

* The library loads and exports exactly the symbols include/mote_hip.h
  declares.
* Every argument rejection and every empty-problem early return of the
  reference's shims happens before any device work, so their status codes are
  checked here with stand-in pointers that are never dereferenced
  (crates/mote-backend-hip/src/quantized_linear.hip:64-76, rms_norm.hip:75-83,
  fused_add_rms_norm.hip:107-122, rope.hip:109-130, hipblaslt_shim.cpp:259-324).
* The dispatch context's host-side state (variants, forcing, plan lookup).
"""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mote_hip.h")

FAKE = 0x10000  # stand-in device pointer: every call below returns before using it
STREAM = 0x20000


@pytest.fixture(scope="module")
def lib():
    from mote_amd import _ffi

    if not os.path.exists(_ffi.LIBRARY):
        from mote_amd import build

        build.build()
    return _ffi.lib()


def declared_symbols() -> set[str]:
    with open(HEADER, encoding="utf-8") as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(mote_\w+)\s*\(", text))


def test_exports_match_header(lib):
    from mote_amd import _ffi

    declared = declared_symbols()
    out = subprocess.run(["nm", "-D", "--defined-only", _ffi.LIBRARY], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert declared, "no declarations parsed"
    assert declared == exported, (sorted(declared - exported), sorted(exported - declared))
    assert declared == set(_ffi.SIGNATURES), "ctypes signature table out of sync with the header"
    for name in declared:
        assert getattr(lib, name) is not None


def test_q4_0_linear_status_codes(lib):
    for fn in (lib.mote_hip_quantized_linear_q4_0_f16, lib.mote_hip_quantized_linear_q4_0_f32):
        assert fn(None, FAKE, FAKE, 1, 1, 32, STREAM) == 1
        assert fn(FAKE, None, FAKE, 1, 1, 32, STREAM) == 1
        assert fn(FAKE, FAKE, None, 1, 1, 32, STREAM) == 1
        assert fn(FAKE, FAKE, FAKE, 1, 1, 32, None) == 1
        assert fn(FAKE, FAKE, FAKE, 1, 1, 33, STREAM) == 1  # K % 32 != 0
        assert fn(FAKE, FAKE, FAKE, 0, 5, 32, STREAM) == 0   # empty: no launch
        assert fn(FAKE, FAKE, FAKE, 5, 0, 32, STREAM) == 0
        assert fn(FAKE, FAKE, FAKE, 0, 5, 33, STREAM) == 1   # K checked before emptiness
        assert fn(FAKE, FAKE, FAKE, 1 << 32, 1, 32, STREAM) == 9
        assert fn(FAKE, FAKE, FAKE, 65536, 65536, 32, STREAM) == 9  # rows * N > UINT_MAX
        # K >= 2^31 launches (64-bit path), as in the reference: tested on the GPU


def test_gate_up_and_decode_status_codes(lib):
    g = lib.mote_hip_q4_0_gate_up_silu_f32
    assert g(None, FAKE, FAKE, FAKE, 1, 1, 32, STREAM) == 1
    assert g(FAKE, FAKE, None, FAKE, 1, 1, 48, STREAM) == 1
    assert g(FAKE, FAKE, None, FAKE, 0, 1, 32, STREAM) == 0
    d = lib.mote_hip_dequantize_q4_0_f32
    assert d(None, FAKE, 1, 32, STREAM) == 1
    assert d(FAKE, FAKE, 1, 31, STREAM) == 1
    assert d(FAKE, FAKE, 0, 32, STREAM) == 0
    assert d(FAKE, FAKE, 4, 0, STREAM) == 0


def test_k_quant_status_codes(lib):
    """Q4_K / Q6_K: the Q4_0 statuses with K % 256 and each format's storage
    alignment (crates/mote-types/src/lib.rs:67-73: Q4_K 4, Q6_K 2)."""
    for name, walign in (("q4_k", 4), ("q6_k", 2)):
        for out, oalign in (("f16", 2), ("f32", 4)):
            fn = getattr(lib, f"mote_hip_quantized_linear_{name}_{out}")
            assert fn(None, FAKE, FAKE, 1, 1, 256, STREAM) == 1
            assert fn(FAKE, FAKE, FAKE, 1, 1, 256, None) == 1
            assert fn(FAKE, FAKE, FAKE, 1, 1, 288, STREAM) == 1   # K % 256 != 0
            assert fn(FAKE, FAKE + walign // 2, FAKE, 1, 1, 256, STREAM) == 1  # weights misaligned
            assert fn(FAKE + 1, FAKE, FAKE, 1, 1, 256, STREAM) == 1  # odd input address
            assert fn(FAKE, FAKE, FAKE + oalign // 2, 1, 1, 256, STREAM) == 1
            assert fn(FAKE, FAKE, FAKE, 0, 5, 256, STREAM) == 0
            assert fn(FAKE, FAKE, FAKE, 5, 0, 256, STREAM) == 0
            assert fn(FAKE, FAKE, FAKE, 65536, 65536, 256, STREAM) == 9
            assert fn(FAKE, FAKE, FAKE, 1, 1, 1 << 31, STREAM) == 9
        d = getattr(lib, f"mote_hip_dequantize_{name}_f32")
        assert d(None, FAKE, 1, 256, STREAM) == 1
        assert d(FAKE, FAKE, 1, 128, STREAM) == 1
        assert d(FAKE + walign // 2, FAKE, 1, 256, STREAM) == 1
        assert d(FAKE, FAKE + 2, 1, 256, STREAM) == 1
        assert d(FAKE, FAKE, 0, 256, STREAM) == 0
        assert d(FAKE, FAKE, 4, 0, STREAM) == 0


def test_norm_status_codes(lib):
    r = lib.mote_hip_rms_norm_f16
    assert r(None, FAKE, FAKE, 1, 8, 1e-6, STREAM) == -1
    assert r(FAKE, FAKE, FAKE, 1, 8, 1e-6, None) == -1
    assert r(FAKE, FAKE, FAKE, 0, 8, 1e-6, STREAM) == 0
    assert r(FAKE, FAKE, FAKE, 3, 0, 1e-6, STREAM) == 0
    assert r(FAKE, FAKE, FAKE, 1 << 32, 8, 1e-6, STREAM) == -1
    f = lib.mote_hip_fused_add_rms_norm_f16
    assert f(FAKE, FAKE + 64, FAKE, FAKE + 64, 1, 8, 1e-6, STREAM) == -1  # output == residual
    for eps in (-1e-6, float("nan"), float("inf")):
        assert f(FAKE, FAKE + 64, FAKE, FAKE + 128, 1, 8, eps, STREAM) == -1
    assert f(FAKE, FAKE + 64, FAKE, FAKE + 128, 0, 8, 1e-6, STREAM) == 0
    assert f(None, FAKE + 64, FAKE, FAKE + 128, 1, 8, 1e-6, STREAM) == -1


def test_rope_status_codes(lib):
    r = lib.mote_hip_rope_f16
    assert r(FAKE, FAKE, FAKE, FAKE, 2, 3, 8, 7, 0, STREAM) == -1
    assert r(FAKE, FAKE, FAKE, FAKE, 2, 3, 8, 10, 0, STREAM) == -1
    assert r(FAKE, FAKE, FAKE, FAKE, 2, 3, 8, 8, 2, STREAM) == -1
    assert r(FAKE, None, FAKE, FAKE, 2, 3, 8, 8, 0, STREAM) == -1
    assert r(None, FAKE, FAKE, FAKE, 2, 3, 8, 8, 0, STREAM) == -1
    assert r(FAKE, FAKE, FAKE, FAKE, 2, 3, 8, 8, 0, None) == -1
    assert r(FAKE, FAKE, FAKE, FAKE, 0, 3, 8, 8, 0, STREAM) == 0
    assert r(FAKE, FAKE, FAKE, FAKE, 2, 0, 8, 8, 0, STREAM) == 0
    assert r(FAKE, FAKE, FAKE, FAKE, 1 << 31, 1 << 31, 8, 8, 0, STREAM) == -1
    qk = lib.mote_hip_rope_qk_f16
    assert qk(FAKE, None, FAKE, FAKE, FAKE, None, 2, 4, 1, 8, 8, 0, STREAM) == -1  # k heads but no k
    assert qk(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 4, 1, 8, 9, 0, STREAM) == -1
    assert qk(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 0, 4, 1, 8, 8, 0, STREAM) == 0
    assert qk(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 0, 0, 8, 8, 0, STREAM) == 0
    t = lib.mote_hip_rope_tables_f32
    assert t(FAKE, FAKE, FAKE, 4, 7, 10000.0, STREAM) == -1
    assert t(FAKE, FAKE, FAKE, 4, 8, 0.0, STREAM) == -1
    assert t(FAKE, FAKE, FAKE, 4, 8, float("nan"), STREAM) == -1
    assert t(None, FAKE, FAKE, 4, 8, 10000.0, STREAM) == -1
    assert t(FAKE, FAKE, FAKE, 0, 8, 10000.0, STREAM) == 0


def test_runtime_wrappers_reject_null_out_parameters(lib):
    assert lib.mote_hip_get_device_count(None) == -1
    assert lib.mote_hip_malloc(None, 16) == -1
    assert lib.mote_hip_stream_create(None) == -1
    assert lib.mote_hip_mem_get_info(None, None) == -1


def test_dispatch_context_host_state(lib):
    names = [lib.mote_q4_0_variant_name(i).decode() for i in range(lib.mote_q4_0_variant_count())]
    assert len(names) == len(set(names)) and "generic" in names and "gateup_generic" in names
    assert lib.mote_q4_0_variant_name(-1) is None
    assert lib.mote_q4_0_variant_name(len(names)) is None
    h = ctypes.c_void_p()
    assert lib.mote_q4_0_dispatch_create(ctypes.byref(h)) == 0 and h.value
    try:
        assert lib.mote_q4_0_dispatch_force_variant(h, b"no_such_kernel") == 1
        assert b"no_such_kernel" in lib.mote_q4_0_dispatch_last_error(h)
        assert lib.mote_q4_0_dispatch_force_variant(h, names[0].encode()) == 0
        assert lib.mote_q4_0_dispatch_force_variant(h, None) == 0
        assert lib.mote_q4_0_dispatch_set_autotune(h, 1) == 0
        buf = ctypes.create_string_buffer(64)
        assert lib.mote_q4_0_dispatch_plan(h, 1, 4096, 4096, 0, 0, buf, 64) == 500  # nothing cached
        # argument errors surface through last_error without touching a device
        assert lib.mote_q4_0_dispatch_linear(h, None, FAKE, FAKE, 1, 1, 32, 0, STREAM) == 1
        assert lib.mote_q4_0_dispatch_last_error(h) != b""
        assert lib.mote_q4_0_dispatch_linear(h, FAKE, FAKE, FAKE, 0, 1, 32, 0, STREAM) == 0
        assert lib.mote_q4_0_dispatch_gate_up_silu(h, FAKE, FAKE, None, FAKE, 1, 1, 40, 0, STREAM) == 1
    finally:
        lib.mote_q4_0_dispatch_destroy(h)
    assert lib.mote_q4_0_dispatch_create(None) == 1
    assert lib.mote_q4_0_dispatch_linear(None, FAKE, FAKE, FAKE, 1, 1, 32, 0, STREAM) == 1
    assert lib.mote_q4_0_dispatch_set_autotune(None, 1) == 1


def test_dense_matmul_argument_errors_without_a_device(lib):
    """The hipBLASLt boundary's host-side checks (no device, no library load):
    a null out-parameter or context is -1, a null context has no message."""
    assert lib.mote_hipblaslt_create(None) == -1
    assert lib.mote_hipblaslt_last_error(None) is None
    lib.mote_hipblaslt_destroy(None)
    assert lib.mote_hipblaslt_matmul_f16_f32(None, 1, 1, 1, FAKE, FAKE, FAKE, FAKE, 1 << 20, STREAM) == -1


def test_read_probe_is_a_separate_library(lib):
    """The HBM read probe of bench.py --read-floor lives in libmote_probe.so,
    not in the drop-in library; bad arguments return 1 before any launch:
    null pointers, a size that is not a multiple of 16, unsupported thread or
    in-flight counts."""
    assert not hasattr(lib, "mote_hip_read_probe_u128")
    path = os.path.join(ROOT, "mote_amd", "libmote_probe.so")
    probe = ctypes.CDLL(path)
    fn = probe.mote_probe_read_u128
    P, U32 = ctypes.c_void_p, ctypes.c_uint32
    fn.restype = ctypes.c_int
    fn.argtypes = [P, ctypes.c_size_t, U32, U32, U32, ctypes.c_int, P, P]
    assert fn(None, 16, 1, 256, 2, 0, FAKE, STREAM) == 1
    assert fn(FAKE, 17, 1, 256, 2, 0, FAKE, STREAM) == 1
    assert fn(FAKE, 16, 1, 300, 2, 0, FAKE, STREAM) == 1
    assert fn(FAKE, 16, 1, 256, 3, 1, FAKE, STREAM) == 1
    assert fn(FAKE, 0, 1, 256, 2, 0, FAKE, STREAM) == 0  # nothing to read
    copy = probe.mote_probe_copy_rows
    copy.restype = ctypes.c_int
    copy.argtypes = [P, P, U32, U32, P]
    assert copy(None, FAKE, 1, 16, STREAM) == 1
    assert copy(FAKE, FAKE, 1, 24, STREAM) == 1  # row bytes not a multiple of 16
    assert copy(FAKE + 8, FAKE, 1, 16, STREAM) == 1  # misaligned
    assert copy(FAKE, FAKE, 0, 16, STREAM) == 0  # nothing to copy
    # the skinny kernel's timeline instantiation (bench.py --timeline-skinny):
    # 16 words per wave; only its form's K, 1-64 tokens, aligned x and w
    words = probe.mote_probe_skinny_record_words
    words.restype, words.argtypes = U32, []
    assert words() == 16
    tl = probe.mote_probe_skinny_timeline
    tl.restype = ctypes.c_int
    tl.argtypes = [P, P, P, U32, U32, U32, P, ctypes.c_size_t, P]
    assert tl(None, FAKE, FAKE, 16, 4096, 4096, FAKE, 1 << 20, STREAM) == 1
    assert tl(FAKE, FAKE, FAKE, 16, 4096, 4096, None, 1 << 20, STREAM) == 1
    assert tl(FAKE, FAKE, FAKE, 16, 4096, 2048, FAKE, 1 << 20, STREAM) == 1  # not the form's K
    assert tl(FAKE, FAKE, FAKE, 0, 4096, 4096, FAKE, 1 << 20, STREAM) == 1
    assert tl(FAKE, FAKE, FAKE, 65, 4096, 4096, FAKE, 1 << 20, STREAM) == 1
    assert tl(FAKE + 8, FAKE, FAKE, 16, 4096, 4096, FAKE, 1 << 20, STREAM) == 1  # x not 16-byte aligned
    assert tl(FAKE, FAKE + 2, FAKE, 16, 4096, 4096, FAKE, 1 << 20, STREAM) == 1  # w not 4-byte aligned


def test_python_wrappers_raise_hip_error(lib):
    from mote_amd import HipError, ops

    with pytest.raises(HipError) as e:
        ops.quantized_linear_q4_0_f32(FAKE, FAKE, FAKE, 1, 1, 33, STREAM)
    assert e.value.status == 1 and "Q4_0" in str(e.value)
    with pytest.raises(HipError):
        ops.rope_f16(FAKE, FAKE, FAKE, FAKE, 2, 3, 8, 7, ops.HALF_SPLIT, STREAM)
    d = ops.Q4_0Dispatch()
    with pytest.raises(HipError) as e:
        d.force("no_such_kernel")
    assert "no_such_kernel" in str(e.value)
    d.close()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from mote_amd import _ffi

    monkeypatch.setattr(_ffi, "_lib", None)
    monkeypatch.setattr(_ffi, "LIBRARY", str(tmp_path / "absent.so"))
    with pytest.raises(_ffi.LibraryNotBuilt):
        _ffi.lib()
