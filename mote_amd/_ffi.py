"""ctypes binding of ``libmote_hip.so`` (the C ABI of ``include/mote_hip.h``).

Loading fails loudly: there is no CPU fallback for any operation in this
package.  ``lib()`` raises :class:`LibraryNotBuilt` when the shared library is
absent; build it with ``python -m mote_amd.build``.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libmote_hip.so")


class LibraryNotBuilt(RuntimeError):
    pass


class HipError(RuntimeError):
    """A non-zero status from the C ABI (the reference's HipError::Runtime,
    crates/mote-backend-hip/src/error.rs:8-12,125-131)."""

    def __init__(self, operation: str, status: int, message: str = ""):
        self.operation = operation
        self.status = status
        text = f"HIP {operation} failed with status {status}"
        super().__init__(text + (f": {message}" if message else ""))


_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_SZ = ctypes.c_size_t
_I = ctypes.c_int

# name -> (restype, argtypes); the full exported surface of include/mote_hip.h
SIGNATURES = {
    "mote_hip_get_device_count": (_I, [ctypes.POINTER(_I)]),
    "mote_hip_set_device": (_I, [_I]),
    "mote_hip_malloc": (_I, [ctypes.POINTER(_P), _SZ]),
    "mote_hip_free": (_I, [_P]),
    "mote_hip_memcpy_host_to_device": (_I, [_P, _P, _SZ]),
    "mote_hip_memcpy_device_to_host": (_I, [_P, _P, _SZ]),
    "mote_hip_stream_create": (_I, [ctypes.POINTER(_P)]),
    "mote_hip_stream_destroy": (_I, [_P]),
    "mote_hip_stream_synchronize": (_I, [_P]),
    "mote_hip_mem_get_info": (_I, [ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]),
    "mote_hip_quantized_linear_q4_0_f16": (_I, [_P, _P, _P, _U64, _U64, _U64, _P]),
    "mote_hip_quantized_linear_q4_0_f32": (_I, [_P, _P, _P, _U64, _U64, _U64, _P]),
    "mote_hip_quantized_linear_q4_0_f32_no_alloc": (_I, [_P, _P, _P, _U64, _U64, _U64, _P]),
    "mote_hip_quantized_linear_q8_0_f16": (_I, [_P, _P, _P, _U64, _U64, _U64, _P]),
    "mote_hip_quantized_linear_q8_0_f32": (_I, [_P, _P, _P, _U64, _U64, _U64, _P]),
    "mote_hip_q4_0_gate_up_silu_f32": (_I, [_P, _P, _P, _P, _U64, _U64, _U64, _P]),
    "mote_hip_dequantize_q4_0_f32": (_I, [_P, _P, _U64, _U64, _P]),
    "mote_hip_quantized_linear_q4_k_f16": (_I, [_P, _P, _P, _U64, _U64, _U64, _P]),
    "mote_hip_quantized_linear_q4_k_f32": (_I, [_P, _P, _P, _U64, _U64, _U64, _P]),
    "mote_hip_quantized_linear_q6_k_f16": (_I, [_P, _P, _P, _U64, _U64, _U64, _P]),
    "mote_hip_quantized_linear_q6_k_f32": (_I, [_P, _P, _P, _U64, _U64, _U64, _P]),
    "mote_hip_dequantize_q4_k_f32": (_I, [_P, _P, _U64, _U64, _P]),
    "mote_hip_dequantize_q6_k_f32": (_I, [_P, _P, _U64, _U64, _P]),
    "mote_q4_0_dispatch_create": (_I, [ctypes.POINTER(_P)]),
    "mote_q4_0_dispatch_destroy": (None, [_P]),
    "mote_q4_0_dispatch_last_error": (ctypes.c_char_p, [_P]),
    "mote_q4_0_dispatch_set_autotune": (_I, [_P, _I]),
    "mote_q4_0_dispatch_set_splitk_fold": (_I, [_P, _I]),
    "mote_q4_0_dispatch_force_variant": (_I, [_P, ctypes.c_char_p]),
    "mote_q4_0_dispatch_linear": (_I, [_P, _P, _P, _P, _U64, _U64, _U64, _I, _P]),
    "mote_q4_0_dispatch_linear_q8_0": (_I, [_P, _P, _P, _P, _U64, _U64, _U64, _I, _P]),
    "mote_q4_0_dispatch_gate_up_silu": (_I, [_P, _P, _P, _P, _P, _U64, _U64, _U64, _I, _P]),
    "mote_q4_0_dispatch_plan": (_I, [_P, _U64, _U64, _U64, _I, _I, ctypes.c_char_p, _SZ]),
    "mote_q4_0_dispatch_select": (_I, [_P, _U64, _U64, _U64, _I, ctypes.c_char_p, _SZ]),
    "mote_q4_0_dispatch_candidates": (_I, [_P, _U64, _U64, _U64, _I, ctypes.c_char_p, _SZ]),
    "mote_q4_0_variant_count": (_I, []),
    "mote_q4_0_variant_name": (ctypes.c_char_p, [_I]),
    "mote_hipblaslt_create": (_I, [ctypes.POINTER(_P)]),
    "mote_hipblaslt_destroy": (None, [_P]),
    "mote_hipblaslt_last_error": (ctypes.c_char_p, [_P]),
    "mote_hipblaslt_matmul_f16_f32": (_I, [_P, _U64, _U64, _U64, _P, _P, _P, _P, _SZ, _P]),
    "mote_hip_rms_norm_f16": (_I, [_P, _P, _P, _U64, _U64, ctypes.c_float, _P]),
    "mote_hip_fused_add_rms_norm_f16": (_I, [_P, _P, _P, _P, _U64, _U64, ctypes.c_float, _P]),
    "mote_hip_rope_f16": (_I, [_P, _P, _P, _P, _U64, _U64, _U64, _U64, ctypes.c_uint32, _P]),
    "mote_hip_rope_qk_f16": (
        _I,
        [_P, _P, _P, _P, _P, _P, _U64, _U64, _U64, _U64, _U64, ctypes.c_uint32, _P],
    ),
    "mote_hip_rope_tables_f32": (_I, [_P, _P, _P, _U64, _U64, ctypes.c_double, _P]),
}

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library with every signature declared."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            raise LibraryNotBuilt(
                f"{LIBRARY} is missing: build it with `python -m mote_amd.build` "
                "(there is no fallback implementation)"
            )
        handle = ctypes.CDLL(LIBRARY)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def check(status: int, operation: str) -> None:
    if status != 0:
        raise HipError(operation, status)
