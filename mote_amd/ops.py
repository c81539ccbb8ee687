"""Launch wrappers over the raw C ABI (device pointers as ints, streams as
:class:`mote_amd.device.Stream`).  Every call enqueues asynchronously and
raises :class:`mote_amd._ffi.HipError` on a non-zero status."""

from __future__ import annotations

import ctypes

from ._ffi import HipError, check, lib

HALF_SPLIT = 0
INTERLEAVED = 1


def _s(stream) -> int:
    return stream.handle if hasattr(stream, "handle") else int(stream)


def quantized_linear_q4_0_f16(x, w, y, rows, n, k, stream) -> None:
    check(lib().mote_hip_quantized_linear_q4_0_f16(x, w, y, rows, n, k, _s(stream)), "launch Q4_0 linear kernel")


def quantized_linear_q4_0_f32(x, w, y, rows, n, k, stream) -> None:
    check(lib().mote_hip_quantized_linear_q4_0_f32(x, w, y, rows, n, k, _s(stream)), "launch Q4_0 linear kernel")


def quantized_linear_q4_0_f32_no_alloc(x, w, y, rows, n, k, stream) -> None:
    """The f32 linear without any device allocation (split-K scratch in the
    library's static device array; overlapping calls on one GPU race)."""
    check(lib().mote_hip_quantized_linear_q4_0_f32_no_alloc(x, w, y, rows, n, k, _s(stream)),
          "launch Q4_0 linear kernel (no allocation)")


def quantized_linear_q8_0_f16(x, w, y, rows, n, k, stream) -> None:
    check(lib().mote_hip_quantized_linear_q8_0_f16(x, w, y, rows, n, k, _s(stream)), "launch Q8_0 linear kernel")


def quantized_linear_q8_0_f32(x, w, y, rows, n, k, stream) -> None:
    check(lib().mote_hip_quantized_linear_q8_0_f32(x, w, y, rows, n, k, _s(stream)), "launch Q8_0 linear kernel")


def q4_0_gate_up_silu_f32(x, w_gate, w_up, y, rows, n, k, stream) -> None:
    check(
        lib().mote_hip_q4_0_gate_up_silu_f32(x, w_gate, w_up, y, rows, n, k, _s(stream)),
        "launch Q4_0 gate/up kernel",
    )


def dequantize_q4_0_f32(w, out, rows, k, stream) -> None:
    check(lib().mote_hip_dequantize_q4_0_f32(w, out, rows, k, _s(stream)), "launch Q4_0 decode kernel")


def quantized_linear_q4_k_f16(x, w, y, rows, n, k, stream) -> None:
    check(lib().mote_hip_quantized_linear_q4_k_f16(x, w, y, rows, n, k, _s(stream)), "launch Q4_K linear kernel")


def quantized_linear_q4_k_f32(x, w, y, rows, n, k, stream) -> None:
    check(lib().mote_hip_quantized_linear_q4_k_f32(x, w, y, rows, n, k, _s(stream)), "launch Q4_K linear kernel")


def quantized_linear_q6_k_f16(x, w, y, rows, n, k, stream) -> None:
    check(lib().mote_hip_quantized_linear_q6_k_f16(x, w, y, rows, n, k, _s(stream)), "launch Q6_K linear kernel")


def quantized_linear_q6_k_f32(x, w, y, rows, n, k, stream) -> None:
    check(lib().mote_hip_quantized_linear_q6_k_f32(x, w, y, rows, n, k, _s(stream)), "launch Q6_K linear kernel")


def dequantize_q4_k_f32(w, out, rows, k, stream) -> None:
    check(lib().mote_hip_dequantize_q4_k_f32(w, out, rows, k, _s(stream)), "launch Q4_K decode kernel")


def dequantize_q6_k_f32(w, out, rows, k, stream) -> None:
    check(lib().mote_hip_dequantize_q6_k_f32(w, out, rows, k, _s(stream)), "launch Q6_K decode kernel")


def rms_norm_f16(x, weight, y, rows, hidden, eps, stream) -> None:
    check(lib().mote_hip_rms_norm_f16(x, weight, y, rows, hidden, eps, _s(stream)), "launch RMSNorm kernel")


def fused_add_rms_norm_f16(x, residual, weight, y, rows, hidden, eps, stream) -> None:
    check(
        lib().mote_hip_fused_add_rms_norm_f16(x, residual, weight, y, rows, hidden, eps, _s(stream)),
        "launch fused add + RMSNorm kernel",
    )


def rope_f16(x, cos, sin, y, tokens, heads, head_dim, rotary_dim, layout, stream) -> None:
    check(
        lib().mote_hip_rope_f16(x, cos, sin, y, tokens, heads, head_dim, rotary_dim, layout, _s(stream)),
        "launch RoPE kernel",
    )


def rope_qk_f16(q, k, cos, sin, q_out, k_out, tokens, q_heads, k_heads, head_dim, rotary_dim, layout, stream) -> None:
    check(
        lib().mote_hip_rope_qk_f16(
            q, k, cos, sin, q_out, k_out, tokens, q_heads, k_heads, head_dim, rotary_dim, layout, _s(stream)
        ),
        "launch fused q/k RoPE kernel",
    )


def rope_tables_f32(positions, cos, sin, tokens, rotary_dim, theta, stream) -> None:
    check(
        lib().mote_hip_rope_tables_f32(positions, cos, sin, tokens, rotary_dim, float(theta), _s(stream)),
        "launch RoPE table kernel",
    )


def variant_names() -> list[str]:
    h = lib()
    return [h.mote_q4_0_variant_name(i).decode() for i in range(h.mote_q4_0_variant_count())]


class Q4_0Dispatch:
    """A dispatch context: per-(M, N, K) plan cache with optional autotuning."""

    def __init__(self, autotune: bool = False) -> None:
        handle = ctypes.c_void_p()
        check(lib().mote_q4_0_dispatch_create(ctypes.byref(handle)), "create Q4_0 dispatch context")
        self.handle = handle.value
        if autotune:
            self.set_autotune(True)

    def _check(self, status: int, operation: str) -> None:
        if status != 0:
            msg = lib().mote_q4_0_dispatch_last_error(self.handle)
            raise HipError(operation, status, msg.decode() if msg else "")

    def set_autotune(self, enabled: bool) -> None:
        self._check(lib().mote_q4_0_dispatch_set_autotune(self.handle, int(enabled)), "set autotune")

    def set_splitk_fold(self, enabled: bool) -> None:
        self._check(lib().mote_q4_0_dispatch_set_splitk_fold(self.handle, int(enabled)), "set split-K fold")

    def force(self, name: str | None) -> None:
        self._check(
            lib().mote_q4_0_dispatch_force_variant(self.handle, name.encode() if name else None),
            "force Q4_0 variant",
        )

    def linear(self, x, w, y, rows, n, k, stream, f16_out: bool = False) -> None:
        self._check(
            lib().mote_q4_0_dispatch_linear(self.handle, x, w, y, rows, n, k, int(f16_out), _s(stream)),
            "launch Q4_0 linear",
        )

    def linear_q8_0(self, x, w, y, rows, n, k, stream, f16_out: bool = False) -> None:
        self._check(
            lib().mote_q4_0_dispatch_linear_q8_0(self.handle, x, w, y, rows, n, k, int(f16_out), _s(stream)),
            "launch Q8_0 linear",
        )

    def gate_up_silu(self, x, w_gate, w_up, y, rows, n, k, stream, f16_out: bool = False) -> None:
        self._check(
            lib().mote_q4_0_dispatch_gate_up_silu(
                self.handle, x, w_gate, w_up, y, rows, n, k, int(f16_out), _s(stream)
            ),
            "launch Q4_0 gate/up",
        )

    def plan(self, rows, n, k, gate_up: bool = False, f16_out: bool = False, q8_0: bool = False) -> str | None:
        buf = ctypes.create_string_buffer(64)
        op = 2 if q8_0 else int(gate_up)
        status = lib().mote_q4_0_dispatch_plan(self.handle, rows, n, k, op, int(f16_out), buf, 64)
        return buf.value.decode() if status == 0 else None

    def select(self, rows, n, k, gate_up: bool = False, q8_0: bool = False) -> str:
        """The variant a call of this shape would plan (aligned operands),
        chosen on the host without launching anything."""
        buf = ctypes.create_string_buffer(64)
        op = 2 if q8_0 else int(gate_up)
        self._check(lib().mote_q4_0_dispatch_select(self.handle, rows, n, k, op, buf, 64), "select Q4_0 variant")
        return buf.value.decode()

    def candidates(self, rows, n, k, gate_up: bool = False, q8_0: bool = False) -> list[str]:
        """The variants the autotuner would time for this shape (aligned
        operands), the rule-based heuristic's pick included; host only."""
        buf = ctypes.create_string_buffer(1 << 14)
        op = 2 if q8_0 else int(gate_up)
        self._check(lib().mote_q4_0_dispatch_candidates(self.handle, rows, n, k, op, buf, len(buf)),
                    "list Q4_0 candidates")
        return [v for v in buf.value.decode().split(",") if v]

    def close(self) -> None:
        if self.handle:
            lib().mote_q4_0_dispatch_destroy(self.handle)
            self.handle = 0

    def __del__(self) -> None:  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass


class DenseMatmul:
    """A hipBLASLt matmul context (the reference's HipBlasLt handle,
    crates/mote-backend-hip/src/ffi.rs:341-419): row-major f32 C[m, n] =
    f16 A[m, k] B[k, n], one tuned plan per shape, a caller-owned workspace."""

    WORKSPACE_BYTES = 32 * 1024 * 1024  # the reference context's workspace (src/context.rs:11)

    def __init__(self) -> None:
        handle = ctypes.c_void_p()
        check(lib().mote_hipblaslt_create(ctypes.byref(handle)), "create hipBLASLt context")
        self.handle = handle.value

    def last_error(self) -> str:
        msg = lib().mote_hipblaslt_last_error(self.handle)
        return msg.decode() if msg else ""

    def matmul_f16_f32(self, m, n, k, lhs, rhs, out, workspace, workspace_bytes, stream) -> None:
        status = lib().mote_hipblaslt_matmul_f16_f32(
            self.handle, m, n, k, lhs, rhs, out, workspace, workspace_bytes, _s(stream)
        )
        if status != 0:
            raise HipError("F16/F32 matmul", status, self.last_error())

    def close(self) -> None:
        if self.handle:
            lib().mote_hipblaslt_destroy(self.handle)
            self.handle = 0

    def __del__(self) -> None:  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass
