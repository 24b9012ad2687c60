"""ctypes binding of libqwen_gpu.so / libnebula_moe.so.

Mirrors the reference's binding (qwen/test_gpu.py:12-61): a SIGNATURES table
bound onto ``qg_*`` symbols, ``call()`` raising on a nonzero status with the
text of ``qg_error``, and a ``Device`` wrapper over ``qg_alloc/write/read``.
Loading fails loudly when the native library is missing: there is no Python
or CPU fallback for any operator.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIBDIR = Path(__file__).resolve().parent / "lib"
P, I, F, Z, D64, U64 = C.c_void_p, C.c_int, C.c_float, C.c_size_t, C.c_double, C.c_uint64

SIGNATURES = {
    # runtime (gpu.h:11-36)
    "alloc": ([Z], P), "free": ([P], None), "write": ([P, P, Z], I), "read": ([P, P, Z], I),
    "copy": ([P, P, Z], I), "zero": ([P, Z], I), "sync": ([], I), "error": ([I], C.c_char_p),
    "memory": ([P, P], I), "tensor_bytes": ([I, P, P], I),
    "graph_begin": ([P], I), "graph_end": ([P], I), "graph_launch": ([P], I), "graph_destroy": ([P], None),
    "upload_create": ([Z], P), "upload_destroy": ([P], None), "upload_expert": ([P, P, P, Z, P, Z, P, Z], I),
    "upload_seconds": ([P], D64),
    # operators (gpu.h:37-43,62-78)
    "matmul": ([P, P, I, I, I, P, I], I), "gather": ([P, P, I, I, I], I),
    "norm": ([P, P, P, I, I, I, I, I, F], I), "unary": ([P, P, I, I, F], I), "binary": ([P, P, P, I, I], I),
    "route": ([P, P, P, I], I), "prune_routes": ([P, P, P, I, D64, P], I),
    "moe_map": ([P, P, I], I), "moe_gather": ([P, P, P, I], I), "moe_scatter": ([P, P, P, P, P, I, I], I),
    "moe_reduce": ([P, P, I], I), "mtp_moe": ([P, P, P, P, P, P, I, P, I, P, I, I], I),
    "dequant": ([P, P, I, I, I], I), "shared_add": ([P, P, P, I], I),
    # additions
    "moe_configure": ([I, I], I), "moe_configure_thread": ([I, I], I), "moe_dispatch": ([P, P, P, P, P, I], I),
    "moe_workspace_bytes": ([I, I, I], Z), "moe_phase_events": ([P, I], I), "moe_forward": ([P, P, P, P, P, P, I, P, P, Z], I),
    "moe_forward_noalloc": ([P, P, P, P, P, P, I, P], I),
    "moe_forward_residual": ([P, P, P, P, P, P, P, I, P, P, Z], I), "moe_kernel_events": ([P, I], I),
    "event_create": ([], P), "event_destroy": ([P], None), "event_record": ([P], I), "event_elapsed": ([P, P, P], I),
    "device_info": ([P, Z, P, P, P, P], I),
    "synth_matrix": ([P, I, U64, U64, I, I, F], I), "synth_experts": ([P, I, U64, I, I, I, I, F], I), "prefill_int8_dense": ([I], I),
    "moe_handoff_pack": ([P, P, P, P, P, P, P, P, P, I, I], I), "moe_handoff_merge": ([P, P, P, P, I, I], I),
    "moe_handoff_notify": ([P, P], I), "host_alloc": ([Z], P), "host_free": ([P], None),
}

# nm_cpu_moe_fn of include/nebula_moe.h: (ctx, out, x, ids, weights, tokens) -> 0 on success
CPU_MOE_FN = C.CFUNCTYPE(I, P, P, P, P, P, I)

HOST_SIGNATURES = {
    "stack_create": ([P, I, I, I], P), "stack_destroy": ([P], None), "stack_hidden": ([P], P),
    "stack_forward": ([P, I, I], I), "stack_record": ([P, I, P, P, P, P], I), "last_error": ([], C.c_char_p),
    "handoff_scratch_bytes": ([I, I], Z),
    "moe_handoff": ([P, P, P, P, P, P, I, I, P, Z, CPU_MOE_FN, P, P], I),
    "handoff_reserve": ([I, I], I), "device_reads": ([], C.c_uint64),
}


# libnebula_moe.so's qwen_* surface (include/qwen_moe.h, after qwen.h)
QWEN_CPU_MOE_FN = C.CFUNCTYPE(I, P, P, P, P, P, I, P, I, P, I, P, I)
QWEN_SIGNATURES = {
    "validate_index": ([C.c_char_p], I), "open": ([C.c_char_p, I, I, I], P), "close": ([P], None),
    "last_error": ([], C.c_char_p), "max_draft": ([], I), "set_hotlist": ([P, P, I, I], I),
    "set_cpu_threads": ([P, I], I), "cpu_threads": ([P], I), "get_cpu_stats": ([P, P], None),
    "handoff_version": ([], I), "get_prune_stats": ([P, P], I), "get_handoff_profile": ([P, P], None),
    "get_stats": ([P, P], None), "profile_routes": ([P, C.c_char_p], I), "set_cpu_moe": ([P, QWEN_CPU_MOE_FN, P], I),
    "moe_shape": ([P, P, P, P, P], I), "moe": ([P, I, P, P, I, I], I),
}


class QwenStats(C.Structure):
    """qwen_stats (qwen.h:11-18)."""
    _fields_ = [(k, C.c_uint64) for k in (
        "gpu_weight_bytes", "gpu_state_bytes", "gpu_workspace_bytes", "gpu_arena_bytes", "target_tokens", "mtp_tokens",
        "expert_handoffs", "expert_upload_bytes", "expert_hits", "expert_requests", "metadata_read_bytes", "ple_read_bytes",
        "host_weight_bytes", "host_staging_bytes")] + [(k, C.c_double) for k in (
        "target_seconds", "mtp_seconds", "expert_handoff_host_seconds", "expert_dma_seconds", "ple_lookup_seconds",
        "core_load_seconds", "host_load_seconds")] + [(k, C.c_int) for k in (
        "target_position", "mtp_position", "context", "resident_per_layer")]


class QwenHandoffProfile(C.Structure):
    """qwen_handoff_profile (qwen.h:19-21)."""
    _fields_ = [("layer_calls", C.c_uint64 * 48), ("layer_handoffs", C.c_uint64 * 48)]


class QwenCpuStats(C.Structure):
    """qwen_cpu_stats (qwen.h:68-71)."""
    _fields_ = [(k, C.c_uint64) for k in ("layer_handoffs", "token_layers", "missing_selections", "activation_bytes")] + [
        ("compute_seconds", C.c_double), ("handoff_seconds", C.c_double)]


class PruneStats(C.Structure):
    _fields_ = [(k, C.c_uint64) for k in ("token_layers", "missing_selections", "skipped_selections", "avoided_token_handoffs")] + [
        ("skipped_mass", C.c_double)]


class MoeLayer(C.Structure):
    """qg_moe_layer of include/qwen_gpu.h."""
    _fields_ = [("width", I), ("ff", I), ("router", P), ("gate", P), ("up", P), ("down", P),
                ("gate_type", I), ("up_type", I), ("down_type", I),
                ("sh_gate", P), ("sh_up", P), ("sh_down", P), ("sh_gate_type", I), ("sh_up_type", I), ("sh_down_type", I),
                ("sh_gate_inp", P), ("resident", P), ("threshold", D64), ("router_bias", P)]


_LIB = None
_HOST = None


def lib() -> C.CDLL:
    """libqwen_gpu.so with every SIGNATURES entry bound (raises if not built)."""
    global _LIB
    if _LIB is None:
        path = LIBDIR / "libqwen_gpu.so"
        if not path.exists():
            raise RuntimeError(f"{path} is not built; run __graft_entry__.build() or python -m nebula_amd.build")
        handle = C.CDLL(str(path))
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(handle, "qg_" + name)
            fn.argtypes, fn.restype = args, res
        _LIB = handle
    return _LIB


def host() -> C.CDLL:
    global _HOST
    if _HOST is None:
        lib()
        path = LIBDIR / "libnebula_moe.so"
        if not path.exists():
            raise RuntimeError(f"{path} is not built")
        handle = C.CDLL(str(path))
        for name, (args, res) in HOST_SIGNATURES.items():
            fn = getattr(handle, "nm_" + name)
            fn.argtypes, fn.restype = args, res
        _HOST = handle
    return _HOST


_QWEN = None


def qwen() -> C.CDLL:
    """libnebula_moe.so with the qwen_* surface bound."""
    global _QWEN
    if _QWEN is None:
        handle = host()
        for name, (args, res) in QWEN_SIGNATURES.items():
            fn = getattr(handle, "qwen_" + name)
            fn.argtypes, fn.restype = args, res
        _QWEN = handle
    return _QWEN


def call(name: str, *args) -> None:
    code = getattr(lib(), "qg_" + name)(*args)
    if code:
        raise RuntimeError(f"qg_{name}: {lib().qg_error(code).decode()} ({code})")


class Device:
    """Device copy of a numpy array (qg_alloc + qg_write); .get() reads it back."""

    def __init__(self, x=None, *, nbytes: int | None = None, dtype=np.uint8, shape=None):
        if x is None:
            shape = shape if shape is not None else (nbytes,)
            x = np.zeros(shape, dtype)
            self.x = x
            self.p = lib().qg_alloc(max(x.nbytes, 1))
            if not self.p:
                raise MemoryError("qg_alloc")
            call("zero", self.p, x.nbytes)
        else:
            self.x = np.ascontiguousarray(x)
            self.p = lib().qg_alloc(max(self.x.nbytes, 1))
            if not self.p:
                raise MemoryError("qg_alloc")
            call("write", self.p, self.x.ctypes.data, self.x.nbytes)

    @property
    def nbytes(self) -> int:
        return self.x.nbytes

    def get(self) -> np.ndarray:
        out = np.empty_like(self.x)
        call("read", out.ctypes.data, self.p, out.nbytes)
        return out

    def set(self, x) -> None:
        """Overwrite the buffer's leading bytes with x (same or smaller size)."""
        x = np.ascontiguousarray(x)
        if x.nbytes > self.x.nbytes:
            raise ValueError(f"{x.nbytes} bytes do not fit a {self.x.nbytes}-byte buffer")
        call("write", self.p, x.ctypes.data, x.nbytes)

    def free(self) -> None:
        if getattr(self, "p", None):
            lib().qg_free(self.p)
            self.p = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        self.p = lib().qg_event_create()
        if not self.p:
            raise RuntimeError("qg_event_create")

    def record(self) -> None:
        call("event_record", self.p)

    def __del__(self):
        if getattr(self, "p", None):
            lib().qg_event_destroy(self.p)


def elapsed_ms(begin: Event, end: Event) -> float:
    ms = C.c_float()
    call("event_elapsed", C.byref(ms), begin.p, end.p)
    return float(ms.value)


def row_bytes(typ: int, cols: int) -> int:
    return {0: cols * 4, 12: cols // 256 * 144, 20: cols // 32 * 18, 1: cols * 2, 30: cols * 2,
            2: cols // 32 * 18, 6: cols // 32 * 22, 7: cols // 32 * 24, 8: cols // 32 * 34,
            13: cols // 256 * 176, 14: cols // 256 * 210}[typ]
