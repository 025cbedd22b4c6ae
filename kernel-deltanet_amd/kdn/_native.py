"""ctypes binding of libkdn.so, the C ABI declared in include/kdn.h.

The shared library is built in-tree (kdn.build.build_native) and loaded from this directory.  There
is no fallback: if the library is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
# KDN_LIBRARY selects another build of the same library (the host-sanitized one of the host-path tests)
LIB_PATH = os.environ.get("KDN_LIBRARY") or os.path.join(_HERE, "libkdn.so")

KDN_OK = 0
KDN_DTYPE_F32 = 0
KDN_DTYPE_BF16 = 1

# Exported symbols of include/kdn.h (checked by tests/test_abi.py).
EXPORTED = (
    "kdn_strerror",
    "kdn_abi_version",
    "kdn_build_omega",
    "kdn_fwht",
    "kdn_fwht_lift",
    "kdn_fwht_lift_bits",
    "kdn_fwht_lift_factored",
    "kdn_scan_workspace_bytes",
    "kdn_delta_scan_fwd",
    "kdn_delta_scan_fwd_noalloc",
    "kdn_scan_prep",
    "kdn_scan_state",
    "kdn_scan_output",
    "kdn_scan_prep_fused",
    "kdn_scan_chain",
    "kdn_scan_schedule",
    "kdn_scan_segment_chunks",
    "kdn_scan_workspace_bytes_pipelined",
    "kdn_delta_scan_fwd_pipelined",
    "kdn_delta_scan_fwd_streams",
    "kdn_ragged_workspace_bytes",
    "kdn_ragged_step",
    "kdn_slot_step_workspace_bytes",
    "kdn_slot_step",
    "kdn_pool_create",
    "kdn_pool_destroy",
    "kdn_pool_allocate",
    "kdn_pool_fork",
    "kdn_pool_release",
    "kdn_pool_active",
    "kdn_pool_allocated_bytes",
    "kdn_pool_free_bytes",
    "kdn_scan_bwd_workspace_bytes",
    "kdn_delta_scan_bwd",
    "kdn_delta_scan_bwd_streams",
    "kdn_scan_bwd_phase",
    "kdn_scan_bwd_segments",
    "kdn_fwht_lift_bits_butterfly",
    "kdn_fwht_lift_factored_bwd",
)

KDN_ERR_CAPACITY = -6
KDN_ERR_WORKSPACE_TOO_SMALL = -3
NOALLOC_SCRATCH_BYTES = 256 << 20   # KDN_NOALLOC_SCRATCH_BYTES of include/kdn.h

_i64 = ctypes.c_int64
_i64x3 = ctypes.c_int64 * 3
_i64x4 = ctypes.c_int64 * 4


class ScanArgs(ctypes.Structure):
    """Mirror of struct kdn_scan_args (include/kdn.h); field order and types must match exactly."""

    _fields_ = [
        ("B", _i64), ("T", _i64), ("H", _i64),
        ("d_k", ctypes.c_int), ("D", ctypes.c_int), ("d_v", ctypes.c_int),
        ("in_dtype", ctypes.c_int), ("out_dtype", ctypes.c_int), ("normalize_input", ctypes.c_int),
        ("inv_tau", ctypes.c_float),
        ("q", ctypes.c_void_p), ("q_stride", _i64x3),
        ("k", ctypes.c_void_p), ("k_stride", _i64x3),
        ("v", ctypes.c_void_p), ("v_stride", _i64x3),
        ("beta", ctypes.c_void_p), ("beta_stride", _i64x3),
        ("decay", ctypes.c_void_p), ("decay_stride", _i64x3),
        ("omega_bf16", ctypes.c_void_p),
        ("phase", ctypes.c_void_p),
        ("initial_state", ctypes.c_void_p), ("init_stride", _i64x4),
        ("final_state", ctypes.c_void_p), ("final_stride", _i64x4),
        ("y", ctypes.c_void_p), ("y_stride", _i64x3),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("segment_chunks", _i64),
        ("omega_lo", ctypes.c_void_p),
        ("omega_head_stride", _i64),
        ("phase_head_stride", _i64),
        ("inv_tau_head", ctypes.c_void_p),
        ("no_renorm", ctypes.c_int),
        ("feature_mode", ctypes.c_int),
        ("rule", ctypes.c_int),
        ("cu_seqlens", ctypes.c_void_p),
        ("state_slots", ctypes.c_void_p),
    ]


_i64x2 = ctypes.c_int64 * 2


class RaggedArgs(ctypes.Structure):
    """Mirror of struct kdn_ragged_args (include/kdn.h)."""

    _fields_ = [
        ("num_seqs", _i64), ("H", _i64),
        ("d_k", ctypes.c_int), ("D", ctypes.c_int), ("d_v", ctypes.c_int),
        ("in_dtype", ctypes.c_int), ("out_dtype", ctypes.c_int), ("normalize_input", ctypes.c_int),
        ("rule", ctypes.c_int),
        ("inv_tau", ctypes.c_float),
        ("cu_seqlens", ctypes.c_void_p),
        ("cu_seqlens_host", ctypes.c_void_p),
        ("slots", ctypes.c_void_p),
        ("q", ctypes.c_void_p), ("q_stride", _i64x2),
        ("k", ctypes.c_void_p), ("k_stride", _i64x2),
        ("v", ctypes.c_void_p), ("v_stride", _i64x2),
        ("beta", ctypes.c_void_p), ("beta_stride", _i64x2),
        ("decay", ctypes.c_void_p), ("decay_stride", _i64x2),
        ("omega_bf16", ctypes.c_void_p), ("phase", ctypes.c_void_p),
        ("states", ctypes.c_void_p), ("state_stride", _i64x4),
        ("y", ctypes.c_void_p), ("y_stride", _i64x2),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("num_slots", _i64),
    ]


class SlotStepArgs(ctypes.Structure):
    """Mirror of struct kdn_slot_step_args (include/kdn.h)."""

    _fields_ = [
        ("num_tokens", _i64), ("H", _i64),
        ("d_k", ctypes.c_int), ("D", ctypes.c_int), ("d_v", ctypes.c_int),
        ("in_dtype", ctypes.c_int), ("out_dtype", ctypes.c_int), ("normalize_input", ctypes.c_int),
        ("rule", ctypes.c_int),
        ("inv_tau", ctypes.c_float),
        ("slot_mapping", ctypes.c_void_p),
        ("slot_bytes", ctypes.c_int),
        ("q", ctypes.c_void_p), ("q_stride", _i64x2),
        ("k", ctypes.c_void_p), ("k_stride", _i64x2),
        ("v", ctypes.c_void_p), ("v_stride", _i64x2),
        ("beta", ctypes.c_void_p), ("beta_stride", _i64x2),
        ("decay", ctypes.c_void_p), ("decay_stride", _i64x2),
        ("omega_bf16", ctypes.c_void_p), ("phase", ctypes.c_void_p),
        ("states", ctypes.c_void_p), ("state_stride", _i64x4),
        ("num_slots", _i64),
        ("y", ctypes.c_void_p), ("y_stride", _i64x2),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("status", ctypes.c_void_p),
    ]


class ScanBwdArgs(ctypes.Structure):
    """Mirror of struct kdn_scan_bwd_args (include/kdn.h)."""

    _fields_ = [
        ("fwd", ctypes.c_void_p),
        ("dy", ctypes.c_void_p), ("dy_stride", _i64x3),
        ("d_final_state", ctypes.c_void_p), ("dfinal_stride", _i64x4),
        ("dq", ctypes.c_void_p), ("dq_stride", _i64x3),
        ("dk", ctypes.c_void_p), ("dk_stride", _i64x3),
        ("dv", ctypes.c_void_p), ("dv_stride", _i64x3),
        ("dbeta", ctypes.c_void_p), ("dbeta_stride", _i64x3),
        ("ddecay", ctypes.c_void_p), ("ddecay_stride", _i64x3),
        ("d_initial_state", ctypes.c_void_p), ("dinit_stride", _i64x4),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("dinv_tau", ctypes.c_void_p),
    ]


_lib = None
_lock = threading.Lock()


class NativeLibraryMissing(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """The loaded library (raises NativeLibraryMissing if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NativeLibraryMissing(
                    f"kernel-deltanet_amd: native library not built ({LIB_PATH} missing); "
                    "run __graft_entry__.build() (hipcc --offload-arch=gfx950)")
            L = ctypes.CDLL(LIB_PATH)
            vp, i64, ci, cf, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
            L.kdn_strerror.argtypes = [ci]
            L.kdn_strerror.restype = ctypes.c_char_p
            L.kdn_abi_version.argtypes = []
            L.kdn_abi_version.restype = ci
            L.kdn_build_omega.argtypes = [vp, ci, ci, vp, ci, vp]
            L.kdn_build_omega.restype = ci
            L.kdn_fwht.argtypes = [vp, i64, i64, ci, ci, vp, i64, vp]
            L.kdn_fwht.restype = ci
            L.kdn_fwht_lift.argtypes = [vp, i64, i64, ci, ci, vp, vp, ci, ci, cf, vp, i64, ci, vp]
            L.kdn_fwht_lift.restype = ci
            L.kdn_fwht_lift_bits.argtypes = [vp, i64, i64, ci, ci, vp, ci, cf, vp, ci, vp, i64, ci, vp]
            L.kdn_fwht_lift_bits_butterfly.argtypes = L.kdn_fwht_lift_bits.argtypes
            L.kdn_fwht_lift_bits.restype = ci
            L.kdn_fwht_lift_bits_butterfly.restype = ci
            L.kdn_scan_workspace_bytes.argtypes = [ctypes.POINTER(ScanArgs)]
            L.kdn_scan_workspace_bytes.restype = sz
            L.kdn_delta_scan_fwd.argtypes = [ctypes.POINTER(ScanArgs), vp]
            L.kdn_delta_scan_fwd.restype = ci
            L.kdn_delta_scan_fwd_noalloc.argtypes = [ctypes.POINTER(ScanArgs), vp]
            L.kdn_delta_scan_fwd_noalloc.restype = ci
            L.kdn_scan_workspace_bytes_pipelined.argtypes = [ctypes.POINTER(ScanArgs)]
            L.kdn_scan_workspace_bytes_pipelined.restype = sz
            L.kdn_delta_scan_fwd_pipelined.argtypes = [ctypes.POINTER(ScanArgs), vp, vp]
            L.kdn_delta_scan_fwd_pipelined.restype = ci
            L.kdn_delta_scan_fwd_streams.argtypes = [ctypes.POINTER(ScanArgs), vp, vp, vp]
            L.kdn_delta_scan_fwd_streams.restype = ci
            L.kdn_scan_schedule.argtypes = [ctypes.POINTER(ScanArgs)]
            L.kdn_scan_schedule.restype = ci
            L.kdn_scan_segment_chunks.argtypes = [ctypes.POINTER(ScanArgs), ci]
            L.kdn_scan_segment_chunks.restype = i64
            for nm in ("kdn_scan_prep", "kdn_scan_state", "kdn_scan_output", "kdn_scan_prep_fused", "kdn_scan_chain"):
                fn = getattr(L, nm)
                fn.argtypes = [ctypes.POINTER(ScanArgs), i64, i64, vp]
                fn.restype = ci
            L.kdn_ragged_workspace_bytes.argtypes = [ctypes.POINTER(RaggedArgs)]
            L.kdn_ragged_workspace_bytes.restype = sz
            L.kdn_ragged_step.argtypes = [ctypes.POINTER(RaggedArgs), vp, vp]
            L.kdn_ragged_step.restype = ci
            L.kdn_slot_step_workspace_bytes.argtypes = [ctypes.POINTER(SlotStepArgs)]
            L.kdn_slot_step_workspace_bytes.restype = sz
            L.kdn_slot_step.argtypes = [ctypes.POINTER(SlotStepArgs), vp, vp]
            L.kdn_slot_step.restype = ci
            L.kdn_pool_create.argtypes = [i64, i64, ctypes.POINTER(vp)]
            L.kdn_pool_create.restype = ci
            L.kdn_pool_destroy.argtypes = [vp]
            L.kdn_pool_destroy.restype = None
            L.kdn_pool_allocate.argtypes = [vp, vp, vp]
            L.kdn_pool_allocate.restype = ci
            L.kdn_pool_fork.argtypes = [vp, ci, vp, vp]
            L.kdn_pool_fork.restype = ci
            L.kdn_pool_release.argtypes = [vp, ci]
            L.kdn_pool_release.restype = ci
            for nm in ("kdn_pool_active", "kdn_pool_allocated_bytes", "kdn_pool_free_bytes"):
                fn = getattr(L, nm)
                fn.argtypes = [vp]
                fn.restype = i64
            L.kdn_scan_bwd_workspace_bytes.argtypes = [ctypes.POINTER(ScanBwdArgs)]
            L.kdn_scan_bwd_workspace_bytes.restype = sz
            L.kdn_delta_scan_bwd.argtypes = [ctypes.POINTER(ScanBwdArgs), vp]
            L.kdn_delta_scan_bwd.restype = ci
            L.kdn_delta_scan_bwd_streams.argtypes = [ctypes.POINTER(ScanBwdArgs), vp, vp]
            L.kdn_delta_scan_bwd_streams.restype = ci
            L.kdn_fwht_lift_factored.argtypes = [vp, i64, i64, ci, vp, vp, vp, vp, cf, vp, i64, ci, vp]
            L.kdn_fwht_lift_factored.restype = ci
            L.kdn_fwht_lift_factored_bwd.argtypes = [vp, i64, i64, ci, vp, vp, vp, vp, cf, vp, i64, vp, i64, vp]
            L.kdn_fwht_lift_factored_bwd.restype = ci
            L.kdn_scan_bwd_phase.argtypes = [ctypes.POINTER(ScanBwdArgs), ci, i64, vp]
            L.kdn_scan_bwd_phase.restype = ci
            L.kdn_scan_bwd_segments.argtypes = [ctypes.POINTER(ScanBwdArgs), ctypes.POINTER(ctypes.c_int64)]
            L.kdn_scan_bwd_segments.restype = i64
            _lib = L
    return _lib


def check(status: int, what: str) -> None:
    if status != KDN_OK:
        msg = lib().kdn_strerror(int(status)).decode()
        raise RuntimeError(f"{what} failed: status {status} ({msg})")
