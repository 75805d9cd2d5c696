"""ctypes binding of the C-ABI library ``libmingru_hip.so``.

Every entry point takes raw device pointers, int64 sizes, a workspace
pointer/size and a ``hipStream_t``, and returns an int status
(``include/mingru_hip.h``).  This module only loads the library and declares
the signatures; it raises ``ImportError`` if the library has not been built.
"""

from __future__ import annotations

import ctypes
import os

from .build import LIB_PATH

MG_OK = 0
MG_STATUS = {
    0: "ok",
    1: "invalid argument",
    2: "kernel launch failed",
    3: "workspace too small",
    4: "problem too large for the static scratch",
    5: "HIP runtime call failed",
    6: "one-time device set-up requested under stream capture",
}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_SZ = ctypes.c_size_t

_SIGNATURES = {
    "mg_linear_scan_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "mg_log_scan_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "mg_linear_scan_fwd": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "mg_linear_scan_bwd": (_I32, [_P] * 8 + [_I64, _I64, _I64, _P, _SZ, _P]),
    "mg_linear_scan_fwd_noalloc": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "mg_linear_scan_noalloc_errors": (_I32, [ctypes.POINTER(ctypes.c_uint), _P]),
    "mg_signed_gate_scan_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "mg_signed_gate_scan_fwd": (_I32, [_P] * 5 + [_I64, _I64, _I64, _I32, _P, _SZ, _P]),
    "mg_signed_gate_scan_bwd": (_I32, [_P] * 10 + [_I64, _I64, _I64, _I32, _P, _SZ, _P]),
    "mg_signed_gate_scan_decay_fwd": (_I32, [_P] * 7 + [_I64, _I64, _I64, _I32, _P, _SZ, _P]),
    "mg_signed_gate_scan_decay_bwd": (_I32, [_P] * 14 + [_I64, _I64, _I64, _I32, _P, _SZ, _P]),
    "mg_mingru_gate_scan_decay_fwd": (_I32, [_P] * 6 + [_I64, _I64, _I64, _P, _SZ, _P]),
    "mg_mingru_gate_scan_decay_bwd": (_I32, [_P] * 12 + [_I64, _I64, _I64, _P, _SZ, _P]),
    "mg_gate_decay_dlam_rows": (_I64, [_I64, _I64, _I64]),
    "mg_gate_decay_ddt_rows": (_I64, [_I64, _I64, _I64]),
    "mg_mingru_gate_scan_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "mg_mingru_gate_scan_fwd": (_I32, [_P] * 4 + [_I64, _I64, _I64, _P, _SZ, _P]),
    "mg_mingru_gate_scan_bwd": (_I32, [_P] * 8 + [_I64, _I64, _I64, _P, _SZ, _P]),
    "mg_gate_step": (_I32, [_I32] + [_P] * 6 + [_I64, _P]),
    "mg_delta_step": (_I32, [_P] * 8 + [_I64, _I32, _I32, _I32, _P]),
    "mg_log_scan_state_bytes": (_SZ, [_I64, _I64, _I64]),
    "mg_log_scan_fwd": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "mg_log_scan_bwd": (_I32, [_P] * 7 + [_I64, _I64, _I64, _P, _SZ, _P]),
    "mg_scan_workspace_errors": (_I32, [_P, ctypes.POINTER(ctypes.c_uint), _P]),
    "mg_affine_scan_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I32, _I32]),
    "mg_affine_scan_fwd": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _P, _SZ, _P]),
    "mg_affine_scan_bwd": (_I32, [_P] * 8 + [_I64, _I64, _I64, _I32, _I32, _P, _SZ, _P]),
    "mg_angle_scan_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I32]),
    "mg_angle_scan_state_bytes": (_SZ, [_I64, _I64, _I64, _I32]),
    "mg_angle_scan_fwd": (
        _I32, [_P] * 7 + [_I64, _I64, _I64, _I32, _I32, _I32, _I32, _P, _SZ, _P],
    ),
    "mg_angle_scan_bwd": (
        _I32, [_P] * 12 + [_I64, _I64, _I64, _I32, _I32, _I32, _I32, _P, _SZ, _P],
    ),
    "mg_angle_scan_gated_fwd": (_I32, [_P] * 8 + [_I64, _I64, _I64, _I32, _I32, _I32, _P, _SZ, _P]),
    "mg_angle_scan_gated_bwd": (
        _I32, [_P] * 15 + [_I64, _I64, _I64, _I32, _I32, _I32, _P, _SZ, _P],
    ),
    "mg_angle_scan_tables_state_bytes": (_SZ, [_I64, _I64, _I64, _I32]),
    "mg_angle_scan_tables_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I32]),
    "mg_angle_scan_tables_fwd": (
        _I32, [_P] * 10 + [_I64, _I64, _I64] + [_I32] * 4 + [_P, _SZ, _P],
    ),
    "mg_angle_scan_tables_bwd": (
        _I32, [_P] * 15 + [_I64, _I64, _I64] + [_I32] * 4 + [_P, _SZ, _P],
    ),
    "mg_delta_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I32, _I32, _I32, _I32]),
    "mg_delta_state_bytes": (_SZ, [_I64, _I64, _I64, _I32, _I32, _I32, _I32]),
    "mg_delta_fwd": (
        _I32,
        [_P] * 5 + [_P] * 3 + [_I64, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _P, _SZ, _P],
    ),
    "mg_delta_bwd": (
        _I32,
        [_P] * 7 + [_P] * 5 + [_I64, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _P, _SZ, _P],
    ),
    "mg_delta_gated_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I32, _I32, _I32, _I32]),
    "mg_delta_gated_fwd": (
        _I32, [_P] * 9 + [_I64, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _P, _SZ, _P],
    ),
    "mg_delta_gated_bwd": (
        _I32, [_P] * 14 + [_I64, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _P, _SZ, _P],
    ),
}

_lib = None


def load():
    """Load the library once and declare every exported signature present."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"HIP library not built: {LIB_PATH} is missing (run `python -m mingru_amd.build`)"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_names():
    """Names from the signature table that the loaded library exports."""
    lib = load()
    return [n for n in _SIGNATURES if getattr(lib, n, None) is not None]


def check(rc: int, what: str) -> None:
    if rc != MG_OK:
        raise RuntimeError(f"{what} failed: status {rc} ({MG_STATUS.get(rc, 'unknown')})")
