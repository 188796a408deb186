"""ctypes binding of libdfmi.so (the C ABI declared in include/dfmi.h).

The library is loaded once per process.  When it is missing every operator
raises: there is no CPU or eager-PyTorch substitute for the kernels.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libdfmi.so")

DFMI_OK = 0
DFMI_EINVAL = -1
DFMI_ELAUNCH = -2
DFMI_ENOSPC = -3

DFMI_BF16 = 0
DFMI_F16 = 1
DFMI_F32 = 2

DFMI_QMM_RECORD_BYTES = 1024

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_size = ctypes.c_size_t
_float = ctypes.c_float


class QmmTuning(ctypes.Structure):
    """dfmi_qmm_tuning: path (1 general, 2 streaming), tiles_per_wave,
    waves_per_block (general kernel K split), k_splits (streaming kernel K
    split across workgroups), rows_per_block (streaming kernel, 64 or 128);
    0 = automatic."""
    _fields_ = [("path", ctypes.c_int), ("tiles_per_wave", ctypes.c_int),
                ("waves_per_block", ctypes.c_int), ("k_splits", ctypes.c_int),
                ("rows_per_block", ctypes.c_int)]


class QmmSegment(ctypes.Structure):
    """dfmi_qmm_segment: one matrix of a shared-activation launch (sb_pairs:
    its pair table or NULL)."""
    _fields_ = [("w_q", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("biases", ctypes.c_void_p), ("y", ctypes.c_void_p), ("N", ctypes.c_int64),
                ("sb_pairs", ctypes.c_void_p)]


class QmmPlanInfo(ctypes.Structure):
    """dfmi_qmm_plan_info: the streaming launch a qmm call makes."""
    _fields_ = [(n, ctypes.c_int) for n in ("streaming", "waves", "k_splits", "whole_blocks",
                                             "blocks", "workgroups", "pair_streaming",
                                             "rows_per_block")]


# name -> (restype, argtypes)
_SIGNATURES = {
    "dfmi_version": (ctypes.c_char_p, []),
    "dfmi_last_error": (ctypes.c_char_p, []),
    "dfmi_qmm_affine": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                               _i64, _i64, _i64, _int, _int, _c_void_p, _size, _c_void_p]),
    "dfmi_qmm_affine_ex": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                  _i64, _i64, _i64, _int, _int, _c_void_p, _size,
                                  ctypes.POINTER(QmmTuning), _c_void_p]),
    "dfmi_qmm_workspace_bytes": (_size, [_i64, _i64, _i64, _int, _int]),
    "dfmi_qmm_general": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _c_void_p, _int, _c_void_p,
                                _i64, _i64, _i64, _int, _int, _int, _c_void_p, _size,
                                _c_void_p]),
    "dfmi_qmm_affine_pairs": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                     _c_void_p, _i64, _i64, _i64, _int, _int, _c_void_p, _size,
                                     ctypes.POINTER(QmmTuning), _c_void_p]),
    "dfmi_sb_pairs": (_int, [_c_void_p, _c_void_p, _int, _i64, _i64, _c_void_p, _c_void_p]),
    "dfmi_qmm_plan": (_int, [_i64, _i64, ctypes.POINTER(ctypes.c_int64), _int, _int, _int,
                             ctypes.POINTER(QmmTuning), ctypes.POINTER(QmmPlanInfo)]),
    "dfmi_qmm_kernel_name": (ctypes.c_char_p, [_i64, _i64, _i64, _int, _int,
                                               ctypes.POINTER(QmmTuning)]),
    "dfmi_qmm_workspace_bytes_ex": (_size, [_i64, _i64, _i64, _int, _int,
                                            ctypes.POINTER(QmmTuning)]),
    "dfmi_qmm_affine_noalloc": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _c_void_p,
                                       _c_void_p, _i64, _i64, _i64, _int, _int, _c_void_p]),
    "dfmi_qmm_noalloc_scratch_bytes": (_size, []),
    "dfmi_qmm_affine_multi": (_int, [_c_void_p, _int, ctypes.POINTER(QmmSegment), _int, _i64,
                                     _i64, _int, _int, _c_void_p, _size, _c_void_p]),
    "dfmi_qmm_affine_multi_fused": (_int, [_c_void_p, _int, ctypes.POINTER(QmmSegment), _int,
                                           _c_void_p, _i64, _i64, _int, _int, _c_void_p, _size,
                                           _c_void_p]),
    "dfmi_qmm_multi_workspace_bytes": (_size, [_i64, _i64, ctypes.POINTER(ctypes.c_int64), _int,
                                               _int, _int]),
    "dfmi_qmm_multi_kernel_name": (ctypes.c_char_p, [_i64, _i64, ctypes.POINTER(ctypes.c_int64),
                                                     _int, _int, _int]),
    "dfmi_qmm_prepare": (_int, [_int, ctypes.POINTER(QmmSegment), _int, _c_void_p, _i64, _i64,
                                _i64, _int, _int, _c_void_p, _size, _c_void_p, _size]),
    "dfmi_qmm_run": (_int, [_c_void_p] * 7),
    "dfmi_gather_qmm_affine": (_int, [_c_void_p, _int, _i64, _c_void_p, _c_void_p, _c_void_p,
                                      _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64,
                                      _int, _int, _c_void_p]),
    "dfmi_gather_qmm_swiglu": (_int, [_c_void_p, _int, _i64, _c_void_p, _c_void_p, _c_void_p,
                                      _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                      _c_void_p, _i64, _i64, _i64, _i64, _int, _int, _c_void_p]),
    "dfmi_gather_qmm_affine_pairs": (_int, [_c_void_p, _int, _i64, _c_void_p, _c_void_p,
                                            _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                            _c_void_p, _i64, _i64, _i64, _i64, _int, _int,
                                            _c_void_p, _size, _c_void_p]),
    "dfmi_gather_qmm_swiglu_pairs": (_int, [_c_void_p, _int, _i64, _c_void_p, _c_void_p,
                                            _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
                                            _i64, _i64, _i64, _int, _int, _c_void_p, _size,
                                            _c_void_p]),
    "dfmi_gather_workspace_bytes": (_size, []),
    "dfmi_moe_pairs": (_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _int, _i64, _i64,
                              _i64, _c_void_p, _c_void_p]),
    "dfmi_moe_combine": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _c_void_p, _i64, _i64,
                                _i64, _c_void_p]),
    "dfmi_greedy_accept": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _i64, _i64, _c_void_p,
                                  _c_void_p, _c_void_p, _c_void_p, _size, _c_void_p]),
    "dfmi_greedy_workspace_bytes": (_size, [_i64]),
    "dfmi_lmhead_greedy_accept": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _c_void_p,
                                         _c_void_p, _float, _c_void_p, _i64, _i64, _i64, _int,
                                         _int, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                         _c_void_p, _size, _c_void_p]),
    "dfmi_lmhead_workspace_bytes": (_size, [_i64]),
    "dfmi_lmhead_greedy_accept_pairs": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _c_void_p,
                                               _c_void_p, _c_void_p, _float, _c_void_p, _i64,
                                               _i64, _i64, _int, _int, _c_void_p, _c_void_p,
                                               _c_void_p, _c_void_p, _c_void_p, _size,
                                               _c_void_p]),
    "dfmi_match_acceptance_length": (_int, [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p]),
    "dfmi_gated_delta_tape": (_int, [_c_void_p] * 10 + [_i64] * 6 + [_int] * 5 + [_c_void_p]),
    "dfmi_tape_replay": (_int, [_c_void_p] * 6 + [_i64] * 6 + [_int] * 4 + [_c_void_p]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib = None


class DfmiError(RuntimeError):
    """A libdfmi call failed (status < 0)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"libdfmi status {status}: {message}")
        self.status = status


class DfmiUnsupported(DfmiError):
    """The kernels do not cover this shape / dtype (DFMI_EINVAL)."""


def load():
    """Load libdfmi.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} not found: build it with __graft_entry__.build() "
                    "(hipcc --offload-arch=gfx950); there is no fallback implementation")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name, None)
                if fn is None:
                    continue  # reported by missing_symbols(); calling it raises AttributeError
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def missing_symbols() -> list[str]:
    """Names of the C-ABI entry points that the loaded library does not export."""
    lib = load()
    return [name for name in _SIGNATURES if getattr(lib, name, None) is None]


def last_error() -> str:
    return load().dfmi_last_error().decode("utf-8", "replace")


def check(status: int, what: str) -> None:
    if status == DFMI_OK:
        return
    msg = last_error()
    if status == DFMI_EINVAL:
        raise DfmiUnsupported(status, f"{what}: {msg}")
    raise DfmiError(status, f"{what}: {msg}")
