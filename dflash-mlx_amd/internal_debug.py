# The flag names, defaults and parsing in this file follow
# dflash_mlx/internal_debug.py of dflash-mlx 0.1.7:
#   Copyright 2026 bstnxbt
#   Licensed under the Apache License, Version 2.0
#   Based on DFlash (arXiv:2602.06036)
# They are kept identical because users set these environment variables.

"""Kernel-debug flag surface (same names, defaults and parsing as
dflash_mlx/internal_debug.py:10-37).  Read at call time, never cached."""

from __future__ import annotations

import os
from typing import Optional


def _env_int(name: str, default: int) -> int:
    try:
        return int(os.environ.get(name, str(default)))
    except ValueError:
        return int(default)


def verify_linear_override() -> Optional[bool]:
    """DFLASH_VERIFY_LINEAR: "1" -> True, "0" -> False, else None."""
    raw = os.environ.get("DFLASH_VERIFY_LINEAR", "").strip()
    if raw == "1":
        return True
    if raw == "0":
        return False
    return None


def verify_qmm_enabled() -> bool:
    """DFLASH_VERIFY_QMM == "1" enables the verify kernels in direct calls."""
    return os.environ.get("DFLASH_VERIFY_QMM", "") == "1"


def verify_qmm_variant() -> str:
    return os.environ.get("DFLASH_VERIFY_VARIANT", "auto")


def verify_qmm_kparts(default: int) -> int:
    return _env_int("DFLASH_VERIFY_QMM_KPARTS", default)


def verify_max_n(default: int) -> int:
    return _env_int("DFLASH_VERIFY_MAX_N", default)


def verify_include() -> str:
    return os.environ.get("DFLASH_VERIFY_INCLUDE", "all").strip().lower()
