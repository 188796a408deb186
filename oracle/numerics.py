"""Floating-point helpers for the oracle (test infrastructure only).

bf16 values are carried as ``uint16`` bit patterns.  Conversion float32 -> bf16
is round-to-nearest-even on the upper 16 bits (the IEEE rounding MLX, PyTorch
and the gfx950 ``v_cvt_pk_bf16_f32`` instruction all use); NaN stays NaN.
"""

from __future__ import annotations

import numpy as np

DTYPES = ("bf16", "f16", "f32")


def f32_to_bf16_bits(a) -> np.ndarray:
    """float32 -> bf16 bit pattern (uint16), round to nearest even."""
    f = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    nan = np.isnan(f)
    if nan.any():
        rounded = np.where(nan, ((u >> 16) | 0x40).astype(np.uint32), rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    """bf16 bit pattern (uint16) -> float32 (exact)."""
    u = np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16
    return u.view(np.float32)


def to_f32(a, dtype: str) -> np.ndarray:
    """Decode an oracle tensor stored in ``dtype`` into float32 values."""
    if dtype == "bf16":
        return bf16_bits_to_f32(a)
    if dtype == "f16":
        return np.asarray(a, dtype=np.float16).astype(np.float32)
    if dtype == "f32":
        return np.asarray(a, dtype=np.float32)
    raise ValueError(f"unknown dtype {dtype!r}")


def round_to_dtype(a, dtype: str) -> np.ndarray:
    """Round float values (any float dtype) to ``dtype``'s storage form.

    float64 inputs are first rounded to float32 (as a float32 accumulator
    would hold them) and then to the target dtype; the double rounding can
    differ from a direct float64 -> bf16 rounding only on exact float32 ties,
    which the parity tolerance absorbs.
    """
    f = np.asarray(a, dtype=np.float32)
    if dtype == "bf16":
        return f32_to_bf16_bits(f)
    if dtype == "f16":
        return f.astype(np.float16)
    if dtype == "f32":
        return f
    raise ValueError(f"unknown dtype {dtype!r}")


def from_f32(a, dtype: str) -> np.ndarray:
    """Alias of :func:`round_to_dtype` for readability at call sites."""
    return round_to_dtype(a, dtype)
