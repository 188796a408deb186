"""Affine group-quantized matmul oracle (test infrastructure only).

Layout (restated from the reference kernels' unpack,
dflash_mlx/verify_qmm.py:97-115, 243-249, 8-bit 593-598): ``w_q`` is uint32
``[N, K*bits/32]``; word ``j`` of row ``n`` holds ``32/bits`` consecutive k
values, the first in the lowest bits.  ``scales`` / ``biases`` are
``[N, K/group_size]`` in the activation dtype.  Dequantised weight:
``w[n, k] = q[n, k] * scales[n, k // gs] + biases[n, k // gs]``.
"""

from __future__ import annotations

import numpy as np

from .numerics import round_to_dtype, to_f32

SUPPORTED_BITS = (2, 4, 8)


def pack(q: np.ndarray, bits: int) -> np.ndarray:
    """Pack integer codes ``q[N, K]`` (0 <= q < 2**bits) into uint32 words."""
    if bits not in SUPPORTED_BITS:
        raise ValueError(f"bits must be one of {SUPPORTED_BITS}")
    q = np.asarray(q)
    n, k = q.shape
    per = 32 // bits
    if k % per:
        raise ValueError(f"K={k} not a multiple of {per}")
    if q.size and (q.min() < 0 or q.max() >= (1 << bits)):
        raise ValueError("code out of range")
    q = q.astype(np.uint32).reshape(n, k // per, per)
    out = np.zeros((n, k // per), dtype=np.uint32)
    for i in range(per):
        out |= q[:, :, i] << np.uint32(bits * i)
    return out


def unpack(w_q: np.ndarray, bits: int) -> np.ndarray:
    """Inverse of :func:`pack`: uint32 words -> int codes ``[N, K]``."""
    if bits not in SUPPORTED_BITS:
        raise ValueError(f"bits must be one of {SUPPORTED_BITS}")
    w = np.asarray(w_q, dtype=np.uint32)
    per = 32 // bits
    shifts = (np.arange(per, dtype=np.uint32) * bits)[None, None, :]
    mask = np.uint32((1 << bits) - 1)
    q = (w[..., None] >> shifts) & mask
    return q.reshape(*w.shape[:-1], w.shape[-1] * per).astype(np.int64)


def quantize(w, group_size: int = 64, bits: int = 4, out_dtype: str = "bf16"):
    """Affine quantisation with MLX's rule (restated, parity unpinned vs MLX).

    Per group of ``group_size`` consecutive k: ``w_min``, ``w_max``;
    ``scale = max((w_max - w_min) / (2**bits - 1), 1e-7)``, negated unless
    ``|w_min| > |w_max|``; ``edge`` is ``w_min`` in the first case else
    ``w_max``; ``q0 = round(edge / scale)``; when ``q0 != 0`` the scale is
    snapped to ``edge / q0`` and the bias is ``edge`` (else the bias is 0).
    Codes are ``clip(round((w - bias) / scale), 0, 2**bits - 1)``.

    Arithmetic is float32.  The codes are computed against the float32
    scale and bias; scales and biases are then cast to ``out_dtype`` (MLX's
    ``affine_quantize`` order: the packing step divides by the unrounded
    scale, and the returned scales / biases are cast afterwards).

    Returns ``(w_q uint32 [N, K*bits/32], scales, biases)`` with scales and
    biases in ``out_dtype`` storage form (uint16 bits for bf16).
    """
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % group_size:
        raise ValueError(f"K={k} not a multiple of group_size={group_size}")
    n_bins = np.float32((1 << bits) - 1)
    g = w.reshape(n, k // group_size, group_size)
    w_max = g.max(axis=-1)
    w_min = g.min(axis=-1)
    mask = np.abs(w_min) > np.abs(w_max)
    scale = np.maximum((w_max - w_min) / n_bins, np.float32(1e-7)).astype(np.float32)
    scale = np.where(mask, scale, -scale).astype(np.float32)
    edge = np.where(mask, w_min, w_max).astype(np.float32)
    q0 = np.round(edge / scale).astype(np.float32)
    nz = q0 != 0
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.where(nz, edge / np.where(nz, q0, 1), scale).astype(np.float32)
    bias = np.where(nz, edge, np.float32(0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        qf = np.round((g - bias[..., None]) / scale[..., None])
    qf[np.isnan(qf)] = 0.0
    q = np.clip(qf, 0, n_bins).astype(np.uint8).reshape(n, k)
    return pack(q, bits), round_to_dtype(scale, out_dtype), round_to_dtype(bias, out_dtype)


def dequantize(w_q, scales, biases, group_size: int, bits: int, dtype: str) -> np.ndarray:
    """Exact float64 dequantisation ``q * s + b`` -> ``[..., N, K]``."""
    q = unpack(w_q, bits).astype(np.float64)
    s = to_f32(scales, dtype).astype(np.float64)
    b = to_f32(biases, dtype).astype(np.float64)
    s = np.repeat(s, group_size, axis=-1)
    b = np.repeat(b, group_size, axis=-1)
    if s.shape != q.shape:
        raise ValueError(f"scales {s.shape} do not cover codes {q.shape}")
    return q * s + b


def quantized_matmul(x, w_q, scales, biases, *, transpose: bool = True,
                     group_size: int = 64, bits: int = 4, dtype: str = "bf16",
                     out_dtype: str | None = None):
    """``y = x . dequant(W)^T`` with float64 accumulation.

    ``x`` is ``[..., K]`` in ``dtype`` storage.  Returns float64 ``[..., N]``
    when ``out_dtype`` is None, else the result rounded to ``out_dtype``.

    ``transpose=False`` is ``y = x . dequant(W)`` with ``w_q [K, N*bits/32]``
    quantised along its last axis and ``scales / biases [K, N/gs]``: the
    other orientation of ``mx.quantized_matmul`` (called by the reference's
    fallbacks with the caller's ``transpose``, dflash_mlx/verify_qmm.py:
    915-919; MLX's documented contract, third-party, not vendored).
    """
    if not transpose:
        xf = to_f32(x, dtype).astype(np.float64)
        w = dequantize(w_q, scales, biases, group_size, bits, dtype)  # [K, N]
        y = xf @ w
        return y if out_dtype is None else round_to_dtype(y, out_dtype)
    xf = to_f32(x, dtype).astype(np.float64)
    n = w_q.shape[0]
    step = 2048  # dequantise in row blocks to bound memory on large weights
    y = np.empty(xf.shape[:-1] + (n,), dtype=np.float64)
    for n0 in range(0, n, step):
        n1 = min(n, n0 + step)
        w = dequantize(w_q[n0:n1], scales[n0:n1], biases[n0:n1], group_size, bits, dtype)
        y[..., n0:n1] = xf @ w.T
    return y if out_dtype is None else round_to_dtype(y, out_dtype)


def gather_qmm(x, w_q, scales, biases, lhs_indices, rhs_indices, *,
               group_size: int = 64, bits: int = 4, dtype: str = "bf16",
               out_dtype: str | None = None):
    """mx.gather_qmm(transpose=True) on explicit index pairs.

    ``x`` is ``[B, M, K]`` (batch of row blocks), ``w_q`` ``[E, N, K*bits/32]``.
    Pair ``p`` computes ``x[lhs[p]] . dequant(W[rhs[p]])^T`` -> ``y[p]`` of
    shape ``[M, N]``; output ``[P, M, N]``.
    """
    lhs = np.asarray(lhs_indices, dtype=np.int64).reshape(-1)
    rhs = np.asarray(rhs_indices, dtype=np.int64).reshape(-1)
    if lhs.shape != rhs.shape:
        raise ValueError("lhs/rhs index counts differ")
    xf = to_f32(x, dtype).astype(np.float64)
    out = []
    cache = {}
    for p in range(lhs.shape[0]):
        e = int(rhs[p])
        if e not in cache:
            cache[e] = dequantize(w_q[e], scales[e], biases[e], group_size, bits, dtype)
        out.append(xf[int(lhs[p])] @ cache[e].T)
    y = np.stack(out, axis=0) if out else np.zeros((0,) + x.shape[1:-1] + (w_q.shape[1],))
    return y if out_dtype is None else round_to_dtype(y, out_dtype)


def parity_metrics(y, y_ref):
    """Reference parity metric (tests/test_verify_qmm_parity.py:69-70).

    Returns ``(max_abs, max_rel)`` with
    ``max_rel = max|y - y_ref| / (max|y_ref| + 1e-3)``.
    """
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    if y.size == 0:
        return 0.0, 0.0
    max_abs = float(np.max(np.abs(y - y_ref)))
    return max_abs, float(max_abs / (np.max(np.abs(y_ref)) + 1e-3))
