"""Affine group quantisation of weights (load-time weight preparation, not
on the verify path).

Implements MLX's affine rule (the ``mx.quantize`` that ``nn.QuantizedLinear``
uses and the reference tests call, tests/test_verify_qmm_parity.py:29-30) in
torch: per group ``scale = max((max - min) / (2**bits - 1), 1e-7)``, negated
unless ``|min| > |max|``, ``edge`` = min or max accordingly, the scale is
snapped to ``edge / round(edge / scale)`` and the bias is ``edge`` (0 when
that rounds to 0); codes ``clip(round((w - bias) / scale), 0, 2**bits - 1)``
against the float32 scale and bias, which are then cast to the output dtype
(MLX's order).  Packing: word j of row n holds ``32/bits`` consecutive k,
first k in the lowest bits.
"""

from __future__ import annotations

import torch


def quantize(w: torch.Tensor, group_size: int = 64, bits: int = 4,
             dtype: torch.dtype | None = None):
    """``w [N, K]`` -> ``(w_q int32 [N, K*bits/32], scales, biases)``.

    Scales / biases are stored in ``dtype`` (default: ``w``'s dtype when it is
    a 16-bit float, else bfloat16).
    """
    if bits not in (2, 4, 8):
        raise ValueError("bits must be 2, 4 or 8")
    if w.dim() != 2 or w.shape[1] % group_size:
        raise ValueError(f"weight {tuple(w.shape)} not divisible by group_size={group_size}")
    if dtype is None:
        dtype = w.dtype if w.dtype in (torch.bfloat16, torch.float16) else torch.bfloat16
    n, k = w.shape
    wf = w.to(torch.float32).reshape(n, k // group_size, group_size)
    n_bins = float((1 << bits) - 1)
    w_max = wf.amax(dim=-1)
    w_min = wf.amin(dim=-1)
    mask = w_min.abs() > w_max.abs()
    scale = torch.clamp((w_max - w_min) / n_bins, min=1e-7)
    scale = torch.where(mask, scale, -scale)
    edge = torch.where(mask, w_min, w_max)
    q0 = torch.round(edge / scale)
    nz = q0 != 0
    scale = torch.where(nz, edge / torch.where(nz, q0, torch.ones_like(q0)), scale)
    bias = torch.where(nz, edge, torch.zeros_like(edge))
    q = torch.round((wf - bias.unsqueeze(-1)) / scale.unsqueeze(-1))
    scales = scale.to(dtype)
    biases = bias.to(dtype)
    q = torch.nan_to_num(q, nan=0.0, posinf=n_bins, neginf=0.0).clamp_(0, n_bins)
    q = q.to(torch.int64).reshape(n, k)
    per = 32 // bits
    shifts = torch.arange(per, device=w.device, dtype=torch.int64) * bits
    words = (q.reshape(n, k // per, per) << shifts).sum(dim=-1)
    w_q = (words & 0xFFFFFFFF).to(torch.int64)
    w_q = torch.where(w_q >= 2**31, w_q - 2**32, w_q).to(torch.int32)
    return w_q, scales, biases


def dequantize(w_q: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """float32 ``q * s + b`` (load-time inspection helper, never on the verify path)."""
    per = 32 // bits
    words = w_q.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(per, device=w_q.device, dtype=torch.int64) * bits
    q = ((words.unsqueeze(-1) >> shifts) & ((1 << bits) - 1)).reshape(*w_q.shape[:-1], -1)
    s = scales.to(torch.float32).repeat_interleave(group_size, dim=-1)
    b = biases.to(torch.float32).repeat_interleave(group_size, dim=-1)
    return q.to(torch.float32) * s + b
