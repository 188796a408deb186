"""Greedy token selection (mirrors dflash_mlx/engine/sampling.py:29-55).

``greedy_tokens_with_mask`` runs the HIP argmax kernel (``dfmi_greedy_accept``):
argmax over the last axis of ``where(mask, dtype(-1e9), logits)``, lowest index
on ties, NaN never selected unless the row is all NaN.  Token ids come back as
int32 tensors holding the reference's uint32 values (ids < 2**31).
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import torch

from . import _lib, _runtime

_MAX_ROWS = 32


def build_suppress_token_mask(vocab_size: int, suppress_token_ids: Optional[Sequence[int]],
                              device: Optional[torch.device] = None) -> Optional[torch.Tensor]:
    """dflash_mlx/engine/sampling.py:29-45: bool ``[vocab_size]`` mask of the
    in-range ids, or None when there are none."""
    token_ids = sorted({int(t) for t in (suppress_token_ids or []) if 0 <= int(t) < vocab_size})
    if not token_ids:
        return None
    mask = torch.zeros((vocab_size,), dtype=torch.bool, device=device)
    mask[torch.tensor(token_ids, dtype=torch.long, device=device)] = True
    return mask


def _mask_ptr(mask: Optional[torch.Tensor], V: int, device) -> tuple[int, Optional[torch.Tensor]]:
    if mask is None:
        return 0, None
    if mask.dtype not in (torch.bool, torch.uint8) or mask.numel() != V:
        raise ValueError(f"suppress mask must be bool/uint8 of {V} entries")
    _runtime.require_device(mask, "suppress_token_mask")
    mask = mask.contiguous()
    return mask.data_ptr(), mask


def greedy_rows(logits2: torch.Tensor, mask_ptr: int, ids: Optional[torch.Tensor],
                posterior: torch.Tensor, accept: Optional[torch.Tensor],
                bonus: Optional[torch.Tensor]) -> None:
    """One ``dfmi_greedy_accept`` launch over ``[M <= 32, V]`` logits."""
    lib = _lib.load()
    M, V = int(logits2.shape[0]), int(logits2.shape[1])
    dev = logits2.device
    ws, ws_bytes = _runtime.workspace(dev, int(lib.dfmi_greedy_workspace_bytes(M)), "greedy")
    status = lib.dfmi_greedy_accept(
        logits2.data_ptr(), _runtime.dtype_code(logits2.dtype), mask_ptr,
        ids.data_ptr() if ids is not None else 0, M, V, posterior.data_ptr(),
        accept.data_ptr() if accept is not None else 0,
        bonus.data_ptr() if bonus is not None else 0, ws, ws_bytes, _runtime.stream_ptr(dev))
    _lib.check(status, "dfmi_greedy_accept")


def greedy_tokens_with_mask(logits: torch.Tensor,
                            suppress_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """dflash_mlx/engine/sampling.py:48-55 on the GPU."""
    _runtime.require_device(logits, "logits")
    V = int(logits.shape[-1])
    M = math.prod(int(d) for d in logits.shape[:-1])
    mask_ptr, _keep = _mask_ptr(suppress_token_mask, V, logits.device)
    flat = logits.reshape(M, V).contiguous()
    out = torch.empty((M,), dtype=torch.int32, device=logits.device)
    for r0 in range(0, M, _MAX_ROWS):
        r1 = min(M, r0 + _MAX_ROWS)
        greedy_rows(flat[r0:r1], mask_ptr, None, out[r0:r1], None, None)
    return out.reshape(logits.shape[:-1])
