"""Accept-prefix length (mirrors dflash_mlx/engine/acceptance.py:9-16).

``match_acceptance_length(drafted, posterior)`` = length of the longest
prefix on which the two token arrays agree (0 for empty input), computed on
the GPU by ``dfmi_match_acceptance_length``; returns a 0-d int32 tensor.
"""

from __future__ import annotations

import torch

from . import _lib, _runtime


def _as_u32_words(t: torch.Tensor) -> torch.Tensor:
    if t.dtype in (torch.int32, torch.uint32):
        return t.contiguous()
    return t.to(torch.int32).contiguous()


def match_acceptance_length(drafted_tokens: torch.Tensor,
                            posterior_tokens: torch.Tensor) -> torch.Tensor:
    _runtime.require_device(drafted_tokens, "drafted_tokens")
    dev = drafted_tokens.device
    out = torch.empty((), dtype=torch.int32, device=dev)
    L = int(drafted_tokens.shape[0])
    if L and int(posterior_tokens.shape[0]) != L:
        raise ValueError("drafted and posterior lengths differ")
    d = _as_u32_words(drafted_tokens.reshape(-1))
    p = _as_u32_words(posterior_tokens.reshape(-1)) if L else d
    status = _lib.load().dfmi_match_acceptance_length(
        d.data_ptr(), p.data_ptr(), L, out.data_ptr(), _runtime.stream_ptr(dev))
    _lib.check(status, "dfmi_match_acceptance_length")
    return out
