"""lm_head + greedy + accept for one verify cycle.

The reference computes ``verify_logits = lm_head(hidden)`` with a stock
quantized matmul (dflash_mlx/engine/target_qwen_gdn.py:774-778; Gemma adds a
tanh softcap, engine/target_gemma4.py:33-40, 336-355), then
``posterior = greedy_tokens_with_mask(logits[0], mask)`` and
``accept = match_acceptance_length(verify_ids[1:], posterior[:-1])``,
``bonus = posterior[accept]`` (engine/spec_epoch.py:2067-2072, 2129).

``lm_head_greedy_accept`` does all of it in one HIP kernel
(``dfmi_lmhead_greedy_accept``): the vocabulary sweep of the int4 lm_head
reduces every logit into a per-row argmax key in its epilogue, so the
``[M, V]`` logits are written only when ``return_logits=True``.
``greedy_accept`` is the same greedy/accept stage over logits already in
memory (``dfmi_greedy_accept``).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib, _runtime
from .sampling import _mask_ptr, greedy_rows

_MAX_ROWS = 32


@dataclass
class GreedyAcceptResult:
    posterior: torch.Tensor              # int32 [M] greedy token per verify row
    accept_len: Optional[torch.Tensor]   # int32 [1] (None without verify_ids)
    bonus: Optional[torch.Tensor]        # int32 [1] posterior[accept_len]
    logits: Optional[torch.Tensor] = None  # [M, V] when requested


def _ids(verify_ids: Optional[torch.Tensor], M: int) -> Optional[torch.Tensor]:
    if verify_ids is None:
        return None
    _runtime.require_device(verify_ids, "verify_ids")
    ids = verify_ids.reshape(-1)
    if int(ids.shape[0]) != M:
        raise ValueError(f"verify_ids must hold {M} tokens (one per verify row)")
    return ids.to(torch.int32).contiguous() if ids.dtype not in (torch.int32, torch.uint32) \
        else ids.contiguous()


def lm_head_greedy_accept(h: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                          biases: torch.Tensor, *, verify_ids: Optional[torch.Tensor] = None,
                          suppress_token_mask: Optional[torch.Tensor] = None,
                          softcap: Optional[float] = None, group_size: int = 64, bits: int = 4,
                          return_logits: bool = False,
                          pairs: Optional[torch.Tensor] = None) -> GreedyAcceptResult:
    """Fused int4 lm_head + greedy argmax + accept/bonus for ``h [..., K]``
    with at most 32 verify rows.  ``pairs``: the lm_head's pair table
    (``_runtime.build_sb_pairs``); when None, the one cached for ``scales``
    is used where the pair-streaming loop applies.  Outputs do not depend
    on it."""
    for t, name in ((h, "h"), (w, "w"), (scales, "scales"), (biases, "biases")):
        _runtime.require_device(t, name)
    lib = _lib.load()
    K = int(h.shape[-1])
    M = math.prod(int(d) for d in h.shape[:-1])
    if M < 1 or M > _MAX_ROWS:
        raise _lib.DfmiUnsupported(_lib.DFMI_EINVAL, f"{M} verify rows (1..{_MAX_ROWS})")
    V = int(w.shape[0])
    dev = h.device
    h2 = _runtime.aligned_contiguous(h.reshape(M, K))
    wq = _runtime.weight_words(w)
    s = _runtime.aligned_contiguous(scales)
    b = _runtime.aligned_contiguous(biases)
    ids = _ids(verify_ids, M)
    mask_ptr, _keep = _mask_ptr(suppress_token_mask, V, dev)
    posterior = torch.empty((M,), dtype=torch.int32, device=dev)
    accept = torch.empty((1,), dtype=torch.int32, device=dev) if ids is not None else None
    bonus = torch.empty((1,), dtype=torch.int32, device=dev) if ids is not None else None
    logits = torch.empty((M, V), dtype=h.dtype, device=dev) if return_logits else None
    ws, ws_bytes = _runtime.workspace(dev, int(lib.dfmi_lmhead_workspace_bytes(M)), "greedy")
    if pairs is None and _runtime.pair_shape(M, K, V, group_size, bits):
        pairs = _runtime.PAIRS.get(s, b)
    status = lib.dfmi_lmhead_greedy_accept_pairs(
        h2.data_ptr(), _runtime.dtype_code(h2.dtype), wq.data_ptr(), s.data_ptr(), b.data_ptr(),
        pairs.data_ptr() if pairs is not None else 0, mask_ptr, float(softcap) if softcap else 0.0, ids.data_ptr() if ids is not None else 0,
        M, K, V, int(group_size), int(bits), posterior.data_ptr(),
        accept.data_ptr() if accept is not None else 0,
        bonus.data_ptr() if bonus is not None else 0,
        logits.data_ptr() if logits is not None else 0, ws, ws_bytes, _runtime.stream_ptr(dev))
    _lib.check(status, "dfmi_lmhead_greedy_accept")
    return GreedyAcceptResult(posterior, accept, bonus, logits)


def draft_tokens_from_hidden(draft_hidden: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                             biases: torch.Tensor, *,
                             suppress_token_mask: Optional[torch.Tensor] = None,
                             softcap: Optional[float] = None, group_size: int = 64,
                             bits: int = 4) -> torch.Tensor:
    """Draft block tokens from the draft model's hidden states.

    dflash_mlx/draft_backend.py:142-149: the target's lm_head over
    ``draft_hidden[:, 1:, :]`` (block_len - 1 rows, e.g. 15) followed by
    ``greedy_tokens_with_mask(...).squeeze(0)``.  One fused kernel: the
    lm_head epilogue reduces to the per-row argmax, no logits are written
    and no accept step runs.  ``draft_hidden`` is ``[1, block_len, K]``
    (or ``[block_len, K]``); returns int32 ``[block_len - 1]``."""
    h = draft_hidden[0] if draft_hidden.dim() == 3 else draft_hidden
    if h.dim() != 2 or int(h.shape[0]) < 2:
        raise ValueError("draft_hidden must be [1, block_len, K] with block_len > 1")
    res = lm_head_greedy_accept(h[1:], w, scales, biases, suppress_token_mask=suppress_token_mask,
                                softcap=softcap, group_size=group_size, bits=bits)
    return res.posterior


def greedy_accept(logits: torch.Tensor, *, verify_ids: Optional[torch.Tensor] = None,
                  suppress_token_mask: Optional[torch.Tensor] = None) -> GreedyAcceptResult:
    """Greedy + accept/bonus over ``logits [..., V]`` (at most 32 rows)."""
    _runtime.require_device(logits, "logits")
    V = int(logits.shape[-1])
    M = math.prod(int(d) for d in logits.shape[:-1])
    if M < 1 or M > _MAX_ROWS:
        raise _lib.DfmiUnsupported(_lib.DFMI_EINVAL, f"{M} verify rows (1..{_MAX_ROWS})")
    dev = logits.device
    ids = _ids(verify_ids, M)
    mask_ptr, _keep = _mask_ptr(suppress_token_mask, V, dev)
    posterior = torch.empty((M,), dtype=torch.int32, device=dev)
    accept = torch.empty((1,), dtype=torch.int32, device=dev) if ids is not None else None
    bonus = torch.empty((1,), dtype=torch.int32, device=dev) if ids is not None else None
    greedy_rows(logits.reshape(M, V).contiguous(), mask_ptr, ids, posterior, accept, bonus)
    return GreedyAcceptResult(posterior, accept, bonus, None)
