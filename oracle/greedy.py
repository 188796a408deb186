"""Greedy sampling / acceptance oracle (test infrastructure only).

Restates dflash_mlx/engine/sampling.py:29-55, engine/acceptance.py:9-16,
engine/spec_epoch.py:2011-2021, 2067-2072, 2129 and the Gemma softcap of
engine/target_gemma4.py:33-40.
"""

from __future__ import annotations

import numpy as np

from .numerics import round_to_dtype, to_f32


def build_suppress_token_mask(vocab_size: int, suppress_token_ids):
    """Boolean ``[vocab_size]`` mask, or None when no id is in range.

    dflash_mlx/engine/sampling.py:29-45: ids outside ``[0, vocab_size)`` are
    dropped; an empty set yields None.
    """
    ids = sorted({int(t) for t in (suppress_token_ids or []) if 0 <= int(t) < vocab_size})
    if not ids:
        return None
    mask = np.zeros((vocab_size,), dtype=bool)
    mask[np.asarray(ids, dtype=np.int64)] = True
    return mask


def _argmax_first(values: np.ndarray) -> np.ndarray:
    """Row-wise index of the maximum; lowest index wins ties; NaN never wins
    unless the whole row is NaN (then index 0)."""
    v = np.asarray(values, dtype=np.float64)
    v = np.where(np.isnan(v), -np.inf, v)
    out = np.argmax(v, axis=-1)  # numpy returns the first maximal index
    return out.astype(np.int64)


def greedy_tokens_with_mask(logits, suppress_token_mask=None, *, dtype: str = "bf16"):
    """dflash_mlx/engine/sampling.py:48-55.

    ``argmax(where(mask, dtype(-1e9), logits), -1)`` on the values of the
    logits dtype.  Returns int64 token ids (the reference casts to uint32).
    """
    vals = to_f32(logits, dtype).astype(np.float64)
    if suppress_token_mask is not None:
        floor = float(to_f32(round_to_dtype(np.float32(-1e9), dtype), dtype).reshape(-1)[0])
        vals = np.where(np.asarray(suppress_token_mask, dtype=bool), floor, vals)
    return _argmax_first(vals)


def match_acceptance_length(drafted_tokens, posterior_tokens) -> int:
    """dflash_mlx/engine/acceptance.py:9-16: length of the equal prefix."""
    d = np.asarray(drafted_tokens, dtype=np.int64).reshape(-1)
    p = np.asarray(posterior_tokens, dtype=np.int64).reshape(-1)
    if d.shape[0] == 0:
        return 0
    if d.shape != p.shape:
        raise ValueError("drafted and posterior lengths differ")
    matches = (d == p).astype(np.int64)
    return int(np.cumprod(matches).sum())


def verify_cycle_accept(verify_ids, posterior):
    """One verify cycle's accept / bonus (dflash_mlx/engine/spec_epoch.py).

    ``verify_ids = [staged_first, d_1 .. d_{L-1}]`` (2011-2021);
    ``accept = match_acceptance_length(verify_ids[1:], posterior[:-1])``
    (2070-2072); ``bonus = posterior[accept]`` (2129).
    """
    ids = np.asarray(verify_ids, dtype=np.int64).reshape(-1)
    post = np.asarray(posterior, dtype=np.int64).reshape(-1)
    accept = match_acceptance_length(ids[1:], post[:-1])
    return accept, int(post[accept])


def logit_softcap(logits, softcap, *, dtype: str = "bf16"):
    """Gemma final-logit softcap ``tanh(l / cap) * cap`` (target_gemma4.py:33-40).

    Each MLX op rounds to the logits dtype: ``t1 = rnd(l / cap)``,
    ``t2 = rnd(tanh(t1))``, ``out = rnd(t2 * cap)``; the Python scalar cap is
    first cast to the logits dtype.  ``softcap`` None or <= 0 is the identity.
    """
    if softcap is None or float(softcap) <= 0.0:
        return logits
    cap = float(to_f32(round_to_dtype(np.float32(softcap), dtype), dtype).reshape(-1)[0])
    l = to_f32(logits, dtype)
    t1 = to_f32(round_to_dtype(l / np.float32(cap), dtype), dtype)
    t2 = to_f32(round_to_dtype(np.tanh(t1), dtype), dtype)
    return round_to_dtype(t2 * np.float32(cap), dtype)
