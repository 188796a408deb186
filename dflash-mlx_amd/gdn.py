"""GDN rollback pair: gated-delta recurrence with innovation tape, and tape replay.

Gated-delta-net (GDN) targets keep a recurrent state per value head.  While
the rollback cache is armed, the verify forward runs the recurrence with
``gated_delta_kernel_with_tape`` (dflash_mlx/kernels.py:11-219, called from
dflash_mlx/engine/target_qwen_gdn.py:615-625), which also records the
per-step innovation ``(v - S.k) * beta`` as an fp32 tape.  After acceptance
the cache restores its snapshot and replays the first ``accepted + 1``
steps of the tape with ``tape_replay_kernel`` (dflash_mlx/kernels.py:691-866,
dflash_mlx/recurrent_rollback_cache.py:142-165) instead of re-running the
layer.  Both run as HIP kernels (``dfmi_gated_delta_tape``,
``dfmi_tape_replay``); there is no CPU path.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib, _runtime


def _mask_u8(mask: Optional[torch.Tensor], B: int, T: int) -> Optional[torch.Tensor]:
    if mask is None:
        return None
    _runtime.require_device(mask, "mask")
    if tuple(mask.shape) != (B, T):
        raise ValueError(f"mask must be [B, T] = [{B}, {T}], got {tuple(mask.shape)}")
    return mask.to(torch.uint8).contiguous()


def _gate(g: torch.Tensor, B: int, T: int, Hv: int, Dk: int) -> Tuple[torch.Tensor, int]:
    if g.dim() == 3 and tuple(g.shape) == (B, T, Hv):
        return g.contiguous(), 0
    if g.dim() == 4 and tuple(g.shape) == (B, T, Hv, Dk):
        return g.contiguous(), 1
    raise ValueError(f"Unsupported gating shape {tuple(g.shape)}")


def gated_delta_kernel_with_tape(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                 g: torch.Tensor, beta: torch.Tensor, state: torch.Tensor,
                                 mask: Optional[torch.Tensor] = None
                                 ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(y [B,T,Hv,Dv] in q's dtype, state_out [B,Hv,Dv,Dk] in state's dtype,
    innovation tape [B,T,Hv,Dv] fp32) for q, k [B,T,Hk,Dk], v [B,T,Hv,Dv],
    g [B,T,Hv] or [B,T,Hv,Dk], beta [B,T,Hv], state [B,Hv,Dv,Dk]."""
    for t, name in ((q, "q"), (k, "k"), (v, "v"), (g, "g"), (beta, "beta"), (state, "state")):
        _runtime.require_device(t, name)
    B, T, Hk, Dk = (int(d) for d in k.shape)
    Hv, Dv = int(v.shape[2]), int(v.shape[3])
    if Hv % Hk != 0:
        raise ValueError(f"Cannot align K heads {Hk} to V heads {Hv}")
    if tuple(q.shape) != (B, T, Hk, Dk) or tuple(v.shape[:2]) != (B, T):
        raise ValueError("q, k [B,T,Hk,Dk] and v [B,T,Hv,Dv] must agree")
    if tuple(beta.shape) != (B, T, Hv) or tuple(state.shape) != (B, Hv, Dv, Dk):
        raise ValueError("beta must be [B,T,Hv] and state [B,Hv,Dv,Dk]")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k and v must share a dtype")
    gc, per_key = _gate(g, B, T, Hv, Dk)
    m = _mask_u8(mask, B, T)
    qc, kc, vc, bc, sc = (t.contiguous() for t in (q, k, v, beta, state))
    dev = q.device
    y = torch.empty((B, T, Hv, Dv), dtype=q.dtype, device=dev)
    state_out = torch.empty_like(sc)
    tape = torch.empty((B, T, Hv, Dv), dtype=torch.float32, device=dev)
    lib = _lib.load()
    _lib.check(lib.dfmi_gated_delta_tape(
        qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), gc.data_ptr(), bc.data_ptr(), sc.data_ptr(),
        m.data_ptr() if m is not None else None, y.data_ptr(), state_out.data_ptr(),
        tape.data_ptr(), B, T, Hk, Hv, Dk, Dv, _runtime.dtype_code(q.dtype),
        _runtime.dtype_code(gc.dtype), _runtime.dtype_code(bc.dtype),
        _runtime.dtype_code(sc.dtype), per_key, _runtime.stream_ptr(dev)),
        "dfmi_gated_delta_tape")
    return y, state_out, tape


def tape_replay_kernel(tape: torch.Tensor, k: torch.Tensor, g: torch.Tensor,
                       state: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """State [B,Hv,Dv,Dk] (state's dtype) after replaying tape [B,T,Hv,Dv]
    (fp32) with keys k [B,T,Hk,Dk] and gates g from ``state``."""
    for t, name in ((tape, "tape"), (k, "k"), (g, "g"), (state, "state")):
        _runtime.require_device(t, name)
    B, T, Hk, Dk = (int(d) for d in k.shape)
    Hv, Dv = int(tape.shape[2]), int(tape.shape[3])
    if Hv % Hk != 0:
        raise ValueError(f"Cannot align K heads {Hk} to tape heads {Hv}")
    if tuple(tape.shape[:2]) != (B, T) or tuple(state.shape) != (B, Hv, Dv, Dk):
        raise ValueError("tape [B,T,Hv,Dv], k [B,T,Hk,Dk] and state [B,Hv,Dv,Dk] must agree")
    gc, per_key = _gate(g, B, T, Hv, Dk)
    m = _mask_u8(mask, B, T)
    tc = tape.to(torch.float32).contiguous()
    kc, sc = k.contiguous(), state.contiguous()
    out = torch.empty_like(sc)
    lib = _lib.load()
    _lib.check(lib.dfmi_tape_replay(
        tc.data_ptr(), kc.data_ptr(), gc.data_ptr(), sc.data_ptr(),
        m.data_ptr() if m is not None else None, out.data_ptr(), B, T, Hk, Hv, Dk, Dv,
        _runtime.dtype_code(kc.dtype), _runtime.dtype_code(gc.dtype),
        _runtime.dtype_code(sc.dtype), per_key, _runtime.stream_ptr(tape.device)),
        "dfmi_tape_replay")
    return out


__all__ = ["gated_delta_kernel_with_tape", "tape_replay_kernel"]
