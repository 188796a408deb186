"""Gated-delta recurrence with innovation tape, and tape replay (TEST INFRASTRUCTURE ONLY).

Restates, in float64 numpy, the two GDN rollback kernels of the reference:

* ``gated_delta_with_tape`` -- dflash_mlx/kernels.py:11-118 (the GPU kernel
  ``gated_delta_tape``) and its ops form ``_gated_delta_ops_with_tape``
  (kernels.py:125-166).  Per batch b, value head hv (key head
  hk = hv // (Hv / Hk)), step t with mask[b, t] true:
      S    = S * g_t                      (g: [B,T,Hv] scalar or [B,T,Hv,Dk])
      kv   = S . k_t                      (per state row dv)
      d    = (v_t[dv] - kv) * beta_t
      S    = S + d * k_t
      y_t  = S . q_t
      tape_t[dv] = d
  A masked step leaves S unchanged, records tape 0 and y 0 (the ops form's
  value; the GPU kernel leaves that y unwritten).  S is carried in fp32 by
  the GPU kernel (here float64); y is rounded to the input dtype, tape is
  fp32, the final state is rounded to the state dtype.
* ``tape_replay`` -- dflash_mlx/kernels.py:691-866 (``tape_replay`` kernel and
  ``_tape_replay_ops``), called by dflash_mlx/recurrent_rollback_cache.py:142-165
  over the accepted steps: per unmasked step
      S = S * g_t + tape_t * k_t
  with S rounded to the state dtype after every step (the GPU kernel's
  ``static_cast<InT>`` per step).

Pinned in tests/test_oracle.py by: a brute-force per-element loop on tiny
shapes, closed forms (beta = 0: the state only decays and the tape is zero;
a single step from a zero state: S = beta v k^T, y = beta v (k . q)), masked
steps leaving the state untouched, and the rollback invariant that replaying
the full fp32 tape over the same steps reproduces the recurrence's final
state exactly.
"""

from __future__ import annotations

import numpy as np

from .numerics import round_to_dtype, to_f32


def _f64(a, dtype):
    return to_f32(a, dtype).astype(np.float64)


def gated_delta_with_tape(q, k, v, g, beta, state, mask=None, *, in_dtype="bf16",
                          state_dtype="f32", g_dtype=None, beta_dtype=None):
    """Returns (y [B,T,Hv,Dv] in in_dtype, state_out [B,Hv,Dv,Dk] in state_dtype,
    tape [B,T,Hv,Dv] float32)."""
    qf, kf, vf = _f64(q, in_dtype), _f64(k, in_dtype), _f64(v, in_dtype)
    gf = _f64(g, g_dtype or in_dtype)
    bf = _f64(beta, beta_dtype or in_dtype)
    S = _f64(state, state_dtype).copy()
    B, T, Hk, Dk = kf.shape
    Hv, Dv = vf.shape[2:]
    if Hv % Hk:
        raise ValueError(f"Cannot align K heads {Hk} to V heads {Hv}")
    hk_of = np.arange(Hv) // (Hv // Hk)
    y = np.zeros((B, T, Hv, Dv))
    tape = np.zeros((B, T, Hv, Dv))
    for b in range(B):
        for t in range(T):
            if mask is not None and not bool(mask[b, t]):
                continue
            kt = kf[b, t, hk_of]                      # [Hv, Dk]
            qt = qf[b, t, hk_of]
            decay = gf[b, t][:, None, None] if gf.ndim == 3 else gf[b, t][:, None, :]
            S[b] = S[b] * decay
            kv = np.einsum("hvk,hk->hv", S[b], kt)
            d = (vf[b, t] - kv) * bf[b, t][:, None]
            S[b] = S[b] + d[:, :, None] * kt[:, None, :]
            y[b, t] = np.einsum("hvk,hk->hv", S[b], qt)
            tape[b, t] = d
    return round_to_dtype(y, in_dtype), round_to_dtype(S, state_dtype), tape.astype(np.float32)


def tape_replay(tape, k, g, state, mask=None, *, k_dtype="bf16", state_dtype="f32",
                g_dtype=None):
    """Returns the state [B,Hv,Dv,Dk] in state_dtype after replaying the tape."""
    tf = np.asarray(tape, dtype=np.float32).astype(np.float64)
    kf = _f64(k, k_dtype)
    gf = _f64(g, g_dtype or k_dtype)
    S = _f64(state, state_dtype).copy()
    B, T, Hk, Dk = kf.shape
    Hv = tf.shape[2]
    if Hv % Hk:
        raise ValueError(f"Cannot align K heads {Hk} to tape heads {Hv}")
    hk_of = np.arange(Hv) // (Hv // Hk)
    for b in range(B):
        for t in range(T):
            if mask is not None and not bool(mask[b, t]):
                continue
            kt = kf[b, t, hk_of]
            decay = gf[b, t][:, None, None] if gf.ndim == 3 else gf[b, t][:, None, :]
            S[b] = S[b] * decay + tf[b, t][:, :, None] * kt[:, None, :]
            S[b] = to_f32(round_to_dtype(S[b], state_dtype), state_dtype).astype(np.float64)
    return round_to_dtype(S, state_dtype)


def gated_delta_with_tape_loops(q, k, v, g, beta, state, mask=None):
    """Scalar-loop restatement on float64 arrays (tiny shapes only): the
    brute-force check of the vectorised form above."""
    q, k, v, g, beta = (np.asarray(a, dtype=np.float64) for a in (q, k, v, g, beta))
    S = np.array(state, dtype=np.float64)
    B, T, Hk, Dk = k.shape
    Hv, Dv = v.shape[2:]
    rep = Hv // Hk
    y = np.zeros((B, T, Hv, Dv))
    tape = np.zeros((B, T, Hv, Dv))
    for b in range(B):
        for hv in range(Hv):
            hk = hv // rep
            for dv in range(Dv):
                row = S[b, hv, dv].copy()
                for t in range(T):
                    if mask is not None and not bool(mask[b, t]):
                        continue
                    for i in range(Dk):
                        row[i] *= g[b, t, hv] if g.ndim == 3 else g[b, t, hv, i]
                    kv = sum(row[i] * k[b, t, hk, i] for i in range(Dk))
                    d = (v[b, t, hv, dv] - kv) * beta[b, t, hv]
                    for i in range(Dk):
                        row[i] += d * k[b, t, hk, i]
                    y[b, t, hv, dv] = sum(row[i] * q[b, t, hk, i] for i in range(Dk))
                    tape[b, t, hv, dv] = d
                S[b, hv, dv] = row
    return y, S, tape
