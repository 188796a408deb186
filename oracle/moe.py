"""Routed-expert (MoE) oracle (test infrastructure only).

Restates the mlx-lm call site that reaches ``mx.gather_qmm`` on the verify
path (``SwitchGLU`` -> ``QuantizedSwitchLinear``, reached from the decoder
layer call at dflash_mlx/engine/target_qwen_gdn.py:865,874) and the Qwen MoE
block around it: softmax router, top-k, optional renormalisation,
``down(silu(gate(x)) * up(x))`` per (token, expert) pair, weighted sum.
mlx-lm is not vendored; the rounding points follow its op sequence (each
MLX op rounds to its output dtype).  Parity against mlx-lm itself is
unpinned; the gather arithmetic reduces to :func:`oracle.qmm.quantized_matmul`.
"""

from __future__ import annotations

import numpy as np

from .numerics import round_to_dtype, to_f32
from .qmm import dequantize


def route_topk(router_logits, top_k: int, renormalize: bool = True):
    """Softmax over experts, top-k per token (descending score, lowest expert
    id first on ties), optional renormalisation.  float64 in, float32 scores."""
    lg = np.asarray(router_logits, dtype=np.float64)
    z = lg - lg.max(axis=-1, keepdims=True)
    p = np.exp(z)
    p /= p.sum(axis=-1, keepdims=True)
    order = np.argsort(-p, axis=-1, kind="stable")[:, :top_k]
    scores = np.take_along_axis(p, order, axis=-1)
    if renormalize:
        scores = scores / scores.sum(axis=-1, keepdims=True)
    return order.astype(np.int64), scores.astype(np.float32)


def _silu_mul(gate_st, up_st, dtype):
    """``silu(gate) * up`` with op-by-op rounding: sigmoid, gate*sig, *up."""
    g = to_f32(gate_st, dtype).astype(np.float64)
    u = to_f32(up_st, dtype).astype(np.float64)
    sig = to_f32(round_to_dtype(1.0 / (1.0 + np.exp(-g)), dtype), dtype).astype(np.float64)
    silu = to_f32(round_to_dtype(g * sig, dtype), dtype).astype(np.float64)
    return round_to_dtype(silu * u, dtype)


def switch_glu(x, inds, gate, up, down, *, group_size=64, bits=4, dtype="bf16"):
    """Per-pair SwitchGLU outputs.

    ``x`` ``[T, D]``; ``inds`` ``[T, k]``; ``gate``/``up``/``down`` are
    ``(w_q [E, N, K*bits/32], scales, biases)`` triples.  Returns
    ``(h [T*k, I], y [T*k, D])`` where pair ``p = t*k + j`` uses token ``t``
    and expert ``inds[t, j]``; ``h`` is the SwiGLU activation and ``y`` the
    down projection, both rounded to ``dtype``.
    """
    xf = to_f32(x, dtype).astype(np.float64)
    inds = np.asarray(inds, dtype=np.int64)
    t_count, k = inds.shape
    cache = {}

    def deq(name, trip, e):
        key = (name, e)
        if key not in cache:
            wq, s, b = trip
            cache[key] = dequantize(wq[e], s[e], b[e], group_size, bits, dtype)
        return cache[key]

    hs, ys = [], []
    for t in range(t_count):
        for j in range(k):
            e = int(inds[t, j])
            g = round_to_dtype(xf[t] @ deq("g", gate, e).T, dtype)
            u = round_to_dtype(xf[t] @ deq("u", up, e).T, dtype)
            h = _silu_mul(g, u, dtype)
            hf = to_f32(h, dtype).astype(np.float64)
            y = round_to_dtype(hf @ deq("d", down, e).T, dtype)
            hs.append(h)
            ys.append(y)
    return np.stack(hs), np.stack(ys)


def moe_combine(y_pairs, scores, *, dtype="bf16", out_dtype=None):
    """``out[t] = sum_j scores[t, j] * y[t*k + j]`` (float64 accumulate).

    ``y_pairs`` ``[T*k, D]`` in ``dtype``; ``scores`` ``[T, k]`` float32.
    Returns float64 ``[T, D]`` or rounded to ``out_dtype``.
    """
    sc = np.asarray(scores, dtype=np.float64)
    t_count, k = sc.shape
    y = to_f32(y_pairs, dtype).astype(np.float64).reshape(t_count, k, -1)
    out = (y * sc[..., None]).sum(axis=1)
    return out if out_dtype is None else round_to_dtype(out, out_dtype)
