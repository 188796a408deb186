"""Routed-expert (MoE) operators of the verify path.

On a MoE target the verify forward reaches ``mx.gather_qmm`` through
mlx-lm's ``SwitchGLU`` / ``QuantizedSwitchLinear`` (the decoder layer call
at dflash_mlx/engine/target_qwen_gdn.py:865,874):

    x_up   = gather_qmm(x, up.weight,   ..., rhs_indices=inds, transpose=True)
    x_gate = gather_qmm(x, gate.weight, ..., rhs_indices=inds, transpose=True)
    h      = silu(x_gate) * x_up
    y      = gather_qmm(h, down.weight, ..., rhs_indices=inds, transpose=True)
    out    = (y * scores[..., None]).sum(axis=-2)

(mlx-lm sorts the pairs by expert when there are >= 64 of them and passes
``sorted_indices=True``.)  Here every (token, expert) pair is explicit:
pair ``p = t*k + j`` reads activation row ``t`` (or ``lhs_indices[p]``) and
expert ``rhs_indices[p]``.  ``gather_qmm`` is ``dfmi_gather_qmm_affine``,
the gate/up pair plus SwiGLU is one ``dfmi_gather_qmm_swiglu`` launch (one
pass over both weight sets), and the weighted sum is ``dfmi_moe_combine``.

Where the expert shapes allow (4-bit, gs 64 / 128, K a multiple of 256,
N a multiple of 128, or 64 for the SwiGLU pair, at most 256 pairs) the
gathers take the experts' (scale, bias) pair table (``dfmi_moe_pairs``,
built once per weight set and cached) and the stream's gather workspace, and
run the pair-streaming main loop (``dfmi_gather_qmm_*_pairs``); otherwise,
and during graph capture before a table exists, the plain entry points.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib, _runtime

Triple = Tuple[torch.Tensor, torch.Tensor, torch.Tensor]


def _indices(t: Optional[torch.Tensor], name: str) -> Optional[torch.Tensor]:
    if t is None:
        return None
    _runtime.require_device(t, name)
    return t.reshape(-1).to(torch.int32).contiguous()


def _expert_weights(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, K: int,
                    group_size: int, bits: int):
    if w.dim() != 3 or scales.dim() != 3 or biases.dim() != 3:
        raise ValueError("expert weights must be [E, N, K*bits/32] with [E, N, K/gs] scales/biases")
    E, N = int(w.shape[0]), int(w.shape[1])
    if int(w.shape[2]) != K * bits // 32:
        raise ValueError(f"w last dim {int(w.shape[2])} does not match K={K}, bits={bits}")
    if tuple(scales.shape) != (E, N, K // group_size) or tuple(biases.shape) != tuple(scales.shape):
        raise ValueError("scales / biases must be [E, N, K/group_size]")
    return (E, N, _runtime.weight_words(w), _runtime.aligned_contiguous(scales),
            _runtime.aligned_contiguous(biases))


def _pairs_ptr(pairs: Optional[torch.Tensor], scales: torch.Tensor, biases: torch.Tensor,
               up: Optional[Tuple[torch.Tensor, torch.Tensor]], K: int, N: int,
               group_size: int, bits: int, use_pairs: bool):
    """Address of the experts' pair table (``dfmi_moe_pairs`` layout), or None.

    An explicit table is checked for shape and device; otherwise the cached
    table of these scales / biases is used when the shape takes one (built on
    first use, never during graph capture)."""
    E, _, G = (int(d) for d in scales.shape)
    cols = 2 * N if up is not None else N
    if pairs is not None:
        _runtime.require_device(pairs, "pairs")
        if (pairs.dtype != torch.int32 or tuple(pairs.shape) != (E, G, cols)
                or not pairs.is_contiguous()):
            raise ValueError(f"pairs must be a contiguous int32 [{E}, {G}, {cols}] table")
        return pairs.data_ptr()
    if not use_pairs or not _runtime.moe_pair_shape(K, N, group_size, bits, up is not None):
        return None
    table = _runtime.PAIRS.get(scales, biases, up, experts=True)
    return table.data_ptr() if table is not None else None


def _workspace(lib, device: torch.device, table_ptr):
    """The stream's gather workspace (tail-split counters and partials), only
    with a pair table (the plain main loops take none)."""
    if table_ptr is None:
        return None, 0
    return _runtime.workspace(device, int(lib.dfmi_gather_workspace_bytes()), kind="gather")


def gather_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               rhs_indices: torch.Tensor, *, lhs_indices: Optional[torch.Tensor] = None,
               transpose: bool = True, group_size: int = 64, bits: int = 4,
               sorted_indices: bool = False, pairs: Optional[torch.Tensor] = None,
               use_pairs: bool = True) -> torch.Tensor:
    """``y[p] = x[lhs[p]] . dequant(W[rhs[p]])^T`` for every pair p.

    ``x`` ``[R, K]`` (bf16/f16), ``w`` ``[E, N, K*bits/32]`` uint32,
    ``rhs_indices`` ``[P]`` expert ids, ``lhs_indices`` ``[P]`` row ids or
    None (row p).  Returns ``[P, N]`` in x's dtype.  ``sorted_indices`` is
    accepted for signature parity: runs of equal experts are found on the
    device either way.  ``pairs`` / ``use_pairs``: the experts' pair table
    (``dfmi_gather_qmm_affine_pairs``), by default the cached one.
    """
    del sorted_indices
    if not transpose:
        raise _lib.DfmiUnsupported(_lib.DFMI_EINVAL, "gather_qmm supports transpose=True only")
    for t, name in ((x, "x"), (w, "w"), (scales, "scales"), (biases, "biases")):
        _runtime.require_device(t, name)
    K = int(x.shape[-1])
    x2 = _runtime.aligned_contiguous(x.reshape(-1, K))
    E, N, w, scales, biases = _expert_weights(w, scales, biases, K, group_size, bits)
    rhs = _indices(rhs_indices, "rhs_indices")
    lhs = _indices(lhs_indices, "lhs_indices")
    P = int(rhs.shape[0])
    if lhs is not None and int(lhs.shape[0]) != P:
        raise ValueError("lhs_indices and rhs_indices must have the same length")
    y = torch.empty((P, N), dtype=x.dtype, device=x.device)
    tp = _pairs_ptr(pairs, scales, biases, None, K, N, group_size, bits, use_pairs)
    lib = _lib.load()
    ws, ws_bytes = _workspace(lib, x.device, tp)
    _lib.check(lib.dfmi_gather_qmm_affine_pairs(
        x2.data_ptr(), _runtime.dtype_code(x.dtype), int(x2.shape[0]), w.data_ptr(),
        scales.data_ptr(), biases.data_ptr(), tp, lhs.data_ptr() if lhs is not None else None,
        rhs.data_ptr(), y.data_ptr(), P, K, N, E, int(group_size), int(bits), ws, ws_bytes,
        _runtime.stream_ptr(x.device)), "dfmi_gather_qmm_affine_pairs")
    return y


def gather_swiglu(x: torch.Tensor, gate: Triple, up: Triple, rhs_indices: torch.Tensor, *,
                  lhs_indices: Optional[torch.Tensor] = None, group_size: int = 64,
                  bits: int = 4, pairs: Optional[torch.Tensor] = None,
                  use_pairs: bool = True) -> torch.Tensor:
    """``silu(gather_qmm(x, gate)) * gather_qmm(x, up)`` per pair in one
    weight pass (each product rounded to x's dtype first, then the MLX
    op-by-op SwiGLU rounding).  Returns ``[P, N]``.  ``pairs`` /
    ``use_pairs``: the interleaved gate/up pair table
    (``dfmi_gather_qmm_swiglu_pairs``), by default the cached one."""
    _runtime.require_device(x, "x")
    K = int(x.shape[-1])
    x2 = _runtime.aligned_contiguous(x.reshape(-1, K))
    Eg, N, wg, sg, bg = _expert_weights(*gate, K, group_size, bits)
    Eu, Nu, wu, su, bu = _expert_weights(*up, K, group_size, bits)
    if (Eg, N) != (Eu, Nu):
        raise ValueError("gate and up expert weights must have the same [E, N]")
    rhs = _indices(rhs_indices, "rhs_indices")
    lhs = _indices(lhs_indices, "lhs_indices")
    P = int(rhs.shape[0])
    h = torch.empty((P, N), dtype=x.dtype, device=x.device)
    tp = _pairs_ptr(pairs, sg, bg, (su, bu), K, N, group_size, bits, use_pairs)
    lib = _lib.load()
    ws, ws_bytes = _workspace(lib, x.device, tp)
    _lib.check(lib.dfmi_gather_qmm_swiglu_pairs(
        x2.data_ptr(), _runtime.dtype_code(x.dtype), int(x2.shape[0]), wg.data_ptr(),
        sg.data_ptr(), bg.data_ptr(), wu.data_ptr(), su.data_ptr(), bu.data_ptr(), tp,
        lhs.data_ptr() if lhs is not None else None, rhs.data_ptr(), h.data_ptr(), P, K, N,
        Eg, int(group_size), int(bits), ws, ws_bytes, _runtime.stream_ptr(x.device)),
        "dfmi_gather_qmm_swiglu_pairs")
    return h


def moe_combine(y: torch.Tensor, scores: torch.Tensor, *,
                y_rows: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``out[t] = sum_j scores[t, j] * y[r(t*k + j)]`` (fp32 accumulate, j in
    order), ``y`` ``[T*k, D]``, ``scores`` ``[T, k]`` -> ``[T, D]``.

    ``r(p) = y_rows[p]`` when given, else ``p``: with ``y`` in expert-sorted
    pair order (what ``gather_qmm`` returns for sorted pairs), ``y_rows`` is
    the inverse of the sort permutation, i.e. mlx-lm SwitchGLU's unsort
    folded into the weighted sum of the Qwen MoE block
    (dflash_mlx/engine/target_qwen_gdn.py:865,874)."""
    _runtime.require_device(y, "y")
    _runtime.require_device(scores, "scores")
    T, k = int(scores.shape[0]), int(scores.shape[1])
    D = int(y.shape[-1])
    if int(y.numel()) != T * k * D:
        raise ValueError("y must hold T*k rows of D")
    rows = _indices(y_rows, "y_rows")
    if rows is not None and int(rows.numel()) != T * k:
        raise ValueError("y_rows must hold T*k row ids")
    yc = y.reshape(T * k, D).contiguous()
    sc = scores.to(torch.float32).contiguous()
    out = torch.empty((T, D), dtype=y.dtype, device=y.device)
    lib = _lib.load()
    _lib.check(lib.dfmi_moe_combine(yc.data_ptr(), _runtime.dtype_code(y.dtype),
                                    rows.data_ptr() if rows is not None else None, sc.data_ptr(),
                                    out.data_ptr(), T, k, D, _runtime.stream_ptr(y.device)),
               "dfmi_moe_combine")
    return out


def switch_glu(x: torch.Tensor, inds: torch.Tensor, gate: Triple, up: Triple, down: Triple, *,
               group_size: int = 64, bits: int = 4) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-pair SwitchGLU for ``x`` ``[T, D]`` and expert ids ``inds``
    ``[T, k]``: returns ``(h [T*k, I], y [T*k, D])``, pair ``p = t*k + j``.
    Pairs are sorted by expert (as mlx-lm does) so each expert's weights are
    streamed once, and the results are returned in pair order."""
    T, k = int(inds.shape[0]), int(inds.shape[1])
    flat = inds.reshape(-1).to(torch.int64)
    order = torch.argsort(flat, stable=True)
    rhs = flat[order].to(torch.int32)
    lhs = (order // k).to(torch.int32)
    h_sorted = gather_swiglu(x, gate, up, rhs, lhs_indices=lhs, group_size=group_size, bits=bits)
    y_sorted = gather_qmm(h_sorted, *down, rhs, group_size=group_size, bits=bits)
    inv = torch.empty_like(order)
    inv[order] = torch.arange(order.numel(), device=order.device)
    return h_sorted[inv], y_sorted[inv]
