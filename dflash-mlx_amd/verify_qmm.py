"""Verify-path quantized matmul with the reference's call surface.

Mirrors dflash_mlx/verify_qmm.py: ``is_enabled`` (15-16), the variant
predicates (21-51), ``_should_use_verify`` (886-903) and ``verify_matmul``
(905-1022).  Every route -- the M=16 K-templated variants, the mma2big /
mma2big_pipe variants, the M=4 k-split variant and the "stock" fallback that
the reference hands to ``mx.quantized_matmul`` -- runs the same hand-written
gfx950 kernel family in libdfmi.so (``dfmi_qmm_affine``).  The route decides
which calls take the verify path (the reference's admission rules, restated
rule for rule); the launch shape is the library's automatic plan, unless
``DFLASH_VERIFY_QMM_KPARTS`` is set, in which case that many workgroups split
K (the meaning the reference gives it).  The reference's built-in K_PARTS
defaults (8 for mma2big_pipe, 1 for mma2big) are Metal launch choices and are
not forced on this GPU.  All shapes compute the same sums in fp32 and differ
only in fp32 summation order.

Tensors: ``x`` bf16/f16 ``[..., K]`` on the GPU; ``w`` int32/uint32 words
``[N, K*bits/32]``; ``scales``/``biases`` ``[N, K/group_size]`` in x's dtype.
"""

from __future__ import annotations

import ctypes
import math
import os
from typing import Optional

import torch

from . import _lib, _runtime
from .internal_debug import (
    verify_qmm_enabled as _debug_verify_qmm_enabled,
    verify_qmm_kparts as _debug_verify_qmm_kparts,
    verify_qmm_variant as _debug_verify_qmm_variant,
)

_KERNEL_DTYPES = (torch.bfloat16, torch.float16)


def is_enabled() -> bool:
    return _debug_verify_qmm_enabled()


def _variant() -> str:
    return _debug_verify_qmm_variant()


def _auto_variant(K: int, N: int) -> tuple[str, int]:
    """dflash_mlx/verify_qmm.py:21-24."""
    if K >= 8192 or N <= 8192:
        return ("mma2big_pipe", 8)
    return ("mma2big", 1)


def _m4_ksplit_np_shape(K: int, N: int, bits: int) -> bool:
    """dflash_mlx/verify_qmm.py:28-29."""
    return int(bits) == 4 and int(N) % 4 == 0 and int(K) % 32 == 0


def _m4_ksplit_np_kparts(N: int) -> int:
    """dflash_mlx/verify_qmm.py:31-32."""
    return 2 if int(N) >= 4096 else 4


def _m16_ktmpl_variant(K: int, N: int, bits: int) -> Optional[str]:
    """dflash_mlx/verify_qmm.py:34-41."""
    if int(bits) != 4:
        return None
    if int(K) % 256 != 0 or int(N) % 16 != 0:
        return None
    if int(K) >= 8192 or int(N) <= 5120:
        return "combo_ktmpl"
    return "super_tree_fp16_ktmpl"


def _resolve_m16_ktmpl_variant(K: int, N: int, bits: int,
                               variant: Optional[str] = None) -> Optional[str]:
    """dflash_mlx/verify_qmm.py:43-51."""
    if int(bits) != 4 or int(K) % 256 != 0 or int(N) % 16 != 0:
        return None
    selected = _variant() if variant is None else str(variant)
    if selected == "auto":
        return _m16_ktmpl_variant(K, N, bits)
    if selected in ("combo_ktmpl", "super_tree_fp16_ktmpl"):
        return selected
    return None


def _tuning(k_parts: int = 0):
    """Launch-shape hint from a K_PARTS value: the number of K splits
    (workgroups on the streaming kernel, wavefronts on the general one, at
    most 8); 0 means automatic."""
    if not k_parts:
        return None
    kp = max(1, min(8, int(k_parts)))
    return _lib.QmmTuning(0, 0, kp, kp)


def _kparts_tuning():
    """The launch shape of an M=16 verify call: automatic, or the split count
    ``DFLASH_VERIFY_QMM_KPARTS`` asks for when the user sets it."""
    raw = os.environ.get("DFLASH_VERIFY_QMM_KPARTS")
    if raw is None:
        return None
    kp = _debug_verify_qmm_kparts(0)
    return _tuning(kp) if kp > 0 else None


def _pairs_of(M: int, K: int, N: int, group_size: int, bits: int, scales, biases,
              pairs) -> Optional[torch.Tensor]:
    """The pair table a launch passes: the given one, else the functional
    cache's for shapes whose plan can use it (None: none)."""
    if pairs is None:
        if not _runtime.pair_shape(M, K, N, group_size, bits):
            return None
        pairs = _runtime.PAIRS.get(scales, biases)
    return pairs


def _pairs_ptr(M: int, K: int, N: int, group_size: int, bits: int, scales, biases,
               pairs) -> int:
    """Device pointer of :func:`_pairs_of`'s table (0: none)."""
    t = _pairs_of(M, K, N, group_size, bits, scales, biases, pairs)
    return t.data_ptr() if t is not None else 0


def qmm_launch(x2: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               N: int, group_size: int, bits: int, tuning=None,
               out: Optional[torch.Tensor] = None,
               pairs: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One ``dfmi_qmm_affine_pairs`` launch on the current stream:
    ``[M, K] -> [M, N]``.  ``pairs`` is the layer's pair table
    (``_runtime.build_sb_pairs``); when None, the one cached for ``scales`` is
    used (built on first use).  The result does not depend on it."""
    lib = _lib.load()
    M, K = int(x2.shape[0]), int(x2.shape[1])
    dev = x2.device
    y = out if out is not None else torch.empty((M, N), dtype=x2.dtype, device=dev)
    tptr = ctypes.byref(tuning) if tuning is not None else None
    need = int(lib.dfmi_qmm_workspace_bytes_ex(M, K, N, int(group_size), int(bits), tptr))
    ws, ws_bytes = _runtime.workspace(dev, need) if need else (0, 0)
    tp = _pairs_ptr(M, K, N, group_size, bits, scales, biases, pairs)
    status = lib.dfmi_qmm_affine_pairs(
        x2.data_ptr(), _runtime.dtype_code(x2.dtype), w.data_ptr(), scales.data_ptr(),
        biases.data_ptr(), tp, y.data_ptr(), M, K, N, int(group_size), int(bits),
        ws, ws_bytes, tptr, _runtime.stream_ptr(dev))
    _lib.check(status, "dfmi_qmm_affine")
    return y


def qmm_multi_launch(x2: torch.Tensor, mats, group_size: int, bits: int,
                     outs=None) -> list:
    """One ``dfmi_qmm_affine_multi`` launch on the current stream: the
    matrices ``mats = [(w, scales, biases[, pairs]), ...]`` (1..4) share
    ``x2 [M, K]``; returns ``[y_i [M, N_i]]``.  A matrix without its pair
    table uses the cached one (see :func:`qmm_launch`)."""
    lib = _lib.load()
    M, K = int(x2.shape[0]), int(x2.shape[1])
    dev = x2.device
    n = len(mats)
    if not 1 <= n <= 4:
        raise ValueError("1..4 matrices per launch")
    Ns = [int(m[0].shape[0]) for m in mats]
    ys = outs if outs is not None else [torch.empty((M, N), dtype=x2.dtype, device=dev)
                                        for N in Ns]
    segs = (_lib.QmmSegment * n)()
    tables = []
    for i, (m, y) in enumerate(zip(mats, ys)):
        w, sc, bi = m[0], m[1], m[2]
        segs[i].w_q, segs[i].scales, segs[i].biases = w.data_ptr(), sc.data_ptr(), bi.data_ptr()
        segs[i].y, segs[i].N = y.data_ptr(), Ns[i]
        t = _pairs_of(M, K, Ns[i], group_size, bits, sc, bi, m[3] if len(m) > 3 else None)
        tables.append(t)
        segs[i].sb_pairs = t.data_ptr() if t is not None else 0
    ns = (ctypes.c_int64 * n)(*Ns)
    need = int(lib.dfmi_qmm_multi_workspace_bytes(M, K, ns, n, int(group_size), int(bits)))
    ws, ws_bytes = _runtime.workspace(dev, need) if need else (0, 0)
    # two or three matrices with tables: the tables side by side, so that the
    # fused kernel starts its first loads without reading a segment table
    fused = (_runtime.FUSED_PAIRS.get(tables)
             if 2 <= n <= 3 and all(t is not None for t in tables) else None)
    if fused is not None:
        status = lib.dfmi_qmm_affine_multi_fused(
            x2.data_ptr(), _runtime.dtype_code(x2.dtype), segs, n, fused.data_ptr(), M, K,
            int(group_size), int(bits), ws, ws_bytes, _runtime.stream_ptr(dev))
        _lib.check(status, "dfmi_qmm_affine_multi_fused")
        return ys
    status = lib.dfmi_qmm_affine_multi(x2.data_ptr(), _runtime.dtype_code(x2.dtype), segs, n, M,
                                       K, int(group_size), int(bits), ws, ws_bytes,
                                       _runtime.stream_ptr(dev))
    _lib.check(status, "dfmi_qmm_affine_multi")
    return ys


_raw_stream = torch._C._cuda_getCurrentRawStream


def current_stream(device_index: int) -> int:
    """The current HIP stream of a device, as a pointer value."""
    return int(_raw_stream(device_index))


class LaunchRecord:
    """One prepared launch (``dfmi_qmm_prepare``): the plan, kernel arguments
    and matrices of a verify linear -- one matrix, or 2..4 sibling matrices
    sharing their input -- computed once for a call shape (M, dtype, stream),
    so that a call is one ``dfmi_qmm_run``.  The reference computes each
    module's route once in ``_build_dispatch`` and launches from a closure
    (dflash_mlx/verify_linear.py:118-309).

    ``mats``: ``[(w, scales, biases, pairs), ...]`` (``pairs`` None, the
    matrix's own table, or its column slice of a wider table when
    ``sb_stride`` names that table's row length); ``fused``: for 2..4
    matrices, their tables side by side.  The record keeps these tensors and
    the stream's workspace alive while it exists; run it only on the stream
    it was prepared for (the workspace is that stream's)."""

    __slots__ = ("_buf", "ptr", "_keep", "M", "Ns", "dtype")

    def __init__(self, M: int, K: int, dtype: torch.dtype, dev: torch.device, mats,
                 group_size: int, bits: int, fused: Optional[torch.Tensor] = None,
                 sb_stride: int = 0):
        lib = _lib.load()
        n = len(mats)
        if not 1 <= n <= 4:
            raise ValueError("1..4 matrices per launch")
        segs = (_lib.QmmSegment * n)()
        keep = []
        Ns = []
        for i, m in enumerate(mats):
            w, sc, bi = m[0], m[1], m[2]
            t = m[3] if len(m) > 3 else None
            for name, ten in (("w", w), ("scales", sc), ("biases", bi)):
                if ten.device != dev:
                    raise ValueError(f"{name} of matrix {i} is on {ten.device}, not {dev}")
            segs[i].w_q, segs[i].scales, segs[i].biases = w.data_ptr(), sc.data_ptr(), bi.data_ptr()
            segs[i].N = int(w.shape[0])
            segs[i].sb_pairs = t.data_ptr() if t is not None else 0
            keep += [w, sc, bi, t]
            Ns.append(int(w.shape[0]))
        if n == 1:
            need = int(lib.dfmi_qmm_workspace_bytes_ex(M, K, Ns[0], int(group_size), int(bits),
                                                        None))
        else:
            ns = (ctypes.c_int64 * n)(*Ns)
            need = int(lib.dfmi_qmm_multi_workspace_bytes(M, K, ns, n, int(group_size),
                                                          int(bits)))
        ws, ws_bytes = _runtime.workspace(dev, need) if need else (0, 0)
        buf = ctypes.create_string_buffer(_lib.DFMI_QMM_RECORD_BYTES + 16)
        ptr = (ctypes.addressof(buf) + 15) // 16 * 16
        status = lib.dfmi_qmm_prepare(_runtime.dtype_code(dtype), segs, n,
                                      fused.data_ptr() if fused is not None else 0,
                                      int(sb_stride), M, K, int(group_size), int(bits), ws,
                                      ws_bytes, ptr, _lib.DFMI_QMM_RECORD_BYTES)
        _lib.check(status, "dfmi_qmm_prepare")
        keep.append(fused)
        self._buf, self.ptr, self._keep = buf, ptr, keep
        self.M, self.Ns, self.dtype = M, Ns, dtype

    def run(self, x2: torch.Tensor, ys, stream: int) -> None:
        """Launch on ``x2 [M, K]`` (contiguous, 16-byte aligned) into ``ys``."""
        p = [y.data_ptr() for y in ys] + [None] * (4 - len(ys))
        status = _lib.load().dfmi_qmm_run(self.ptr, x2.data_ptr(), p[0], p[1], p[2], p[3], stream)
        if status:
            _lib.check(status, "dfmi_qmm_run")


def _prepare(x, w, scales, biases):
    for t, name in ((x, "x"), (w, "w"), (scales, "scales"), (biases, "biases")):
        _runtime.require_device(t, name)
    if scales.dtype != x.dtype or biases is None or biases.dtype != x.dtype:
        raise _lib.DfmiUnsupported(
            _lib.DFMI_EINVAL, "scales and biases must exist and share x's dtype")
    K = int(x.shape[-1])
    M = math.prod(int(d) for d in x.shape[:-1])
    x2 = _runtime.aligned_contiguous(x.reshape(M, K))
    return (x2, _runtime.weight_words(w), _runtime.aligned_contiguous(scales),
            _runtime.aligned_contiguous(biases), M, K)


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                     biases: torch.Tensor, *, transpose: bool = True, group_size: int = 64,
                     bits: int = 4, mode: str = "affine", tuning=None) -> torch.Tensor:
    """The "stock" quantized matmul of this framework (the role
    ``mx.quantized_matmul`` plays for the reference): ``x . dequant(w)^T``
    (``transpose=True``, w ``[N, K*bits/32]``) or ``x . dequant(w)``
    (``transpose=False``, w ``[K, N*bits/32]`` quantised along N).

    Activations and scales in bf16, f16 or f32; the result has their common
    dtype when they share one, else float32 (MLX's promotion).  x and scales
    of one 16-bit dtype with ``transpose=True`` take the verify kernels; the
    other cases ``dfmi_qmm_general``'s fp32 kernels.  Raises
    :class:`_lib.DfmiUnsupported` for bits other than 4 and 8, group sizes
    other than 32 / 64 / 128 and non-affine modes.
    """
    if mode != "affine":
        raise _lib.DfmiUnsupported(_lib.DFMI_EINVAL, f"mode {mode!r} is not implemented")
    if transpose and x.dtype in _KERNEL_DTYPES and scales.dtype == x.dtype:
        x2, wq, s, b, M, K = _prepare(x, w, scales, biases)
        N = int(wq.shape[0])
        y = qmm_launch(x2, wq, s, b, N, group_size, bits, tuning)
        return y.reshape(*x.shape[:-1], N)
    return _general(x, w, scales, biases, transpose, int(group_size), int(bits))


_FLOAT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _general(x, w, scales, biases, transpose: bool, group_size: int, bits: int):
    """``dfmi_qmm_general`` on the inputs the verify kernels do not take."""
    for t, name in ((x, "x"), (w, "w"), (scales, "scales"), (biases, "biases")):
        _runtime.require_device(t, name)
    if x.dtype not in _FLOAT_DTYPES or scales.dtype not in _FLOAT_DTYPES:
        raise _lib.DfmiUnsupported(_lib.DFMI_EINVAL,
                                   f"dtypes x {x.dtype}, scales {scales.dtype} unsupported")
    if biases is None or biases.dtype != scales.dtype:
        raise _lib.DfmiUnsupported(_lib.DFMI_EINVAL, "biases must exist and share the scales' dtype")
    if bits not in (4, 8):
        raise _lib.DfmiUnsupported(_lib.DFMI_EINVAL, f"bits={bits} unsupported (4 or 8)")
    wq = _runtime.weight_words(w)
    if wq.dim() != 2:
        raise ValueError(f"w must be 2-D packed words, got shape {tuple(wq.shape)}")
    K = int(x.shape[-1])
    M = math.prod(int(d) for d in x.shape[:-1])
    if transpose:
        N, kw = int(wq.shape[0]), int(wq.shape[1]) * 32 // bits
        if kw != K:
            raise ValueError(f"w covers K={kw}, x has K={K}")
        groups = (N, K // group_size if group_size else 0)
    else:
        N = int(wq.shape[1]) * 32 // bits
        if int(wq.shape[0]) != K:
            raise ValueError(f"w has {int(wq.shape[0])} rows, x has K={K}")
        groups = (K, N // group_size if group_size else 0)
    if tuple(scales.shape) != groups or tuple(biases.shape) != groups:
        raise ValueError(f"scales / biases must be {groups}, got {tuple(scales.shape)} / "
                         f"{tuple(biases.shape)}")
    x2 = _runtime.aligned_contiguous(x.reshape(M, K))
    s, b = _runtime.aligned_contiguous(scales), _runtime.aligned_contiguous(biases)
    ydt = x.dtype if x.dtype == scales.dtype else torch.float32
    y = torch.empty((M, N), dtype=ydt, device=x.device)
    lib = _lib.load()
    need = 0
    if transpose and x.dtype == scales.dtype and x.dtype != torch.float32:
        need = int(lib.dfmi_qmm_workspace_bytes(M, K, N, group_size, bits))
    ws, ws_bytes = _runtime.workspace(x.device, need) if need else (0, 0)
    status = lib.dfmi_qmm_general(
        x2.data_ptr(), _runtime.dtype_code(x2.dtype), wq.data_ptr(), s.data_ptr(), b.data_ptr(),
        _runtime.dtype_code(s.dtype), y.data_ptr(), M, K, N, group_size, bits, int(bool(transpose)),
        ws, ws_bytes, _runtime.stream_ptr(x.device))
    _lib.check(status, "dfmi_qmm_general")
    return y.reshape(*x.shape[:-1], N)


def quantized_matmul_multi(x: torch.Tensor, weights, *, group_size: int = 64,
                           bits: int = 4) -> list:
    """``[x . dequant(W_i)^T for W_i in weights]`` in one launch, for sibling
    projections that read the same input (q/k/v, gate/up).  ``weights`` is a
    list of 1..4 ``(w, scales, biases)``; the reference calls ``verify_matmul``
    once per projection (dflash_mlx/verify_linear.py:266-286).  Each result is
    within fp32 summation order of :func:`quantized_matmul` on that matrix."""
    if x.dtype not in _KERNEL_DTYPES:
        raise _lib.DfmiUnsupported(_lib.DFMI_EINVAL, f"x dtype {x.dtype} unsupported")
    mats = []
    x2 = None
    for (w, scales, biases) in weights:
        x2, wq, s, b, M, K = _prepare(x, w, scales, biases)
        mats.append((wq, s, b))
    ys = qmm_multi_launch(x2, mats, group_size, bits)
    return [y.reshape(*x.shape[:-1], int(y.shape[-1])) for y in ys]


def _should_use_verify(x: torch.Tensor, group_size: int, bits: int, transpose: bool) -> bool:
    """dflash_mlx/verify_qmm.py:886-903."""
    if not is_enabled():
        return False
    if bits not in (4, 8) or group_size not in (32, 64, 128):
        return False
    if x.dtype not in _KERNEL_DTYPES:
        return False
    if not transpose:
        return False
    m = math.prod(int(d) for d in x.shape[:-1])
    return m in (4, 16)


def verify_route(M: int, K: int, N: int, bits: int,
                 variant: Optional[str] = None) -> tuple[str, object]:
    """Route of ``verify_matmul`` for an enabled M in {4, 16} call
    (dflash_mlx/verify_qmm.py:933-1022): ``(name, tuning)``; name "stock"
    means the reference would fall back to mx.quantized_matmul."""
    if M == 4:
        if not _m4_ksplit_np_shape(K, N, bits):
            return "stock", None
        return "m4_ksplit_np", None
    selected = _variant() if variant is None else variant
    ktmpl = _resolve_m16_ktmpl_variant(K, N, bits, selected)
    if ktmpl is not None:
        return ktmpl, None
    auto_kp = None
    if selected == "auto":
        selected, auto_kp = _auto_variant(K, N)
    k_parts = auto_kp if auto_kp is not None else _debug_verify_qmm_kparts(4)
    if selected == "mma2big_pipe":
        if N % 32 != 0 or k_parts <= 0 or K % (32 * k_parts) != 0:
            return "stock", None
        return "mma2big_pipe", _kparts_tuning()
    if N % 32 != 0 or K % 32 != 0:
        return "stock", None
    return "mma2big", _kparts_tuning()


def verify_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                  biases: torch.Tensor, *, transpose: bool = True, group_size: int = 64,
                  bits: int = 4) -> torch.Tensor:
    """dflash_mlx/verify_qmm.py:905-1022 -- verify kernels for M in {4, 16}
    when ``DFLASH_VERIFY_QMM=1``, else the stock quantized matmul."""
    if not _should_use_verify(x, group_size, bits, transpose):
        return quantized_matmul(x, w, scales, biases, transpose=transpose,
                                group_size=group_size, bits=bits)
    x2, wq, s, b, M, K = _prepare(x, w, scales, biases)
    N = int(wq.shape[0])
    route, tuning = verify_route(M, K, N, bits)
    if route == "stock":
        return quantized_matmul(x, w, scales, biases, transpose=transpose,
                                group_size=group_size, bits=bits)
    y = qmm_launch(x2, wq, s, b, N, group_size, bits, tuning)
    return y.reshape(*x.shape[:-1], N)
