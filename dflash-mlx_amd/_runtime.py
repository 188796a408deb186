"""Device plumbing for the operators: dtype codes, streams, workspaces.

PyTorch only supplies device memory and the current HIP stream; all
arithmetic on the verify path happens in libdfmi.so.
"""

from __future__ import annotations

import threading
import weakref
from typing import Optional, Tuple

import torch

from . import _lib

_DTYPE_CODES = {
    torch.bfloat16: _lib.DFMI_BF16,
    torch.float16: _lib.DFMI_F16,
    torch.float32: _lib.DFMI_F32,
}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dt]
    except KeyError:
        raise _lib.DfmiUnsupported(_lib.DFMI_EINVAL, f"dtype {dt} unsupported") from None


def require_device(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (got {getattr(t, 'device', type(t))})")


def stream_ptr(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


def aligned_contiguous(t: torch.Tensor) -> torch.Tensor:
    """Contiguous tensor whose data pointer is 16-byte aligned (copy if needed)."""
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def weight_words(w: torch.Tensor) -> torch.Tensor:
    """Packed weights as 32-bit words (int32 / uint32 storage, same bits)."""
    if w.dtype not in (torch.int32, torch.uint32):
        raise ValueError(f"packed weights must be int32/uint32 words, got {w.dtype}")
    return aligned_contiguous(w)


class _WorkspaceCache:
    """One zero-initialised scratch buffer per (device, stream, kind).

    ``kind`` names the function family ("qmm", "greedy"): each family lays out
    its own counters, so families never share a buffer.

    The kernels leave every counter they touch at zero, so a buffer is
    zero-filled only when it is created or grown.  Growing is not allowed
    while a HIP graph is being captured: reserve the size beforehand
    (``reserve``), e.g. through ``prewarm_verify_kernels``.  A buffer that a
    larger one replaces stays allocated: a graph captured earlier still
    launches kernels on its address (each replacement at least doubles the
    size, so the retired buffers total less than the live one).
    """

    def __init__(self):
        self._lock = threading.Lock()
        self._bufs: dict[tuple[int, int, str], torch.Tensor] = {}
        self._retired: list[torch.Tensor] = []

    def get(self, device: torch.device, nbytes: int, kind: str = "qmm") -> torch.Tensor:
        nbytes = max(int(nbytes), 256)
        key = (device.index if device.index is not None else torch.cuda.current_device(),
               stream_ptr(device), kind)
        with self._lock:
            buf = self._bufs.get(key)
            if buf is None or buf.numel() < nbytes:
                if torch.cuda.is_current_stream_capturing():
                    raise RuntimeError(
                        f"libdfmi workspace must grow to {nbytes} bytes during graph capture; "
                        "reserve it before capturing")
                size = max(nbytes, 2 * (buf.numel() if buf is not None else 0))
                if buf is not None:
                    self._retired.append(buf)
                buf = torch.zeros(size + 256, dtype=torch.uint8, device=device)
                self._bufs[key] = buf
        return buf

    def reserve(self, device: torch.device, nbytes: int, kind: str = "qmm") -> None:
        self.get(device, nbytes, kind)


WORKSPACES = _WorkspaceCache()


def workspace(device: torch.device, nbytes: int, kind: str = "qmm") -> tuple[int, int]:
    """(aligned pointer, usable bytes) of this stream's scratch buffer for ``kind``."""
    buf = WORKSPACES.get(device, nbytes + 256, kind)
    base = buf.data_ptr()
    aligned = (base + 255) // 256 * 256
    return aligned, buf.numel() - (aligned - base)


def pair_shape(M: int, K: int, N: int, group_size: int, bits: int) -> bool:
    """Shapes whose streaming plan can take a pair table (``dfmi_qmm_affine_pairs``):
    4-bit, gs 64 / 128, M <= 32, whole 256-k steps (mirrors the library's rule)."""
    return (int(bits) == 4 and int(group_size) in (64, 128) and 1 <= int(M) <= 32
            and int(K) % 256 == 0 and int(K) % (8 * int(group_size)) == 0
            and (int(N) + 63) // 64 <= 16384)


def build_sb_pairs(scales: torch.Tensor, biases: torch.Tensor) -> torch.Tensor:
    """The ``[K/gs][N]`` uint32 pair table of a layer (``dfmi_sb_pairs``), on
    the current stream."""
    N, G = int(scales.shape[-2]), int(scales.shape[-1])
    pairs = torch.empty((G, N), dtype=torch.int32, device=scales.device)
    lib = _lib.load()
    status = lib.dfmi_sb_pairs(scales.data_ptr(), biases.data_ptr(), dtype_code(scales.dtype),
                               N, G, pairs.data_ptr(), stream_ptr(scales.device))
    _lib.check(status, "dfmi_sb_pairs")
    return pairs


def moe_pair_shape(K: int, N: int, group_size: int, bits: int, swiglu: bool) -> bool:
    """Expert shapes the pair-streaming gather takes (``dfmi_gather_qmm_*_pairs``):
    4-bit, gs 64 / 128, whole 256-k steps, N a multiple of 64 (SwiGLU) or 128
    (mirrors the library's rule; the pair count is checked per call)."""
    return (int(bits) == 4 and int(group_size) in (64, 128) and int(K) >= 256
            and int(K) % 256 == 0 and int(N) > 0 and int(N) % (64 if swiglu else 128) == 0)


def build_moe_pairs(scales: torch.Tensor, biases: torch.Tensor,
                    up_scales: Optional[torch.Tensor] = None,
                    up_biases: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The ``[E][K/gs][N]`` (or SwiGLU-interleaved ``[E][K/gs][2N]``) uint32
    pair table of routed experts (``dfmi_moe_pairs``), on the current stream."""
    E, N, G = (int(d) for d in scales.shape)
    cols = 2 * N if up_scales is not None else N
    pairs = torch.empty((E, G, cols), dtype=torch.int32, device=scales.device)
    lib = _lib.load()
    status = lib.dfmi_moe_pairs(scales.data_ptr(), biases.data_ptr(),
                                up_scales.data_ptr() if up_scales is not None else None,
                                up_biases.data_ptr() if up_biases is not None else None,
                                dtype_code(scales.dtype), E, N, G, pairs.data_ptr(),
                                stream_ptr(scales.device))
    _lib.check(status, "dfmi_moe_pairs")
    return pairs


class _PairCache:
    """Pair tables of the (scales, biases) tensors the functional operators
    see, built on first use and kept while the tensors live.  An entry is
    valid only for the same tensor objects at the same versions (an in-place
    update rebuilds it).  Nothing is built during graph capture: the caller
    then runs without a table (dense matmuls: the same plan, bit-identical
    result; gathers: the plain gather's main loop).  ``experts`` selects the
    routed-expert layout (``dfmi_moe_pairs``; with ``up`` the SwiGLU
    interleave of two sets)."""

    def __init__(self):
        self._lock = threading.Lock()
        self._entries: dict[tuple, tuple] = {}

    def _drop(self, key: tuple):
        with self._lock:
            self._entries.pop(key, None)

    def get(self, scales: torch.Tensor, biases: torch.Tensor,
            up: Optional[Tuple[torch.Tensor, torch.Tensor]] = None, *, experts: bool = False):
        tensors = (scales, biases) + (tuple(up) if up is not None else ())
        key = (id(scales), id(up[0]) if up is not None else 0, bool(experts))
        ver = tuple(t._version for t in tensors)
        with self._lock:
            ent = self._entries.get(key)
        if ent is not None:
            refs, ever, pairs = ent
            if ever == ver and all(r() is t for r, t in zip(refs, tensors)):
                return pairs
        if torch.cuda.is_current_stream_capturing():
            return None
        if experts:
            pairs = build_moe_pairs(scales, biases, *(up if up is not None else ()))
        else:
            pairs = build_sb_pairs(scales, biases)
        refs = tuple(weakref.ref(t, lambda _r, k=key: self._drop(k)) for t in tensors)
        with self._lock:
            self._entries[key] = (refs, ver, pairs)
        return pairs


PAIRS = _PairCache()


class _FusedPairCache:
    """Pair tables of sibling matrices side by side (``[K/gs][N0 + N1 (+ N2)]``,
    the per-matrix tables concatenated along the columns), for
    ``dfmi_qmm_affine_multi_fused``; built on first use from the tables given,
    kept while they live, never built during graph capture (the caller then
    launches with the per-matrix tables: the same sums)."""

    def __init__(self):
        self._lock = threading.Lock()
        self._entries: dict[tuple, tuple] = {}

    def _drop(self, key: tuple):
        with self._lock:
            self._entries.pop(key, None)

    def get(self, tables) -> Optional[torch.Tensor]:
        key = tuple(id(t) for t in tables)
        ver = tuple(t._version for t in tables)
        with self._lock:
            ent = self._entries.get(key)
        if ent is not None:
            refs, ever, fused = ent
            if ever == ver and all(r() is t for r, t in zip(refs, tables)):
                return fused
        if torch.cuda.is_current_stream_capturing():
            return None
        fused = torch.cat(list(tables), dim=1).contiguous()
        refs = tuple(weakref.ref(t, lambda _r, k=key: self._drop(k)) for t in tables)
        with self._lock:
            self._entries[key] = (refs, ver, fused)
        return fused


FUSED_PAIRS = _FusedPairCache()
