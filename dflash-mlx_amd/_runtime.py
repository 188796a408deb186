"""Device plumbing for the operators: dtype codes, streams, workspaces.

PyTorch only supplies device memory and the current HIP stream; all
arithmetic on the verify path happens in libdfmi.so.
"""

from __future__ import annotations

import threading

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
