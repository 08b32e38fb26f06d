"""Look-back workspaces for the single-pass scans.

A workspace is a zero-filled device buffer that one stream reuses across
launches (its header resets itself at the end of every launch and carries an
epoch that invalidates stale carry words).  One buffer is kept per
(device, stream) and grown when a launch needs more; launches on different
streams therefore never share one.
"""
from __future__ import annotations

import threading

import torch

from . import _lib

_lock = threading.Lock()
_cache: dict[tuple[int, int], torch.Tensor] = {}


def get(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    with _lock:
        buf = _cache.get(key)
        if buf is None or buf.numel() < nbytes:
            # zero-filled on the current stream, so it is ordered before the scan
            buf = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
            _cache[key] = buf
        return buf


def error_flag(buf: torch.Tensor, clear: bool = True) -> int:
    """Sticky look-back timeout flag of a workspace (synchronous; tests only)."""
    import ctypes
    out = ctypes.c_int(0)
    _lib.call("tssm_workspace_error", buf.data_ptr(), int(clear), ctypes.byref(out))
    return out.value


def clear() -> None:
    with _lock:
        _cache.clear()
