"""Device workspaces of the fused scans, and the look-back error check.

A workspace is a zero-filled device buffer that one stream reuses across
launches.  Two kinds never share a buffer:

``lookback``  the single-pass scans (multihead, selective, elementwise):
              tagged carry words {value, epoch} after a 256-byte header whose
              first word is a sticky error flag.  The epoch advances on every
              launch, so stale words never match and no per-launch clearing
              is needed -- provided nothing but tagged words is ever written
              there.
``ssd``       the SSD passes: raw fp32 chunk states and decays.  Kept apart
              because an arbitrary fp32 pair read as a carry word could carry
              a current epoch in its upper half.

One buffer is kept per (device, stream, kind) and grown when a launch needs
more; launches on different streams therefore never share one.

A bounded look-back wait that expires (a predecessor tile that never
published, ~1 s of polling) sets the sticky flag and the kernel finishes with
that tile's carry incomplete.  ``check()`` synchronises, reads every lookback
workspace's flag (and the no-allocation scratch's) and raises ``TssmError``
if one is set.
"""
from __future__ import annotations

import ctypes
import threading

import torch

from . import _lib

LOOKBACK = "lookback"
SSD = "ssd"
KINDS = (LOOKBACK, SSD)

_lock = threading.Lock()
_cache: dict[tuple[int, int, str], torch.Tensor] = {}


def _dev_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def get(device: torch.device, stream: int, nbytes: int, kind: str = LOOKBACK) -> torch.Tensor:
    if kind not in KINDS:
        raise ValueError(f"unknown workspace kind {kind!r}")
    key = (_dev_index(device), stream, kind)
    with _lock:
        buf = _cache.get(key)
        if buf is None or buf.numel() < nbytes:
            # zero-filled on the current stream, so it is ordered before the scan
            buf = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
            _cache[key] = buf
        return buf


def error_flag(buf: torch.Tensor, clear: bool = True) -> int:
    """Sticky look-back timeout flag of one workspace (a synchronous read)."""
    out = ctypes.c_int(0)
    _lib.call("tssm_workspace_error", buf.data_ptr(), int(clear), ctypes.byref(out))
    return out.value


def check(device: torch.device | int | None = None, clear: bool = True) -> None:
    """Synchronise and raise ``TssmError`` if a look-back wait expired.

    Reads the sticky flag of every lookback workspace (of ``device``, or of
    every device when None) and of the no-allocation entry point's scratch on
    those devices and the current one.  A set flag means that some launch on
    that workspace since the last check produced outputs without its full
    carry; the flag is cleared (with ``clear``) before raising, so later
    launches can be checked afresh.
    """
    want = None if device is None else (device if isinstance(device, int) else
                                        _dev_index(torch.device(device)))
    with _lock:
        items = [(k, b) for k, b in _cache.items() if k[2] == LOOKBACK and
                 (want is None or k[0] == want)]
    bad = []
    for (dev_idx, stream, _), buf in items:
        torch.cuda.synchronize(dev_idx)
        if error_flag(buf, clear):
            bad.append(f"device {dev_idx} stream {stream:#x}")
    devs = {k[0] for k, _ in items}
    if want is not None:
        devs.add(want)
    elif torch.cuda.is_initialized():
        devs.add(torch.cuda.current_device())
    for dev_idx in sorted(devs):
        with torch.cuda.device(dev_idx):
            torch.cuda.synchronize(dev_idx)
            out = ctypes.c_int(0)
            _lib.call("tssm_workspace_error", None, int(clear), ctypes.byref(out))
            if out.value:
                bad.append(f"device {dev_idx} no-allocation scratch")
    if bad:
        raise _lib.TssmError(
            "a bounded look-back wait expired (a predecessor tile never published its carry); "
            "outputs of fused scans since the last check are invalid: " + ", ".join(bad))


def clear() -> None:
    with _lock:
        _cache.clear()
