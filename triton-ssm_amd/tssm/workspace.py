"""Device workspaces of the fused scans, and the look-back error check.

A workspace is a zero-filled device buffer that one stream reuses across
launches.  Two kinds never share a buffer:

``lookback``  the single-pass scans (multihead, selective, elementwise):
              tagged carry words {value, epoch} after a 256-byte header whose
              first word is a sticky error flag.  The epoch advances on every
              launch, so stale words never match and no per-launch clearing
              is needed -- provided nothing but tagged words is ever written
              there.
``ssd``       raw fp32 data: the SSD passes' chunk states and decays, and the
              three-pass selective scan's chunk states, dt sums and produced
              dt.  Kept apart because an arbitrary fp32 pair read as a carry
              word could carry a current epoch in its upper half.

One buffer is kept per (device, stream, kind) and grown when a launch needs
more; launches on different streams therefore never share one.

A bounded look-back wait that expires (a predecessor tile that never
published, ~1 s of polling) sets the sticky flag and the kernel finishes with
that tile's carry incomplete.  Two ways report it:

* without a synchronisation: every lookback workspace gets a pinned host int
  attached (``tssm_workspace_attach_host_flag``) that the failing kernel also
  sets.  ``get()`` -- called by every fused launch before it launches -- reads
  that int for the buffer it hands out and raises ``TssmError`` if a launch
  on it has failed since (the int lands when that kernel finishes, so the
  report comes with the first launch on the workspace after it);
* ``check()`` synchronises, reads every lookback workspace's flag (and the
  no-allocation scratch's) and raises ``TssmError`` if one is set.
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
# pinned host int per lookback workspace (same key), set by a failing kernel
_host_flags: dict[tuple[int, int, str], torch.Tensor] = {}

_EXPIRED = ("a bounded look-back wait expired (a predecessor tile never published its "
            "carry); outputs of fused scans since the last check are invalid: ")


def _dev_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def _raise_if_flagged(key) -> None:
    """Host-side poll of a workspace's attached flag (no synchronisation)."""
    flag = _host_flags.get(key)
    if flag is not None and int(flag[0]) != 0:
        flag[0] = 0
        raise _lib.TssmError(_EXPIRED + f"device {key[0]} stream {key[1]:#x} (reported by the "
                             "workspace's host flag; the device word stays set for check())")


def get(device: torch.device, stream: int, nbytes: int, kind: str = LOOKBACK) -> torch.Tensor:
    if kind not in KINDS:
        raise ValueError(f"unknown workspace kind {kind!r}")
    key = (_dev_index(device), stream, kind)
    with _lock:
        _raise_if_flagged(key)
        buf = _cache.get(key)
        if buf is None or buf.numel() < nbytes:
            # zero-filled on the current stream, so it is ordered before the scan
            buf = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
            _cache[key] = buf
            if kind == LOOKBACK:
                flag = _host_flags.get(key)
                if flag is None:
                    flag = torch.zeros(1, dtype=torch.int32, pin_memory=True)
                    _host_flags[key] = flag
                # the header's flag address is written by a synchronous copy,
                # after the zero fill above
                _lib.call("tssm_workspace_attach_host_flag", buf.data_ptr(), flag.data_ptr())
        return buf


def host_flag(device: torch.device, stream: int) -> torch.Tensor | None:
    """The pinned int attached to the lookback workspace of (device, stream)."""
    return _host_flags.get((_dev_index(device), stream, LOOKBACK))


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
    with _lock:
        for k, _ in items:
            flag = _host_flags.get(k)
            if flag is not None:
                flag[0] = 0   # reported here, with the device word
    if bad:
        raise _lib.TssmError(_EXPIRED + ", ".join(bad))


def clear() -> None:
    with _lock:
        _cache.clear()
        _host_flags.clear()
