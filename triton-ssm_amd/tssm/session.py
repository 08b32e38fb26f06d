"""Streaming session state: save and restore (format ``TSSMSES1``).

A streaming caller carries state between steps: the recurrent state ``h``
(streaming_inference_kernel.py:9, [B, H] fp32, or bf16 for the bf16 step
kernel :41-71; the SSD stream state [S, H, P, N] fp32 of ``ssd_stream_step``)
and, for the ring kernel (:75-80), the ring buffers ``ring_V``/``ring_M``
[B, KRING, H] fp32, ``ring_tau`` [B, KRING] fp32 and ``ring_head`` [B] int32.
The reference keeps these only in device memory.  This module is their
on-disk and wire form, so a stream can stop and resume bit for bit.

File layout (little-endian):

    0    8 B   magic b"TSSMSES1"
    8    u32   format version (1)
    12   u32   number of tensors n
    16   u64   file size in bytes
    24   u32   metadata length m
    28   u32   CRC-32 of bytes [32, 32 + 112 n + m) (tensor records + metadata)
    32   n tensor records of 112 bytes:
           name      32 B UTF-8, NUL-padded (1..32 bytes, unique)
           dtype     u32  0 f32, 1 bf16, 2 f16 (the library's codes), 3 i32, 4 u8
           ndim      u32  0..6
           shape     6 x i64 (unused dims 0)
           offset    u64  from the file start, a multiple of 64
           nbytes    u64  = prod(shape) * itemsize
           crc32     u32  of the data bytes
           reserved  u32  0
    32 + 112 n   metadata: a UTF-8 JSON object (m bytes)
    data blocks, C-contiguous, at their records' offsets (ascending, no overlap)

Large device tensors are moved in bounded pieces (``_PIECE`` bytes) in both
directions, so saving a 4 GiB SSD state does not hold a second host copy.
"""
from __future__ import annotations

import io
import json
import os
import struct
import zlib
from typing import BinaryIO, Mapping

import numpy as np
import torch

MAGIC = b"TSSMSES1"
VERSION = 1
_HEAD = struct.Struct("<8sIIQII")        # 32 bytes
_REC = struct.Struct("<32sII6qQQII")     # 112 bytes
_ALIGN = 64
_MAXDIM = 6
_PIECE = 64 << 20

_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.int32: 3, torch.uint8: 4}
_DTYPES = {v: k for k, v in _CODES.items()}
# host views of each dtype as raw integers of the same width (bf16 has no numpy type)
_RAW = {torch.float32: torch.int32, torch.bfloat16: torch.int16, torch.float16: torch.int16,
        torch.int32: torch.int32, torch.uint8: torch.uint8}
_NP = {torch.int32: np.int32, torch.int16: np.int16, torch.uint8: np.uint8}

assert _HEAD.size == 32 and _REC.size == 112


class SessionFormatError(ValueError):
    """The bytes are not a valid session of this format version."""


def _align(n: int) -> int:
    return (n + _ALIGN - 1) // _ALIGN * _ALIGN


def _check_tensor(name: str, t) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if t.dtype not in _CODES:
        raise TypeError(f"{name}: unsupported dtype {t.dtype}")
    if t.dim() > _MAXDIM:
        raise ValueError(f"{name}: at most {_MAXDIM} dimensions")
    raw = name.encode("utf-8")
    if not 1 <= len(raw) <= 32 or b"\0" in raw:
        raise ValueError(f"tensor name {name!r}: 1..32 UTF-8 bytes, no NUL")
    return t


def _pieces(t: torch.Tensor):
    """Host byte pieces of t (C order), at most _PIECE bytes each."""
    flat = t.detach().contiguous().view(-1).view(_RAW[t.dtype])
    step = max(1, _PIECE // flat.element_size())
    for i in range(0, flat.numel(), step):
        yield flat[i:i + step].cpu().numpy().tobytes()


def save(dst, tensors: Mapping[str, torch.Tensor], meta: Mapping | None = None) -> None:
    """Write ``tensors`` (and the JSON-serialisable ``meta``) to a path or a
    binary file object.  A path is written to a temporary file and renamed, so
    an interrupted save never leaves a partial session under that name."""
    items = [(k, _check_tensor(k, v)) for k, v in tensors.items()]
    metab = json.dumps(dict(meta or {}), sort_keys=True).encode("utf-8")
    n = len(items)
    pos = _align(_HEAD.size + n * _REC.size + len(metab))
    layout = []
    for name, t in items:
        nbytes = t.numel() * t.element_size()
        layout.append((name, t, pos, nbytes))
        pos = _align(pos + nbytes)
    size = pos
    if isinstance(dst, (str, os.PathLike)):
        tmp = os.fspath(dst) + ".tmp"
        with open(tmp, "wb") as f:
            _write(f, layout, metab, size)
            f.flush()
            os.fsync(f.fileno())
        os.replace(tmp, dst)
    else:
        _write(dst, layout, metab, size)


def _write(f: BinaryIO, layout, metab: bytes, size: int) -> None:
    table_pos = _HEAD.size
    # header and table are written last (the data CRCs come first); reserve them
    f.write(b"\0" * table_pos)
    f.write(b"\0" * (len(layout) * _REC.size))
    f.write(metab)
    written = table_pos + len(layout) * _REC.size + len(metab)
    recs = []
    for name, t, off, nbytes in layout:
        f.write(b"\0" * (off - written))
        crc = 0
        for piece in _pieces(t):
            crc = zlib.crc32(piece, crc)
            f.write(piece)
        written = off + nbytes
        shape = list(t.shape) + [0] * (_MAXDIM - t.dim())
        recs.append(_REC.pack(name.encode("utf-8"), _CODES[t.dtype], t.dim(), *shape, off, nbytes,
                              crc, 0))
    f.write(b"\0" * (size - written))
    table = b"".join(recs) + metab
    head = _HEAD.pack(MAGIC, VERSION, len(layout), size, len(metab), zlib.crc32(table))
    end = f.tell()
    f.seek(end - size)
    f.write(head)
    f.write(b"".join(recs))
    f.seek(end)


def dumps(tensors: Mapping[str, torch.Tensor], meta: Mapping | None = None) -> bytes:
    """The session as bytes (the wire form)."""
    buf = io.BytesIO()
    save(buf, tensors, meta)
    return buf.getvalue()


def load(src, device=None):
    """Read a session from a path, a binary file object or bytes.  Returns
    ``(tensors, meta)``; tensors are placed on ``device`` (default: CPU).
    Raises SessionFormatError on any inconsistency (magic, version, sizes,
    offsets, CRCs)."""
    if isinstance(src, (bytes, bytearray, memoryview)):
        return _read(io.BytesIO(bytes(src)), len(src), device)
    if isinstance(src, (str, os.PathLike)):
        with open(src, "rb") as f:
            return _read(f, os.fstat(f.fileno()).st_size, device)
    start = src.tell()
    src.seek(0, io.SEEK_END)
    avail = src.tell() - start
    src.seek(start)
    return _read(src, avail, device)


def loads(data: bytes, device=None):
    return load(data, device)


def _read(f: BinaryIO, avail: int, device):
    base = f.tell()
    head = f.read(_HEAD.size)
    if len(head) != _HEAD.size:
        raise SessionFormatError("truncated header")
    magic, version, n, size, mlen, tcrc = _HEAD.unpack(head)
    if magic != MAGIC:
        raise SessionFormatError("not a TSSM session (bad magic)")
    if version != VERSION:
        raise SessionFormatError(f"unsupported session format version {version}")
    if size > avail:
        raise SessionFormatError(f"truncated session: {avail} of {size} bytes")
    table_end = _HEAD.size + n * _REC.size + mlen
    if table_end > size:
        raise SessionFormatError("tensor table runs past the end of the session")
    table = f.read(n * _REC.size + mlen)
    if zlib.crc32(table) != tcrc:
        raise SessionFormatError("tensor table checksum mismatch")
    try:
        meta = json.loads(table[n * _REC.size:].decode("utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as e:
        raise SessionFormatError(f"bad metadata: {e}") from None
    if not isinstance(meta, dict):
        raise SessionFormatError("metadata is not a JSON object")
    recs = []
    for i in range(n):
        name, code, ndim, *rest = _REC.unpack_from(table, i * _REC.size)
        shape, (off, nbytes, crc, _) = rest[:_MAXDIM], rest[_MAXDIM:]
        try:
            name = name.rstrip(b"\0").decode("utf-8")
        except UnicodeDecodeError:
            raise SessionFormatError(f"record {i}: bad name") from None
        if code not in _DTYPES or ndim > _MAXDIM:
            raise SessionFormatError(f"{name}: bad dtype code {code} or ndim {ndim}")
        dtype = _DTYPES[code]
        shape = tuple(int(s) for s in shape[:ndim])
        if any(s < 0 for s in shape):
            raise SessionFormatError(f"{name}: negative dimension")
        if int(np.prod(shape, dtype=np.int64)) * torch.empty(0, dtype=dtype).element_size() != nbytes:
            raise SessionFormatError(f"{name}: byte count does not match its shape")
        recs.append((name, dtype, shape, off, nbytes, crc))
    names = [r[0] for r in recs]
    if len(set(names)) != len(names):
        raise SessionFormatError("duplicate tensor names")
    prev = _align(table_end)
    for name, _, _, off, nbytes, _ in sorted(recs, key=lambda r: r[3]):
        if off % _ALIGN or off < prev or off + nbytes > size:
            raise SessionFormatError(f"{name}: data block out of place")
        prev = off + nbytes
    out = {}
    for name, dtype, shape, off, nbytes, crc in recs:
        t = torch.empty(shape, dtype=dtype, device=device)
        flat = t.view(-1).view(_RAW[dtype])
        f.seek(base + off)
        got, pos = 0, 0
        step = max(1, _PIECE // flat.element_size())
        while pos < flat.numel():
            cnt = min(step, flat.numel() - pos)
            piece = f.read(cnt * flat.element_size())
            if len(piece) != cnt * flat.element_size():
                raise SessionFormatError(f"{name}: truncated data")
            got = zlib.crc32(piece, got)
            host = torch.from_numpy(np.frombuffer(piece, dtype=_NP[flat.dtype]).copy())
            flat[pos:pos + cnt].copy_(host)
            pos += cnt
        if got != crc:
            raise SessionFormatError(f"{name}: data checksum mismatch")
        out[name] = t
    f.seek(base + size)
    return out, meta


class RingSession:
    """State of ``streaming_interp_then_ssm_kernel`` (streaming_inference_kernel.py:75-156)
    for B streams of H features with a ring of KRING = K+1 observations, plus
    ``step`` to advance it and ``save``/``load`` to persist it."""

    KIND = "ring"
    FIELDS = ("ring_V", "ring_M", "ring_tau", "ring_head", "h")

    def __init__(self, B: int, H: int, K: int, block_h: int = 128, device=None):
        if B <= 0 or H <= 0 or K < 0 or block_h <= 0:
            raise ValueError("B, H, BLOCK_H must be positive and K non-negative")
        self.B, self.H, self.K, self.block_h = int(B), int(H), int(K), int(block_h)
        kr = self.K + 1
        f32 = dict(dtype=torch.float32, device=device)
        self.ring_V = torch.zeros(B, kr, H, **f32)
        self.ring_M = torch.zeros(B, kr, H, **f32)
        self.ring_tau = torch.zeros(B, kr, **f32)
        self.ring_head = torch.zeros(B, dtype=torch.int32, device=device)
        self.h = torch.zeros(B, H, **f32)

    @property
    def device(self):
        return self.h.device

    def step(self, v_new, m_new, tau_new, Abar, Bbar, C, D, y=None):
        """Insert one observation per stream and advance the state; returns y [B, H]."""
        from streaming_inference_kernel import streaming_interp_then_ssm_kernel
        B, H = self.B, self.H
        y = torch.empty(B, H, dtype=torch.float32, device=self.device) if y is None else y
        streaming_interp_then_ssm_kernel[(B, -(-H // self.block_h))](
            self.ring_V, self.ring_M, self.ring_tau, self.ring_head, v_new, m_new, tau_new,
            self.h, Abar, Bbar, C, D, y, B, H, self.K, self.ring_V.stride(0),
            self.ring_V.stride(1), self.ring_V.stride(2), v_new.stride(0), v_new.stride(1),
            self.h.stride(0), self.h.stride(1), C.stride(0), C.stride(1),
            BLOCK_H=self.block_h, KRING=self.K + 1)
        return y

    def state_dict(self):
        return {k: getattr(self, k) for k in self.FIELDS}

    def meta(self):
        return {"kind": self.KIND, "B": self.B, "H": self.H, "K": self.K,
                "BLOCK_H": self.block_h}

    def save(self, dst) -> None:
        if self.device.type == "cuda":
            torch.cuda.synchronize(self.device)
        save(dst, self.state_dict(), self.meta())

    def dumps(self) -> bytes:
        buf = io.BytesIO()
        self.save(buf)
        return buf.getvalue()

    @classmethod
    def load(cls, src, device=None) -> "RingSession":
        tensors, meta = load(src, device)
        if meta.get("kind") != cls.KIND:
            raise SessionFormatError(f"not a ring session (kind {meta.get('kind')!r})")
        try:
            s = cls.__new__(cls)
            s.B, s.H, s.K, s.block_h = (int(meta[k]) for k in ("B", "H", "K", "BLOCK_H"))
        except (KeyError, TypeError, ValueError):
            raise SessionFormatError("ring session metadata incomplete") from None
        want = {"ring_V": ((s.B, s.K + 1, s.H), torch.float32),
                "ring_M": ((s.B, s.K + 1, s.H), torch.float32),
                "ring_tau": ((s.B, s.K + 1), torch.float32),
                "ring_head": ((s.B,), torch.int32),
                "h": ((s.B, s.H), torch.float32)}
        for k, (shape, dtype) in want.items():
            t = tensors.get(k)
            if t is None or tuple(t.shape) != shape or t.dtype != dtype:
                raise SessionFormatError(f"ring session field {k}: missing or wrong shape/dtype")
            setattr(s, k, t)
        head = s.ring_head.cpu()
        if bool(((head < 0) | (head > s.K)).any()):
            raise SessionFormatError("ring_head outside [0, K]")
        return s
