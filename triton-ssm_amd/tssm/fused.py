"""Fused single-pass entry points (API additions beyond the reference's
kernel set; the reference's own recurrence and discretization, one launch).

``multihead_ssm_forward``  DIAG multihead scan: multihead_ssm_kernel.py's three
                           phases (:20-187) fused, discretization in the load
                           stage, decoupled look-back across chunks.
"""
from __future__ import annotations

import torch

from . import _lib, workspace
from .launch import as_f32, dcode, need_gpu, ptr, stream_handle

_DISC = {"euler": _lib.DISC_EULER, "zoh": _lib.DISC_ZOH}


def _disc_code(disc: str) -> int:
    try:
        return _DISC[disc]
    except KeyError:
        raise ValueError(f"disc must be 'euler' or 'zoh', got {disc!r}") from None


def _inner_unit(t: torch.Tensor, what: str) -> None:
    if t.stride(-1) != 1:
        raise ValueError(f"{what}: innermost dimension must be contiguous")


def multihead_ssm_forward(u, A_log, B, C, dt, D=None, *, chunk=128, disc="euler", h0=None,
                          return_state=False, out=None):
    """Fused DIAG multihead selective scan.

    u      [Bsz, L, nh*hd]  float32 / bfloat16 / float16
    A_log  [nh, hd] (per channel) or [nh] (per head); stores log(-a)
    B, C   [Bsz, L, nh, hd] same dtype as u
    dt     [Bsz, L, nh]     (read as float32)
    D      [nh*hd] or None  skip weights (y += sum_p D*u)
    h0     [Bsz, nh, hd] float32 or None (zero initial state)
    disc   'euler' (Bbar = dt*B, multihead_ssm_kernel.py:73) or 'zoh'
           (Bbar = expm1(dt*a)/a * B, discretize_kernel.py:50-54)

    For each (b, head, channel p): h_t = exp(dt a_p) h_{t-1} + Bbar_t u_t,
    y[b,t,head*hd + q] = sum_p C_t[p] h_t[p] + sum_p D[p] u_t[p] for every q
    (the per-head value broadcast over the head's channels,
    multihead_ssm_kernel.py:168-187).  Returns y (dtype of u) and, with
    ``return_state``, the final state [Bsz, nh, hd] float32.
    """
    for t, w in ((u, "u"), (B, "B"), (C, "C"), (dt, "dt"), (A_log, "A_log")):
        need_gpu(t, w)
    if u.dim() != 3 or B.dim() != 4 or C.shape != B.shape or dt.dim() != 3:
        raise ValueError("expected u [Bsz,L,nh*hd], B/C [Bsz,L,nh,hd], dt [Bsz,L,nh]")
    Bsz, L, nh, hd = B.shape
    if u.shape != (Bsz, L, nh * hd) or dt.shape != (Bsz, L, nh):
        raise ValueError(f"shape mismatch: u {tuple(u.shape)}, B {tuple(B.shape)}, "
                         f"dt {tuple(dt.shape)}")
    if B.dtype != u.dtype or C.dtype != u.dtype:
        raise TypeError("u, B and C must share one dtype")
    code = dcode(u, "u")
    a_per_head = A_log.dim() == 1
    if A_log.shape not in ((nh,), (nh, hd)):
        raise ValueError(f"A_log must be [nh] or [nh, hd], got {tuple(A_log.shape)}")
    A_log = as_f32(A_log, "A_log").contiguous()
    dt = as_f32(dt, "dt")
    for t, w in ((u, "u"), (B, "B"), (C, "C")):
        _inner_unit(t, w)
    if D is not None:
        need_gpu(D, "D")
        if D.numel() != nh * hd:
            raise ValueError("D must have nh*hd elements")
        D = as_f32(D, "D").contiguous()
    if h0 is not None:
        need_gpu(h0, "h0")
        if tuple(h0.shape) != (Bsz, nh, hd):
            raise ValueError("h0 must be [Bsz, nh, hd]")
        h0 = as_f32(h0, "h0").contiguous()
    y = torch.empty_like(u, memory_format=torch.contiguous_format) if out is None else out
    need_gpu(y, "out")
    if y.shape != u.shape or y.dtype != u.dtype:
        raise ValueError("out must match u in shape and dtype")
    _inner_unit(y, "out")
    h_last = torch.empty(Bsz, nh, hd, device=u.device, dtype=torch.float32) if return_state else None

    L_ = _lib.lib()
    nbytes = L_.tssm_mh_scan_workspace_bytes(Bsz, L, nh, hd, int(chunk))
    if nbytes < 0:
        raise ValueError(f"unsupported head_dim {hd} (multiple of 8, <= 128) or chunk {chunk}")
    stream = stream_handle(u)
    ws = workspace.get(u.device, stream, nbytes)
    _lib.call("tssm_mh_scan_fused", code, _disc_code(disc), u.data_ptr(), A_log.data_ptr(),
              B.data_ptr(), C.data_ptr(), dt.data_ptr(), ptr(D), ptr(h0), y.data_ptr(),
              ptr(h_last), Bsz, L, nh, hd, int(a_per_head), u.stride(0), u.stride(1),
              B.stride(0), B.stride(1), B.stride(2), C.stride(0), C.stride(1), C.stride(2),
              dt.stride(0), dt.stride(1), dt.stride(2), y.stride(0), y.stride(1), int(chunk),
              ws.data_ptr(), ws.numel(), stream)
    return (y, h_last) if return_state else y
