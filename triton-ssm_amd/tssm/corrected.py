"""Opt-in "corrected" interpolation: per-feature neighbours with observed
values kept (the intent stated at fused_interp_kernel.py:49-50).  The
reference's behaviour -- neighbours decided per FTILE-wide tile, observed
values overwritten whenever a neighbour exists -- stays the default of every
reference-named kernel; these entry points exist next to it and change
results on purpose.

* ``time_aware_interp_corrected(V, M, tau, K=10)``: for each (b, t, f) an
  observed value (M > 0.5) is kept; otherwise the nearest steps within K on
  each side where feature f is observed give the value, with the reference's
  weights w = (tau_t - tau_p) / (tau_n - tau_p) clipped to [0, 1] (0.5 when the
  gap is <= 1e-9) and its one-sided fills; no neighbour: V[t] as stored.
* ``streaming_interp_step_corrected(...)``: the ring insert and race-free head
  update of streaming_interp_then_ssm_kernel, then per feature an observed new
  value is kept and an unobserved one is forward-filled from the most recent
  of the previous KRING-1 slots where that feature was observed (a causal step
  has no later neighbour to weight against), then the in-place step
  h = Abar h + Bbar v, y = C h + D v.
"""
from __future__ import annotations

import torch

from . import _lib
from .launch import dcode, extent, need_gpu, span, stream_handle


def time_aware_interp_corrected(V: torch.Tensor, M: torch.Tensor, tau: torch.Tensor, K: int = 10,
                                out: torch.Tensor | None = None) -> torch.Tensor:
    """V, M [B,T,F] (float32/bfloat16/float16; M any float dtype), tau [B,T];
    returns Vhat [B,T,F] in V's dtype."""
    for t, w in ((V, "V"), (M, "M"), (tau, "tau")):
        need_gpu(t, w)
    if V.dim() != 3 or M.shape != V.shape or tau.dim() != 2 or tuple(tau.shape) != V.shape[:2]:
        raise ValueError("expected V, M [B,T,F] and tau [B,T]")
    K = int(K)
    if not 0 <= K <= 449:   # the workgroup's LDS holds flags of 64 + 2K rows
        raise ValueError("K must be in [0, 449]")
    Bsz, T, F = V.shape
    if V.stride(2) != 1 or M.stride(2) != 1:
        raise ValueError("V and M need a unit feature stride")
    if out is None:
        out = torch.empty_like(V, memory_format=torch.contiguous_format)
    need_gpu(out, "out")
    if out.shape != V.shape or out.dtype != V.dtype or out.stride(2) != 1:
        raise ValueError("out must match V in shape and dtype, with a unit feature stride")
    if Bsz * T * F == 0:
        return out
    extent(V, span([(Bsz, V.stride(0)), (T, V.stride(1)), (F, 1)]), "V")
    extent(M, span([(Bsz, M.stride(0)), (T, M.stride(1)), (F, 1)]), "M")
    extent(tau, span([(Bsz, tau.stride(0)), (T, tau.stride(1))]), "tau")
    extent(out, span([(Bsz, out.stride(0)), (T, out.stride(1)), (F, 1)]), "out")
    _lib.call("tssm_time_aware_interp_corrected", dcode(V, "V"), dcode(M, "M"), dcode(tau, "tau"),
              V.data_ptr(), M.data_ptr(), tau.data_ptr(), out.data_ptr(), Bsz, T, F,
              V.stride(0), V.stride(1), M.stride(0), M.stride(1), tau.stride(0), tau.stride(1),
              out.stride(0), out.stride(1), K, stream_handle(V))
    return out


def streaming_interp_step_corrected(ring_V, ring_M, ring_tau, ring_head, v_new, m_new, tau_new,
                                    h, Abar, Bbar, C, D, y) -> None:
    """ring_V/ring_M [S,KRING,H] f32, ring_tau [S,KRING] f32, ring_head [S]
    int32 (all updated in place), v_new/m_new [S,H] (m_new with v_new's batch
    stride), tau_new [S], h [S,H] (updated in place), Abar/Bbar/D [H], C [S,H],
    y [S,H] (v_new's batch stride) -- the layout of
    streaming_interp_then_ssm_kernel."""
    names = ("ring_V", "ring_M", "ring_tau", "v_new", "m_new", "tau_new", "h", "Abar", "Bbar", "C",
             "D", "y")
    ts = dict(zip(names, (ring_V, ring_M, ring_tau, v_new, m_new, tau_new, h, Abar, Bbar, C, D,
                          y)))
    for k, t in ts.items():
        need_gpu(t, k)
        if t.dtype != torch.float32:
            raise TypeError(f"{k} must be float32")
    need_gpu(ring_head, "ring_head")
    if ring_head.dtype != torch.int32:
        raise TypeError("ring_head must be int32")
    if ring_V.dim() != 3 or ring_M.shape != ring_V.shape:
        raise ValueError("ring_V, ring_M must be [S, KRING, H]")
    S, KR, H = ring_V.shape
    if v_new.shape != (S, H) or m_new.shape != (S, H) or h.shape != (S, H) or C.shape != (S, H):
        raise ValueError("v_new, m_new, h, C must be [S, H]")
    if tuple(ring_tau.shape) != (S, KR) or tuple(tau_new.shape) != (S,) or \
            tuple(ring_head.shape) != (S,):
        raise ValueError("ring_tau [S, KRING], tau_new and ring_head [S] expected")
    if ring_V.stride() != ring_M.stride() or m_new.stride(0) != v_new.stride(0) or \
            y.stride(0) != v_new.stride(0):
        raise ValueError("ring_M must share ring_V's strides; m_new and y v_new's batch stride")
    for k in ("ring_V", "v_new", "m_new", "h", "C", "y"):
        if ts[k].stride(-1) != 1:
            raise ValueError(f"{k}: unit feature stride expected")
    for k in ("Abar", "Bbar", "D"):
        if ts[k].numel() < H or ts[k].stride(-1) != 1:
            raise ValueError(f"{k}: H contiguous values expected")
    if ring_tau.stride(1) != 1 or ring_tau.stride(0) != KR:
        raise ValueError("ring_tau must be contiguous [S, KRING]")
    if tau_new.stride(0) != 1 or ring_head.stride(0) != 1:
        raise ValueError("tau_new and ring_head must be contiguous")
    if S == 0 or H == 0:
        return
    extent(ring_V, span([(S, ring_V.stride(0)), (KR, ring_V.stride(1)), (H, 1)]), "ring_V")
    extent(ring_M, span([(S, ring_M.stride(0)), (KR, ring_M.stride(1)), (H, 1)]), "ring_M")
    extent(ring_tau, S * KR - 1, "ring_tau")
    for k in ("v_new", "m_new", "y"):
        extent(ts[k], span([(S, v_new.stride(0)), (H, 1)]), k)
    extent(h, span([(S, h.stride(0)), (H, 1)]), "h")
    extent(C, span([(S, C.stride(0)), (H, 1)]), "C")
    extent(tau_new, S - 1, "tau_new")
    extent(ring_head, S - 1, "ring_head")
    _lib.call("tssm_stream_interp_step_corrected", ring_V.data_ptr(), ring_M.data_ptr(),
              ring_tau.data_ptr(), ring_head.data_ptr(), v_new.data_ptr(), m_new.data_ptr(),
              tau_new.data_ptr(), h.data_ptr(), Abar.data_ptr(), Bbar.data_ptr(), C.data_ptr(),
              D.data_ptr(), y.data_ptr(), S, H, ring_V.stride(0), ring_V.stride(1),
              v_new.stride(0), h.stride(0), C.stride(0), KR, stream_handle(v_new))
