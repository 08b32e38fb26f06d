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


def _ws(nbytes, t, what, kind=workspace.LOOKBACK):
    if nbytes < 0:
        raise ValueError(f"{what}: unsupported shape for the fused kernel")
    stream = stream_handle(t)
    return workspace.get(t.device, stream, nbytes, kind), stream


def ssd_scan_forward(x, dt, A_log, B, C, D=None, *, chunk=256, disc="zoh", h0=None,
                     return_state=False, out=None, fused=True):
    """SSD selective scan: one decay per head, state [P, N] per (batch, head).

    x      [Bsz, L, H, P]  float32 / bfloat16 / float16 (P <= 64)
    dt     [Bsz, L, H]     (read as float32)
    A_log  [H]             log(-a) per head
    B, C   [Bsz, L, H, N]  dtype of x, N in {8, 16, 32, 64}
    D      [H, P] / [H*P] or None
    h0     [Bsz, H, P, N] float32 or None

    h_t[p,n] = exp(dt_t a) h_{t-1}[p,n] + Bbar_t x_t[p] B_t[n];
    y_t[p] = sum_n C_t[n] h_t[p,n] + D[p] x_t[p].  Returns y (dtype of x)
    and, with ``return_state``, the final state [Bsz, H, P, N] float32.

    bf16 with P = 64, N = 16 and 256-step chunks runs in one launch
    (tssm_ssd_scan_fused: two sweeps per segment around a decoupled
    look-back) unless ``fused=False``, which keeps the three tile passes.
    """
    for t, w in ((x, "x"), (dt, "dt"), (A_log, "A_log"), (B, "B"), (C, "C")):
        need_gpu(t, w)
    if x.dim() != 4 or B.dim() != 4 or C.shape != B.shape or dt.dim() != 3:
        raise ValueError("expected x [Bsz,L,H,P], B/C [Bsz,L,H,N], dt [Bsz,L,H]")
    Bsz, L, H, P = x.shape
    N = B.shape[-1]
    if B.shape[:3] != (Bsz, L, H) or dt.shape != (Bsz, L, H) or A_log.shape != (H,):
        raise ValueError("shape mismatch between x, B, C, dt and A_log")
    if B.dtype != x.dtype or C.dtype != x.dtype:
        raise TypeError("x, B and C must share one dtype")
    code = dcode(x, "x")
    for t, w in ((x, "x"), (B, "B"), (C, "C")):
        _inner_unit(t, w)
    A_log = as_f32(A_log, "A_log").contiguous()
    dt = as_f32(dt, "dt")
    if D is not None:
        need_gpu(D, "D")
        if D.numel() != H * P:
            raise ValueError("D must have H*P elements")
        D = as_f32(D, "D").contiguous()
    if h0 is not None:
        need_gpu(h0, "h0")
        if tuple(h0.shape) != (Bsz, H, P, N):
            raise ValueError("h0 must be [Bsz, H, P, N]")
        h0 = as_f32(h0, "h0").contiguous()
    y = torch.empty(Bsz, L, H, P, device=x.device, dtype=x.dtype) if out is None else out
    need_gpu(y, "out")
    if y.shape != x.shape or y.dtype != x.dtype:
        raise ValueError("out must match x in shape and dtype")
    _inner_unit(y, "out")
    h_last = torch.empty(Bsz, H, P, N, device=x.device, dtype=torch.float32) if return_state else None
    L_ = _lib.lib()
    args = (x.data_ptr(), dt.data_ptr(), A_log.data_ptr(), B.data_ptr(), C.data_ptr(), ptr(D),
            ptr(h0), y.data_ptr(), ptr(h_last), Bsz, L, H, P, N, *x.stride()[:3], *dt.stride(),
            *B.stride()[:3], *C.stride()[:3], *y.stride()[:3], int(chunk))
    if fused and L_.tssm_ssd_scan_fused_supported(code, *args):
        # one launch with a decoupled look-back: a look-back workspace
        ws, stream = _ws(L_.tssm_ssd_scan_fused_workspace_bytes(Bsz, L, H, P, N, int(chunk)), x,
                         "ssd_scan")
        _lib.call("tssm_ssd_scan_fused", code, _disc_code(disc), *args, ws.data_ptr(),
                  ws.numel(), stream)
    else:
        ws, stream = _ws(L_.tssm_ssd_scan_workspace_bytes(Bsz, L, H, P, N, int(chunk)), x,
                         "ssd_scan", workspace.SSD)
        _lib.call("tssm_ssd_scan", code, _disc_code(disc), *args, ws.data_ptr(), ws.numel(),
                  stream)
    return (y, h_last) if return_state else y


def ssd_stream_step(x, dt, A_log, B, C, D, state, *, disc="zoh", out=None):
    """One streaming SSD step, the state updated in place in HBM.

    x [S, H, P], dt [S] (one per stream) or [S, H], A_log [H], B/C [S, H, N],
    D [H, P] / [H*P] or None, state [S, H, P, N], out [S, H, P] or None; all
    float32.  Returns y [S, H, P].  Shapes and dtypes are checked before the
    devices, and everything before the launch.
    """
    named = [(x, "x"), (dt, "dt"), (A_log, "A_log"), (B, "B"), (C, "C"), (state, "state")]
    if D is not None:
        named.append((D, "D"))
    if out is not None:
        named.append((out, "out"))
    for t, w in named:
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{w}: expected a torch.Tensor, got {type(t).__name__}")
        if t.dtype != torch.float32:
            raise TypeError(f"{w} must be float32")
    if x.dim() != 3:
        raise ValueError("x must be [S, H, P]")
    S, H, P = x.shape
    if B.dim() != 3:
        raise ValueError("B must be [S, H, N]")
    N = B.shape[-1]
    if B.shape != (S, H, N) or C.shape != (S, H, N) or tuple(state.shape) != (S, H, P, N):
        raise ValueError("expected B/C [S,H,N] and state [S,H,P,N]")
    if A_log.shape != (H,):
        raise ValueError(f"A_log must be [H] = [{H}], got {tuple(A_log.shape)}")
    if D is not None and tuple(D.shape) not in ((H, P), (H * P,)):
        raise ValueError(f"D must be [H, P] or [H*P], got {tuple(D.shape)}")
    if out is not None and tuple(out.shape) != (S, H, P):
        raise ValueError(f"out must be [S, H, P] = {(S, H, P)}, got {tuple(out.shape)}")
    if not state.is_contiguous():
        raise ValueError("state must be contiguous")
    if dt.shape == (S,):
        sdt = (dt.stride(0), 0)
    elif dt.shape == (S, H):
        sdt = dt.stride()
    else:
        raise ValueError("dt must be [S] or [S, H]")
    for t, w in ((x, "x"), (B, "B"), (C, "C")) + (((out, "out"),) if out is not None else ()):
        _inner_unit(t, w)
    for t, w in named:
        need_gpu(t, w)
    A_log = A_log.contiguous()
    if D is not None:
        D = D.contiguous()
    y = torch.empty(S, H, P, device=x.device, dtype=torch.float32) if out is None else out
    _lib.call("tssm_ssd_stream_step", _disc_code(disc), x.data_ptr(), dt.data_ptr(),
              A_log.data_ptr(), B.data_ptr(), C.data_ptr(), ptr(D), state.data_ptr(),
              y.data_ptr(), S, H, P, N, *sdt, *x.stride()[:2], *B.stride()[:2],
              *C.stride()[:2], *y.stride()[:2], stream_handle(x))
    return y


def _selective_scan_bcproj(x, dt, A_log, W_bc, D, disc, h0, return_state, dt_is_tau, out):
    """tssm_selective_scan_bcproj: B_t = x_t W_bc[:, :N], C_t = x_t W_bc[:, N:]
    formed inside the scan's first pass (fp32, Dc <= 256)."""
    for t, w in ((x, "x"), (dt, "dt"), (A_log, "A_log"), (W_bc, "bc_proj")):
        need_gpu(t, w)
    if x.dim() != 3 or x.dtype != torch.float32:
        raise ValueError("bc_proj: x must be float32 [Bsz, L, Dc]")
    Bsz, L, Dc = x.shape
    if W_bc.dim() != 2 or W_bc.shape[0] != Dc or W_bc.shape[1] % 2:
        raise ValueError("bc_proj: W_bc must be [Dc, 2N] (columns W_B then W_C)")
    N = W_bc.shape[1] // 2
    if A_log.shape != (Dc, N):
        raise ValueError("shape mismatch between x, bc_proj and A_log")
    if Dc > 256 or Dc % 4 or N not in (8, 16):
        raise ValueError("bc_proj needs Dc <= 256 (a multiple of 4) and N = 8 or 16")
    _inner_unit(x, "x")
    W_bc = as_f32(W_bc, "bc_proj")
    _inner_unit(W_bc, "bc_proj")
    A_log = as_f32(A_log, "A_log").contiguous()
    dt = as_f32(dt, "dt")
    if dt.shape == (Bsz, L):
        sdt = (dt.stride(0), dt.stride(1), 0)
    elif dt.shape == (Bsz, L, Dc) and not dt_is_tau:
        sdt = dt.stride()
    else:
        raise ValueError("dt must be [Bsz, L] (or [Bsz, L, Dc] without dt_is_tau)")
    if D is not None:
        need_gpu(D, "D")
        if D.numel() != Dc:
            raise ValueError("D must have Dc elements")
        D = as_f32(D, "D").contiguous()
    if h0 is not None:
        need_gpu(h0, "h0")
        if tuple(h0.shape) != (Bsz, Dc, N):
            raise ValueError("h0 must be [Bsz, Dc, N]")
        h0 = as_f32(h0, "h0").contiguous()
    y = torch.empty(Bsz, L, Dc, device=x.device, dtype=x.dtype) if out is None else out
    need_gpu(y, "out")
    if y.shape != x.shape or y.dtype != x.dtype:
        raise ValueError("out must match x in shape and dtype")
    _inner_unit(y, "out")
    h_last = torch.empty(Bsz, Dc, N, device=x.device, dtype=torch.float32) if return_state else None
    ws, stream = _ws(_lib.lib().tssm_selective_scan_bcproj_workspace_bytes(Bsz, L, Dc, N), x,
                     "selective_scan bc_proj", workspace.SSD)
    _lib.call("tssm_selective_scan_bcproj", _disc_code(disc), x.data_ptr(), dt.data_ptr(),
              int(bool(dt_is_tau)), A_log.data_ptr(), W_bc.data_ptr(), W_bc.stride(0), ptr(D),
              ptr(h0), y.data_ptr(), ptr(h_last), Bsz, L, Dc, N, x.stride(0), x.stride(1),
              *sdt, y.stride(0), y.stride(1), ws.data_ptr(), ws.numel(), stream)
    return (y, h_last) if return_state else y


def _selective_scan_xproj(x, A_log, xp, D, disc, h0, return_state, out):
    """tssm_selective_scan_xproj: dt, B and C formed from x inside the scan's
    first pass (fp32, Dc <= 256).  xp = (W_x [Dc, R + 2N], W_dt [R, Dc], bias
    [Dc], DT_MIN, DT_MAX)."""
    try:
        W_x, W_dt, bias, dt_min, dt_max = xp
    except (TypeError, ValueError):
        raise ValueError("x_proj must be (W_x, W_dt, bias, DT_MIN, DT_MAX)") from None
    for t, w in ((x, "x"), (A_log, "A_log"), (W_x, "W_x"), (W_dt, "W_dt"), (bias, "bias")):
        need_gpu(t, w)
    if x.dim() != 3 or x.dtype != torch.float32:
        raise ValueError("x_proj: x must be float32 [Bsz, L, Dc]")
    Bsz, L, Dc = x.shape
    if W_dt.dim() != 2 or W_dt.shape[1] != Dc:
        raise ValueError("x_proj: W_dt must be [R, Dc]")
    R = W_dt.shape[0]
    if W_x.dim() != 2 or W_x.shape[0] != Dc or (W_x.shape[1] - R) % 2 or W_x.shape[1] <= R:
        raise ValueError("x_proj: W_x must be [Dc, R + 2N] (columns dt_raw, B, C)")
    N = (W_x.shape[1] - R) // 2
    if A_log.shape != (Dc, N):
        raise ValueError("shape mismatch between x, x_proj and A_log")
    if Dc > 256 or Dc % 4 or N not in (8, 16) or R not in (16, 32, 48, 64):
        raise ValueError("x_proj needs Dc <= 256 (a multiple of 4), N = 8 or 16, R in 16..64 "
                         "(a multiple of 16)")
    if bias.numel() != Dc:
        raise ValueError("x_proj: bias must have Dc elements")
    _inner_unit(x, "x")
    W_x = as_f32(W_x, "W_x")
    _inner_unit(W_x, "W_x")
    W_dt = as_f32(W_dt, "W_dt")
    if W_dt.stride(1) != 1 or W_dt.stride(0) % 4:
        W_dt = W_dt.contiguous()
    bias = as_f32(bias, "bias").contiguous()
    A_log = as_f32(A_log, "A_log").contiguous()
    if D is not None:
        need_gpu(D, "D")
        if D.numel() != Dc:
            raise ValueError("D must have Dc elements")
        D = as_f32(D, "D").contiguous()
    if h0 is not None:
        need_gpu(h0, "h0")
        if tuple(h0.shape) != (Bsz, Dc, N):
            raise ValueError("h0 must be [Bsz, Dc, N]")
        h0 = as_f32(h0, "h0").contiguous()
    y = torch.empty(Bsz, L, Dc, device=x.device, dtype=x.dtype) if out is None else out
    need_gpu(y, "out")
    if y.shape != x.shape or y.dtype != x.dtype:
        raise ValueError("out must match x in shape and dtype")
    _inner_unit(y, "out")
    h_last = torch.empty(Bsz, Dc, N, device=x.device, dtype=torch.float32) if return_state else None
    ws, stream = _ws(_lib.lib().tssm_selective_scan_xproj_workspace_bytes(Bsz, L, Dc, N), x,
                     "selective_scan x_proj", workspace.SSD)
    _lib.call("tssm_selective_scan_xproj", _disc_code(disc), x.data_ptr(), A_log.data_ptr(),
              W_x.data_ptr(), W_x.stride(0), R, W_dt.data_ptr(), W_dt.stride(0),
              bias.data_ptr(), float(dt_min), float(dt_max), ptr(D), ptr(h0), y.data_ptr(),
              ptr(h_last), Bsz, L, Dc, N, x.stride(0), x.stride(1), y.stride(0), y.stride(1),
              ws.data_ptr(), ws.numel(), stream)
    return (y, h_last) if return_state else y


def selective_scan_forward(x, dt, A_log, B=None, C=None, D=None, *, chunk=128, disc="zoh",
                           h0=None, return_state=False, dt_is_tau=False, out=None, dt_proj=None,
                           bc_proj=None, x_proj=None):
    """Mamba-1 selective scan over lanes (channel d, state n).

    x      [Bsz, L, Dc]        float32 / bfloat16 / float16
    dt     [Bsz, L] (one per step, shared by the channels) or [Bsz, L, Dc];
           with ``dt_is_tau`` it holds timestamps and dt_t = tau_t - tau_{t-1},
           dt_0 = tau_0; with ``dt_proj`` it holds dt_raw [Bsz, L, rank]
    A_log  [Dc, N]             log(-a) per lane
    B, C   [Bsz, L, N]         dtype of x; N a multiple of 8, <= 128
    D      [Dc] or None;  h0 [Bsz, Dc, N] float32 or None
    dt_proj  (W [rank, Dc], bias [Dc], DT_MIN, DT_MAX) or None: dt is produced
           in the scan's load stage as clamp(softplus(dt_raw @ W + bias),
           DT_MIN, DT_MAX) -- dt_project_softplus_kernel
           (discretize_kernel.py:166-213) fused into the scan; rank <= 64
    bc_proj  W_bc [Dc, 2N] or None (then B and C are None): B_t = x_t W_bc[:, :N]
           and C_t = x_t W_bc[:, N:] (the input projection's B and C columns)
           are formed inside the scan (fp32, Dc <= 256, N = 8 or 16)
    x_proj  (W_x [Dc, R + 2N], W_dt [R, Dc], bias [Dc], DT_MIN, DT_MAX) or None
           (then dt, B and C are None): the whole input projection in the scan,
           x_dbl = x @ W_x split into dt_raw, B, C and dt = clamp(softplus(
           dt_raw @ W_dt + bias), DT_MIN, DT_MAX) (fp32, Dc <= 256, N = 8 or
           16, R = 16, 32, 48 or 64)

    h_t[d,n] = exp(dt_t a[d,n]) h_{t-1}[d,n] + Bbar_t[d,n] B_t[n] x_t[d];
    y_t[d] = sum_n C_t[n] h_t[d,n] + D[d] x_t[d].
    """
    if x_proj is not None:
        if dt is not None or B is not None or C is not None or dt_proj is not None \
                or bc_proj is not None:
            raise ValueError("x_proj replaces dt, B and C (pass None for them)")
        return _selective_scan_xproj(x, A_log, x_proj, D, disc, h0, return_state, out)
    if bc_proj is not None:
        if B is not None or C is not None or dt_proj is not None:
            raise ValueError("bc_proj replaces B and C (and does not combine with dt_proj)")
        return _selective_scan_bcproj(x, dt, A_log, bc_proj, D, disc, h0, return_state,
                                      dt_is_tau, out)
    if B is None or C is None:
        raise ValueError("B and C are required unless bc_proj is given")
    for t, w in ((x, "x"), (dt, "dt"), (A_log, "A_log"), (B, "B"), (C, "C")):
        need_gpu(t, w)
    if x.dim() != 3 or B.dim() != 3 or C.shape != B.shape:
        raise ValueError("expected x [Bsz,L,Dc] and B/C [Bsz,L,N]")
    Bsz, L, Dc = x.shape
    N = B.shape[-1]
    if B.shape[:2] != (Bsz, L) or A_log.shape != (Dc, N):
        raise ValueError("shape mismatch between x, B, C and A_log")
    if B.dtype != x.dtype or C.dtype != x.dtype:
        raise TypeError("x, B and C must share one dtype")
    code = dcode(x, "x")
    for t, w in ((x, "x"), (B, "B"), (C, "C")):
        _inner_unit(t, w)
    dt = as_f32(dt, "dt")
    proj = None
    if dt_proj is not None:
        if dt_is_tau:
            raise ValueError("dt_proj and dt_is_tau are exclusive")
        W, bias, dt_min, dt_max = dt_proj
        need_gpu(W, "W")
        need_gpu(bias, "bias")
        if dt.dim() != 3 or dt.shape[:2] != (Bsz, L):
            raise ValueError("with dt_proj, dt holds dt_raw [Bsz, L, rank]")
        rank = dt.shape[2]
        if W.shape != (rank, Dc) or bias.shape != (Dc,):
            raise ValueError(f"dt_proj: W must be [rank, Dc] = {(rank, Dc)} and bias [Dc]")
        if not 1 <= rank <= 64:
            raise ValueError("dt_proj: rank must be in 1..64")
        if not float(dt_min) <= float(dt_max):
            raise ValueError("dt_proj: DT_MIN must not exceed DT_MAX")
        _inner_unit(dt, "dt_raw")
        W = as_f32(W, "W")
        _inner_unit(W, "W")
        proj = (W, as_f32(bias, "bias").contiguous(), float(dt_min), float(dt_max), rank)
    elif dt.shape == (Bsz, L):
        sdt = (dt.stride(0), dt.stride(1), 0)
    elif dt.shape == (Bsz, L, Dc) and not dt_is_tau:
        sdt = dt.stride()
    else:
        raise ValueError("dt must be [Bsz, L] (or [Bsz, L, Dc] without dt_is_tau)")
    A_log = as_f32(A_log, "A_log").contiguous()
    if D is not None:
        need_gpu(D, "D")
        if D.numel() != Dc:
            raise ValueError("D must have Dc elements")
        D = as_f32(D, "D").contiguous()
    if h0 is not None:
        need_gpu(h0, "h0")
        if tuple(h0.shape) != (Bsz, Dc, N):
            raise ValueError("h0 must be [Bsz, Dc, N]")
        h0 = as_f32(h0, "h0").contiguous()
    y = torch.empty(Bsz, L, Dc, device=x.device, dtype=x.dtype) if out is None else out
    need_gpu(y, "out")
    if y.shape != x.shape or y.dtype != x.dtype:
        raise ValueError("out must match x in shape and dtype")
    _inner_unit(y, "out")
    h_last = torch.empty(Bsz, Dc, N, device=x.device, dtype=torch.float32) if return_state else None
    L_ = _lib.lib()
    # the three-pass path writes raw fp32 chunk states (and the produced dt)
    # into its workspace, the single-pass kernel tagged look-back words: the
    # two never share a buffer
    if proj is not None:
        W, bias, dt_min, dt_max, rank = proj
        passes = L_.tssm_selective_scan_takes_passes(
            code, Bsz, L, Dc, N, 1, 0, dt.data_ptr(), W.data_ptr(), bias.data_ptr(), rank,
            dt.stride(0), dt.stride(1), W.stride(0))
        nbytes = L_.tssm_selective_scan_dtproj_workspace_bytes(Bsz, L, Dc, N, int(chunk))
    else:
        passes = L_.tssm_selective_scan_takes_passes(
            code, Bsz, L, Dc, N, sdt[2], int(bool(dt_is_tau)), dt.data_ptr(), None, None, 0,
            0, 0, 0)
        nbytes = L_.tssm_selective_scan_workspace_bytes(Bsz, L, Dc, N, int(chunk))
    ws, stream = _ws(nbytes, x, "selective_scan",
                     workspace.SSD if passes else workspace.LOOKBACK)
    if proj is not None:
        _lib.call("tssm_selective_scan_dtproj", code, _disc_code(disc), x.data_ptr(),
                  dt.data_ptr(), W.data_ptr(), bias.data_ptr(), dt_min, dt_max,
                  A_log.data_ptr(), B.data_ptr(), C.data_ptr(), ptr(D), ptr(h0), y.data_ptr(),
                  ptr(h_last), Bsz, L, Dc, N, rank, x.stride(0), x.stride(1), dt.stride(0),
                  dt.stride(1), W.stride(0), B.stride(0), B.stride(1), C.stride(0),
                  C.stride(1), y.stride(0), y.stride(1), int(chunk), ws.data_ptr(), ws.numel(),
                  stream)
    else:
        _lib.call("tssm_selective_scan", code, _disc_code(disc), x.data_ptr(), dt.data_ptr(),
                  int(bool(dt_is_tau)), A_log.data_ptr(), B.data_ptr(), C.data_ptr(), ptr(D),
                  ptr(h0), y.data_ptr(), ptr(h_last), Bsz, L, Dc, N, x.stride(0), x.stride(1),
                  *sdt, B.stride(0), B.stride(1), C.stride(0), C.stride(1), y.stride(0),
                  y.stride(1), int(chunk), ws.data_ptr(), ws.numel(), stream)
    return (y, h_last) if return_state else y


def _interp_scan_fused(V, M, tau32, A_log, B, C, D, Vhat, K, FTILE, disc, h0, return_state):
    """tssm_interp_selective_scan (the interpolation formed inside the scan's
    first pass) when it supports the operands, else None."""
    Bsz, T, F = V.shape
    if B.dim() != 3 or B.shape[:2] != (Bsz, T) or C.shape != B.shape:
        return None
    N = B.shape[-1]
    if (B.dtype != V.dtype or C.dtype != V.dtype or V.dtype not in (torch.float32, torch.bfloat16)
            or M.dtype != torch.float32 or A_log.shape != (F, N)):
        return None
    L_ = _lib.lib()
    code = dcode(V, "V")
    if not L_.tssm_interp_selective_scan_supported(code, _lib.F32, _lib.F32, Bsz, T, F, N,
                                                   int(K), int(FTILE), M.data_ptr(),
                                                   M.stride(0), M.stride(1), V.stride(1)):
        return None
    for t, w in ((A_log, "A_log"), (B, "B"), (C, "C")):
        need_gpu(t, w)
    _inner_unit(B, "B")
    _inner_unit(C, "C")
    A_log = as_f32(A_log, "A_log").contiguous()
    if D is not None:
        need_gpu(D, "D")
        if D.numel() != F:
            raise ValueError("D must have F elements")
        D = as_f32(D, "D").contiguous()
    if h0 is not None:
        need_gpu(h0, "h0")
        if tuple(h0.shape) != (Bsz, F, N):
            raise ValueError("h0 must be [Bsz, F, N]")
        h0 = as_f32(h0, "h0").contiguous()
    y = torch.empty(Bsz, T, F, device=V.device, dtype=V.dtype)
    h_last = torch.empty(Bsz, F, N, device=V.device, dtype=torch.float32) if return_state else None
    ws, stream = _ws(L_.tssm_interp_selective_scan_workspace_bytes(Bsz, T, F, N), V,
                     "interp_selective_scan", workspace.SSD)
    _lib.call("tssm_interp_selective_scan", code, _disc_code(disc), V.data_ptr(), M.data_ptr(),
              tau32.data_ptr(), A_log.data_ptr(), B.data_ptr(), C.data_ptr(), ptr(D), ptr(h0),
              Vhat.data_ptr(), y.data_ptr(), ptr(h_last), Bsz, T, F, N, V.stride(0),
              V.stride(1), M.stride(0), M.stride(1), tau32.stride(0), tau32.stride(1),
              B.stride(0), B.stride(1), C.stride(0), C.stride(1), Vhat.stride(0),
              Vhat.stride(1), y.stride(0), y.stride(1), int(K), int(FTILE), ws.data_ptr(),
              ws.numel(), stream)
    return (Vhat, y, h_last) if return_state else (Vhat, y)


def fused_interp_ssm_forward(V, M, tau, A_log, B, C, D=None, *, K=10, FTILE=128, disc="zoh",
                             chunk=256, h0=None, return_state=False):
    """Interpolation of irregular observations followed by a Mamba-1 scan.

    V, M [Bsz, T, F] (M > 0.5 observed, tested through FTILE-wide tile sums as
    in fused_interp_kernel.py), tau [Bsz, T] sorted timestamps.  Vhat is the
    reference's time-aware interpolation (K, FTILE honoured); the scan then
    runs over channels F with dt_t = tau_t - tau_{t-1} (dt_0 = tau_0) computed
    in the scan's load stage.  Returns (Vhat, y[, h_last]).

    Large problems with fp32 masks (tssm_interp_selective_scan_supported) form
    Vhat inside the scan's first pass: written once, consumed there as x,
    never read back.  Others run the interpolation kernel, then the scan.
    """
    for t, w in ((V, "V"), (M, "M"), (tau, "tau")):
        need_gpu(t, w)
    if V.dim() != 3 or M.shape != V.shape or tau.shape != V.shape[:2]:
        raise ValueError("expected V, M [Bsz,T,F] and tau [Bsz,T]")
    Bsz, T, F = V.shape
    _inner_unit(V, "V")
    _inner_unit(M, "M")
    Vhat = torch.empty(Bsz, T, F, device=V.device, dtype=V.dtype)
    tau32 = as_f32(tau, "tau").contiguous()
    fused = _interp_scan_fused(V, M, tau32, A_log, B, C, D, Vhat, K, FTILE, disc, h0,
                               return_state)
    if fused is not None:
        return fused
    nt = -(-F // int(FTILE))
    nbytes = _lib.lib().tssm_time_aware_interp_workspace_bytes(T, F, int(K), int(FTILE), Bsz, T, nt)
    ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=V.device)
    _lib.call("tssm_time_aware_interp", dcode(V, "V"), dcode(M, "M"), dcode(tau32, "tau"),
              V.data_ptr(), M.data_ptr(), tau32.data_ptr(), Vhat.data_ptr(), Bsz, T, F,
              V.stride(0), V.stride(1), M.stride(0), M.stride(1), tau32.stride(0),
              tau32.stride(1), Vhat.stride(0), Vhat.stride(1), int(K), int(FTILE), Bsz, T,
              nt, ws.data_ptr(), ws.numel(), stream_handle(V))
    res = selective_scan_forward(Vhat, tau32, A_log, B, C, D, chunk=chunk, disc=disc, h0=h0,
                                 return_state=return_state, dt_is_tau=True)
    if return_state:
        return Vhat, res[0], res[1]
    return Vhat, res
