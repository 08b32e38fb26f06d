"""Drop-in for Triton-SSM ``ssm_scan.py`` on MI355X (HIP, gfx950).

Elementwise chunked linear scan  h_t = A_t h_{t-1} + B_t u_t,
y_t = C_t h_t + D u_t  over contiguous [batch, seqlen, H] tensors.

Kernels (same names, parameters, grids and intermediate layouts):
  ssm_fwd_local_kernel      ssm_scan.py:18-50
  ssm_carry_scan_kernel     :54-65
  ssm_fwd_apply_kernel      :69-98
  ssm_output_kernel         :102-124
  ssm_bwd_local_kernel      :136-170
  ssm_bwd_carry_scan_kernel :174-185
  ssm_bwd_apply_kernel      :189-231
Host functions: ``_nxt_pow2`` (:234-236), ``ssm_forward`` (:239-264),
``ssm_backward`` (:267-289), with the same signatures and return tuples.
As in the reference, ``ssm_backward``'s du omits the D*dY term and no dD is
returned (:226).
"""
from __future__ import annotations

import torch

from tssm import _lib
from tssm.launch import HipKernel, dcode, extent, ival, need_gpu, stream_handle

__all__ = [
    "_combine", "_combine_bwd", "ssm_fwd_local_kernel", "ssm_carry_scan_kernel",
    "ssm_fwd_apply_kernel", "ssm_output_kernel", "ssm_bwd_local_kernel",
    "ssm_bwd_carry_scan_kernel", "ssm_bwd_apply_kernel", "_nxt_pow2", "ssm_forward",
    "ssm_backward",
]


def _combine(aL, xL, aR, xR):
    """(aL,xL) o (aR,xR) = (aR*aL, aR*xL + xR) (ssm_scan.py:13-14)."""
    return aR * aL, aR * xL + xR


def _combine_bwd(aR, xR, aL, xL):
    """Reverse-time operator (ssm_scan.py:130-132)."""
    return aL * aR, aL * xR + xL


def _same_dtype(a, keys):
    """All tensors of one kernel share a dtype; every [B, L, H] operand and the
    carry buffer must cover the offsets the reference formulas address."""
    ts = [need_gpu(a[k], k) for k in keys]
    d = ts[0].dtype
    for t, k in zip(ts, keys):
        if t.dtype != d:
            raise TypeError(f"{k}: every tensor of this kernel must share one dtype "
                            f"({keys[0]} is {d}, {k} is {t.dtype})")
    Bsz, L, H = _dims(a)
    nblk = ival(a.get("NBLK", 1), "NBLK")
    for t, k in zip(ts, keys):
        if k == "carry_ptr":
            extent(t, 2 * Bsz * H * nblk - 1, k)
        elif k == "D_ptr":
            extent(t, H - 1, k)
        else:
            extent(t, Bsz * L * H - 1, k)
    return ts, dcode(ts[0], keys[0])


def _dims(a):
    return ival(a["B"], "B"), ival(a["L"], "L"), ival(a["H"], "H")


def _launch_fwd_local(grid, a):
    ts, code = _same_dtype(a, ["u_ptr", "A_ptr", "B_ptr", "loc_a_ptr", "loc_x_ptr", "carry_ptr"])
    _lib.call("tssm_ssm_fwd_local", code, *(t.data_ptr() for t in ts), *_dims(a),
              ival(a["BLK"], "BLK"), ival(a["NBLK"], "NBLK"), grid[0], grid[1],
              stream_handle(ts[0]))


def _launch_carry(reverse):
    def launch(grid, a):
        carry = need_gpu(a["carry_ptr"], "carry_ptr")
        extent(carry, 2 * ival(a["nrows"], "nrows") * ival(a["NBLK"], "NBLK") - 1, "carry_ptr")
        _lib.call("tssm_carry_scan", dcode(carry, "carry_ptr"), carry.data_ptr(),
                  ival(a["nrows"], "nrows"), ival(a["NBLK"], "NBLK"), reverse, grid[0],
                  stream_handle(carry))
    return launch


def _launch_fwd_apply(grid, a):
    ts, code = _same_dtype(a, ["loc_a_ptr", "loc_x_ptr", "carry_ptr", "h_out_ptr"])
    _lib.call("tssm_ssm_fwd_apply", code, *(t.data_ptr() for t in ts), *_dims(a),
              ival(a["BLK"], "BLK"), ival(a["NBLK"], "NBLK"), grid[0], grid[1],
              stream_handle(ts[0]))


def _launch_output(grid, a):
    ts, code = _same_dtype(a, ["h_ptr", "C_ptr", "D_ptr", "u_ptr", "y_ptr"])
    _lib.call("tssm_ssm_output", code, *(t.data_ptr() for t in ts), *_dims(a),
              ival(a["BLK"], "BLK"), grid[0], grid[1], stream_handle(ts[0]))


def _launch_bwd_local(grid, a):
    ts, code = _same_dtype(a, ["A_ptr", "C_ptr", "dY_ptr", "loc_a_ptr", "loc_dh_ptr", "carry_ptr"])
    _lib.call("tssm_ssm_bwd_local", code, *(t.data_ptr() for t in ts), *_dims(a),
              ival(a["BLK"], "BLK"), ival(a["NBLK"], "NBLK"), grid[0], grid[1],
              stream_handle(ts[0]))


def _launch_bwd_apply(grid, a):
    ts, code = _same_dtype(a, ["loc_a_ptr", "loc_dh_ptr", "carry_ptr", "u_ptr", "A_ptr", "B_ptr",
                               "h_ptr", "dY_ptr", "du_ptr", "dA_ptr", "dB_ptr", "dC_ptr"])
    _lib.call("tssm_ssm_bwd_apply", code, *(t.data_ptr() for t in ts), *_dims(a),
              ival(a["BLK"], "BLK"), ival(a["NBLK"], "NBLK"), grid[0], grid[1],
              stream_handle(ts[0]))


_FWD = ["B", "L", "H", "BLK", "NBLK"]
ssm_fwd_local_kernel = HipKernel(
    "ssm_fwd_local_kernel", ["u_ptr", "A_ptr", "B_ptr", "loc_a_ptr", "loc_x_ptr", "carry_ptr", *_FWD],
    _launch_fwd_local, "ssm_scan.py:18-50")
ssm_carry_scan_kernel = HipKernel(
    "ssm_carry_scan_kernel", ["carry_ptr", "nrows", "NBLK"], _launch_carry(0), "ssm_scan.py:54-65")
ssm_fwd_apply_kernel = HipKernel(
    "ssm_fwd_apply_kernel", ["loc_a_ptr", "loc_x_ptr", "carry_ptr", "h_out_ptr", *_FWD],
    _launch_fwd_apply, "ssm_scan.py:69-98")
ssm_output_kernel = HipKernel(
    "ssm_output_kernel", ["h_ptr", "C_ptr", "D_ptr", "u_ptr", "y_ptr", "B", "L", "H", "BLK"],
    _launch_output, "ssm_scan.py:102-124")
ssm_bwd_local_kernel = HipKernel(
    "ssm_bwd_local_kernel", ["A_ptr", "C_ptr", "dY_ptr", "loc_a_ptr", "loc_dh_ptr", "carry_ptr", *_FWD],
    _launch_bwd_local, "ssm_scan.py:136-170")
ssm_bwd_carry_scan_kernel = HipKernel(
    "ssm_bwd_carry_scan_kernel", ["carry_ptr", "nrows", "NBLK"], _launch_carry(1),
    "ssm_scan.py:174-185")
ssm_bwd_apply_kernel = HipKernel(
    "ssm_bwd_apply_kernel",
    ["loc_a_ptr", "loc_dh_ptr", "carry_ptr", "u_ptr", "A_ptr", "B_ptr", "h_ptr", "dY_ptr",
     "du_ptr", "dA_ptr", "dB_ptr", "dC_ptr", *_FWD],
    _launch_bwd_apply, "ssm_scan.py:189-231")


def _nxt_pow2(n):
    """Smallest power of two >= n (1 for n <= 1), ssm_scan.py:234-236."""
    if n <= 1:
        return 1
    return 1 << (n - 1).bit_length()


def _fused_ok(ts, H) -> bool:
    """One launch replaces the four phase kernels when every operand is a
    contiguous tensor of one dtype on the GPU, H % 4 == 0 and the base
    pointers allow 16-byte (fp32) / 8-byte (16-bit) accesses."""
    d = ts[0].dtype
    if d not in (torch.float32, torch.bfloat16, torch.float16) or H % 4:
        return False
    al = 16 if d == torch.float32 else 8
    return all(isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == d and t.is_contiguous()
               and t.data_ptr() % al == 0 for t in ts)


def _fused_ws(t, Bsz, L, H):
    from tssm import workspace
    n = _lib.lib().tssm_ssm_scan_fused_workspace_bytes(Bsz, L, H)
    stream = stream_handle(t)
    return workspace.get(t.device, stream, n), stream


def ssm_forward(u, A, B, C, D, BLK=256):
    """u, A, B, C: [batch, seqlen, H] (A, B already discretized); D: [H].
    Returns (y, h), both [batch, seqlen, H] -- h is the full state trajectory
    (ssm_scan.py:239-264).  Runs as one single-pass launch where the operands
    allow (then BLK, which only shapes the phase kernels' intermediates, does
    not apply), else as the reference's four phase kernels."""
    Bsz, L, H = u.shape
    if _fused_ok([u, A, B, C, D], H) and D.numel() == H and A.shape == u.shape == B.shape == C.shape:
        y_out, h_out = torch.empty_like(u), torch.empty_like(u)
        ws, stream = _fused_ws(u, Bsz, L, H)
        _lib.call("tssm_ssm_forward_fused", dcode(u, "u"), u.data_ptr(), A.data_ptr(),
                  B.data_ptr(), C.data_ptr(), D.data_ptr(), y_out.data_ptr(), h_out.data_ptr(),
                  Bsz, L, H, ws.data_ptr(), ws.numel(), stream)
        return y_out, h_out
    nrows = Bsz * H
    nblk = _nxt_pow2((L + BLK - 1) // BLK)
    loc_a = torch.empty_like(A)
    loc_x = torch.empty_like(A)
    h_out = torch.empty_like(u)
    y_out = torch.empty_like(u)
    carry = torch.empty(2 * nrows * nblk, dtype=u.dtype, device=u.device)
    g1 = (nrows, nblk)
    ssm_fwd_local_kernel[g1](u, A, B, loc_a, loc_x, carry, Bsz, L, H, BLK, nblk)
    ssm_carry_scan_kernel[(nrows,)](carry, nrows, nblk)
    ssm_fwd_apply_kernel[g1](loc_a, loc_x, carry, h_out, Bsz, L, H, BLK, nblk)
    ssm_output_kernel[g1](h_out, C, D, u, y_out, Bsz, L, H, BLK)
    return y_out, h_out


def ssm_backward(u, A, B, C, h, dY, BLK=256):
    """Returns (du, dA, dB, dC) (ssm_scan.py:267-289); one single-pass launch
    where the operands allow, else the reference's four phase kernels."""
    Bsz, L, H = u.shape
    ts = [u, A, B, C, h, dY]
    if _fused_ok(ts, H) and all(t.shape == u.shape for t in ts):
        du, dA, dB, dC = (torch.empty_like(u) for _ in range(4))
        ws, stream = _fused_ws(u, Bsz, L, H)
        _lib.call("tssm_ssm_backward_fused", dcode(u, "u"), *(t.data_ptr() for t in ts),
                  du.data_ptr(), dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), Bsz, L, H,
                  ws.data_ptr(), ws.numel(), stream)
        return du, dA, dB, dC
    nrows = Bsz * H
    nblk = _nxt_pow2((L + BLK - 1) // BLK)
    loc_a = torch.empty_like(A)
    loc_dh = torch.empty_like(A)
    carry = torch.empty(2 * nrows * nblk, dtype=u.dtype, device=u.device)
    du = torch.empty_like(u)
    dA = torch.empty_like(A)
    dB = torch.empty_like(B)
    dC = torch.empty_like(C)
    g1 = (nrows, nblk)
    ssm_bwd_local_kernel[g1](A, C, dY, loc_a, loc_dh, carry, Bsz, L, H, BLK, nblk)
    ssm_bwd_carry_scan_kernel[(nrows,)](carry, nrows, nblk)
    ssm_bwd_apply_kernel[g1](loc_a, loc_dh, carry, u, A, B, h, dY, du, dA, dB, dC,
                             Bsz, L, H, BLK, nblk)
    return du, dA, dB, dC
