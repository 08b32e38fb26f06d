"""Drop-in for Triton-SSM ``multihead_ssm_kernel.py`` on MI355X (HIP, gfx950).

Same symbols, same parameter lists, same launch convention
(``kernel[grid](...)``), same intermediate layouts:

  multihead_ssm_fwd_local_kernel   (multihead_ssm_kernel.py:20-102)
  multihead_ssm_carry_scan_kernel  (:106-117)
  multihead_ssm_output_kernel      (:121-187)
  _scan_combine                    (:15-16)

The reference's local kernel cannot be traced by Triton (scalar indexing of a
block at :101-102, :151-152); these kernels implement its evident intent: a
per-lane carry store/load.

``multihead_ssm_forward`` (new) runs all three phases as ONE single-pass HIP
kernel with the discretization fused into its load stage.

  residual_add_kernel / dropout_residual_kernel  (:190-222)
      flat over the first min(N, grid*BLOCK) elements; the dropout keep mask
      is uint8 (or bool).
"""
from __future__ import annotations

from tssm import _lib
from tssm.fused import multihead_ssm_forward  # noqa: F401
from tssm import layers
from tssm.launch import (HipKernel, as_f32, dcode, extent, ival, need_gpu, span,
                         stream_handle)

__all__ = [
    "_scan_combine", "multihead_ssm_fwd_local_kernel", "multihead_ssm_carry_scan_kernel",
    "multihead_ssm_output_kernel", "residual_add_kernel", "dropout_residual_kernel",
    "multihead_ssm_forward",
]


def _scan_combine(aL, xL, aR, xR):
    """(aL,xL) o (aR,xR) = (aR*aL, aR*xL + xR) (multihead_ssm_kernel.py:15-16)."""
    return aR * aL, aR * xL + xR


def _sizes(a):
    return (ival(a["B"], "B"), ival(a["L"], "L"), ival(a["H"], "H"),
            ival(a["n_heads"], "n_heads"), ival(a["head_dim"], "head_dim"))


def _check_head_dim(a, hd):
    if ival(a["HEAD_DIM"], "HEAD_DIM") < hd:
        raise ValueError("HEAD_DIM must be >= head_dim (the reference masks lanes >= head_dim "
                         "of a HEAD_DIM-wide block)")


def _launch_fwd_local(grid, a):
    u = need_gpu(a["u_ptr"], "u_ptr")
    Bm = need_gpu(a["B_ptr"], "B_ptr")
    if Bm.dtype != u.dtype:
        raise TypeError("u_ptr and B_ptr must share one dtype")
    A_log = as_f32(a["A_log_ptr"], "A_log_ptr")
    dt = as_f32(a["dt_ptr"], "dt_ptr")
    outs = [need_gpu(a[k], k) for k in ("loc_a_ptr", "loc_x_ptr", "carry_ptr")]
    for t, k in zip(outs, ("loc_a_ptr", "loc_x_ptr", "carry_ptr")):
        if t.dtype.itemsize != 4 or not t.is_floating_point():
            raise TypeError(f"{k} must be float32")
    Bsz, L, H, nh, hd = _sizes(a)
    _check_head_dim(a, hd)
    nblk = ival(a["NBLK"], "NBLK")
    g = lambda k: ival(a[k], k)  # noqa: E731
    extent(u, span([(Bsz, g("stride_ub")), (L, g("stride_ul"))]) + min(H, nh * hd) - 1, "u_ptr")
    extent(Bm, span([(Bsz, g("stride_Bb")), (L, g("stride_Bl")), (nh, g("stride_Bh")), (hd, 1)]),
           "B_ptr")
    extent(dt, span([(Bsz, g("stride_db")), (L, g("stride_dl")), (nh, g("stride_dh"))]), "dt_ptr")
    extent(A_log, span([(nh, g("stride_alh")), (hd, 1)]), "A_log_ptr")
    extent(outs[0], Bsz * L * nh * hd - 1, "loc_a_ptr")
    extent(outs[1], Bsz * L * nh * hd - 1, "loc_x_ptr")
    extent(outs[2], 2 * Bsz * nh * hd * nblk - 1, "carry_ptr")
    if grid[0] > Bsz * nh or grid[1] > nblk:
        raise ValueError(f"grid {grid[:2]} exceeds (B*n_heads, NBLK) = ({Bsz * nh}, {nblk})")
    _lib.call("tssm_mh_fwd_local", dcode(u, "u_ptr"), u.data_ptr(), A_log.data_ptr(),
              Bm.data_ptr(), dt.data_ptr(), *(t.data_ptr() for t in outs), Bsz, L, H, nh, hd,
              ival(a["stride_ub"], "stride_ub"), ival(a["stride_ul"], "stride_ul"),
              ival(a["stride_alh"], "stride_alh"), ival(a["stride_Bb"], "stride_Bb"),
              ival(a["stride_Bl"], "stride_Bl"), ival(a["stride_Bh"], "stride_Bh"),
              ival(a["stride_db"], "stride_db"), ival(a["stride_dl"], "stride_dl"),
              ival(a["stride_dh"], "stride_dh"), ival(a["BLK_L"], "BLK_L"),
              ival(a["NBLK"], "NBLK"), grid[0], grid[1], stream_handle(u))


def _launch_carry_scan(grid, a):
    carry = need_gpu(a["carry_ptr"], "carry_ptr")
    extent(carry, 2 * ival(a["total_rows"], "total_rows") * ival(a["NBLK"], "NBLK") - 1,
           "carry_ptr")
    _lib.call("tssm_carry_scan", dcode(carry, "carry_ptr"), carry.data_ptr(),
              ival(a["total_rows"], "total_rows"), ival(a["NBLK"], "NBLK"), 0, grid[0],
              stream_handle(carry))


def _launch_output(grid, a):
    loc_a = need_gpu(a["loc_a_ptr"], "loc_a_ptr")
    loc_x = need_gpu(a["loc_x_ptr"], "loc_x_ptr")
    carry = need_gpu(a["carry_ptr"], "carry_ptr")
    for t, k in ((loc_a, "loc_a_ptr"), (loc_x, "loc_x_ptr"), (carry, "carry_ptr")):
        if t.dtype.itemsize != 4 or not t.is_floating_point():
            raise TypeError(f"{k} must be float32")
    C = need_gpu(a["C_ptr"], "C_ptr")
    u = need_gpu(a["u_ptr"], "u_ptr")
    y = need_gpu(a["y_ptr"], "y_ptr")
    if not (C.dtype == u.dtype == y.dtype):
        raise TypeError("C_ptr, u_ptr and y_ptr must share one dtype")
    D = as_f32(a["D_ptr"], "D_ptr")
    Bsz, L, H, nh, hd = _sizes(a)
    _check_head_dim(a, hd)
    nblk = ival(a["NBLK"], "NBLK")
    g = lambda k: ival(a[k], k)  # noqa: E731
    m = min(H, nh * hd)
    extent(loc_a, Bsz * L * nh * hd - 1, "loc_a_ptr")
    extent(loc_x, Bsz * L * nh * hd - 1, "loc_x_ptr")
    extent(carry, 2 * Bsz * nh * hd * nblk - 1, "carry_ptr")
    extent(C, span([(Bsz, g("stride_Cb")), (L, g("stride_Cl")), (nh, g("stride_Ch")), (hd, 1)]),
           "C_ptr")
    extent(u, span([(Bsz, g("stride_ub")), (L, g("stride_ul"))]) + m - 1, "u_ptr")
    extent(D, m - 1, "D_ptr")
    extent(y, Bsz * L * H - 1, "y_ptr")
    if grid[0] > Bsz * nh or grid[1] > nblk:
        raise ValueError(f"grid {grid[:2]} exceeds (B*n_heads, NBLK) = ({Bsz * nh}, {nblk})")
    _lib.call("tssm_mh_output", dcode(u, "u_ptr"), loc_a.data_ptr(), loc_x.data_ptr(),
              carry.data_ptr(), C.data_ptr(), D.data_ptr(), u.data_ptr(), y.data_ptr(),
              Bsz, L, H, nh, hd, ival(a["stride_ub"], "stride_ub"),
              ival(a["stride_ul"], "stride_ul"), ival(a["stride_Cb"], "stride_Cb"),
              ival(a["stride_Cl"], "stride_Cl"), ival(a["stride_Ch"], "stride_Ch"),
              ival(a["BLK_L"], "BLK_L"), ival(a["NBLK"], "NBLK"), grid[0], grid[1],
              stream_handle(u))


multihead_ssm_fwd_local_kernel = HipKernel(
    "multihead_ssm_fwd_local_kernel",
    ["u_ptr", "A_log_ptr", "B_ptr", "C_ptr", "dt_ptr", "loc_a_ptr", "loc_x_ptr", "carry_ptr",
     "B", "L", "H", "n_heads", "head_dim", "stride_ub", "stride_ul", "stride_uh",
     "stride_alh", "stride_alp", "stride_Bb", "stride_Bl", "stride_Bh", "stride_Bp",
     "stride_Cb", "stride_Cl", "stride_Ch", "stride_Cp", "stride_db", "stride_dl", "stride_dh",
     "BLK_L", "NBLK", "HEAD_DIM"],
    _launch_fwd_local, "multihead_ssm_kernel.py:20-102")

multihead_ssm_carry_scan_kernel = HipKernel(
    "multihead_ssm_carry_scan_kernel", ["carry_ptr", "total_rows", "NBLK"],
    _launch_carry_scan, "multihead_ssm_kernel.py:106-117")

multihead_ssm_output_kernel = HipKernel(
    "multihead_ssm_output_kernel",
    ["loc_a_ptr", "loc_x_ptr", "carry_ptr", "C_ptr", "D_ptr", "u_ptr", "y_ptr", "B", "L", "H",
     "n_heads", "head_dim", "stride_ub", "stride_ul", "stride_uh", "stride_Cb", "stride_Cl",
     "stride_Ch", "stride_Cp", "BLK_L", "NBLK", "HEAD_DIM"],
    _launch_output, "multihead_ssm_kernel.py:121-187")

residual_add_kernel = HipKernel(
    "residual_add_kernel", ["x_ptr", "res_ptr", "out_ptr", "N", "BLOCK"],
    layers.launch_residual_add, "multihead_ssm_kernel.py:190-201")

dropout_residual_kernel = HipKernel(
    "dropout_residual_kernel", ["x_ptr", "res_ptr", "mask_ptr", "out_ptr", "N", "p_keep", "BLOCK"],
    layers.launch_dropout_residual, "multihead_ssm_kernel.py:204-222")
