"""Drop-in for Triton-SSM ``fused_ssm_interp.py`` on MI355X (HIP, gfx950).

  fused_interp_ssm_step_kernel  fused_ssm_interp.py:12-101
      interpolation at one step t_cur (same rules as fused_interp_kernel.py)
      fused with one SSM step h_out = A_bar*h_in + B_bar*vhat.  Grid
      (B, ceil(F/FTILE)); V/Vhat in any float dtype, A_bar, B_bar, h_in, h_out
      float32.
  _combine_fwd                  :7-8

  layernorm_kernel / layernorm_bwd_kernel   :104-171
      one wave per (b, l) row; BLOCK_H >= H honoured as the reference's block
      (its masked lanes enter the variance); dw/db accumulated in a fixed
      order instead of atomically.
  swiglu_kernel / swiglu_bwd_kernel         :173-217
"""
from __future__ import annotations

from tssm import _lib
from tssm import layers
from tssm.launch import HipKernel, as_f32, dcode, extent, ival, need_gpu, span, stream_handle

__all__ = ["_combine_fwd", "fused_interp_ssm_step_kernel", "layernorm_kernel",
           "layernorm_bwd_kernel", "swiglu_kernel", "swiglu_bwd_kernel"]


def _combine_fwd(aL, xL, aR, xR):
    """(aL,xL) o (aR,xR) = (aR*aL, aR*xL + xR) (fused_ssm_interp.py:7-8)."""
    return aR * aL, aR * xL + xR


def _launch_step(grid, a):
    V = need_gpu(a["V_ptr"], "V_ptr")
    M = need_gpu(a["M_ptr"], "M_ptr")
    tau = need_gpu(a["tau_ptr"], "tau_ptr")
    Ab = as_f32(a["A_bar_ptr"], "A_bar_ptr")
    Bb = as_f32(a["B_bar_ptr"], "B_bar_ptr")
    hin = as_f32(a["h_in_ptr"], "h_in_ptr")
    O = need_gpu(a["Vhat_ptr"], "Vhat_ptr")
    hout = need_gpu(a["h_out_ptr"], "h_out_ptr")
    if O.dtype != V.dtype:
        raise TypeError("Vhat_ptr must have V_ptr's dtype")
    if hout.dtype.itemsize != 4 or not hout.is_floating_point():
        raise TypeError("h_out_ptr must be float32")
    nb, T, F = ival(a["B"], "B"), ival(a["T"], "T"), ival(a["F"], "F")
    K, FT, t_cur = ival(a["K"], "K"), ival(a["FTILE"], "FTILE"), ival(a["t_cur"], "t_cur")
    g = lambda k: ival(a[k], k)  # noqa: E731
    gb, gf, _ = grid
    if gb > nb:
        raise ValueError(f"grid {grid} exceeds B = {nb}")
    if not 0 <= t_cur < T:
        raise ValueError(f"t_cur {t_cur} outside [0, {T})")
    if FT <= 0:
        raise ValueError("FTILE must be positive")
    fc = min(F, gf * FT)
    extent(V, span([(gb, g("stride_vb")), (T, g("stride_vt")), (fc, 1)]), "V_ptr")
    extent(M, span([(gb, g("stride_mb")), (T, g("stride_mt")), (fc, 1)]), "M_ptr")
    extent(tau, span([(gb, g("stride_tb")), (T, g("stride_tt"))]), "tau_ptr")
    extent(O, span([(gb, g("stride_ob")), (1, 0), (fc, 1)]) + t_cur * g("stride_ot"), "Vhat_ptr")
    extent(Ab, fc - 1, "A_bar_ptr")
    extent(Bb, fc - 1, "B_bar_ptr")
    extent(hin, min(nb * F - 1, span([(gb, g("stride_hib")), (fc, 1)])), "h_in_ptr")
    extent(hout, span([(gb, g("stride_hob")), (fc, 1)]), "h_out_ptr")
    _lib.call("tssm_interp_ssm_step", dcode(V, "V_ptr"), dcode(M, "M_ptr"), dcode(tau, "tau_ptr"),
              V.data_ptr(), M.data_ptr(), tau.data_ptr(), Ab.data_ptr(), Bb.data_ptr(),
              hin.data_ptr(), O.data_ptr(), hout.data_ptr(), nb, T, F, g("stride_vb"),
              g("stride_vt"), g("stride_mb"), g("stride_mt"), g("stride_tb"), g("stride_tt"),
              g("stride_ob"), g("stride_ot"), g("stride_hib"), g("stride_hob"), t_cur, K, FT,
              gb, gf, stream_handle(V))


fused_interp_ssm_step_kernel = HipKernel(
    "fused_interp_ssm_step_kernel",
    ["V_ptr", "M_ptr", "tau_ptr", "A_bar_ptr", "B_bar_ptr", "h_in_ptr", "Vhat_ptr", "h_out_ptr",
     "B", "T", "F", "stride_vb", "stride_vt", "stride_vf", "stride_mb", "stride_mt", "stride_mf",
     "stride_tb", "stride_tt", "stride_ob", "stride_ot", "stride_of", "stride_hib", "stride_hif",
     "stride_hob", "stride_hof", "t_cur", "K", "FTILE"],
    _launch_step, "fused_ssm_interp.py:12-101")

layernorm_kernel = HipKernel(
    "layernorm_kernel",
    ["x_ptr", "w_ptr", "bias_ptr", "out_ptr", "B", "L", "H", "stride_b", "stride_l", "stride_h",
     "EPS", "BLOCK_H"],
    layers.launch_layernorm, "fused_ssm_interp.py:104-130")
layernorm_bwd_kernel = HipKernel(
    "layernorm_bwd_kernel",
    ["dout_ptr", "x_ptr", "w_ptr", "dx_ptr", "dw_ptr", "db_ptr", "B", "L", "H", "stride_b",
     "stride_l", "EPS", "BLOCK_H"],
    layers.launch_layernorm_bwd, "fused_ssm_interp.py:133-171")
swiglu_kernel = HipKernel(
    "swiglu_kernel", ["gate_ptr", "up_ptr", "out_ptr", "B", "L", "H", "stride_b", "stride_l", "BLOCK_H"],
    layers.launch_swiglu, "fused_ssm_interp.py:173-191")
swiglu_bwd_kernel = HipKernel(
    "swiglu_bwd_kernel",
    ["dout_ptr", "gate_ptr", "up_ptr", "dgate_ptr", "dup_ptr", "B", "L", "H", "stride_b",
     "stride_l", "BLOCK_H"],
    layers.launch_swiglu_bwd, "fused_ssm_interp.py:193-217")
