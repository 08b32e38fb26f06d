"""Drop-in for Triton-SSM ``discretize_kernel.py`` on MI355X (HIP, gfx950).

ZOH discretization of a diagonal continuous-time SSM from irregular time
deltas:  Abar = exp(dt*a),  Bbar = expm1(dt*a) / (a + 1e-12) * B,  a = -exp(A_log).

  zoh_discretize_diag_kernel       discretize_kernel.py:16-57  (fp32 outputs)
  zoh_discretize_diag_bf16_kernel  :61-94  (bf16 outputs, fp32 math)
  zoh_discretize_bwd_kernel        :98-162
  dt_project_softplus_kernel       :166-213

Both forward kernels take the output dtype from the Abar/Bbar tensors, as a
Triton store would.  A_ptr (log(-a)) and dt_ptr are read as float32 (other
float dtypes are converted first, keeping their layout).  expm1 is evaluated
accurately instead of the reference's exp(x)-1 / x+x^2/2 branch (:51-53),
which loses ~1e-4 relative accuracy for 1e-5 < |x| < 1e-3.
"""
from __future__ import annotations

from tssm import _lib
from tssm.launch import HipKernel, as_f32, dcode, extent, ival, need_gpu, not_built, span, stream_handle

__all__ = ["zoh_discretize_diag_kernel", "zoh_discretize_diag_bf16_kernel",
           "zoh_discretize_bwd_kernel", "dt_project_softplus_kernel"]

_PARAMS = ["A_ptr", "B_ptr", "dt_ptr", "Abar_ptr", "Bbar_ptr", "B", "T", "H",
           "stride_Bb", "stride_Bt", "stride_Bh", "stride_db", "stride_dt",
           "stride_ab", "stride_at", "stride_ah", "stride_bb", "stride_bt", "stride_bh", "BLOCK_H"]


def _launch_zoh(grid, a):
    A = as_f32(a["A_ptr"], "A_ptr")
    Bm = need_gpu(a["B_ptr"], "B_ptr")
    dt = as_f32(a["dt_ptr"], "dt_ptr")
    Abar = need_gpu(a["Abar_ptr"], "Abar_ptr")
    Bbar = need_gpu(a["Bbar_ptr"], "Bbar_ptr")
    if Abar.dtype != Bbar.dtype:
        raise TypeError("Abar_ptr and Bbar_ptr must share one dtype")
    nb, T, H = ival(a["B"], "B"), ival(a["T"], "T"), ival(a["H"], "H")
    g = lambda k: ival(a[k], k)  # noqa: E731
    gb, gt, gh = grid
    if gb > nb or gt > T:
        raise ValueError(f"grid {grid} exceeds (B, T) = ({nb}, {T})")
    hc = min(H, gh * g("BLOCK_H"))
    extent(A, hc - 1, "A_ptr")
    extent(Bm, span([(gb, g("stride_Bb")), (gt, g("stride_Bt")), (hc, 1)]), "B_ptr")
    extent(dt, span([(gb, g("stride_db")), (gt, g("stride_dt"))]), "dt_ptr")
    extent(Abar, span([(gb, g("stride_ab")), (gt, g("stride_at")), (hc, 1)]), "Abar_ptr")
    extent(Bbar, span([(gb, g("stride_bb")), (gt, g("stride_bt")), (hc, 1)]), "Bbar_ptr")
    _lib.call("tssm_zoh_discretize", dcode(Bm, "B_ptr"), dcode(Abar, "Abar_ptr"), A.data_ptr(),
              Bm.data_ptr(), dt.data_ptr(), Abar.data_ptr(), Bbar.data_ptr(), nb, T, H, gb, gt, hc,
              g("stride_Bb"), g("stride_Bt"), g("stride_db"), g("stride_dt"), g("stride_ab"),
              g("stride_at"), g("stride_bb"), g("stride_bt"), stream_handle(Bm))


zoh_discretize_diag_kernel = HipKernel(
    "zoh_discretize_diag_kernel", _PARAMS, _launch_zoh, "discretize_kernel.py:16-57")
zoh_discretize_diag_bf16_kernel = HipKernel(
    "zoh_discretize_diag_bf16_kernel", _PARAMS, _launch_zoh, "discretize_kernel.py:61-94")

zoh_discretize_bwd_kernel = HipKernel(
    "zoh_discretize_bwd_kernel",
    ["A_ptr", "B_ptr", "dt_ptr", "Abar_ptr", "dAbar_ptr", "dBbar_ptr", "dA_ptr", "dB_ptr",
     "ddt_ptr", "B", "T", "H", "stride_Bb", "stride_Bt", "stride_Bh", "stride_db", "stride_dt",
     "stride_ab", "stride_at", "stride_ah", "stride_bb", "stride_bt", "stride_bh", "BLOCK_H"],
    not_built("zoh_discretize_bwd_kernel", "discretize_kernel.py:98-162", "not built yet"),
    "discretize_kernel.py:98-162")

dt_project_softplus_kernel = HipKernel(
    "dt_project_softplus_kernel",
    ["dt_raw_ptr", "W_ptr", "bias_ptr", "dt_out_ptr", "B", "T", "H", "dt_rank",
     "stride_rb", "stride_rt", "stride_rr", "stride_wb", "stride_wh",
     "stride_ob", "stride_ot", "stride_oh", "DT_MIN", "DT_MAX", "BLOCK_H", "BLOCK_R"],
    not_built("dt_project_softplus_kernel", "discretize_kernel.py:166-213", "not built yet"),
    "discretize_kernel.py:166-213")
