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

import torch

from tssm import _lib
from tssm.launch import HipKernel, as_f32, dcode, extent, ival, need_gpu, span, stream_handle

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

_BWD_PARAMS = ["A_ptr", "B_ptr", "dt_ptr", "Abar_ptr", "dAbar_ptr", "dBbar_ptr", "dA_ptr",
               "dB_ptr", "ddt_ptr", "B", "T", "H", "stride_Bb", "stride_Bt", "stride_Bh",
               "stride_db", "stride_dt", "stride_ab", "stride_at", "stride_ah", "stride_bb",
               "stride_bt", "stride_bh", "BLOCK_H"]


def _launch_zoh_bwd(grid, a):
    """discretize_kernel.py:98-162.  dA_ptr is accumulated into (the reference's
    atomic_add, :156); ddt_ptr is overwritten with the sum over the covered
    lanes (the intent of :159-162); dB_ptr uses B's strides (:157)."""
    A = as_f32(a["A_ptr"], "A_ptr")
    dt = as_f32(a["dt_ptr"], "dt_ptr")
    Bm = need_gpu(a["B_ptr"], "B_ptr")
    Abar = need_gpu(a["Abar_ptr"], "Abar_ptr")
    dAbar = need_gpu(a["dAbar_ptr"], "dAbar_ptr")
    dBbar = need_gpu(a["dBbar_ptr"], "dBbar_ptr")
    dA = need_gpu(a["dA_ptr"], "dA_ptr")
    dB = need_gpu(a["dB_ptr"], "dB_ptr")
    ddt = need_gpu(a["ddt_ptr"], "ddt_ptr")
    for t, w in ((Abar, "Abar_ptr"), (dAbar, "dAbar_ptr"), (dBbar, "dBbar_ptr"), (dB, "dB_ptr")):
        if t.dtype != Bm.dtype:
            raise TypeError(f"{w}: must have B_ptr's dtype {Bm.dtype}, got {t.dtype}")
    for t, w in ((dA, "dA_ptr"), (ddt, "ddt_ptr")):
        if t.dtype != torch.float32:
            raise TypeError(f"{w}: gradients accumulated across lanes must be float32")
    nb, T, H = ival(a["B"], "B"), ival(a["T"], "T"), ival(a["H"], "H")
    g = lambda k: ival(a[k], k)  # noqa: E731
    gb, gt, gh = grid
    if gb > nb or gt > T:
        raise ValueError(f"grid {grid} exceeds (B, T) = ({nb}, {T})")
    hc = min(H, gh * g("BLOCK_H"))
    extent(A, hc - 1, "A_ptr")
    extent(dA, hc - 1, "dA_ptr")
    for t, w, sb, st in ((Bm, "B_ptr", "stride_Bb", "stride_Bt"), (dB, "dB_ptr", "stride_Bb", "stride_Bt"),
                         (Abar, "Abar_ptr", "stride_ab", "stride_at"),
                         (dAbar, "dAbar_ptr", "stride_ab", "stride_at"),
                         (dBbar, "dBbar_ptr", "stride_bb", "stride_bt")):
        extent(t, span([(gb, g(sb)), (gt, g(st)), (hc, 1)]), w)
    for t, w in ((dt, "dt_ptr"), (ddt, "ddt_ptr")):
        extent(t, span([(gb, g("stride_db")), (gt, g("stride_dt"))]), w)
    nbytes = _lib.lib().tssm_zoh_discretize_bwd_workspace_bytes(gb, gt, hc)
    ws = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=Bm.device)
    _lib.call("tssm_zoh_discretize_bwd", dcode(Bm, "B_ptr"), A.data_ptr(), Bm.data_ptr(),
              dt.data_ptr(), Abar.data_ptr(), dAbar.data_ptr(), dBbar.data_ptr(), dA.data_ptr(),
              dB.data_ptr(), ddt.data_ptr(), nb, T, H, gb, gt, hc, g("stride_Bb"), g("stride_Bt"),
              g("stride_db"), g("stride_dt"), g("stride_ab"), g("stride_at"), g("stride_bb"),
              g("stride_bt"), ws.data_ptr(), ws.numel(), stream_handle(Bm))


zoh_discretize_bwd_kernel = HipKernel(
    "zoh_discretize_bwd_kernel", _BWD_PARAMS, _launch_zoh_bwd, "discretize_kernel.py:98-162")

_DTP_PARAMS = ["dt_raw_ptr", "W_ptr", "bias_ptr", "dt_out_ptr", "B", "T", "H", "dt_rank",
               "stride_rb", "stride_rt", "stride_rr", "stride_wb", "stride_wh",
               "stride_ob", "stride_ot", "stride_oh", "DT_MIN", "DT_MAX", "BLOCK_H", "BLOCK_R"]


def _launch_dt_project(grid, a):
    """discretize_kernel.py:166-213: dt = clamp(softplus(dt_raw @ W + bias)).
    BLOCK_R only tiles the reference's loop over r; every r < dt_rank is summed.
    Innermost strides (stride_rr, stride_wh, stride_oh) are unit, as in the
    reference, which accepts them but never uses them."""
    raw = as_f32(a["dt_raw_ptr"], "dt_raw_ptr")
    W = as_f32(a["W_ptr"], "W_ptr")
    bias = as_f32(a["bias_ptr"], "bias_ptr")
    out = need_gpu(a["dt_out_ptr"], "dt_out_ptr")
    nb, T, H, R = (ival(a[k], k) for k in ("B", "T", "H", "dt_rank"))
    g = lambda k: ival(a[k], k)  # noqa: E731
    if g("BLOCK_R") <= 0:
        raise ValueError("BLOCK_R must be positive")
    gb, gt, gh = grid
    if gb > nb or gt > T:
        raise ValueError(f"grid {grid} exceeds (B, T) = ({nb}, {T})")
    hc = min(H, gh * g("BLOCK_H"))
    if hc > 0 and gb * gt > 0:
        extent(raw, span([(gb, g("stride_rb")), (gt, g("stride_rt")), (R, 1)]), "dt_raw_ptr")
        extent(W, span([(R, g("stride_wb")), (hc, 1)]), "W_ptr")
        extent(bias, hc - 1, "bias_ptr")
        extent(out, span([(gb, g("stride_ob")), (gt, g("stride_ot")), (hc, 1)]), "dt_out_ptr")
    _lib.call("tssm_dt_project_softplus", dcode(out, "dt_out_ptr"), raw.data_ptr(), W.data_ptr(),
              bias.data_ptr(), out.data_ptr(), nb, T, H, R, gb, gt, hc, g("stride_rb"),
              g("stride_rt"), g("stride_wb"), g("stride_ob"), g("stride_ot"),
              float(a["DT_MIN"]), float(a["DT_MAX"]), stream_handle(out))


dt_project_softplus_kernel = HipKernel(
    "dt_project_softplus_kernel", _DTP_PARAMS, _launch_dt_project, "discretize_kernel.py:166-213")
