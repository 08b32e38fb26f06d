"""Drop-in for Triton-SSM ``streaming_inference_kernel.py`` on MI355X (HIP, gfx950).

  streaming_ssm_inplace_kernel       streaming_inference_kernel.py:7-37
  streaming_ssm_inplace_bf16_kernel  :41-71   (state stored as bf16, as the reference)
  streaming_interp_then_ssm_kernel   :75-156  (ring-buffer insert, forward fill, step)

Grid (B, ceil(H/BLOCK_H)).  The ring kernel runs one workgroup per stream, so
the ring head is read once for all feature tiles and advanced once after them
(the reference reads it in every tile program but advances it from tile 0,
:106,115-117 -- a race whenever H > BLOCK_H).  BLOCK_H stays the width of the
"any lane observed" test.  Its grid must cover every tile of H.

  mean_pool_logit_kernel             :159-194  (per-batch reduction in a fixed order)
  masked_fill_zero_kernel            :197-214  (mask [B,T] broadcast over H; float, int32,
                                                uint8 or bool masks)
"""
from __future__ import annotations

import torch

from tssm import _lib
from tssm import layers
from tssm.launch import HipKernel, dcode, extent, ival, need_gpu, span, stream_handle

__all__ = ["streaming_ssm_inplace_kernel", "streaming_ssm_inplace_bf16_kernel",
           "streaming_interp_then_ssm_kernel", "mean_pool_logit_kernel",
           "masked_fill_zero_kernel"]

_STEP = ["vhat_ptr", "h_ptr", "Abar_ptr", "Bbar_ptr", "C_ptr", "D_ptr", "y_ptr", "B", "H",
         "stride_vb", "stride_vh", "stride_hb", "stride_hh", "stride_cb", "stride_ch", "BLOCK_H"]


def _launch_step(grid, a):
    keys = ["vhat_ptr", "h_ptr", "Abar_ptr", "Bbar_ptr", "C_ptr", "D_ptr", "y_ptr"]
    ts = [need_gpu(a[k], k) for k in keys]
    for t, k in zip(ts, keys):
        if t.dtype != ts[0].dtype:
            raise TypeError(f"{k}: all tensors of this kernel must share one dtype")
    nb, H = ival(a["B"], "B"), ival(a["H"], "H")
    g = lambda k: ival(a[k], k)  # noqa: E731
    gb, gh, _ = grid
    if gb > nb:
        raise ValueError(f"grid {grid} exceeds B = {nb}")
    hc = min(H, gh * g("BLOCK_H"))
    v, h, Ab, Bb, C, D, y = ts
    extent(v, span([(gb, g("stride_vb")), (hc, 1)]), "vhat_ptr")
    extent(h, span([(gb, g("stride_hb")), (hc, 1)]), "h_ptr")
    extent(C, span([(gb, g("stride_cb")), (hc, 1)]), "C_ptr")
    extent(y, span([(gb, g("stride_vb")), (hc, 1)]), "y_ptr")
    for t, k in ((Ab, "Abar_ptr"), (Bb, "Bbar_ptr"), (D, "D_ptr")):
        extent(t, hc - 1, k)
    _lib.call("tssm_stream_step", dcode(v, "vhat_ptr"), *(t.data_ptr() for t in ts), nb, H, gb, hc,
              g("stride_vb"), g("stride_hb"), g("stride_cb"), stream_handle(v))


streaming_ssm_inplace_kernel = HipKernel(
    "streaming_ssm_inplace_kernel", _STEP, _launch_step, "streaming_inference_kernel.py:7-37")
streaming_ssm_inplace_bf16_kernel = HipKernel(
    "streaming_ssm_inplace_bf16_kernel", _STEP, _launch_step, "streaming_inference_kernel.py:41-71")


def _launch_ring(grid, a):
    fk = ["ring_V_ptr", "ring_M_ptr", "ring_tau_ptr", "v_new_ptr", "m_new_ptr", "tau_new_ptr",
          "h_ptr", "Abar_ptr", "Bbar_ptr", "C_ptr", "D_ptr", "y_ptr"]
    ts = {k: need_gpu(a[k], k) for k in fk}
    for k, t in ts.items():
        if t.dtype != torch.float32:
            raise TypeError(f"{k} must be float32")
    head = need_gpu(a["ring_head_ptr"], "ring_head_ptr")
    if head.dtype != torch.int32:
        raise TypeError("ring_head_ptr must be int32")
    nb, H = ival(a["B"], "B"), ival(a["H"], "H")
    g = lambda k: ival(a[k], k)  # noqa: E731
    BH, KR = g("BLOCK_H"), g("KRING")
    gb, gh, _ = grid
    if gb > nb:
        raise ValueError(f"grid {grid} exceeds B = {nb}")
    if gh * BH < H:
        raise ValueError("the ring kernel's grid must cover every BLOCK_H tile of H")
    extent(ts["ring_V_ptr"], span([(gb, g("stride_rb")), (KR, g("stride_rk")), (H, 1)]), "ring_V_ptr")
    extent(ts["ring_M_ptr"], span([(gb, g("stride_rb")), (KR, g("stride_rk")), (H, 1)]), "ring_M_ptr")
    extent(ts["ring_tau_ptr"], gb * KR - 1, "ring_tau_ptr")
    extent(head, gb - 1, "ring_head_ptr")
    extent(ts["tau_new_ptr"], gb - 1, "tau_new_ptr")
    for k in ("v_new_ptr", "m_new_ptr", "y_ptr"):
        extent(ts[k], span([(gb, g("stride_vb")), (H, 1)]), k)
    extent(ts["h_ptr"], span([(gb, g("stride_hb")), (H, 1)]), "h_ptr")
    extent(ts["C_ptr"], span([(gb, g("stride_cb")), (H, 1)]), "C_ptr")
    for k in ("Abar_ptr", "Bbar_ptr", "D_ptr"):
        extent(ts[k], H - 1, k)
    _lib.call("tssm_stream_interp_step", ts["ring_V_ptr"].data_ptr(), ts["ring_M_ptr"].data_ptr(),
              ts["ring_tau_ptr"].data_ptr(), head.data_ptr(), ts["v_new_ptr"].data_ptr(),
              ts["m_new_ptr"].data_ptr(), ts["tau_new_ptr"].data_ptr(), ts["h_ptr"].data_ptr(),
              ts["Abar_ptr"].data_ptr(), ts["Bbar_ptr"].data_ptr(), ts["C_ptr"].data_ptr(),
              ts["D_ptr"].data_ptr(), ts["y_ptr"].data_ptr(), nb, H, g("stride_rb"),
              g("stride_rk"), g("stride_vb"), g("stride_hb"), g("stride_cb"), BH, KR, gb,
              stream_handle(head))


streaming_interp_then_ssm_kernel = HipKernel(
    "streaming_interp_then_ssm_kernel",
    ["ring_V_ptr", "ring_M_ptr", "ring_tau_ptr", "ring_head_ptr", "v_new_ptr", "m_new_ptr",
     "tau_new_ptr", "h_ptr", "Abar_ptr", "Bbar_ptr", "C_ptr", "D_ptr", "y_ptr", "B", "H", "K",
     "stride_rb", "stride_rk", "stride_rh", "stride_vb", "stride_vh", "stride_hb", "stride_hh",
     "stride_cb", "stride_ch", "BLOCK_H", "KRING"],
    _launch_ring, "streaming_inference_kernel.py:75-156")

mean_pool_logit_kernel = HipKernel(
    "mean_pool_logit_kernel",
    ["h_ptr", "W_ptr", "bias_ptr", "out_ptr", "B", "T", "H", "stride_b", "stride_t", "stride_h",
     "BLOCK_H", "BLOCK_T"],
    layers.launch_mean_pool_logit, "streaming_inference_kernel.py:159-194")
masked_fill_zero_kernel = HipKernel(
    "masked_fill_zero_kernel", ["x_ptr", "mask_ptr", "out_ptr", "B", "T", "H", "BLOCK"],
    layers.launch_masked_fill_zero, "streaming_inference_kernel.py:197-214")
