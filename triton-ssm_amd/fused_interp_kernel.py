"""Drop-in for Triton-SSM ``fused_interp_kernel.py`` on MI355X (HIP, gfx950).

Time-aware linear interpolation of irregular observations:

  fused_time_aware_interp_kernel  fused_interp_kernel.py:10-100   (fp32)
  fused_interp_bf16_kernel        :104-181  (bf16 V/Vhat, fp32 math)
  fused_interp_fp16_kernel        :187-257  (fp16 V/Vhat, fp32 math)

Grid (B, T, ceil(F/FTILE)).  The reference's semantics are kept because they
change results: K (search window) and FTILE (width of the per-tile "any lane
observed" aggregate, :49-54) are honoured as given; the nearest observed tile
within K on each side is the neighbour; an observed current value is replaced
whenever a neighbour exists (:94-97).  The three kernels share one launcher:
V/Vhat dtype comes from the tensors, M and tau may be any float dtype.
"""
from __future__ import annotations

import torch

from tssm import _lib
from tssm.launch import HipKernel, dcode, extent, ival, need_gpu, span, stream_handle

__all__ = ["fused_time_aware_interp_kernel", "fused_interp_bf16_kernel",
           "fused_interp_fp16_kernel"]

_PARAMS = ["V_ptr", "M_ptr", "tau_ptr", "Vhat_ptr", "B", "T", "F",
           "stride_vb", "stride_vt", "stride_vf", "stride_mb", "stride_mt", "stride_mf",
           "stride_tb", "stride_tt", "stride_ob", "stride_ot", "stride_of", "K", "FTILE"]


def _launch_interp(grid, a):
    V = need_gpu(a["V_ptr"], "V_ptr")
    M = need_gpu(a["M_ptr"], "M_ptr")
    tau = need_gpu(a["tau_ptr"], "tau_ptr")
    O = need_gpu(a["Vhat_ptr"], "Vhat_ptr")
    if O.dtype != V.dtype:
        raise TypeError("Vhat_ptr must have V_ptr's dtype")
    nb, T, F = ival(a["B"], "B"), ival(a["T"], "T"), ival(a["F"], "F")
    K, FT = ival(a["K"], "K"), ival(a["FTILE"], "FTILE")
    g = lambda k: ival(a[k], k)  # noqa: E731
    gb, gt, gf = grid
    if gb > nb or gt > T:
        raise ValueError(f"grid {grid} exceeds (B, T) = ({nb}, {T})")
    if FT <= 0:
        raise ValueError("FTILE must be positive")
    fc = min(F, gf * FT)
    extent(V, span([(gb, g("stride_vb")), (T, g("stride_vt")), (fc, 1)]), "V_ptr")
    extent(M, span([(gb, g("stride_mb")), (T, g("stride_mt")), (fc, 1)]), "M_ptr")
    extent(tau, span([(gb, g("stride_tb")), (T, g("stride_tt"))]), "tau_ptr")
    extent(O, span([(gb, g("stride_ob")), (gt, g("stride_ot")), (fc, 1)]), "Vhat_ptr")
    ws = interp_workspace(T, F, K, FT, gb, gt, gf, V.device)
    _lib.call("tssm_time_aware_interp", dcode(V, "V_ptr"), dcode(M, "M_ptr"),
              dcode(tau, "tau_ptr"), V.data_ptr(), M.data_ptr(), tau.data_ptr(), O.data_ptr(),
              nb, T, F, g("stride_vb"), g("stride_vt"), g("stride_mb"), g("stride_mt"),
              g("stride_tb"), g("stride_tt"), g("stride_ob"), g("stride_ot"), K, FT, gb, gt, gf,
              ws.data_ptr(), ws.numel(), stream_handle(V))


def interp_workspace(T, F, K, FTILE, gb, gt, gf, device):
    """Scratch for the per-(b, t, tile) observed flags (freed by torch's
    caching allocator after the launch is enqueued)."""
    n = _lib.lib().tssm_time_aware_interp_workspace_bytes(T, F, K, FTILE, gb, gt, gf)
    if n < 0:
        raise ValueError("invalid interpolation sizes")
    return torch.empty(max(int(n), 1), dtype=torch.uint8, device=device)


fused_time_aware_interp_kernel = HipKernel(
    "fused_time_aware_interp_kernel", _PARAMS, _launch_interp, "fused_interp_kernel.py:10-100")
fused_interp_bf16_kernel = HipKernel(
    "fused_interp_bf16_kernel", _PARAMS, _launch_interp, "fused_interp_kernel.py:104-181")
fused_interp_fp16_kernel = HipKernel(
    "fused_interp_fp16_kernel", _PARAMS, _launch_interp, "fused_interp_kernel.py:187-257")
