"""Launchers of the model-layer kernels (LayerNorm, SwiGLU, residual/dropout,
mean-pool logit head, padding mask) behind the reference's Triton launch
convention; the reference-named modules bind them to their kernel names.

Semantics follow the reference kernels, including what their launch
parameters decide: the grid selects the rows (or the flat prefix) that are
computed, and LayerNorm's ``BLOCK_H`` enters the variance through the masked
lanes H..BLOCK_H-1 (fused_ssm_interp.py:118-123).  A ``BLOCK_H`` smaller than
H (a partial row in the reference) is rejected.  All float tensors of one
launch share one dtype (float32, bfloat16 or float16); arithmetic is fp32.
"""
from __future__ import annotations

import torch

from . import _lib
from .launch import dcode, extent, ival, need_gpu, span, stream_handle


def _same_dtype(ts: dict) -> torch.Tensor:
    first = next(iter(ts.values()))
    for k, t in ts.items():
        if t.dtype != first.dtype:
            raise TypeError(f"{k}: all float tensors of this kernel must share one dtype "
                            f"({first.dtype}), got {t.dtype}")
    dcode(first, "tensors")
    return first


def _rows(grid, a, nb_key="B", nl_key="L"):
    nb, nl = ival(a[nb_key], nb_key), ival(a[nl_key], nl_key)
    gb, gl, _ = grid
    if gb > nb or gl > nl:
        raise ValueError(f"grid {grid} exceeds ({nb_key}, {nl_key}) = ({nb}, {nl})")
    return nb, nl, gb, gl


def _block_h(a, H):
    bh = ival(a["BLOCK_H"], "BLOCK_H")
    if bh < H:
        raise ValueError(f"BLOCK_H = {bh} < H = {H}: the reference would process a partial "
                         "row; use BLOCK_H >= H")
    return bh


def _gpu(a, keys):
    return {k: need_gpu(a[k], k) for k in keys}


def launch_layernorm(grid, a):
    ts = _gpu(a, ["x_ptr", "w_ptr", "bias_ptr", "out_ptr"])
    x = _same_dtype(ts)
    nb, nl, gb, gl = _rows(grid, a)
    H = ival(a["H"], "H")
    if H <= 0:
        raise ValueError("H must be positive")
    bh = _block_h(a, H)
    sb, sl = ival(a["stride_b"], "stride_b"), ival(a["stride_l"], "stride_l")
    rows = span([(gb, sb), (gl, sl), (H, 1)])
    extent(x, rows, "x_ptr")
    extent(ts["out_ptr"], rows, "out_ptr")
    extent(ts["w_ptr"], H - 1, "w_ptr")
    extent(ts["bias_ptr"], H - 1, "bias_ptr")
    _lib.call("tssm_layernorm_fwd", dcode(x), x.data_ptr(), ts["w_ptr"].data_ptr(),
              ts["bias_ptr"].data_ptr(), ts["out_ptr"].data_ptr(), nb, nl, H, sb, sl,
              float(a["EPS"]), bh, gb, gl, stream_handle(x))


def launch_layernorm_bwd(grid, a):
    ts = _gpu(a, ["dout_ptr", "x_ptr", "w_ptr", "dx_ptr", "dw_ptr", "db_ptr"])
    _same_dtype(ts)
    x = ts["x_ptr"]
    nb, nl, gb, gl = _rows(grid, a)
    H = ival(a["H"], "H")
    if H <= 0:
        raise ValueError("H must be positive")
    bh = _block_h(a, H)
    sb, sl = ival(a["stride_b"], "stride_b"), ival(a["stride_l"], "stride_l")
    rows = span([(gb, sb), (gl, sl), (H, 1)])
    for k in ("dout_ptr", "x_ptr", "dx_ptr"):
        extent(ts[k], rows, k)
    for k in ("w_ptr", "dw_ptr", "db_ptr"):
        extent(ts[k], H - 1, k)
    L_ = _lib.lib()
    nbytes = L_.tssm_layernorm_bwd_workspace_bytes(gb, gl, H)
    ws = torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=x.device)
    _lib.call("tssm_layernorm_bwd", dcode(x), ts["dout_ptr"].data_ptr(), x.data_ptr(),
              ts["w_ptr"].data_ptr(), ts["dx_ptr"].data_ptr(), ts["dw_ptr"].data_ptr(),
              ts["db_ptr"].data_ptr(), nb, nl, H, sb, sl, float(a["EPS"]), bh, gb, gl,
              ws.data_ptr(), ws.numel(), stream_handle(x))


def _swiglu_common(grid, a, keys):
    ts = _gpu(a, keys)
    x = _same_dtype(ts)
    nb, nl, gb, gl = _rows(grid, a)
    H = ival(a["H"], "H")
    _block_h(a, H)
    sb, sl = ival(a["stride_b"], "stride_b"), ival(a["stride_l"], "stride_l")
    rows = span([(gb, sb), (gl, sl), (H, 1)])
    for k in keys:
        extent(ts[k], rows, k)
    return ts, x, nb, nl, gb, gl, H, sb, sl


def launch_swiglu(grid, a):
    keys = ["gate_ptr", "up_ptr", "out_ptr"]
    ts, x, nb, nl, gb, gl, H, sb, sl = _swiglu_common(grid, a, keys)
    _lib.call("tssm_swiglu_fwd", dcode(x), *(ts[k].data_ptr() for k in keys), nb, nl, H, sb, sl,
              gb, gl, stream_handle(x))


def launch_swiglu_bwd(grid, a):
    keys = ["dout_ptr", "gate_ptr", "up_ptr", "dgate_ptr", "dup_ptr"]
    ts, x, nb, nl, gb, gl, H, sb, sl = _swiglu_common(grid, a, keys)
    _lib.call("tssm_swiglu_bwd", dcode(x), *(ts[k].data_ptr() for k in keys), nb, nl, H, sb, sl,
              gb, gl, stream_handle(x))


def _flat_cover(grid, a, n_key, block_key="BLOCK"):
    n = ival(a[n_key], n_key)
    blk = ival(a[block_key], block_key)
    if n < 0 or blk <= 0:
        raise ValueError(f"{n_key} must be >= 0 and {block_key} > 0")
    return min(n, grid[0] * blk)


def launch_residual_add(grid, a):
    ts = _gpu(a, ["x_ptr", "res_ptr", "out_ptr"])
    x = _same_dtype(ts)
    n = _flat_cover(grid, a, "N")
    for k, t in ts.items():
        extent(t, n - 1, k)
    _lib.call("tssm_residual_add", dcode(x), x.data_ptr(), ts["res_ptr"].data_ptr(), None,
              ts["out_ptr"].data_ptr(), n, 1.0, stream_handle(x))


def launch_dropout_residual(grid, a):
    ts = _gpu(a, ["x_ptr", "res_ptr", "out_ptr"])
    x = _same_dtype(ts)
    keep = need_gpu(a["mask_ptr"], "mask_ptr")
    if keep.dtype not in (torch.uint8, torch.bool):
        raise TypeError("mask_ptr must be uint8 (or bool)")
    p_keep = float(a["p_keep"])
    if not p_keep > 0.0:
        raise ValueError("p_keep must be positive")
    n = _flat_cover(grid, a, "N")
    for k, t in ts.items():
        extent(t, n - 1, k)
    extent(keep, n - 1, "mask_ptr")
    _lib.call("tssm_residual_add", dcode(x), x.data_ptr(), ts["res_ptr"].data_ptr(),
              keep.data_ptr(), ts["out_ptr"].data_ptr(), n, p_keep, stream_handle(x))


def launch_mean_pool_logit(grid, a):
    ts = _gpu(a, ["h_ptr", "W_ptr", "bias_ptr", "out_ptr"])
    h = _same_dtype(ts)
    nb, nt, gb, _ = _rows(grid, a, "B", "T")
    H = ival(a["H"], "H")
    if nt <= 0 or H <= 0:
        raise ValueError("T and H must be positive")
    sb, st = ival(a["stride_b"], "stride_b"), ival(a["stride_t"], "stride_t")
    extent(h, span([(gb, sb), (nt, st), (H, 1)]), "h_ptr")
    extent(ts["W_ptr"], H - 1, "W_ptr")
    extent(ts["bias_ptr"], 0, "bias_ptr")
    extent(ts["out_ptr"], gb - 1, "out_ptr")
    L_ = _lib.lib()
    nbytes = L_.tssm_mean_pool_logit_workspace_bytes(gb, nt)
    ws = torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=h.device)
    _lib.call("tssm_mean_pool_logit", dcode(h), h.data_ptr(), ts["W_ptr"].data_ptr(),
              ts["bias_ptr"].data_ptr(), ts["out_ptr"].data_ptr(), nb, nt, H, sb, st, gb,
              ws.data_ptr(), ws.numel(), stream_handle(h))


_MASK_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.int32: 3,
              torch.uint8: 4, torch.bool: 4}


def launch_masked_fill_zero(grid, a):
    ts = _gpu(a, ["x_ptr", "out_ptr"])
    x = _same_dtype(ts)
    m = need_gpu(a["mask_ptr"], "mask_ptr")
    if m.dtype not in _MASK_CODE:
        raise TypeError(f"mask_ptr: unsupported dtype {m.dtype}")
    nb, nt, H, blk = (ival(a[k], k) for k in ("B", "T", "H", "BLOCK"))
    if H <= 0 or nb < 0 or nt < 0 or blk <= 0:
        raise ValueError("H and BLOCK must be positive, B and T non-negative")
    n = min(nb * nt * H, grid[0] * blk)
    for k, t in ts.items():
        extent(t, n - 1, k)
    extent(m, (n - 1) // H if n > 0 else -1, "mask_ptr")
    _lib.call("tssm_masked_fill_zero", dcode(x), _MASK_CODE[m.dtype], x.data_ptr(), m.data_ptr(),
              ts["out_ptr"].data_ptr(), n, H, stream_handle(x))
