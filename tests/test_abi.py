"""CPU checks of the C ABI and the launcher plumbing (no GPU compute).

* the built library loads and exports every function include/tssm.h declares;
* argument errors come back as negative status codes before anything is
  launched (NULL pointers), and map to ValueError;
* the Triton-convention launchers bind the reference parameter lists.
"""
import ctypes

import pytest
import torch

from tssm import _lib
from tssm.launch import HipKernel, normalize_grid, span


def test_header_parses_and_library_exports_every_symbol():
    decl = _lib.declared_functions()
    assert len(decl) >= 18
    cdll = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in decl if not hasattr(cdll, n)]
    assert not missing, missing
    assert _lib.lib().tssm_abi_version() >= 1


def test_strerror_and_status_mapping():
    assert _lib.strerror(0) == "ok"
    assert "NULL" in _lib.strerror(-1)
    with pytest.raises(ValueError, match="TSSM_ERR_NULL"):
        _lib.check(-1, "x")
    with pytest.raises(_lib.TssmError):
        _lib.check(1, "x")


def test_null_pointers_rejected_before_launch():
    L = _lib.lib()
    assert L.tssm_carry_scan(0, None, 4, 8, 0, 4, None) == -1
    assert L.tssm_ssm_fwd_local(0, None, None, None, None, None, None, 1, 1, 1, 1, 1, 1, 1, None) == -1
    assert L.tssm_mh_scan_workspace_bytes(8, 4096, 16, 64, 128) > 0
    assert L.tssm_mh_scan_workspace_bytes(8, 4096, 16, 12, 128) == -1   # head_dim % 8 != 0
    with pytest.raises(ValueError):
        _lib.call("tssm_time_aware_interp", 0, 0, 0, None, None, None, None, 1, 1, 1,
                  1, 1, 1, 1, 1, 1, 1, 1, 10, 128, 1, 1, 1, None, 0, None)


def test_every_reference_symbol_is_exported():
    import discretize_kernel, fused_interp_kernel, fused_ssm_interp  # noqa: E401
    import multihead_ssm_kernel, ssm_scan, streaming_inference_kernel  # noqa: E401
    expect = {
        discretize_kernel: ["zoh_discretize_diag_kernel", "zoh_discretize_diag_bf16_kernel",
                            "zoh_discretize_bwd_kernel", "dt_project_softplus_kernel"],
        ssm_scan: ["_combine", "ssm_fwd_local_kernel", "ssm_carry_scan_kernel",
                   "ssm_fwd_apply_kernel", "ssm_output_kernel", "_combine_bwd",
                   "ssm_bwd_local_kernel", "ssm_bwd_carry_scan_kernel", "ssm_bwd_apply_kernel",
                   "_nxt_pow2", "ssm_forward", "ssm_backward"],
        multihead_ssm_kernel: ["_scan_combine", "multihead_ssm_fwd_local_kernel",
                               "multihead_ssm_carry_scan_kernel", "multihead_ssm_output_kernel",
                               "residual_add_kernel", "dropout_residual_kernel"],
        fused_interp_kernel: ["fused_time_aware_interp_kernel", "fused_interp_bf16_kernel",
                              "fused_interp_fp16_kernel"],
        fused_ssm_interp: ["_combine_fwd", "fused_interp_ssm_step_kernel", "layernorm_kernel",
                           "layernorm_bwd_kernel", "swiglu_kernel", "swiglu_bwd_kernel"],
        streaming_inference_kernel: ["streaming_ssm_inplace_kernel",
                                     "streaming_ssm_inplace_bf16_kernel",
                                     "streaming_interp_then_ssm_kernel",
                                     "mean_pool_logit_kernel", "masked_fill_zero_kernel"],
    }
    for mod, names in expect.items():
        for n in names:
            assert hasattr(mod, n), f"{mod.__name__}.{n}"


def test_reference_parameter_lists():
    import multihead_ssm_kernel as mk
    import ssm_scan as ss
    assert mk.multihead_ssm_fwd_local_kernel.arg_names[:8] == [
        "u_ptr", "A_log_ptr", "B_ptr", "C_ptr", "dt_ptr", "loc_a_ptr", "loc_x_ptr", "carry_ptr"]
    assert len(mk.multihead_ssm_fwd_local_kernel.arg_names) == 32
    assert len(mk.multihead_ssm_output_kernel.arg_names) == 22
    assert ss.ssm_fwd_local_kernel.arg_names == [
        "u_ptr", "A_ptr", "B_ptr", "loc_a_ptr", "loc_x_ptr", "carry_ptr", "B", "L", "H", "BLK", "NBLK"]
    assert ss._nxt_pow2(1) == 1 and ss._nxt_pow2(5) == 8 and ss._nxt_pow2(8) == 8
    assert ss._combine(2.0, 3.0, 5.0, 7.0) == (10.0, 22.0)
    assert ss._combine_bwd(2.0, 3.0, 5.0, 7.0) == (10.0, 22.0)


def test_launcher_binding():
    seen = {}

    def launch(grid, bound):
        seen["grid"], seen["bound"] = grid, bound

    k = HipKernel("k", ["a_ptr", "n", "BLOCK"], launch, "x.py:1")
    k[(3, 2)](1, 2, BLOCK=64, num_warps=4)
    assert seen["grid"] == (3, 2, 1) and seen["bound"] == {"a_ptr": 1, "n": 2, "BLOCK": 64}
    k[lambda meta: (meta["n"],)](1, 5, 8)
    assert seen["grid"] == (5, 1, 1)
    with pytest.raises(TypeError):
        k[(1,)](1, 2)                 # missing BLOCK
    with pytest.raises(TypeError):
        k[(1,)](1, 2, 3, bogus=1)     # unknown keyword
    with pytest.raises(TypeError):
        k(1, 2, 3)                    # must be launched with a grid
    assert normalize_grid(4) == (4, 1, 1)
    assert span([(3, 10), (2, 1)]) == 21 and span([(0, 5)]) == -1


def test_layer_launchers_validate_on_host():
    """Model-layer drop-ins bind the reference's parameter lists and reject
    host tensors before any library call."""
    import fused_ssm_interp as fs
    import multihead_ssm_kernel as mk
    import streaming_inference_kernel as sk
    x = torch.zeros(2, 3, 8)
    w = torch.zeros(8)
    with pytest.raises(ValueError):
        fs.layernorm_kernel[(2, 3)](x, w, w, x, 2, 3, 8, 24, 8, 1, 1e-5, 8)
    with pytest.raises(ValueError):
        fs.swiglu_kernel[(2, 3)](x, x, x, 2, 3, 8, 24, 8, BLOCK_H=8)
    with pytest.raises(ValueError):
        mk.residual_add_kernel[(1,)](x, x, x, 48, BLOCK=64)
    with pytest.raises(ValueError):
        sk.masked_fill_zero_kernel[(1,)](x, torch.ones(2, 3), x, 2, 3, 8, BLOCK=64)
    with pytest.raises(TypeError):
        sk.mean_pool_logit_kernel[(2,)](x, w, w, w)   # missing arguments


def test_selective_scan_path_query():
    """tssm_selective_scan_takes_passes (host logic only): which problems the
    three-pass path takes, so the caller can give it a raw-float workspace."""
    L = _lib.lib()
    F32, BF16, F16 = _lib.F32, _lib.BF16, _lib.F16
    A = 1 << 20   # 16-byte aligned stand-in addresses (never dereferenced)
    # interpolation workload's scan: dt shared (timestamps), 16 x 4 x 64 blocks
    assert L.tssm_selective_scan_takes_passes(F32, 16, 2048, 256, 16, 0, 1, A, None, None, 0,
                                              0, 0, 0) == 1
    # too few blocks of 64 channels x 32 steps, N outside {8, 16}, fp16 I/O
    assert L.tssm_selective_scan_takes_passes(F32, 2, 256, 16, 16, 0, 0, A, None, None, 0,
                                              0, 0, 0) == 0
    assert L.tssm_selective_scan_takes_passes(F32, 16, 2048, 256, 32, 0, 0, A, None, None, 0,
                                              0, 0, 0) == 0
    assert L.tssm_selective_scan_takes_passes(F16, 16, 2048, 256, 16, 0, 0, A, None, None, 0,
                                              0, 0, 0) == 0
    # per-channel timestamps are not supported by the passes
    assert L.tssm_selective_scan_takes_passes(BF16, 16, 2048, 256, 16, 1, 1, A, None, None, 0,
                                              0, 0, 0) == 0
    # projected dt: 16-byte raw rows of rank 16 take the passes; rank 7 does not
    assert L.tssm_selective_scan_takes_passes(F32, 16, 2048, 256, 16, 1, 0, A, A, A, 16,
                                              2048 * 16, 16, 256) == 1
    assert L.tssm_selective_scan_takes_passes(F32, 16, 2048, 256, 16, 1, 0, A, A, A, 7,
                                              2048 * 7, 7, 256) == 0
    assert L.tssm_selective_scan_takes_passes(F32, 16, 2048, 256, 16, 1, 0, A + 4, A, A, 16,
                                              2048 * 16, 16, 256) == 0   # unaligned raw rows
    # the dtproj workspace adds the produced-dt table to the passes' workspace
    base = L.tssm_selective_scan_workspace_bytes(16, 2048, 256, 16, 256)
    big = L.tssm_selective_scan_dtproj_workspace_bytes(16, 2048, 256, 16, 256)
    assert big >= base + 16 * 2048 * 256 * 4
