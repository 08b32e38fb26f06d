"""tssm -- MI355X (gfx950) selective-SSM kernels behind a C ABI.

The reference-named modules next to this package (``discretize_kernel``,
``ssm_scan``, ``multihead_ssm_kernel``, ``fused_interp_kernel``,
``fused_ssm_interp``, ``streaming_inference_kernel``) are the drop-in surface;
this package holds the shared host code: the ctypes binding (``_lib``), the
Triton-convention launchers (``launch``), look-back workspaces
(``workspace``), the fused entry points (``fused``), the opt-in corrected
interpolation (``corrected``) and the seeded synthetic workloads
(``workloads``).
"""
from . import _lib, launch, workspace  # noqa: F401
from ._lib import TssmError  # noqa: F401
from .corrected import streaming_interp_step_corrected, time_aware_interp_corrected  # noqa: F401
from .fused import (fused_interp_ssm_forward, multihead_ssm_forward,  # noqa: F401
                    selective_scan_forward, ssd_scan_forward, ssd_stream_step)
from .workspace import check  # noqa: F401

__all__ = ["multihead_ssm_forward", "selective_scan_forward", "ssd_scan_forward",
           "ssd_stream_step", "fused_interp_ssm_forward", "time_aware_interp_corrected",
           "streaming_interp_step_corrected", "check", "TssmError"]
