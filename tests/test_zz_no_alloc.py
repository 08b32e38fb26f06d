"""GPU parity of the no-allocation entry point tssm_mh_scan_fused_noalloc
against tssm_mh_scan_fused (same kernel, caller workspace), called through the
C ABI: two calls in a row, the second smaller, so the second runs over the
fixed scratch the first left behind.  Also: a problem larger than the scratch
is refused before any launch, the scratch's look-back error word reads 0, and
one launch captured in a HIP graph takes a fresh look-back tag on every replay
(the scratch's epoch is advanced on the device by a kernel captured with the
scan; a tag fixed at capture would let a tile fold the previous replay's
words): three replays with new inputs copied into the captured buffers and
eager work between them, each checked against the eager result and the
float64 oracle.
"""
import ctypes

import numpy as np
import pytest
import torch

from helpers import assert_close
from oracle import ssm_oracle as O
from tssm import _lib, workspace

pytestmark = pytest.mark.gpu


def _inputs(dev, Bsz, L, nh, hd, seed):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(Bsz, L, nh * hd, generator=g)
    B = torch.randn(Bsz, L, nh, hd, generator=g) / hd ** 0.5
    C = torch.randn(Bsz, L, nh, hd, generator=g) / hd ** 0.5
    dt = torch.nn.functional.softplus(torch.randn(Bsz, L, nh, generator=g)) * \
        torch.empty(Bsz, L, 1).exponential_(1.0, generator=g)
    A_log = torch.rand(nh, generator=g) * np.log(16.0)
    D = torch.randn(nh * hd, generator=g)
    h0 = torch.randn(Bsz, nh, hd, generator=g)
    return {k: v.to(dev) for k, v in dict(u=u, B=B, C=C, dt=dt, A_log=A_log, D=D, h0=h0).items()}


def _args(d, y, h_last, chunk):
    u, B, C, dt = d["u"], d["B"], d["C"], d["dt"]
    Bsz, L, nh, hd = B.shape
    return [_lib.F32, _lib.DISC_ZOH, u.data_ptr(), d["A_log"].data_ptr(), B.data_ptr(),
            C.data_ptr(), dt.data_ptr(), d["D"].data_ptr(), d["h0"].data_ptr(), y.data_ptr(),
            h_last.data_ptr(), Bsz, L, nh, hd, 1, u.stride(0), u.stride(1), B.stride(0),
            B.stride(1), B.stride(2), C.stride(0), C.stride(1), C.stride(2), dt.stride(0),
            dt.stride(1), dt.stride(2), y.stride(0), y.stride(1), chunk]


def _both(dev, d, chunk=128):
    """y and h_last from the workspace entry point and from the no-allocation one."""
    Bsz, L, nh, hd = d["B"].shape
    stream = torch.cuda.current_stream(dev).cuda_stream
    lib = _lib.lib()
    nbytes = lib.tssm_mh_scan_workspace_bytes(Bsz, L, nh, hd, chunk)
    assert 0 < nbytes <= _lib_scratch_bytes()
    ws = workspace.get(dev, stream, nbytes)
    y_ws, y_na = torch.empty_like(d["u"]), torch.empty_like(d["u"])
    h_ws, h_na = (torch.empty(Bsz, nh, hd, device=dev) for _ in range(2))
    _lib.call("tssm_mh_scan_fused", *_args(d, y_ws, h_ws, chunk), ws.data_ptr(), ws.numel(),
              stream)
    _lib.call("tssm_mh_scan_fused_noalloc", *_args(d, y_na, h_na, chunk), stream)
    torch.cuda.synchronize()
    return (y_ws, h_ws), (y_na, h_na)


def _lib_scratch_bytes():
    return 16 << 20   # TSSM_NOALLOC_SCRATCH_BYTES in include/tssm.h


def _error_word():
    out = ctypes.c_int(-1)
    _lib.call("tssm_workspace_error", None, 1, ctypes.byref(out))
    return out.value


def test_noalloc_matches_workspace_entry_point(dev):
    # first call: 64 rows x 32 chunks of carry words; second: fewer rows and
    # chunks, over what the first left in the scratch
    for shape, seed in (((4, 4096, 16, 64), 1), ((2, 1000, 8, 64), 2)):
        d = _inputs(dev, *shape, seed=seed)
        (y_ws, h_ws), (y_na, h_na) = _both(dev, d)
        assert_close(y_na, y_ws, 1e-5, f"noalloc y {shape}")
        assert_close(h_na, h_ws, 1e-5, f"noalloc h_last {shape}")
    assert _error_word() == 0


def test_noalloc_refuses_more_than_its_scratch(dev):
    d = _inputs(dev, 1, 64, 1, 64, seed=3)
    y, h = torch.empty_like(d["u"]), torch.empty(1, 1, 64, device=dev)
    args = _args(d, y, h, 128)
    # claim a problem whose look-back words exceed the scratch: refused on the
    # host, before the (too large) sizes could reach a kernel
    args[11:14] = [64, 8192, 16]
    lib = _lib.lib()
    assert lib.tssm_mh_scan_workspace_bytes(64, 8192, 16, 64, 128) > _lib_scratch_bytes()
    stream = torch.cuda.current_stream(dev).cuda_stream
    assert lib.tssm_mh_scan_fused_noalloc(*args, stream) == -8
    with pytest.raises(ValueError, match="TSSM_ERR_SCRATCH"):
        _lib.call("tssm_mh_scan_fused_noalloc", *args, stream)


def test_noalloc_graph_replays_take_fresh_tags(dev):
    shape = (2, 2048, 8, 64)
    Bsz, L, nh, hd = shape
    d = _inputs(dev, *shape, seed=4)
    y = torch.empty_like(d["u"])
    h = torch.empty(Bsz, nh, hd, device=dev)
    # first call on the device outside capture: resolves the scratch address
    _lib.call("tssm_mh_scan_fused_noalloc", *_args(d, y, h, 128),
              torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _lib.call("tssm_mh_scan_fused_noalloc", *_args(d, y, h, 128),
                  torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    for seed in (5, 6, 7):
        new = _inputs(dev, *shape, seed=seed)
        for k in d:
            d[k].copy_(new[k])
        g.replay()
        torch.cuda.synchronize()
        y_g, h_g = y.clone(), h.clone()
        (y_ws, h_ws), _ = _both(dev, d)      # eager work between the replays
        assert_close(y_g, y_ws, 1e-5, f"graph replay seed {seed}: y vs eager")
        assert_close(h_g, h_ws, 1e-5, f"graph replay seed {seed}: h_last vs eager")
        A_log = d["A_log"][:, None].expand(nh, hd)     # one decay per head
        y_ref, h_ref = O.multihead_forward(d["u"], A_log, d["B"], d["C"], d["dt"], d["D"],
                                           disc="zoh", h0=d["h0"])
        e = assert_close(y_g, y_ref, 1e-5, f"graph replay seed {seed}: y vs oracle")
        assert_close(h_g, h_ref, 1e-5, f"graph replay seed {seed}: h_last vs oracle")
        print(f"graph replay seed {seed}: relerr {e:.2e}", flush=True)
    assert _error_word() == 0
