"""GPU: the no-allocation entry point captured in a HIP graph and replayed.

Each replay must take a fresh look-back tag (the scratch's epoch is advanced
on the device by a kernel captured with the scan), or a tile could fold the
previous replay's words as its own.  One launch is captured; it is replayed
three times with new inputs copied into the captured buffers, with eager work
(the workspace entry point on the same inputs) and a synchronisation between
the replays; every replay is checked against that eager result and against
the float64 oracle.
"""
import pytest
import torch

from helpers import assert_close
from oracle import ssm_oracle as O
from tssm import _lib
from test_zz_no_alloc import _args, _both, _error_word, _inputs

pytestmark = pytest.mark.gpu


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
