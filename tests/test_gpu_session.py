"""Streaming sessions on the GPU: a ring stream saved mid-way and restored
continues exactly as the uninterrupted stream; the SSD stream state survives
the same round trip."""
import numpy as np
import pytest
import torch

from helpers import assert_close, np64
from oracle import ssm_oracle as O
from tssm import session as S

pytestmark = pytest.mark.gpu


def _ring_inputs(B, H, steps, seed):
    g = torch.Generator().manual_seed(seed)
    out = []
    for s in range(steps):
        m = (torch.rand(B, H, generator=g) < (0.0 if s % 4 == 2 else 0.1)).float()
        v = torch.randn(B, H, generator=g) * m
        tau = torch.full((B,), 0.5 * s) + torch.rand(B, generator=g) * 0.1
        C = torch.randn(B, H, generator=g)
        out.append((v, m, tau, C))
    return out


def test_ring_session_resume(dev, tmp_path):
    B, H, K, BH, steps, cut = 3, 200, 6, 64, 25, 11
    g = torch.Generator().manual_seed(3)
    Ab, Bb, D = (torch.rand(H, generator=g).to(dev) for _ in range(3))
    seq = [tuple(t.to(dev) for t in x) for x in _ring_inputs(B, H, steps, 9)]

    whole = S.RingSession(B, H, K, block_h=BH, device=dev)
    ys = [whole.step(v, m, tau, Ab, Bb, C, D) for v, m, tau, C in seq]

    first = S.RingSession(B, H, K, block_h=BH, device=dev)
    ys2 = [first.step(v, m, tau, Ab, Bb, C, D) for v, m, tau, C in seq[:cut]]
    path = tmp_path / "ring.tssm"
    first.save(path)
    resumed = S.RingSession.load(path, device=dev)
    ys2 += [resumed.step(v, m, tau, Ab, Bb, C, D) for v, m, tau, C in seq[cut:]]
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(ys, ys2)):
        assert torch.equal(a, b), f"y differs at step {i}"
    for k in S.RingSession.FIELDS:
        assert torch.equal(getattr(whole, k), getattr(resumed, k)), k

    # and the restored stream still follows the oracle
    st = [np.zeros((B, K + 1, H)), np.zeros((B, K + 1, H)), np.zeros((B, K + 1)),
          np.zeros(B, dtype=np.int64), np.zeros((B, H))]
    for v, m, tau, C in seq:
        rV, rM, rt, hd, h_new, y_ref = O.streaming_interp_step(*st[:4], v, m, tau, st[4], Ab, Bb,
                                                               C, D, BH, K + 1)
        st = [rV, rM, rt, hd, h_new]
    assert_close(ys2[-1], y_ref, 1e-5, "y after resume")
    assert_close(resumed.h, st[4], 1e-5, "h after resume")


def test_ssd_stream_state_round_trip(dev):
    from tssm import ssd_stream_step
    g = torch.Generator().manual_seed(4)
    Sn, H, P, N = 8, 4, 64, 16
    A_log = torch.rand(H, generator=g).to(dev)
    state = torch.zeros(Sn, H, P, N, device=dev)

    def step(st, i):
        gg = torch.Generator().manual_seed(100 + i)
        x = torch.randn(Sn, H, P, generator=gg).to(dev)
        dt = (torch.rand(Sn, generator=gg) * 0.2).to(dev)
        Bm = torch.randn(Sn, H, N, generator=gg).to(dev)
        Cm = torch.randn(Sn, H, N, generator=gg).to(dev)
        return ssd_stream_step(x, dt, A_log, Bm, Cm, None, st)

    for i in range(5):
        step(state, i)
    torch.cuda.synchronize()
    blob = S.dumps({"state": state}, {"kind": "ssd_stream", "step": 5})
    out, meta = S.loads(blob, device=dev)
    assert meta["step"] == 5 and torch.equal(out["state"], state)
    restored = out["state"]
    ya = [step(state, i) for i in range(5, 9)]
    yb = [step(restored, i) for i in range(5, 9)]
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(ya, yb))
    assert torch.equal(state, restored)
