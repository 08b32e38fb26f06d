"""Opt-in corrected interpolation on the GPU against the float64 oracle:
offline (per-feature neighbours, observed values kept) and the streaming
step (per-feature forward fill)."""
import numpy as np
import pytest
import torch

from helpers import TOL, assert_close, np64
from oracle import ssm_oracle as O

pytestmark = pytest.mark.gpu


def _inputs(Bsz, T, F, dtype, mdtype, p, seed, dev):
    g = torch.Generator().manual_seed(seed)
    tau = torch.sort(torch.rand(Bsz, T, generator=g) * 50, dim=1).values
    M = (torch.rand(Bsz, T, F, generator=g) < p).to(mdtype)
    V = torch.randn(Bsz, T, F, generator=g).to(dtype)
    return V.to(dev), M.to(dev), tau.to(dev)


@pytest.mark.parametrize("Bsz,T,F,K,p,dtype,mdtype", [
    (2, 150, 100, 10, 0.3, torch.float32, torch.float32),
    (3, 64, 64, 5, 0.05, torch.bfloat16, torch.bfloat16),
    (1, 300, 130, 64, 0.02, torch.float32, torch.float16),     # K = 64, ragged tiles
    (2, 70, 7, 0, 0.5, torch.float16, torch.float32),           # K = 0: identity
    (2, 200, 256, 10, 0.3, torch.float32, torch.float32),       # 16-byte staging path
    (1, 333, 128, 64, 0.05, torch.float32, torch.float32),      # 16-byte staging, K = 64
    (1, 150, 128, 80, 0.02, torch.float32, torch.float32)])     # window past LDS staging
def test_interp_corrected(dev, Bsz, T, F, K, p, dtype, mdtype):
    from tssm import time_aware_interp_corrected
    V, M, tau = _inputs(Bsz, T, F, dtype, mdtype, p, 10 + K, dev)
    out = time_aware_interp_corrected(V, M, tau, K=K)
    torch.cuda.synchronize()
    ref = O.time_aware_interp_corrected(V, M, tau, K)
    tol = 1e-6 if dtype == torch.float32 else TOL[dtype]
    assert_close(out, ref, tol, "corrected interp")
    obs = np64(M) > 0.5
    assert np.array_equal(np64(out)[obs], np64(V)[obs])       # observed values kept


def test_interp_corrected_strided_and_out(dev):
    from tssm import time_aware_interp_corrected
    V, M, tau = _inputs(2, 80, 40, torch.float32, torch.float32, 0.2, 3, dev)
    Vw = torch.zeros(2, 80, 48, device=dev)
    Vw[..., :40] = V
    Vs = Vw[..., :40]                                          # row stride 48
    out = torch.full((2, 80, 40), float("nan"), device=dev)
    time_aware_interp_corrected(Vs, M, tau, K=7, out=out)
    torch.cuda.synchronize()
    assert_close(out, O.time_aware_interp_corrected(V, M, tau, 7), 1e-6, "strided")
    with pytest.raises(ValueError):   # flags of 64 + 2K rows must fit the workgroup's LDS
        time_aware_interp_corrected(V, M, tau, K=450)


@pytest.mark.parametrize("S,H,KR", [(3, 100, 5), (4, 1000, 11),   # 16-byte rows
                                    (3, 130, 17),                 # H % 4 != 0: scalar rows
                                    (2, 64, 24)])                 # 24: slot walk
def test_streaming_corrected(dev, S, H, KR):
    from tssm import streaming_interp_step_corrected
    g = torch.Generator().manual_seed(S + H)
    ring_V = torch.zeros(S, KR, H, device=dev)
    ring_M = torch.zeros_like(ring_V)
    ring_tau = torch.zeros(S, KR, device=dev)
    head = torch.zeros(S, dtype=torch.int32, device=dev)
    h = torch.randn(S, H, generator=g).to(dev)
    Ab, Bb, D = (torch.rand(H, generator=g).to(dev) for _ in range(3))
    st = [np64(ring_V), np64(ring_M), np64(ring_tau), np.zeros(S, dtype=np.int64), np64(h)]
    for step in range(KR + 6):
        m = (torch.rand(S, H, generator=g) < (0.0 if step % 4 == 2 else 0.2)).float().to(dev)
        v = torch.randn(S, H, generator=g).to(dev) * m
        tau = torch.full((S,), float(step), device=dev)
        C = torch.randn(S, H, generator=g).to(dev)
        y = torch.empty_like(v)
        streaming_interp_step_corrected(ring_V, ring_M, ring_tau, head, v, m, tau, h, Ab, Bb, C,
                                        D, y)
        out = O.streaming_interp_step_corrected(*st[:4], v, m, tau, st[4], Ab, Bb, C, D, KR)
        st = list(out[:5])
        torch.cuda.synchronize()
        assert_close(y, out[5], 1e-5, f"y step {step}")
        assert np.array_equal(head.cpu().numpy(), out[3])
    assert_close(h, st[4], 1e-5, "h")
    assert_close(ring_V, st[0], 0, "ring_V")
