"""The C restatement (timed CPU baseline) agrees with the float64 oracle."""
import numpy as np
import pytest

from helpers import assert_close
from oracle import cport
from oracle import ssm_oracle as O


@pytest.mark.parametrize("disc", ["euler", "zoh"])
@pytest.mark.parametrize("per_head", [False, True])
def test_multihead(disc, per_head):
    r = np.random.default_rng(1)
    Bsz, L, nh, hd = 2, 130, 3, 16
    u = r.normal(size=(Bsz, L, nh * hd))
    A_log = r.uniform(0, np.log(16), size=(nh,) if per_head else (nh, hd))
    B, C = r.normal(size=(Bsz, L, nh, hd)) / 4, r.normal(size=(Bsz, L, nh, hd)) / 4
    dt = r.uniform(0.001, 2.0, size=(Bsz, L, nh))
    D = r.normal(size=nh * hd)
    y, hl = cport.multihead_scan(u, A_log, B, C, dt, D, disc=disc)
    Af = np.repeat(A_log[:, None], hd, 1) if per_head else A_log
    y_ref, h_ref = O.multihead_forward(u, Af, B, C, dt, D, disc=disc)
    assert_close(y, y_ref, 1e-5, "y")
    assert_close(hl, h_ref, 1e-5, "h")


def test_ssd_selective_stream():
    r = np.random.default_rng(2)
    Bsz, L, H, P, N = 2, 60, 2, 8, 4
    x = r.normal(size=(Bsz, L, H, P))
    dt = np.exp(r.normal(-3, 1.5, size=(Bsz, L, H)))
    A_log = r.uniform(0, np.log(16), size=H)
    B, C = r.normal(size=(Bsz, L, H, N)) / 2, r.normal(size=(Bsz, L, H, N)) / 2
    D = r.normal(size=(H, P))
    h0 = r.normal(size=(Bsz, H, P, N))
    y, hl = cport.ssd_scan(x, dt, A_log, B, C, D, h0)
    y_ref, h_ref = O.ssd_scan(x, dt, A_log, B, C, D, h0)
    assert_close(y, y_ref, 1e-5, "ssd y")
    assert_close(hl, h_ref, 1e-5, "ssd h")
    state = np.zeros((Bsz, H, P, N), np.float32)
    st_ref = np.zeros((Bsz, H, P, N))
    for t in range(5):
        dts = dt[:, t, 0]
        ys = cport.ssd_stream_step(x[:, t], dts, A_log, B[:, t], C[:, t], D, state)
        yr = O.ssd_stream_step(x[:, t], dts, A_log, B[:, t], C[:, t], D, st_ref)
        assert_close(ys, yr, 1e-5, "stream y")
    xs = r.normal(size=(Bsz, L, 6))
    dts = r.uniform(0.001, 0.2, size=(Bsz, L))
    Al = r.uniform(np.log(0.5), np.log(5), size=(6, N))
    Bm, Cm = r.normal(size=(Bsz, L, N)) / 2, r.normal(size=(Bsz, L, N)) / 2
    y, hl = cport.selective_scan(xs, dts, Al, Bm, Cm, np.ones(6))
    y_ref, h_ref = O.selective_scan(xs, dts, Al, Bm, Cm, np.ones(6))
    assert_close(y, y_ref, 1e-5, "mamba1 y")
    assert cport.threads() >= 1


def test_interp():
    r = np.random.default_rng(3)
    Bsz, T, F = 2, 90, 40
    # fp32 inputs for both sides: the weight (tau_t - tau_p) / (tau_n - tau_p)
    # amplifies timestamp rounding
    tau = np.sort(r.uniform(0, 10, size=(Bsz, T)), axis=1).astype(np.float32)
    M = (r.random((Bsz, T, F)) < 0.05).astype(np.float32)
    V = (r.normal(size=(Bsz, T, F)) * M).astype(np.float32)
    for K, FT in ((10, 128), (3, 8)):
        out = cport.time_aware_interp(V, M, tau, K, FT)
        assert_close(out, O.time_aware_interp(V, M, tau, K, FT), 1e-6, f"interp K={K} FTILE={FT}")
