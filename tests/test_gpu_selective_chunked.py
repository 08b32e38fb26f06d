"""GPU parity of the three-pass Mamba-1 selective scan (csrc/selective.hip:
chunk end states, carry scan over chunks, outputs), which tssm_selective_scan
runs for N = 8 or 16 states, fp32 or bf16 I/O and at least 512 waves of 64
channels x 32 steps.  Every case here is above that size (Dc = 320 leaves a
partially filled workgroup, L = 1700 a partial last chunk) and is checked
against the float64 oracle (oracle/ssm_oracle.py selective_scan, the
recurrence of discretize_kernel.py:16-57 and ssm_scan.py:239-264)."""
import numpy as np
import pytest
import torch

from helpers import TOL, assert_close, np64
from oracle import ssm_oracle as O

pytestmark = pytest.mark.gpu

BSZ, L, DC = 2, 1700, 320   # 2 x ceil(320/64) x ceil(1700/32) = 540 waves


def _inputs(dev, N, dtype, dt_mode, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(BSZ, L, DC, generator=g).to(dtype)
    if dt_mode == "tau":
        # timestamps with gaps of mean 0.05; dt_0 = tau_0
        tau = torch.cumsum(torch.empty(BSZ, L).exponential_(20.0, generator=g), 1)
        dt_in, dt_ref = tau, torch.diff(tau, dim=1, prepend=torch.zeros(BSZ, 1))
    else:
        shape = (BSZ, L, DC) if dt_mode == "channel" else (BSZ, L)
        dt_in = torch.empty(shape).exponential_(20.0, generator=g).clamp_(1e-3, 1.0)
        dt_ref = dt_in
    A_log = torch.empty(DC, N).uniform_(np.log(0.5), np.log(5.0), generator=g)
    Bm = (torch.randn(BSZ, L, N, generator=g) / N ** 0.5).to(dtype)
    Cm = (torch.randn(BSZ, L, N, generator=g) / N ** 0.5).to(dtype)
    D = torch.randn(DC, generator=g)
    h0 = torch.randn(BSZ, DC, N, generator=g)
    host = dict(x=x, dt=dt_ref, A_log=A_log, B=Bm, C=Cm, D=D, h0=h0)
    gpu = {k: v.to(dev) for k, v in dict(host, dt=dt_in).items()}
    return host, gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("disc", ["zoh", "euler"])
@pytest.mark.parametrize("N", [8, 16])
@pytest.mark.parametrize("dt_mode", ["shared", "channel", "tau"])
def test_three_pass_selective_scan(dev, dtype, disc, N, dt_mode):
    from tssm import selective_scan_forward
    host, d = _inputs(dev, N, dtype, dt_mode, seed=N * 10 + len(dt_mode))
    y, h = selective_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], d["D"],
                                  h0=d["h0"], disc=disc, return_state=True,
                                  dt_is_tau=dt_mode == "tau")
    torch.cuda.synchronize()
    y_ref, h_ref = O.selective_scan(host["x"], host["dt"], host["A_log"], host["B"], host["C"],
                                    host["D"], h0=np64(host["h0"]), disc=disc)
    assert_close(y, y_ref, TOL[dtype], f"three-pass y {dtype} {disc} N={N} dt={dt_mode}")
    assert_close(h, h_ref, TOL[dtype], "three-pass h_last")


def test_three_pass_many_chunks(dev):
    """1 x 9000 steps: 282 chunks per sequence, so the carry pass walks eight
    full register batches of 32 chunks and a remainder of 26."""
    from tssm import selective_scan_forward
    g = torch.Generator().manual_seed(11)
    Lm, Dm, N = 9000, 128, 16
    x = torch.randn(1, Lm, Dm, generator=g)
    dt = torch.empty(1, Lm).exponential_(20.0, generator=g).clamp_(1e-3, 1.0)
    A_log = torch.empty(Dm, N).uniform_(np.log(0.5), np.log(5.0), generator=g)
    Bm = torch.randn(1, Lm, N, generator=g) / N ** 0.5
    Cm = torch.randn(1, Lm, N, generator=g) / N ** 0.5
    h0 = torch.randn(1, Dm, N, generator=g)
    y, h = selective_scan_forward(*(t.to(dev) for t in (x, dt, A_log, Bm, Cm)), None,
                                  h0=h0.to(dev), return_state=True)
    torch.cuda.synchronize()
    y_ref, h_ref = O.selective_scan(x, dt, A_log, Bm, Cm, h0=np64(h0))
    assert_close(y, y_ref, 1e-5, "three-pass y, 282 chunks")
    assert_close(h, h_ref, 1e-5, "three-pass h_last, 282 chunks")


def test_three_pass_without_skip_or_state_and_reuse(dev):
    """No D, no h0, no h_last; then a second, smaller call on the same stream
    (the workspace is reused) whose result must not depend on the first."""
    from tssm import selective_scan_forward
    host, d = _inputs(dev, 16, torch.float32, "shared", seed=7)
    y = selective_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], None)
    x2 = d["x"][:, : L - 40].contiguous()
    B2, C2, dt2 = (d[k][:, : L - 40].contiguous() for k in ("B", "C", "dt"))
    y2 = selective_scan_forward(x2, dt2, d["A_log"], B2, C2, None)
    torch.cuda.synchronize()
    y_ref, _ = O.selective_scan(host["x"], host["dt"], host["A_log"], host["B"], host["C"])
    assert_close(y, y_ref, 1e-5, "three-pass y, no skip term")
    assert_close(y2, y_ref[:, : L - 40], 1e-5, "three-pass prefix")


@pytest.mark.parametrize("dt_mode", ["shared", "channel"])
def test_three_pass_few_chunks_ragged_lanes(dev, dt_mode):
    """L = 70: three chunks, so of the carry pass's four waves per lane group
    the last walks no chunk (its entry state is h_last); Dc = 100 with N = 8
    gives 800 (d, n) entries per batch, a partial last group of 64 lanes."""
    from tssm import selective_scan_forward
    g = torch.Generator().manual_seed(23)
    Bn, Lm, Dm, N = 100, 70, 100, 8
    x = torch.randn(Bn, Lm, Dm, generator=g)
    shape = (Bn, Lm, Dm) if dt_mode == "channel" else (Bn, Lm)
    dt = torch.empty(shape).exponential_(20.0, generator=g).clamp_(1e-3, 1.0)
    A_log = torch.empty(Dm, N).uniform_(np.log(0.5), np.log(5.0), generator=g)
    Bm = torch.randn(Bn, Lm, N, generator=g) / N ** 0.5
    Cm = torch.randn(Bn, Lm, N, generator=g) / N ** 0.5
    h0 = torch.randn(Bn, Dm, N, generator=g)
    y, h = selective_scan_forward(*(t.to(dev) for t in (x, dt, A_log, Bm, Cm)), None,
                                  h0=h0.to(dev), return_state=True)
    torch.cuda.synchronize()
    y_ref, h_ref = O.selective_scan(x, dt, A_log, Bm, Cm, h0=np64(h0))
    assert_close(y, y_ref, 1e-5, f"three-pass y, 3 chunks, dt {dt_mode}")
    assert_close(h, h_ref, 1e-5, f"three-pass h_last, 3 chunks, dt {dt_mode}")


@pytest.mark.parametrize("Bn,Lm,Dm,N,dt_mode", [
    (2, 9000, 36, 8, "channel"),    # 282 chunks: 9 segments, the last of 26 chunks
    (1, 70000, 64, 16, "shared"),   # 2188 chunks: 69 segments, walked in two loads
    (3, 12000, 20, 16, "tau"),      # per-batch timestamps; 320 (d, n) lanes
])
def test_three_pass_segmented_carry(dev, Bn, Lm, Dm, N, dt_mode):
    """Few (batch, channel, state) lanes and many chunks: the carry pass folds
    segments of 32 chunks, carries over the segments and walks each segment
    again from its entry state."""
    from tssm import selective_scan_forward
    g = torch.Generator().manual_seed(Lm + Dm)
    x = torch.randn(Bn, Lm, Dm, generator=g)
    if dt_mode == "tau":
        tau = torch.cumsum(torch.empty(Bn, Lm).exponential_(20.0, generator=g), 1)
        dt_in, dt_ref = tau, torch.diff(tau, dim=1, prepend=torch.zeros(Bn, 1))
    else:
        shape = (Bn, Lm, Dm) if dt_mode == "channel" else (Bn, Lm)
        dt_in = torch.empty(shape).exponential_(40.0, generator=g).clamp_(1e-3, 1.0)
        dt_ref = dt_in
    # decays down to a = -0.2 (dt ~ 0.025): a chunk's entry state still matters
    # several chunks later, so a wrong segment entry shows in the outputs.
    # (Slower decays over 70000 steps leave h_last ~1.2e-5 from the float64
    # oracle on either form of the carry pass: the per-step exp2 rounding
    # accumulated over the state's long memory, not the carry.)
    A_log = torch.empty(Dm, N).uniform_(np.log(0.2), np.log(2.0), generator=g)
    Bm = torch.randn(Bn, Lm, N, generator=g) / N ** 0.5
    Cm = torch.randn(Bn, Lm, N, generator=g) / N ** 0.5
    h0 = torch.randn(Bn, Dm, N, generator=g)
    y, h = selective_scan_forward(x.to(dev), dt_in.to(dev), A_log.to(dev), Bm.to(dev),
                                  Cm.to(dev), None, h0=h0.to(dev), return_state=True,
                                  dt_is_tau=dt_mode == "tau")
    torch.cuda.synchronize()
    y_ref, h_ref = O.selective_scan(x, dt_ref, A_log, Bm, Cm, h0=np64(h0))
    assert_close(y, y_ref, 1e-5, f"three-pass y, segmented carry, {Bn}x{Lm}x{Dm} N={N}")
    assert_close(h, h_ref, 1e-5, f"three-pass h_last, segmented carry, {Bn}x{Lm}x{Dm} N={N}")
