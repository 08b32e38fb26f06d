"""GPU parity of the new fused entry points (SSD scan, streaming SSD step,
Mamba-1 selective scan, interpolation + scan) against the float64 oracle."""
import numpy as np
import pytest
import torch

from helpers import TOL, assert_close, np64
from oracle import ssm_oracle as O

pytestmark = pytest.mark.gpu


def _ssd_inputs(dev, Bsz, L, H, P, N, dtype, seed, heavy=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(Bsz, L, H, P, generator=g).to(dtype)
    Bm = (torch.randn(Bsz, L, H, N, generator=g) / N ** 0.5).to(dtype)
    Cm = (torch.randn(Bsz, L, H, N, generator=g) / N ** 0.5).to(dtype)
    if heavy:
        dt = torch.exp(torch.randn(Bsz, L, H, generator=g) * 1.5 - 3.0)
    else:
        dt = torch.nn.functional.softplus(torch.randn(Bsz, L, H, generator=g)) * 0.3
    A_log = torch.rand(H, generator=g) * np.log(16.0)
    D = torch.randn(H, P, generator=g)
    return {k: v.to(dev) for k, v in dict(x=x, B=Bm, C=Cm, dt=dt, A_log=A_log, D=D).items()}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("disc", ["zoh", "euler"])
@pytest.mark.parametrize("P,N", [(64, 16), (32, 8), (48, 32), (64, 64)])
def test_ssd_scan(dev, dtype, disc, P, N):
    from tssm import ssd_scan_forward
    d = _ssd_inputs(dev, 2, 1100, 3, P, N, dtype, seed=P + N, heavy=True)
    h0 = torch.randn(2, 3, P, N, device=dev)
    y, hl = ssd_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], d["D"], disc=disc,
                             h0=h0, chunk=256, return_state=True)
    torch.cuda.synchronize()
    y_ref, h_ref = O.ssd_scan(d["x"], d["dt"], d["A_log"], d["B"], d["C"], d["D"], h0=np64(h0), disc=disc)
    assert_close(y, y_ref, TOL[dtype], f"ssd y {dtype} {disc} P={P} N={N}")
    assert_close(hl, h_ref, TOL[dtype], "ssd h_last")


@pytest.mark.parametrize("L", [100, 256, 513, 2600])
@pytest.mark.parametrize("disc", ["zoh", "euler"])
@pytest.mark.parametrize("with_d", [False, True])
def test_ssd_scan_matrix_core_path(dev, L, disc, with_d):
    """bf16, P=64, N=16, 256-step tiles run on the MFMA passes: ragged and
    sub-tile lengths, skip term, nonzero h0.  The bar is tighter than the bf16
    tolerance (the fp32 operands of the products are split hi/lo, so only the
    bf16 output rounding should remain)."""
    from tssm import ssd_scan_forward
    d = _ssd_inputs(dev, 2, L, 3, 64, 16, torch.bfloat16, seed=L + with_d, heavy=True)
    h0 = torch.randn(2, 3, 64, 16, device=dev)
    D = d["D"] if with_d else None
    y, hl = ssd_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], D, disc=disc,
                             h0=h0, chunk=256, return_state=True)
    torch.cuda.synchronize()
    y_ref, h_ref = O.ssd_scan(d["x"], d["dt"], d["A_log"], d["B"], d["C"], D, h0=np64(h0), disc=disc)
    assert_close(y, y_ref, 4e-3, f"mfma ssd y L={L} {disc} D={with_d}")
    assert_close(hl, h_ref, 1e-3, "mfma ssd h_last")


def test_ssd_scan_time_broadcast_b(dev):
    """bf16 P=64 N=16 with B broadcast over time (row stride 0): the matrix-core
    tile passes need every row stride to cover a row, so this layout runs the
    generic passes, against the same oracle."""
    from tssm import ssd_scan_forward
    d = _ssd_inputs(dev, 2, 700, 3, 64, 16, torch.bfloat16, seed=77, heavy=True)
    Bb = d["B"][:, :1].expand(-1, 700, -1, -1)
    assert Bb.stride(1) == 0
    y = ssd_scan_forward(d["x"], d["dt"], d["A_log"], Bb, d["C"], d["D"], chunk=256)
    torch.cuda.synchronize()
    y_ref, _ = O.ssd_scan(d["x"], d["dt"], d["A_log"], Bb.contiguous(), d["C"], d["D"])
    assert_close(y, y_ref, TOL[torch.bfloat16], "ssd y, B broadcast over time")


@pytest.mark.parametrize("Bsz,L,H,P", [(2, 300, 3, 64), (2, 200, 4, 32), (1, 130, 8, 48),
                                        (1, 64, 8, 16), (1, 1, 2, 64), (3, 1000, 8, 64)])
@pytest.mark.parametrize("disc", ["zoh", "euler"])
@pytest.mark.parametrize("with_d", [False, True])
def test_ssd_scan_n64_matrix_core_path(dev, Bsz, L, H, P, disc, with_d):
    """bf16 with N = 64 runs one matrix-core pass per (row, 16-channel block):
    ragged blocks of 64 steps, 1-4 channel blocks per row, row counts that are
    and are not multiples of 8 (the two block mappings), skip term, nonzero h0
    and the final state.  Same bar as the other matrix-core path."""
    from tssm import ssd_scan_forward
    d = _ssd_inputs(dev, Bsz, L, H, P, 64, torch.bfloat16, seed=L + P + with_d, heavy=True)
    h0 = torch.randn(Bsz, H, P, 64, device=dev)
    D = d["D"] if with_d else None
    y, hl = ssd_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], D, disc=disc,
                             h0=h0, chunk=256, return_state=True)
    torch.cuda.synchronize()
    y_ref, h_ref = O.ssd_scan(d["x"], d["dt"], d["A_log"], d["B"], d["C"], D, h0=np64(h0), disc=disc)
    assert_close(y, y_ref, 4e-3, f"n64 ssd y L={L} P={P} {disc} D={with_d}")
    assert_close(hl, h_ref, 1e-3, f"n64 ssd h_last L={L} P={P} {disc}")


@pytest.mark.parametrize("cut", [128, 200, 1])
def test_ssd_scan_n64_split_resume(dev, cut):
    """bf16 N = 64 on the one-pass matrix-core kernel: a run split at `cut`
    (the second half starting at an offset view of the same tensors) and
    resumed from the first half's final state reproduces the whole run."""
    from tssm import ssd_scan_forward
    d = _ssd_inputs(dev, 2, 700, 4, 64, 64, torch.bfloat16, seed=cut, heavy=True)
    args = lambda s: (d["x"][:, s], d["dt"][:, s], d["A_log"], d["B"][:, s], d["C"][:, s])  # noqa: E731
    y, h = ssd_scan_forward(*args(slice(None)), d["D"], return_state=True)
    _, h1 = ssd_scan_forward(*args(slice(0, cut)), d["D"], return_state=True)
    y2, h2 = ssd_scan_forward(*args(slice(cut, None)), d["D"], h0=h1, return_state=True)
    torch.cuda.synchronize()
    assert_close(y2, y[:, cut:], 4e-3, f"n64 tail via h0, cut {cut}")
    assert_close(h2, h, 1e-3, f"n64 final state via h0, cut {cut}")


@pytest.mark.parametrize("Bsz,L,H,P,decay", [
    (1, 5000, 2, 64, "slow"),    # 2 rows x 2 channel blocks: 20 segments of 256 steps, ragged end
    (1, 5000, 2, 64, "heavy"),
    (1, 3001, 3, 48, "slow"),    # 3 rows (not a multiple of 8), 3 blocks of 16 channels
    (2, 2000, 1, 16, "slow"),    # one 16-channel block: the step halves of pass 1 added
    (1, 4000, 8, 32, "slow"),    # 8 rows (XCD mapping), one 32-channel block per row
])
@pytest.mark.parametrize("disc", ["zoh", "euler"])
def test_ssd_scan_n64_segments(dev, Bsz, L, H, P, decay, disc):
    """bf16 N = 64 with too few (row, channel block) units to fill the chip:
    the one-pass kernel runs time segments (pass 1 segment end states, the
    prefix pass over segments, pass 3 outputs from each entry state).  Slow
    decays carry the state across every segment; h0, skip term and the final
    state against the float64 oracle."""
    from tssm import ssd_scan_forward
    d = _ssd_inputs(dev, Bsz, L, H, P, 64, torch.bfloat16, seed=L + P + H, heavy=True)
    if decay == "slow":
        g = torch.Generator().manual_seed(L)
        d["A_log"] = torch.full((H,), float(np.log(0.02)), device=dev)
        d["dt"] = (torch.rand(Bsz, L, H, generator=g) * 0.02).to(dev)
    h0 = torch.randn(Bsz, H, P, 64, device=dev)
    y, hl = ssd_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], d["D"], disc=disc,
                             h0=h0, chunk=256, return_state=True)
    torch.cuda.synchronize()
    y_ref, h_ref = O.ssd_scan(d["x"], d["dt"], d["A_log"], d["B"], d["C"], d["D"], h0=np64(h0),
                              disc=disc)
    assert_close(y, y_ref, 4e-3, f"segmented n64 ssd y L={L} P={P} {decay} {disc}")
    assert_close(hl, h_ref, 1e-3, f"segmented n64 ssd h_last L={L} P={P} {decay} {disc}")


@pytest.mark.parametrize("chunk", [64, 1024])
def test_ssd_scan_n64_segments_chunk_slots(dev, chunk):
    """The segment count is bounded by the workspace's chunk slots: with
    1024-step chunks (L=5000: 5 slots) there are fewer segments and one
    sub-segment per segment in pass 1; with 64-step chunks more sub-segments
    fit.  Slow decays, h0, skip term, against the float64 oracle."""
    from tssm import ssd_scan_forward
    Bsz, L, H, P = 1, 5000, 2, 64
    d = _ssd_inputs(dev, Bsz, L, H, P, 64, torch.bfloat16, seed=chunk, heavy=True)
    g = torch.Generator().manual_seed(chunk + 1)
    d["A_log"] = torch.full((H,), float(np.log(0.02)), device=dev)
    d["dt"] = (torch.rand(Bsz, L, H, generator=g) * 0.02).to(dev)
    h0 = torch.randn(Bsz, H, P, 64, device=dev)
    y, hl = ssd_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], d["D"], h0=h0,
                             chunk=chunk, return_state=True)
    torch.cuda.synchronize()
    y_ref, h_ref = O.ssd_scan(d["x"], d["dt"], d["A_log"], d["B"], d["C"], d["D"], h0=np64(h0))
    assert_close(y, y_ref, 4e-3, f"segmented n64 ssd y, chunk {chunk}")
    assert_close(hl, h_ref, 1e-3, f"segmented n64 ssd h_last, chunk {chunk}")


def test_ssd_scan_n64_long_sequence(dev):
    """B=1 L=65536 H=8 P=N=64 bf16, log-normal dt: 16 (row, channel block)
    units, so the one-pass kernel runs 16 segments of 4096 steps.  Heads 0
    and 7 against the float64 oracle over every step, every head against the
    oracle's fp32 C restatement, and split/resume at L/2."""
    import tssm
    from oracle import cport
    from tssm import ssd_scan_forward, workloads
    w = workloads.ssd_long(L=65536, N=64)
    d = {k: w[k].to(dev) for k in ("x", "dt", "A_log", "B", "C")}
    y, h = ssd_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], None, chunk=256,
                            return_state=True)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    heads = [0, 7]
    sl = (slice(None), slice(None), heads)
    y_ref, h_ref = O.ssd_scan(w["x"][sl], w["dt"][sl], w["A_log"][heads], w["B"][sl], w["C"][sl])
    assert_close(y[sl], y_ref, 4e-3, "n64 long y, heads 0 and 7")
    assert_close(h[:, heads], h_ref, 1e-3, "n64 long final state, heads 0 and 7")
    y32, h32 = cport.ssd_scan(w["x"].float(), w["dt"], w["A_log"], w["B"].float(),
                              w["C"].float())
    yc, hc = y.float().cpu(), h.cpu()
    for k in range(w["x"].shape[2]):
        assert_close(yc[:, :, k], y32[:, :, k], 4e-3, f"n64 long y, head {k}")
        assert_close(hc[:, k], h32[:, k], 1e-3, f"n64 long final state, head {k}")
    cut = 32768
    _, h1 = ssd_scan_forward(d["x"][:, :cut], d["dt"][:, :cut], d["A_log"], d["B"][:, :cut],
                             d["C"][:, :cut], None, chunk=256, return_state=True)
    y2, h2 = ssd_scan_forward(d["x"][:, cut:], d["dt"][:, cut:], d["A_log"], d["B"][:, cut:],
                              d["C"][:, cut:], None, chunk=256, h0=h1, return_state=True)
    torch.cuda.synchronize()
    assert_close(y2, y[:, cut:], 4e-3, "n64 long tail via h0")
    assert_close(h2, h, 1e-3, "n64 long final state via h0")
    tssm.check(dev)


def test_ssd_scan_n64_headline_shape(dev):
    """B=8 L=4096 H=16 P=N=64 bf16 (the headline shapes read as SSD), the
    seeded workload of the benchmark: batch 0 and 7, heads 0 and 15 against
    the oracle on those slices; zero initial state."""
    from tssm import ssd_scan_forward, workloads
    Bsz, L, H, P = 8, 4096, 16, 64
    w = workloads.multihead(B=Bsz, L=L, H=H, P=P)
    x = w["u"].view(Bsz, L, H, P)
    d = {k: v.to(dev) for k, v in dict(x=x, B=w["B"], C=w["C"], dt=w["dt"]).items()}
    A_log = w["A_log_h"].to(dev)
    y, hl = ssd_scan_forward(d["x"], d["dt"], A_log, d["B"], d["C"], None, chunk=128,
                             return_state=True)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    for b in (0, 7):
        for hh in (0, 15):
            sl = (slice(b, b + 1), slice(None), slice(hh, hh + 1))
            y_ref, h_ref = O.ssd_scan(x[sl], w["dt"][sl], w["A_log_h"][hh:hh + 1], w["B"][sl],
                                      w["C"][sl])
            assert_close(y[sl], y_ref, 4e-3, f"headline-shape ssd y b={b} h={hh}")
            assert_close(hl[b:b + 1, hh:hh + 1], h_ref, 1e-3, f"headline-shape ssd h b={b} h={hh}")


@pytest.mark.parametrize("chunk", [64, 256, 1024])
def test_ssd_scan_chunks_and_split(dev, chunk):
    from tssm import ssd_scan_forward
    d = _ssd_inputs(dev, 1, 3000, 2, 64, 16, torch.float32, seed=chunk)
    y, h = ssd_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], None, chunk=chunk,
                            return_state=True)
    y_ref, h_ref = O.ssd_scan(d["x"], d["dt"], d["A_log"], d["B"], d["C"], None)
    torch.cuda.synchronize()
    assert_close(y, y_ref, 1e-5, f"chunk {chunk}")
    cut = 1234
    y1, h1 = ssd_scan_forward(d["x"][:, :cut], d["dt"][:, :cut], d["A_log"], d["B"][:, :cut],
                              d["C"][:, :cut], None, chunk=chunk, return_state=True)
    y2 = ssd_scan_forward(d["x"][:, cut:], d["dt"][:, cut:], d["A_log"], d["B"][:, cut:],
                          d["C"][:, cut:], None, chunk=chunk, h0=h1)
    torch.cuda.synchronize()
    assert_close(torch.cat([y1, y2], 1), y_ref, 1e-5, "split/resume")


def test_ssd_long_sequence_shape(dev):
    """B=1 L=262144 H=8 P=64 N=16 bf16, log-normal dt (the long-sequence
    workload, the instance the benchmark times).  Heads 0 and 7 are compared
    with the float64 oracle over all 262144 steps (y and final state), and
    every head, each on its own, with the oracle's fp32 C restatement (itself
    checked against the float64 oracle on the CPU); split/resume of the full
    run at L/2 reproduces the tail."""
    import tssm
    from oracle import cport
    from tssm import ssd_scan_forward, workloads
    w = workloads.ssd_long()
    d = {k: w[k].to(dev) for k in ("x", "dt", "A_log", "B", "C")}
    y, h = ssd_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], None, chunk=256,
                            return_state=True)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    heads = [0, 7]
    sl = (slice(None), slice(None), heads)
    y_ref, h_ref = O.ssd_scan(w["x"][sl], w["dt"][sl], w["A_log"][heads], w["B"][sl], w["C"][sl])
    e = assert_close(y[sl], y_ref, 1e-2, "full-length y, heads 0 and 7")
    assert_close(h[:, heads], h_ref, 1e-3, "final state, heads 0 and 7")
    print(f"ssd long full-length relerr {e:.3e}")
    y32, h32 = cport.ssd_scan(w["x"].float(), w["dt"], w["A_log"], w["B"].float(),
                              w["C"].float())
    H = w["x"].shape[2]
    yc, hc = y.float().cpu(), h.cpu()
    errs = [assert_close(yc[:, :, k], y32[:, :, k], 1e-2, f"full-length y, head {k}")
            for k in range(H)]
    for k in range(H):
        assert_close(hc[:, k], h32[:, k], 1e-3, f"final state, head {k}")
    print("ssd long per-head relerr vs the fp32 restatement: "
          + " ".join(f"{v:.2e}" for v in errs))
    cut = 131072
    _, h1 = ssd_scan_forward(d["x"][:, :cut], d["dt"][:, :cut], d["A_log"], d["B"][:, :cut],
                             d["C"][:, :cut], None, chunk=256, return_state=True)
    y2, h2 = ssd_scan_forward(d["x"][:, cut:], d["dt"][:, cut:], d["A_log"], d["B"][:, cut:],
                              d["C"][:, cut:], None, chunk=256, h0=h1, return_state=True)
    torch.cuda.synchronize()
    assert_close(y2, y[:, cut:], 1e-2, "tail via h0")
    assert_close(h2, h, 1e-3, "final state via h0")
    tssm.check(dev)


@pytest.mark.parametrize("decay,L,Bsz,H,with_d", [
    ("slow", 20000, 1, 2, False),    # no segment forgets: walks fold many aggregates
    ("slow", 70001, 2, 3, True),     # more than 64 segments per row, ragged end, skip term
    ("mixed", 205006, 2, 8, False),  # four-tile segments, forgetting and slow heads together
    ("slow", 70001, 4, 8, False),    # four-tile segments, more than 64 per row, slow decays
])
def test_ssd_scan_fused_lookback(dev, decay, L, Bsz, H, with_d):
    """The one-launch SSD kernel (reverse first sweep, decoupled look-back,
    forward second sweep) against the three tile passes on the same inputs,
    and two heads against the float64 oracle over every step.  Slow decays
    (decay product of a segment far from zero) make every segment publish an
    aggregate and the walks fold long chains, beyond one 64-segment status
    window; "mixed" gives half the heads decays that underflow to exactly
    zero (inclusive state published at once) and half slow ones.  h0 and the
    final state are checked too."""
    import tssm
    from tssm import ssd_scan_forward
    g = torch.Generator().manual_seed(L + H)
    x = torch.randn(Bsz, L, H, 64, generator=g).to(torch.bfloat16)
    Bm = (torch.randn(Bsz, L, H, 16, generator=g) / 4).to(torch.bfloat16)
    Cm = (torch.randn(Bsz, L, H, 16, generator=g) / 4).to(torch.bfloat16)
    slow = torch.full((H,), np.log(0.02))
    if decay == "slow":
        A_log = slow
        dt = torch.rand(Bsz, L, H, generator=g) * 0.02
    else:
        A_log = torch.where(torch.arange(H) % 2 == 0, torch.full((H,), np.log(8.0)), slow)
        dt = torch.exp(torch.randn(Bsz, L, H, generator=g) * 1.5 - 3.0)
    D = torch.randn(H * 64, generator=g) if with_d else None
    h0 = torch.randn(Bsz, H, 64, 16, generator=g)
    d = {k: v.to(dev) for k, v in dict(x=x, B=Bm, C=Cm, A_log=A_log, dt=dt, h0=h0).items()}
    Dd = D.to(dev) if with_d else None
    y, h = ssd_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], Dd, chunk=256,
                            h0=d["h0"], return_state=True)
    y3, h3 = ssd_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], Dd, chunk=256,
                              h0=d["h0"], return_state=True, fused=False)
    torch.cuda.synchronize()
    tssm.check(dev)
    assert_close(y, y3, 4e-3, f"fused vs three passes, y ({decay})")
    assert_close(h, h3, 1e-4, f"fused vs three passes, final state ({decay})")
    heads = [0, H - 1]
    sl = (slice(Bsz - 1, Bsz), slice(None), heads)
    y_ref, h_ref = O.ssd_scan(x[sl], dt[sl], A_log[heads], Bm[sl], Cm[sl],
                              None if D is None else D.view(H, 64)[heads],
                              h0=np64(h0[Bsz - 1:, heads]))
    e = assert_close(y[sl], y_ref, 4e-3, f"fused y vs oracle ({decay})")
    assert_close(h[Bsz - 1:, heads], h_ref, 1e-3, f"fused final state vs oracle ({decay})")
    print(f"ssd fused look-back {decay} L={L}: relerr {e:.2e}")


@pytest.mark.parametrize("L", [65499, 205006])
def test_ssd_scan_multi_tile_segments(dev, L):
    """bf16 P=64 N=16 with 16 rows: the matrix-core passes walk one
    (L=65499) or two (L=205006: 801 tiles, so the last segment holds one
    tile) consecutive 256-step tiles per wave and pass the states between
    those segments; ragged last tile (an odd number of 32-step sub-chunks),
    skip term and h0.  Two heads of the second batch are compared with the
    float64 oracle over every step."""
    from tssm import ssd_scan_forward
    d = _ssd_inputs(dev, 2, L, 8, 64, 16, torch.bfloat16, seed=L % 1000, heavy=True)
    h0 = torch.randn(2, 8, 64, 16, device=dev)
    y, hl = ssd_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], d["D"], disc="zoh",
                             h0=h0, chunk=256, return_state=True)
    torch.cuda.synchronize()
    heads = [2, 7]
    sl = (slice(1, 2), slice(None), heads)
    y_ref, h_ref = O.ssd_scan(d["x"][sl], d["dt"][sl], d["A_log"][heads], d["B"][sl],
                              d["C"][sl], d["D"][heads], h0=np64(h0[1:2, heads]), disc="zoh")
    assert_close(y[sl], y_ref, 4e-3, f"segmented mfma ssd y L={L}")
    assert_close(hl[1:2, heads], h_ref, 1e-3, "segmented mfma ssd h_last")


def test_ssd_then_multihead_on_one_stream(dev):
    """The SSD passes write raw fp32 chunk data into their workspace; a
    look-back scan launched next on the same stream must not read any of it
    as a published carry (the two use separate workspaces)."""
    import tssm
    from tssm import multihead_ssm_forward, ssd_scan_forward
    from test_gpu_multihead import _inputs, _oracle
    # tiny, slowly underflowing decays leave denormal chunk products behind
    s = _ssd_inputs(dev, 2, 3000, 4, 64, 16, torch.float32, seed=3, heavy=True)
    s["A_log"] = torch.full_like(s["A_log"], 4.0)
    for _ in range(2):
        ssd_scan_forward(s["x"], s["dt"], s["A_log"], s["B"], s["C"], None, chunk=256)
        d = _inputs(dev, 2, 3000, 4, 64, torch.float32, seed=4, per_head=True, with_d=False)
        y = multihead_ssm_forward(d["u"], d["A_log"], d["B"], d["C"], d["dt"], None,
                                  disc="zoh", chunk=128)
        torch.cuda.synchronize()
        y_ref, _ = _oracle(d, "zoh")
        assert_close(y, y_ref, 1e-5, "multihead after ssd on one stream")
    tssm.check(dev)


def test_check_reports_a_flag_set_by_the_host(dev):
    """tssm.check raises once a workspace's sticky look-back flag is set (set
    here by a host write, never by a real timeout) and clears it."""
    import tssm
    from tssm import multihead_ssm_forward, workspace
    d = _ssd_inputs(dev, 1, 256, 2, 64, 16, torch.float32, seed=1)
    multihead_ssm_forward(d["x"].view(1, 256, 128), d["A_log"], d["B"].repeat(1, 1, 1, 4),
                          d["C"].repeat(1, 1, 1, 4), d["dt"], None, disc="zoh")
    tssm.check(dev)
    ws = workspace.get(dev, torch.cuda.current_stream(dev).cuda_stream, 0)
    ws[:4].view(torch.int32).fill_(1)
    with pytest.raises(tssm.TssmError, match="look-back wait expired"):
        tssm.check(dev)
    tssm.check(dev)


def test_host_flag_reports_an_expired_wait_without_a_sync(dev):
    """A lookback workspace carries the address of a pinned host int that a
    kernel whose wait expired sets with the sticky word.  The next fused
    launch on that workspace polls it on the host (no synchronisation) and
    raises.  The int is set here by a host write, never by a real timeout."""
    import tssm
    from tssm import multihead_ssm_forward, workspace
    d = _ssd_inputs(dev, 1, 256, 2, 64, 16, torch.float32, seed=2)
    args = (d["x"].view(1, 256, 128), d["A_log"], d["B"].repeat(1, 1, 1, 4),
            d["C"].repeat(1, 1, 1, 4), d["dt"], None)
    multihead_ssm_forward(*args, disc="zoh")
    stream = torch.cuda.current_stream(dev).cuda_stream
    flag = workspace.host_flag(dev, stream)
    assert flag is not None and flag.is_pinned()
    ws = workspace.get(dev, stream, 0)
    assert ws[8:16].view(torch.int64).item() != 0   # header: flag address attached
    torch.cuda.synchronize()
    assert int(flag[0]) == 0                         # healthy launches leave it alone
    flag[0] = 1                                      # what the error path stores
    with pytest.raises(tssm.TssmError, match="host flag"):
        multihead_ssm_forward(*args, disc="zoh")
    assert int(flag[0]) == 0                         # reported once
    multihead_ssm_forward(*args, disc="zoh")         # and the workspace goes on
    tssm.check(dev)                                  # the device word was never set


@pytest.fixture(scope="module")
def stream_wl():
    from tssm import workloads
    return workloads.ssd_stream()


def test_ssd_stream_step_config_size(dev, stream_wl):
    """The streaming workload at its size: 4096 streams, H=32 P=64 N=128, the
    fp32 state [4096,32,64,128] (4 GiB, byte offsets past 2^32) resident and
    updated in place over 50 steps of the benchmark's cycled input pool.  y of
    64 sampled streams (stream 0 and 4095 among them, all 32 heads) is checked
    against the float64 oracle every step, and their state at the end; y of
    every stream is checked against the oracle's fp32 C restatement in the
    first two steps."""
    from oracle import cport
    from tssm import ssd_stream_step
    w = stream_wl
    S, H, P, N = w["S"], w["H"], w["P"], w["N"]
    A_log = w["A_log"].to(dev)
    pool = [{k: v.to(dev) for k, v in st.items()} for st in w["steps"]]
    state = torch.zeros(S, H, P, N, device=dev)
    g = torch.Generator().manual_seed(44)
    idx = torch.cat([torch.tensor([0, S - 1]), torch.randperm(S - 2, generator=g)[:62] + 1])
    idx = torch.sort(idx).values
    st_ref = np.zeros((len(idx), H, P, N))
    st_all = np.zeros((S, H, P, N), np.float32)
    y = torch.empty(S, H, P, device=dev)
    worst = 0.0
    for step in range(50):
        s = pool[step % len(pool)]
        ssd_stream_step(s["x"], s["dt"], A_log, s["B"], s["C"], None, state, out=y)
        cpu = w["steps"][step % len(pool)]
        y_ref = O.ssd_stream_step(cpu["x"][idx], cpu["dt"][idx], w["A_log"], cpu["B"][idx],
                                  cpu["C"][idx], None, st_ref)
        if step < 2:
            y_all = cport.ssd_stream_step(cpu["x"], cpu["dt"], w["A_log"], cpu["B"], cpu["C"],
                                          None, st_all)
        torch.cuda.synchronize()
        worst = max(worst, assert_close(y[idx.to(dev)], y_ref, 1e-5, f"stream y step {step}"))
        if step < 2:
            yc = y.cpu()
            for lo in range(0, S, 512):
                assert_close(yc[lo:lo + 512], y_all[lo:lo + 512], 1e-5,
                             f"stream y step {step}, streams {lo}..{lo + 511}")
    del st_all
    assert_close(state[idx.to(dev)], st_ref, 1e-5, "stream state after 50 steps")
    assert torch.isfinite(state[-1, -1]).all()
    print(f"ssd stream config size: worst y relerr over 50 steps {worst:.3e}")


def test_ssd_stream_step_full_run(dev, stream_wl):
    """The streaming workload over its full run length of 10,000 steps (the
    input pool cycled as the benchmark cycles it): 16 sampled streams (0 and
    4095 among them) follow the oracle's fp32 C restatement step by step; y is
    compared every 100 steps and the state after the last step."""
    from oracle import cport
    from tssm import ssd_stream_step
    w = stream_wl
    S, H, P, N = w["S"], w["H"], w["P"], w["N"]
    A_log = w["A_log"].to(dev)
    pool = [{k: v.to(dev) for k, v in st.items()} for st in w["steps"]]
    g = torch.Generator().manual_seed(45)
    idx = torch.cat([torch.tensor([0, S - 1]), torch.randperm(S - 2, generator=g)[:14] + 1])
    idx = torch.sort(idx).values
    idx_d = idx.to(dev)
    sub = [{k: np.ascontiguousarray(v[idx].numpy(), dtype=np.float32) for k, v in st.items()}
           for st in w["steps"]]
    a32 = w["A_log"].numpy().astype(np.float32)
    state = torch.zeros(S, H, P, N, device=dev)
    st_ref = np.zeros((len(idx), H, P, N), np.float32)
    y = torch.empty(S, H, P, device=dev)
    worst = 0.0
    for step in range(10000):
        s = pool[step % len(pool)]
        ssd_stream_step(s["x"], s["dt"], A_log, s["B"], s["C"], None, state, out=y)
        c = sub[step % len(sub)]
        y_ref = cport.ssd_stream_step(c["x"], c["dt"], a32, c["B"], c["C"], None, st_ref)
        if step % 100 == 99:
            worst = max(worst, assert_close(y[idx_d], y_ref, 1e-5, f"stream y step {step}"))
        if step % 1000 == 999:
            print(f"stream full run: step {step + 1}, worst y relerr {worst:.3e}", flush=True)
    assert_close(state[idx_d], st_ref, 1e-5, "stream state after 10000 steps")
    print(f"ssd stream full run: worst y relerr over 10000 steps {worst:.3e}")


@pytest.mark.parametrize("N", [16, 128])
@pytest.mark.parametrize("per_stream_dt", [True, False])
@pytest.mark.parametrize("P", [64, 40])   # 40: a batch of row passes runs past P
def test_ssd_stream_step(dev, N, per_stream_dt, P):
    from tssm import ssd_stream_step
    g = torch.Generator().manual_seed(N + P)
    S, H = 37, 4
    A_log = (torch.rand(H, generator=g) * np.log(16.0)).to(dev)
    D = torch.randn(H, P, generator=g).to(dev)
    state = torch.zeros(S, H, P, N, device=dev)
    st_ref = np.zeros((S, H, P, N))
    for step in range(12):
        x = torch.randn(S, H, P, generator=g).to(dev)
        dt = (torch.empty(S if per_stream_dt else (S, H)).exponential_(10.0, generator=g)).to(dev)
        Bm = (torch.randn(S, H, N, generator=g) / N ** 0.5).to(dev)
        Cm = (torch.randn(S, H, N, generator=g) / N ** 0.5).to(dev)
        y = ssd_stream_step(x, dt, A_log, Bm, Cm, D, state)
        y_ref = O.ssd_stream_step(x, dt, A_log, Bm, Cm, D, st_ref)
        torch.cuda.synchronize()
        assert_close(y, y_ref, 1e-5, f"stream y step {step}")
    assert_close(state, st_ref, 1e-5, "stream state")


def _mamba1_inputs(dev, Bsz, L, Dc, N, dtype, seed, dt_per_channel=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(Bsz, L, Dc, generator=g).to(dtype)
    shape = (Bsz, L, Dc) if dt_per_channel else (Bsz, L)
    dt = torch.empty(shape).exponential_(20.0, generator=g).clamp_(1e-3, 1.0)
    A_log = torch.empty(Dc, N).uniform_(np.log(0.5), np.log(5.0), generator=g)
    Bm = (torch.randn(Bsz, L, N, generator=g) / N ** 0.5).to(dtype)
    Cm = (torch.randn(Bsz, L, N, generator=g) / N ** 0.5).to(dtype)
    D = torch.randn(Dc, generator=g)
    return {k: v.to(dev) for k, v in dict(x=x, dt=dt, A_log=A_log, B=Bm, C=Cm, D=D).items()}


def test_selective_scan_small_config(dev):
    """B=2 L=256 D=16 N=16 fp32, dt ~ Exp(mean .05) clamped (the small fp32 workload)."""
    from tssm import selective_scan_forward, workloads
    w = workloads.mamba1_small()
    d = {k: w[k].to(dev) for k in w}
    y, h = selective_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], None,
                                  return_state=True)
    torch.cuda.synchronize()
    y_ref, h_ref = O.selective_scan(d["x"], d["dt"], d["A_log"], d["B"], d["C"])
    assert_close(y, y_ref, 1e-5, "mamba1 y")
    assert_close(h, h_ref, 1e-5, "mamba1 h")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N,Dc", [(8, 40), (16, 40), (64, 40), (16, 6), (32, 9), (128, 3)])
@pytest.mark.parametrize("dt_per_channel", [False, True])
def test_selective_scan(dev, dtype, N, Dc, dt_per_channel):
    """Channel counts that do and do not fill the packed 64-lane rows."""
    from tssm import selective_scan_forward
    d = _mamba1_inputs(dev, 3, 700, Dc, N, dtype, seed=N + Dc, dt_per_channel=dt_per_channel)
    h0 = torch.randn(3, Dc, N, device=dev)
    y, h = selective_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], d["D"], h0=h0,
                                  return_state=True, chunk=128)
    torch.cuda.synchronize()
    y_ref, h_ref = O.selective_scan(d["x"], d["dt"], d["A_log"], d["B"], d["C"], d["D"], h0=np64(h0))
    assert_close(y, y_ref, TOL[dtype], f"mamba1 {dtype} N={N}")
    assert_close(h, h_ref, TOL[dtype], "mamba1 h_last")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N,Dc,rank,L", [(16, 40, 16, 700), (8, 24, 1, 333), (64, 6, 33, 520),
                                         (16, 256, 64, 300), (32, 9, 4, 129), (128, 3, 7, 200)])
def test_selective_scan_dtproj(dev, dtype, N, Dc, rank, L):
    """dt produced in the scan's load stage (dt_project_softplus fused into the
    Mamba-1 scan) against the oracle's projection followed by its selective
    scan; the projection spans both clamps; nonzero h0, skip term, ragged L."""
    from tssm import selective_scan_forward
    g = torch.Generator().manual_seed(N * 1000 + Dc + rank)
    x = torch.randn(3, L, Dc, generator=g).to(dtype)
    raw = torch.randn(3, L, rank, generator=g)
    W = torch.randn(rank, Dc, generator=g) * (3.0 / rank ** 0.5)
    bias = torch.empty(Dc).uniform_(-4.0, 0.0, generator=g)
    A_log = torch.empty(Dc, N).uniform_(np.log(0.5), np.log(5.0), generator=g)
    Bm = (torch.randn(3, L, N, generator=g) / N ** 0.5).to(dtype)
    Cm = (torch.randn(3, L, N, generator=g) / N ** 0.5).to(dtype)
    D = torch.randn(Dc, generator=g)
    h0 = torch.randn(3, Dc, N, generator=g)
    DT_MIN, DT_MAX = 2e-3, 0.4
    dt_ref = O.dt_project_softplus(raw, W, bias, DT_MIN, DT_MAX)
    assert (dt_ref == DT_MIN).any() and (dt_ref == DT_MAX).any()   # both clamps hit
    d = {k: v.to(dev) for k, v in dict(x=x, raw=raw, W=W, bias=bias, A_log=A_log, B=Bm, C=Cm,
                                        D=D, h0=h0).items()}
    y, h = selective_scan_forward(d["x"], d["raw"], d["A_log"], d["B"], d["C"], d["D"],
                                  h0=d["h0"], return_state=True,
                                  dt_proj=(d["W"], d["bias"], DT_MIN, DT_MAX))
    torch.cuda.synchronize()
    y_ref, h_ref = O.selective_scan(x, dt_ref, A_log, Bm, Cm, D, h0=np64(h0))
    assert_close(y, y_ref, TOL[dtype], f"dtproj y {dtype} N={N} Dc={Dc} rank={rank}")
    assert_close(h, h_ref, TOL[dtype], "dtproj h_last")


@pytest.mark.parametrize("dtype,N,Dc,rank,L,Bsz", [
    (torch.float32, 16, 100, 20, 2100, 8),    # rank block of 16 + a partial one; 28 lanes past Dc
    (torch.bfloat16, 8, 260, 4, 1000, 16),    # second workgroup holds 4 channels; ragged L
    (torch.float32, 16, 64, 64, 4096, 4),     # four rank blocks
    (torch.float32, 16, 64, 7, 4096, 4),      # rank 7: raw rows not 16-byte vectors, single pass
])
def test_selective_scan_dtproj_three_pass(dev, dtype, N, Dc, rank, L, Bsz):
    """dt produced on the matrix cores inside passes 1 and 3 of the three-pass
    scan (problems large enough for it): against the oracle's projection and
    scan, and against the two-launch path (projection kernel, then the scan
    over the stored dt), with h0 and the skip term."""
    import discretize_kernel as dk
    from tssm import selective_scan_forward
    g = torch.Generator().manual_seed(rank * 100 + Dc + N)
    x = torch.randn(Bsz, L, Dc, generator=g).to(dtype)
    raw = torch.randn(Bsz, L, rank, generator=g)
    W = torch.randn(rank, Dc, generator=g) * (2.0 / rank ** 0.5)
    bias = torch.empty(Dc).uniform_(-4.0, -1.0, generator=g)
    A_log = torch.empty(Dc, N).uniform_(np.log(0.5), np.log(5.0), generator=g)
    Bm = (torch.randn(Bsz, L, N, generator=g) / N ** 0.5).to(dtype)
    Cm = (torch.randn(Bsz, L, N, generator=g) / N ** 0.5).to(dtype)
    D = torch.randn(Dc, generator=g)
    h0 = torch.randn(Bsz, Dc, N, generator=g)
    DT_MIN, DT_MAX = 2e-3, 0.25
    dt_ref = O.dt_project_softplus(raw, W, bias, DT_MIN, DT_MAX)
    assert (dt_ref == DT_MIN).any() and (dt_ref == DT_MAX).any()   # both clamps hit
    d = {k: v.to(dev) for k, v in dict(x=x, raw=raw, W=W, bias=bias, A_log=A_log, B=Bm, C=Cm,
                                        D=D, h0=h0).items()}
    y, h = selective_scan_forward(d["x"], d["raw"], d["A_log"], d["B"], d["C"], d["D"],
                                  h0=d["h0"], return_state=True,
                                  dt_proj=(d["W"], d["bias"], DT_MIN, DT_MAX))
    dt = torch.empty(Bsz, L, Dc, device=dev)
    dk.dt_project_softplus_kernel[(Bsz, L, 1)](
        d["raw"], d["W"], d["bias"], dt, Bsz, L, Dc, rank, *d["raw"].stride(),
        d["W"].stride(0), d["W"].stride(1), *dt.stride(), DT_MIN=DT_MIN, DT_MAX=DT_MAX,
        BLOCK_H=triton_pow2(Dc), BLOCK_R=16)
    y2, h2 = selective_scan_forward(d["x"], dt, d["A_log"], d["B"], d["C"], d["D"], h0=d["h0"],
                                    return_state=True)
    torch.cuda.synchronize()
    y_ref, h_ref = O.selective_scan(x, dt_ref, A_log, Bm, Cm, D, h0=np64(h0))
    e = assert_close(y, y_ref, TOL[dtype], f"dtproj three-pass y {dtype} N={N} Dc={Dc} R={rank}")
    assert_close(h, h_ref, TOL[dtype], "dtproj three-pass h_last")
    assert_close(y, y2, TOL[dtype], "fused vs two-launch y")
    assert_close(h, h2, 1e-5, "fused vs two-launch h_last")
    print(f"dtproj three-pass {dtype} N={N} Dc={Dc} R={rank}: relerr {e:.2e}, "
          f"bitwise equal to the two-launch path: {torch.equal(y, y2)}")


def test_selective_scan_dtproj_workspace_forms(dev):
    """tssm_selective_scan_dtproj through the C ABI with the two workspace
    sizes: tssm_selective_scan_dtproj_workspace_bytes (pass 1 stores the dt it
    produced, pass 3 reads it back) and the smaller
    tssm_selective_scan_workspace_bytes (pass 3 produces dt again).  Both
    produce the same dt on the matrix cores, so y and h_last agree bit for
    bit; both against the oracle."""
    from tssm import _lib
    Bsz, L, Dc, N, R = 8, 1030, 128, 16, 16
    g = torch.Generator().manual_seed(77)
    x = torch.randn(Bsz, L, Dc, generator=g)
    raw = torch.randn(Bsz, L, R, generator=g)
    W = torch.randn(R, Dc, generator=g) * 0.5
    bias = torch.empty(Dc).uniform_(-3.0, -1.0, generator=g)
    A_log = torch.empty(Dc, N).uniform_(np.log(0.5), np.log(5.0), generator=g)
    Bm = torch.randn(Bsz, L, N, generator=g) / N ** 0.5
    Cm = torch.randn(Bsz, L, N, generator=g) / N ** 0.5
    d = {k: v.to(dev) for k, v in dict(x=x, raw=raw, W=W, bias=bias, A_log=A_log, B=Bm,
                                        C=Cm).items()}
    lib = _lib.lib()
    assert lib.tssm_selective_scan_takes_passes(
        _lib.F32, Bsz, L, Dc, N, 1, 0, d["raw"].data_ptr(), d["W"].data_ptr(),
        d["bias"].data_ptr(), R, L * R, R, Dc) == 1
    small = lib.tssm_selective_scan_workspace_bytes(Bsz, L, Dc, N, 256)
    big = lib.tssm_selective_scan_dtproj_workspace_bytes(Bsz, L, Dc, N, 256)
    assert big > small > 0
    stream = torch.cuda.current_stream(dev).cuda_stream
    outs = []
    for nbytes in (big, small):
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        y = torch.empty_like(d["x"])
        h = torch.empty(Bsz, Dc, N, device=dev)
        _lib.call("tssm_selective_scan_dtproj", _lib.F32, _lib.DISC_ZOH, d["x"].data_ptr(),
                  d["raw"].data_ptr(), d["W"].data_ptr(), d["bias"].data_ptr(), 1e-3, 0.5,
                  d["A_log"].data_ptr(), d["B"].data_ptr(), d["C"].data_ptr(), None, None,
                  y.data_ptr(), h.data_ptr(), Bsz, L, Dc, N, R, L * Dc, Dc, L * R, R, Dc,
                  L * N, N, L * N, N, L * Dc, Dc, 256, ws.data_ptr(), nbytes, stream)
        torch.cuda.synchronize()
        outs.append((y, h))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    dt_ref = O.dt_project_softplus(raw, W, bias, 1e-3, 0.5)
    y_ref, h_ref = O.selective_scan(x, dt_ref, A_log, Bm, Cm)
    assert_close(outs[0][0], y_ref, 1e-5, "dtproj y (stored dt table)")
    assert_close(outs[1][1], h_ref, 1e-5, "dtproj h_last (dt produced again)")


@pytest.mark.parametrize("Dc,N,L,Bsz,dt_mode,extras,sliced", [
    (256, 16, 2048, 4, "tau", False, False),      # the interpolation workload's scan shape
    (100, 8, 333, 3, "per_channel", True, False),  # ragged channels and steps, D, h0
    (64, 16, 700, 2, "shared", True, True),       # W as a column slice of a wider x_proj weight
])
def test_selective_scan_bcproj(dev, Dc, N, L, Bsz, dt_mode, extras, sliced):
    """B_t = x_t W_B and C_t = x_t W_C formed inside the scan (bc_proj=):
    against the float64 oracle fed the float64 products, and against the
    unfused path (torch.matmul for B and C, then the scan)."""
    from tssm import selective_scan_forward
    g = torch.Generator().manual_seed(Dc + N + L)
    x = torch.randn(Bsz, L, Dc, generator=g)
    R = 16
    Wx = torch.randn(Dc, R + 2 * N, generator=g) / Dc ** 0.5
    W_bc = Wx[:, R:] if sliced else Wx[:, R:].contiguous()
    if dt_mode == "tau":
        dt = torch.sort(torch.rand(Bsz, L, generator=g) * (L / 20.0), dim=1).values
    elif dt_mode == "shared":
        dt = torch.rand(Bsz, L, generator=g) * 0.1
    else:
        dt = torch.rand(Bsz, L, Dc, generator=g) * 0.1
    A_log = torch.empty(Dc, N).uniform_(np.log(0.5), np.log(5.0), generator=g)
    D = torch.randn(Dc, generator=g) if extras else None
    h0 = torch.randn(Bsz, Dc, N, generator=g) if extras else None
    d = {k: v.to(dev) for k, v in dict(x=x, dt=dt, A_log=A_log).items()}
    Wd = Wx.to(dev)[:, R:] if sliced else W_bc.to(dev)
    if sliced:
        assert Wd.stride(0) == R + 2 * N
    Dd = D.to(dev) if extras else None
    h0d = h0.to(dev) if extras else None
    tau = dt_mode == "tau"
    y, h = selective_scan_forward(d["x"], d["dt"], d["A_log"], None, None, Dd, h0=h0d,
                                  return_state=True, dt_is_tau=tau, bc_proj=Wd)
    Bg = (d["x"] @ Wd[:, :N]).contiguous()
    Cg = (d["x"] @ Wd[:, N:]).contiguous()
    y2, h2 = selective_scan_forward(d["x"], d["dt"], d["A_log"], Bg, Cg, Dd, h0=h0d,
                                    return_state=True, dt_is_tau=tau)
    torch.cuda.synchronize()
    x64, W64 = x.double(), W_bc.double()
    Bref, Cref = x64 @ W64[:, :N], x64 @ W64[:, N:]
    dtr = torch.diff(dt.double(), dim=1, prepend=torch.zeros(Bsz, 1, dtype=torch.float64)) \
        if tau else dt
    y_ref, h_ref = O.selective_scan(x, dtr, A_log, Bref, Cref, D,
                                    h0=None if h0 is None else np64(h0))
    e = assert_close(y, y_ref, 1e-5, f"bcproj y Dc={Dc} N={N} {dt_mode}")
    assert_close(h, h_ref, 1e-5, "bcproj h_last")
    assert_close(y, y2, 1e-5, "bcproj vs matmul + scan")
    assert_close(h, h2, 1e-5, "bcproj h_last vs matmul + scan")
    print(f"bcproj Dc={Dc} N={N} {dt_mode}: relerr {e:.2e}")


@pytest.mark.parametrize("Dc,N,L,Bsz,R,extras,sliced", [
    (256, 16, 2048, 4, 16, False, False),   # Mamba-1 at D = 256: dt rank D / 16
    (100, 8, 333, 3, 32, True, False),      # ragged channels and steps, D, h0
    (64, 16, 700, 2, 64, True, True),       # W_x as a column slice of a wider weight
])
def test_selective_scan_xproj(dev, Dc, N, L, Bsz, R, extras, sliced):
    """The whole input projection inside the scan (x_proj=): x_dbl = x W_x split
    into dt_raw, B and C, dt = clamp(softplus(dt_raw W_dt + bias)), against the
    float64 oracle (its projection and dt_project_softplus fed float64
    products) and against the unfused path (torch.matmul for x_dbl, then the
    scan with dt_proj= over the dt_raw columns and the B/C columns)."""
    from tssm import selective_scan_forward
    g = torch.Generator().manual_seed(Dc + N + L + R)
    x = torch.randn(Bsz, L, Dc, generator=g)
    wide = torch.randn(Dc, R + 2 * N + (8 if sliced else 0), generator=g) / Dc ** 0.5
    W_x = wide[:, :R + 2 * N]
    W_dt = torch.randn(R, Dc, generator=g) * (0.5 / R ** 0.5)
    bias = float(np.log(np.expm1(0.05))) + torch.empty(Dc).uniform_(-0.5, 0.5, generator=g)
    dt_min, dt_max = 1e-3, 0.5
    A_log = torch.empty(Dc, N).uniform_(np.log(0.5), np.log(5.0), generator=g)
    D = torch.randn(Dc, generator=g) if extras else None
    h0 = torch.randn(Bsz, Dc, N, generator=g) if extras else None
    xd, Ad = x.to(dev), A_log.to(dev)
    Wxd = wide.to(dev)[:, :R + 2 * N] if sliced else W_x.contiguous().to(dev)
    if sliced:
        assert Wxd.stride(0) == R + 2 * N + 8
    Wdt, bd = W_dt.to(dev), bias.to(dev)
    Dd = D.to(dev) if extras else None
    h0d = h0.to(dev) if extras else None
    xp = (Wxd, Wdt, bd, dt_min, dt_max)
    y, h = selective_scan_forward(xd, None, Ad, None, None, Dd, h0=h0d, return_state=True,
                                  x_proj=xp)
    xdbl = (xd @ Wxd).contiguous()
    raw = xdbl[..., :R].contiguous()
    Bg, Cg = xdbl[..., R:R + N].contiguous(), xdbl[..., R + N:].contiguous()
    y2, h2 = selective_scan_forward(xd, raw, Ad, Bg, Cg, Dd, h0=h0d, return_state=True,
                                    dt_proj=(Wdt, bd, dt_min, dt_max))
    torch.cuda.synchronize()
    x64 = x.double() @ W_x.double()
    dt_ref = O.dt_project_softplus(x64[..., :R], W_dt, bias, dt_min, dt_max)
    y_ref, h_ref = O.selective_scan(x, dt_ref, A_log, x64[..., R:R + N], x64[..., R + N:], D,
                                    h0=None if h0 is None else np64(h0))
    e = assert_close(y, y_ref, 1e-5, f"xproj y Dc={Dc} N={N} R={R}")
    assert_close(h, h_ref, 1e-5, "xproj h_last")
    assert_close(y, y2, 1e-5, "xproj vs matmul + dt_proj scan")
    assert_close(h, h2, 1e-5, "xproj h_last vs matmul + dt_proj scan")
    print(f"xproj Dc={Dc} N={N} R={R}: relerr {e:.2e}")



def triton_pow2(n):
    return 1 << (n - 1).bit_length()


def test_selective_scan_dtproj_config_shape(dev):
    """B=16 L=2048 D=256 N=16 fp32, rank 16 (the interpolation workload's scan
    shape): the fused projection against the oracle, and against the two-launch
    path (dt_project_softplus_kernel, then the scan over the [B,L,D] dt)."""
    import discretize_kernel as dk
    from tssm import selective_scan_forward, workloads
    w = workloads.dtproj_mamba1()
    d = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in w.items()}
    proj = (d["W"], d["bias"], w["DT_MIN"], w["DT_MAX"])
    y = selective_scan_forward(d["x"], d["dt_raw"], d["A_log"], d["B"], d["C"], None,
                               chunk=256, dt_proj=proj)
    Bsz, L, R = w["dt_raw"].shape
    Dc = w["W"].shape[1]
    dt = torch.empty(Bsz, L, Dc, device=dev)
    dk.dt_project_softplus_kernel[(Bsz, L, Dc // 256)](
        d["dt_raw"], d["W"], d["bias"], dt, Bsz, L, Dc, R, *d["dt_raw"].stride()[:2],
        d["dt_raw"].stride(2), d["W"].stride(0), d["W"].stride(1), *dt.stride(),
        DT_MIN=w["DT_MIN"], DT_MAX=w["DT_MAX"], BLOCK_H=256, BLOCK_R=16)
    y2 = selective_scan_forward(d["x"], dt, d["A_log"], d["B"], d["C"], None, chunk=256)
    torch.cuda.synchronize()
    dt_ref = O.dt_project_softplus(w["dt_raw"], w["W"], w["bias"], w["DT_MIN"], w["DT_MAX"])
    y_ref, _ = O.selective_scan(w["x"], dt_ref, w["A_log"], w["B"], w["C"])
    e = assert_close(y, y_ref, 1e-5, "fused projection y")
    assert_close(y2, y_ref, 1e-5, "two-launch y")
    assert_close(y, y2, 1e-5, "fused vs two-launch")
    print(f"dtproj config shape relerr {e:.2e}")


@pytest.mark.parametrize("FTILE", [16, 128])
def test_fused_interp_ssm_small(dev, FTILE):
    from tssm import fused_interp_ssm_forward
    g = torch.Generator().manual_seed(FTILE)
    Bsz, T, F, N = 3, 300, 64, 16
    tau = torch.sort(torch.rand(Bsz, T, generator=g) * 30, dim=1).values
    M = (torch.rand(Bsz, T, F, generator=g) < 0.3).float()
    V = torch.randn(Bsz, T, F, generator=g) * M
    A_log = torch.empty(F, N).uniform_(np.log(0.5), np.log(5.0), generator=g)
    Bm = torch.randn(Bsz, T, N, generator=g) / 4
    Cm = torch.randn(Bsz, T, N, generator=g) / 4
    d = {k: v.to(dev) for k, v in dict(V=V, M=M, tau=tau, A_log=A_log, B=Bm, C=Cm).items()}
    vhat, y, h = fused_interp_ssm_forward(d["V"], d["M"], d["tau"], d["A_log"], d["B"], d["C"],
                                          K=10, FTILE=FTILE, return_state=True)
    torch.cuda.synchronize()
    v_ref, y_ref, h_ref = O.fused_interp_ssm(d["V"], d["M"], d["tau"], d["A_log"], d["B"],
                                             d["C"], K=10, FTILE=FTILE)
    assert_close(vhat, v_ref, 1e-6, "Vhat")
    assert_close(y, y_ref, 1e-5, "y")
    assert_close(h, h_ref, 1e-5, "h_last")


@pytest.mark.parametrize("dtype,N,F,FTILE,K,T,Bsz,missing,extras", [
    (torch.float32, 16, 256, 16, 5, 2000, 8, 0.97, True),      # 16 tiles per workgroup, gaps
    (torch.bfloat16, 8, 260, 128, 64, 1100, 16, 0.999, False),  # ragged channels, K = 64, sparse
    (torch.float32, 16, 128, 256, 1, 2048, 8, 0.5, False),      # tile wider than F, K = 1
])
def test_interp_scan_fused_forms(dev, dtype, N, F, FTILE, K, T, Bsz, missing, extras):
    """Interpolation formed inside the scan's first pass
    (tssm_interp_selective_scan, taken by fused_interp_ssm_forward for these
    problems) against the oracle and against the two-kernel path (the
    interpolation drop-in, then the selective scan over the stored Vhat):
    Vhat bit for bit, y and h_last within the bars.  Sparse masks leave
    whole tiles unobserved, so steps take every neighbour case (both, one
    side, none within K)."""
    import fused_interp_kernel as fik
    from tssm import _lib, fused_interp_ssm_forward, selective_scan_forward
    g = torch.Generator().manual_seed(F + K + FTILE)
    tau = torch.sort(torch.rand(Bsz, T, generator=g) * (T / 20.0), dim=1).values
    M = (torch.rand(Bsz, T, F, generator=g) >= missing).float()
    V = (torch.randn(Bsz, T, F, generator=g) * M).to(dtype)
    A_log = torch.empty(F, N).uniform_(np.log(0.5), np.log(5.0), generator=g)
    Bm = (torch.randn(Bsz, T, N, generator=g) / N ** 0.5).to(dtype)
    Cm = (torch.randn(Bsz, T, N, generator=g) / N ** 0.5).to(dtype)
    D = torch.randn(F, generator=g) if extras else None
    h0 = torch.randn(Bsz, F, N, generator=g) if extras else None
    d = {k: v.to(dev) for k, v in dict(V=V, M=M, tau=tau, A_log=A_log, B=Bm, C=Cm).items()}
    Dd = D.to(dev) if extras else None
    h0d = h0.to(dev) if extras else None
    assert _lib.lib().tssm_interp_selective_scan_supported(
        _lib.F32 if dtype == torch.float32 else _lib.BF16, _lib.F32, _lib.F32, Bsz, T, F, N, K,
        FTILE, d["M"].data_ptr(),
        d["M"].stride(0), d["M"].stride(1), d["V"].stride(1)) == 1
    vhat, y, h = fused_interp_ssm_forward(d["V"], d["M"], d["tau"], d["A_log"], d["B"], d["C"],
                                          Dd, K=K, FTILE=FTILE, h0=h0d, return_state=True)
    # two-kernel path: the interpolation drop-in, then the scan over its Vhat
    v2 = torch.empty_like(d["V"])
    fik_kernel = fik.fused_time_aware_interp_kernel if dtype == torch.float32 else \
        fik.fused_interp_bf16_kernel
    fik_kernel[(Bsz, T, -(-F // FTILE))](d["V"], d["M"], d["tau"], v2, Bsz, T, F,
                                         *d["V"].stride(), *d["M"].stride(), *d["tau"].stride(),
                                         *v2.stride(), K=K, FTILE=FTILE)
    y2, h2 = selective_scan_forward(v2, d["tau"], d["A_log"], d["B"], d["C"], Dd, h0=h0d,
                                    return_state=True, dt_is_tau=True)
    torch.cuda.synchronize()
    v_ref, y_ref, h_ref = O.fused_interp_ssm(d["V"], d["M"], d["tau"], d["A_log"], d["B"],
                                             d["C"], D, K=K, FTILE=FTILE,
                                             h0=None if h0 is None else np64(h0))
    tol = TOL[dtype]
    dv = (vhat.float() - v2.float()).abs()
    print(f"Vhat vs interpolation kernel: max |diff| {dv.max().item():.3e}, "
          f"{int((dv > 0).sum())} of {dv.numel()} differ", flush=True)
    assert_close(vhat, v_ref, 1e-6 if dtype == torch.float32 else 1e-2, "Vhat vs oracle")
    assert_close(v2, v_ref, 1e-6 if dtype == torch.float32 else 1e-2, "kernel Vhat vs oracle")
    assert torch.equal(vhat, v2), "Vhat differs from the interpolation kernel's"
    e = assert_close(y, y_ref, tol, "y vs oracle")
    assert_close(h, h_ref, tol, "h_last vs oracle")
    assert_close(y, y2, 1e-5 if dtype == torch.float32 else 1e-2, "y vs two-kernel path")
    print(f"interp-in-pass-1 {dtype} F={F} FTILE={FTILE} K={K}: relerr {e:.2e}, "
          f"y bitwise equal to the two-kernel path: {torch.equal(y, y2)}")


def test_fused_interp_ssm_full_shape(dev):
    """B=16 T=2048 F=D=256 N=16 fp32, 30% missing, K=10 FTILE=128."""
    from tssm import fused_interp_ssm_forward, workloads
    w = workloads.interp_mamba1()
    d = {k: w[k].to(dev) for k in w}
    vhat, y = fused_interp_ssm_forward(d["V"], d["M"], d["tau"], d["A_log"], d["B"], d["C"])
    torch.cuda.synchronize()
    v_ref, y_ref, _ = O.fused_interp_ssm(d["V"], d["M"], d["tau"], d["A_log"], d["B"], d["C"])
    assert_close(vhat, v_ref, 1e-6, "Vhat")
    e = assert_close(y, y_ref, 1e-5, "y")
    print(f"interp+ssm full shape relerr {e:.2e}")
