"""GPU parity: multihead DIAG scan (fused entry point and phase-exact drop-ins)
against the float64 oracle on the same (rounded) inputs."""
import numpy as np
import pytest
import torch

from helpers import TOL, assert_close, np64
from oracle import ssm_oracle as O

pytestmark = pytest.mark.gpu


def _inputs(dev, Bsz, L, nh, hd, dtype, seed=0, per_head=False, with_d=True):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(Bsz, L, nh * hd, generator=g).to(dtype)
    B = (torch.randn(Bsz, L, nh, hd, generator=g) / hd ** 0.5).to(dtype)
    C = (torch.randn(Bsz, L, nh, hd, generator=g) / hd ** 0.5).to(dtype)
    dt = torch.nn.functional.softplus(torch.randn(Bsz, L, nh, generator=g)) * \
        torch.empty(Bsz, L, 1).exponential_(1.0, generator=g)
    A_log = torch.rand(nh if per_head else (nh, hd), generator=g) * np.log(16.0)
    D = torch.randn(nh * hd, generator=g) if with_d else None
    d = dict(u=u, A_log=A_log, B=B, C=C, dt=dt, D=D)
    return {k: (v.to(dev) if v is not None else None) for k, v in d.items()}


def _oracle(d, disc, h0=None):
    A_log = np64(d["A_log"])
    nh, hd = d["B"].shape[2], d["B"].shape[3]
    if A_log.ndim == 1:
        A_log = np.repeat(A_log[:, None], hd, axis=1)
    return O.multihead_forward(d["u"], A_log, d["B"], d["C"], d["dt"], d["D"], disc=disc,
                               h0=None if h0 is None else np64(h0))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("disc", ["euler", "zoh"])
@pytest.mark.parametrize("per_head", [False, True])
@pytest.mark.parametrize("with_d", [True, False])
def test_fused_small(dev, dtype, disc, per_head, with_d):
    """Every (dtype, discretization, decay layout, skip term) instance of the
    fused kernel at head_dim 64, ragged length."""
    from tssm import multihead_ssm_forward
    d = _inputs(dev, 2, 300, 3, 64, dtype, seed=1, per_head=per_head, with_d=with_d)
    y, hl = multihead_ssm_forward(d["u"], d["A_log"], d["B"], d["C"], d["dt"], d["D"],
                                  disc=disc, return_state=True)
    torch.cuda.synchronize()
    y_ref, h_ref = _oracle(d, disc)
    assert y.dtype == dtype
    assert_close(y, y_ref, TOL[dtype], f"y {dtype} {disc}")
    assert_close(hl, h_ref, TOL[dtype], f"h_last {dtype} {disc}")
    yh = y.float().view(2, 300, 3, 64)
    assert torch.equal(yh, yh[..., :1].expand_as(yh))


@pytest.mark.parametrize("hd", [8, 16, 32, 128])
@pytest.mark.parametrize("chunk", [64, 128, 256])
def test_fused_head_dims_and_chunks(dev, hd, chunk):
    from tssm import multihead_ssm_forward
    d = _inputs(dev, 2, 517, 2, hd, torch.float32, seed=hd + chunk)
    y = multihead_ssm_forward(d["u"], d["A_log"], d["B"], d["C"], d["dt"], d["D"],
                              disc="zoh", chunk=chunk)
    torch.cuda.synchronize()
    y_ref, _ = _oracle(d, "zoh")
    assert_close(y, y_ref, TOL[torch.float32], f"hd={hd} chunk={chunk}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("hd,nh", [(32, 8), (32, 6), (16, 8), (8, 16), (8, 12)])
@pytest.mark.parametrize("per_head", [False, True])
@pytest.mark.parametrize("bc", ["strided", "shared"])
def test_fused_packed_heads(dev, dtype, hd, nh, per_head, bc):
    """Heads narrower than 64 channels share a 128-lane tile row (128/hd heads)
    when nh allows (else one per row): per-head decay, D, B/C head strides
    (padded, or 0 = one B/C for all heads), h0 and the final state must land
    on the right head."""
    from tssm import multihead_ssm_forward
    Bsz, L = 2, 611
    d = _inputs(dev, Bsz, L, nh, hd, dtype, seed=40 + nh, per_head=per_head)
    for k in ("B", "C"):
        if bc == "strided":
            wide = torch.zeros(Bsz, L, nh, 40, dtype=dtype, device=dev)
            wide[..., :hd] = d[k]
            d[k] = wide[..., :hd]                  # head stride 40 channels
        else:
            d[k] = d[k][:, :, :1].expand(Bsz, L, nh, hd)  # head stride 0
    h0 = torch.randn(Bsz, nh, hd, device=dev)
    y, hl = multihead_ssm_forward(d["u"], d["A_log"], d["B"], d["C"], d["dt"], d["D"],
                                  disc="zoh", chunk=128, h0=h0, return_state=True)
    torch.cuda.synchronize()
    y_ref, h_ref = _oracle(d, "zoh", h0=h0)
    assert_close(y, y_ref, TOL[dtype], f"y packed hd={hd} nh={nh} {dtype}")
    assert_close(hl, h_ref, TOL[dtype], f"h_last packed hd={hd} nh={nh} {dtype}")
    yh = y.float().view(Bsz, L, nh, hd)
    assert torch.equal(yh, yh[..., :1].expand_as(yh))


def test_fused_split_resume_and_repeat(dev):
    """scan(x1 || x2) == scan(x2, h0 = h_last(x1)); repeated launches reuse the
    workspace (epoch advance) and give identical results."""
    from tssm import multihead_ssm_forward
    d = _inputs(dev, 2, 700, 4, 64, torch.float32, seed=5)
    y, h = multihead_ssm_forward(d["u"], d["A_log"], d["B"], d["C"], d["dt"], d["D"],
                                 disc="zoh", return_state=True)
    cut = 333
    sl = lambda k, s: d[k][:, s]  # noqa: E731
    y1, h1 = multihead_ssm_forward(sl("u", slice(0, cut)), d["A_log"], sl("B", slice(0, cut)),
                                   sl("C", slice(0, cut)), sl("dt", slice(0, cut)), d["D"],
                                   disc="zoh", return_state=True)
    y2, h2 = multihead_ssm_forward(sl("u", slice(cut, None)), d["A_log"],
                                   sl("B", slice(cut, None)), sl("C", slice(cut, None)),
                                   sl("dt", slice(cut, None)), d["D"], disc="zoh", h0=h1,
                                   return_state=True)
    torch.cuda.synchronize()
    assert_close(torch.cat([y1, y2], 1), y, 1e-5, "split/resume y")
    assert_close(h2, h, 1e-5, "split/resume h")
    for _ in range(3):
        y_again = multihead_ssm_forward(d["u"], d["A_log"], d["B"], d["C"], d["dt"], d["D"], disc="zoh")
        torch.cuda.synchronize()
        assert torch.equal(y_again, y)


def test_fused_forgetting_tiles(dev):
    """Tiles whose decay product underflows to zero publish their state before
    looking back; rows mixing such tiles with slowly decaying ones (and a
    nonzero h0) must still match the sequential oracle."""
    from tssm import multihead_ssm_forward
    Bsz, L, nh, hd = 2, 1100, 4, 64
    d = _inputs(dev, Bsz, L, nh, hd, torch.float32, seed=21, per_head=True)
    chunk_id = torch.arange(L, device=dev) // 128
    strong = (chunk_id % 3 == 0).view(1, L, 1)
    d["dt"] = torch.where(strong, torch.full_like(d["dt"], 5.0), torch.full_like(d["dt"], 1e-3))
    d["A_log"] = torch.tensor([np.log(16.0), np.log(0.01), 0.0, np.log(4.0)],
                              dtype=torch.float32, device=dev)
    h0 = torch.randn(Bsz, nh, hd, device=dev)
    y, hl = multihead_ssm_forward(d["u"], d["A_log"], d["B"], d["C"], d["dt"], d["D"],
                                  disc="zoh", chunk=128, h0=h0, return_state=True)
    torch.cuda.synchronize()
    y_ref, h_ref = _oracle(d, "zoh", h0=h0)
    assert_close(y, y_ref, TOL[torch.float32], "y, mixed forgetting tiles")
    assert_close(hl, h_ref, TOL[torch.float32], "h_last, mixed forgetting tiles")


@pytest.mark.parametrize("disc", ["zoh", "euler"])
def test_fused_headline_scaling_is_exact(dev, disc):
    """Every output of the benchmarked instance at its full size: the scan is
    linear in u with dt, A, B, C fixed, and doubling is exact in bf16 and in
    every fp32 operation, so y(2u) = 2 y(u) and h_last(2u) = 2 h_last(u) bit
    for bit -- a check of all 33.5 M outputs that needs no reference."""
    import tssm
    from tssm import multihead_ssm_forward, workloads
    w = workloads.multihead()
    d = {k: w[k].to(dev) for k in ("u", "B", "C", "dt", "A_log_h")}
    y1, h1 = multihead_ssm_forward(d["u"], d["A_log_h"], d["B"], d["C"], d["dt"], None,
                                   disc=disc, chunk=128, return_state=True)
    y2, h2 = multihead_ssm_forward(d["u"] * 2, d["A_log_h"], d["B"], d["C"], d["dt"], None,
                                   disc=disc, chunk=128, return_state=True)
    tssm.check(dev)
    assert torch.equal(y2, y1 * 2), "y(2u) != 2 y(u)"
    assert torch.equal(h2, h1 * 2), "h_last(2u) != 2 h_last(u)"


@pytest.mark.parametrize("disc", ["zoh", "euler"])
@pytest.mark.parametrize("a_layout", ["per_head", "per_channel"])
@pytest.mark.parametrize("with_d", [False, True])
def test_fused_full_headline_shape(dev, disc, a_layout, with_d):
    """B=8 L=4096 H=16 P=N=64 bf16 x/B/C, fp32 dt and state.  The instance the
    benchmark times is a_layout="per_head" (A_log [H]: one decay per head),
    with_d=False, ZOH; the others are the per-channel A_log [H, P] layout of
    the reference kernel and the skip term.  Every y of the launch is
    compared against the float64 oracle."""
    import tssm
    from tssm import multihead_ssm_forward, workloads
    w = workloads.multihead()
    d = {k: w[k].to(dev) for k in ("u", "B", "C", "dt")}
    A_log = w["A_log_h" if a_layout == "per_head" else "A_log"].to(dev)
    H, P = w["B"].shape[2], w["B"].shape[3]
    D = torch.randn(H * P, generator=torch.Generator().manual_seed(5)).to(dev) if with_d else None
    y = multihead_ssm_forward(d["u"], A_log, d["B"], d["C"], d["dt"], D, disc=disc, chunk=128)
    torch.cuda.synchronize()
    tssm.check(dev)
    y_ref, _ = O.multihead_forward(d["u"], w["A_log"], d["B"], d["C"], d["dt"], D, disc=disc)
    e = assert_close(y, y_ref, 1e-2, f"headline {disc} {a_layout} D={with_d}")
    print(f"headline {disc} {a_layout} D={with_d} normwise relerr {e:.3e}")
    # The contract is 1e-2 (bf16 inputs, fp32 state); the kernel's observed
    # error is ~2e-3 (the bf16 rounding of y).  A regression bar at 5e-3 keeps
    # an accuracy loss of 2.5x from passing under the contract.
    assert e <= 5e-3, f"headline {disc} {a_layout} D={with_d}: relerr {e:.3e} above 5e-3"


@pytest.mark.parametrize("hd,dtype,BLK,L", [(16, torch.float32, 16, 70),
                                          (64, torch.float32, 128, 300),
                                          (32, torch.bfloat16, 64, 200),
                                          (128, torch.float32, 32, 90),
                                          (24, torch.float32, 16, 50)])   # scalar output path
def test_phase_exact_dropins(dev, hd, dtype, BLK, L):
    """multihead_ssm_fwd_local/carry_scan/output launched exactly as a caller of
    the reference would, intermediates and y checked against the oracle; a
    partial output grid writes exactly its rows and blocks."""
    import multihead_ssm_kernel as mk
    Bsz, nh = 2, 3
    d = _inputs(dev, Bsz, L, nh, hd, dtype, seed=9 + hd)
    u, A_log, B, C, dt, D = (d[k] for k in ("u", "A_log", "B", "C", "dt", "D"))
    H = nh * hd
    nblk = 1 << (((L + BLK - 1) // BLK) - 1).bit_length()
    loc_a = torch.empty(Bsz, L, nh, hd, device=dev)
    loc_x = torch.empty_like(loc_a)
    carry = torch.empty(2 * Bsz * nh * hd * nblk, device=dev)
    y = torch.zeros(Bsz, L, H, device=dev, dtype=dtype)
    mk.multihead_ssm_fwd_local_kernel[(Bsz * nh, nblk)](
        u, A_log, B, C, dt, loc_a, loc_x, carry, Bsz, L, H, nh, hd,
        u.stride(0), u.stride(1), u.stride(2), A_log.stride(0), A_log.stride(1),
        B.stride(0), B.stride(1), B.stride(2), B.stride(3),
        C.stride(0), C.stride(1), C.stride(2), C.stride(3),
        dt.stride(0), dt.stride(1), dt.stride(2), BLK_L=BLK, NBLK=nblk, HEAD_DIM=hd)
    la_ref, lx_ref, c_ref = O.multihead_fwd_local(u, A_log, B, C, dt, nh, hd, BLK, nblk)
    torch.cuda.synchronize()
    assert_close(loc_a, la_ref, 1e-5, "loc_a")
    assert_close(loc_x, lx_ref, 1e-5, "loc_x")
    assert_close(carry, c_ref, 1e-5, "carry (local)")
    mk.multihead_ssm_carry_scan_kernel[(Bsz * nh * hd,)](carry, Bsz * nh * hd, nblk)
    c_ref = O.multihead_carry_scan(c_ref, Bsz * nh * hd, nblk)
    torch.cuda.synchronize()
    assert_close(carry, c_ref, 1e-5, "carry (scanned)")
    mk.multihead_ssm_output_kernel[(Bsz * nh, nblk)](
        loc_a, loc_x, carry, C, D, u, y, Bsz, L, H, nh, hd,
        u.stride(0), u.stride(1), u.stride(2), C.stride(0), C.stride(1), C.stride(2),
        C.stride(3), BLK_L=BLK, NBLK=nblk, HEAD_DIM=hd, num_warps=4)
    torch.cuda.synchronize()
    y_ref, _ = O.multihead_forward(u, A_log, B, C, dt, D, disc="euler")
    tol = 1e-5 if dtype == torch.float32 else TOL[dtype]
    assert_close(y, y_ref, tol, "y (phases)")
    # partial grid: rows (b, h) < Bsz*nh - 1, blocks < nblk - 1 (when there are 2)
    gr, gb = Bsz * nh - 1, max(nblk - 1, 1)
    y2 = torch.zeros_like(y)
    mk.multihead_ssm_output_kernel[(gr, gb)](
        loc_a, loc_x, carry, C, D, u, y2, Bsz, L, H, nh, hd,
        u.stride(0), u.stride(1), u.stride(2), C.stride(0), C.stride(1), C.stride(2),
        C.stride(3), BLK_L=BLK, NBLK=nblk, HEAD_DIM=hd, num_warps=4)
    torch.cuda.synchronize()
    t_end = min(gb * BLK, L)
    yv, y2v = y.view(Bsz, L, nh, hd), y2.view(Bsz, L, nh, hd)
    for r in range(Bsz * nh):
        b_, h_ = divmod(r, nh)
        if r < gr:
            assert torch.equal(y2v[b_, :t_end, h_], yv[b_, :t_end, h_])
            assert torch.all(y2v[b_, t_end:, h_] == 0)
        else:
            assert torch.all(y2v[b_, :, h_] == 0)


def test_launcher_rejects_out_of_bounds(dev):
    import multihead_ssm_kernel as mk
    small = torch.zeros(10, device=dev)
    with pytest.raises(ValueError):
        mk.multihead_ssm_carry_scan_kernel[(4,)](small, 4, 8)


def test_fused_alternating_decays_on_one_workspace(dev):
    """One stream, one workspace, six launches in a row that alternate between
    decays that make most tiles forget their entry state (such a tile
    publishes only its inclusive carry word) and slow decays (every tile
    publishes its aggregate words and walks back), per head and per channel:
    every launch must ignore the words the earlier launches left behind.
    Each result is checked against the float64 oracle."""
    from tssm import multihead_ssm_forward
    for i in range(6):
        per_head = i % 2 == 0
        d = _inputs(dev, 2, 1500, 4, 64, torch.float32, seed=40 + i, per_head=per_head,
                    with_d=False)
        # fast (log a in [2, 2.8]) or slow (log a in [-6, -5]) decay
        d["A_log"] = d["A_log"] * 0.05 + (2.0 if i % 4 < 2 else -6.0)
        y, hl = multihead_ssm_forward(d["u"], d["A_log"], d["B"], d["C"], d["dt"], None,
                                      disc="zoh", return_state=True)
        torch.cuda.synchronize()
        y_ref, h_ref = _oracle(d, "zoh")
        assert_close(y, y_ref, 1e-5, f"launch {i} y")
        assert_close(hl, h_ref, 1e-5, f"launch {i} h_last")
