"""GPU parity of the reference-named drop-in kernels (discretize, elementwise
scan, interpolation, fused interp step, streaming) against the float64 oracle.
Each kernel is launched exactly as a caller of the reference would:
``kernel[grid](*reference_args)``."""
import numpy as np
import pytest
import torch

from helpers import TOL, assert_close, np64
from oracle import ssm_oracle as O

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------------ discretize
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("H", [200, 203])   # 4-lane and 1-lane accesses
def test_zoh_discretize(dev, out_dtype, H):
    import discretize_kernel as dk
    g = torch.Generator().manual_seed(3)
    Bsz, T, BLOCK_H = 3, 50, 64
    A = torch.empty(H).uniform_(np.log(0.5), np.log(5.0), generator=g).to(dev)
    B = torch.randn(Bsz, T, H, generator=g).to(out_dtype).to(dev)
    # include tiny dt*a (1e-5..1e-3 range where the accurate expm1 matters) and large ones
    dt = torch.exp(torch.empty(Bsz, T).uniform_(np.log(1e-6), np.log(3.0), generator=g)).to(dev)
    Abar = torch.empty(Bsz, T, H, device=dev, dtype=out_dtype)
    Bbar = torch.empty_like(Abar)
    kern = dk.zoh_discretize_diag_kernel if out_dtype == torch.float32 else dk.zoh_discretize_diag_bf16_kernel
    kern[(Bsz, T, (H + BLOCK_H - 1) // BLOCK_H)](
        A, B, dt, Abar, Bbar, Bsz, T, H, B.stride(0), B.stride(1), B.stride(2),
        dt.stride(0), dt.stride(1), Abar.stride(0), Abar.stride(1), Abar.stride(2),
        Bbar.stride(0), Bbar.stride(1), Bbar.stride(2), BLOCK_H=BLOCK_H)
    torch.cuda.synchronize()
    Ar, Br = O.zoh_discretize(A, B, dt)
    tol = TOL[out_dtype]
    assert_close(Abar, Ar, tol, "Abar")
    assert_close(Bbar, Br, tol, "Bbar")
    if out_dtype == torch.float32:  # elementwise relative accuracy of the accurate expm1
        rel = np.abs(np64(Bbar) - Br) / np.maximum(np.abs(Br), 1e-30)
        assert rel.max() < 2e-6


def test_zoh_discretize_partial_grid(dev):
    import discretize_kernel as dk
    Bsz, T, H = 2, 4, 100
    A = torch.zeros(H, device=dev)
    B = torch.ones(Bsz, T, H, device=dev)
    dt = torch.full((Bsz, T), 0.1, device=dev)
    Abar = torch.full((Bsz, T, H), -7.0, device=dev)
    Bbar = torch.full_like(Abar, -7.0)
    dk.zoh_discretize_diag_kernel[(1, 2, 1)](
        A, B, dt, Abar, Bbar, Bsz, T, H, *B.stride(), *dt.stride(), *Abar.stride(),
        *Bbar.stride(), BLOCK_H=32)
    torch.cuda.synchronize()
    assert torch.all(Abar[0, :2, :32] != -7.0)
    assert torch.all(Abar[0, :2, 32:] == -7.0) and torch.all(Abar[1] == -7.0)
    assert torch.all(Abar[0, 2:] == -7.0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(3, 50, 200, 64), (2, 70, 300, 128), (1, 3, 5, 4),
                                   (5, 2, 40, 64), (7, 3, 64, 64)])   # rows wrap inside a batch of 4
def test_zoh_discretize_bwd(dev, dtype, shape):
    """zoh_discretize_bwd_kernel[grid](...) against the float64 oracle (itself
    pinned by torch.autograd): dA accumulates into its input, ddt is the full
    lane sum, dB elementwise.  Tiny dt*a exercises the cancellation-free psi."""
    import discretize_kernel as dk
    Bsz, T, H, BLOCK_H = shape
    g = torch.Generator().manual_seed(sum(shape))
    A = torch.empty(H).uniform_(np.log(0.5), np.log(5.0), generator=g).to(dev)
    B = torch.randn(Bsz, T, H, generator=g).to(dtype).to(dev)
    dt = torch.exp(torch.empty(Bsz, T).uniform_(np.log(1e-6), np.log(2.0), generator=g)).to(dev)
    Abar = torch.exp(dt[..., None] * -torch.exp(A)).to(dtype)
    dAbar = torch.randn(Bsz, T, H, generator=g).to(dtype).to(dev)
    dBbar = torch.randn(Bsz, T, H, generator=g).to(dtype).to(dev)
    dA0 = torch.randn(H, generator=g).to(dev)
    dA = dA0.clone()
    dB = torch.empty_like(B)
    ddt = torch.full((Bsz, T), 123.0, device=dev)
    dk.zoh_discretize_bwd_kernel[(Bsz, T, (H + BLOCK_H - 1) // BLOCK_H)](
        A, B, dt, Abar, dAbar, dBbar, dA, dB, ddt, Bsz, T, H, *B.stride(), *dt.stride(),
        *Abar.stride(), *dBbar.stride(), BLOCK_H=BLOCK_H)
    torch.cuda.synchronize()
    dA_r, dB_r, ddt_r = O.zoh_discretize_bwd(A, B, dt, Abar, dAbar, dBbar)
    tol = 1e-5 if dtype == torch.float32 else TOL[dtype]
    assert_close(dA - dA0, dA_r, tol, "dA_log (accumulated)")
    assert_close(dB, dB_r, tol, "dB")
    assert_close(ddt, ddt_r, tol, "ddt")
    # deterministic (fixed reduction order, no atomics): a repeat is bitwise equal
    dA2, ddt2 = dA0.clone(), torch.zeros_like(ddt)
    dk.zoh_discretize_bwd_kernel[(Bsz, T, (H + BLOCK_H - 1) // BLOCK_H)](
        A, B, dt, Abar, dAbar, dBbar, dA2, dB, ddt2, Bsz, T, H, *B.stride(), *dt.stride(),
        *Abar.stride(), *dBbar.stride(), BLOCK_H=BLOCK_H)
    torch.cuda.synchronize()
    assert torch.equal(dA2, dA) and torch.equal(ddt2, ddt)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 33, 300, 16, 64, 8), (3, 20, 64, 5, 32, 4),
                                   (1, 7, 1000, 48, 256, 16), (2, 9, 301, 7, 128, 4),
                                   # matrix-core path: rank 4..20 with partial rank
                                   # blocks, ragged T and H tiles
                                   (2, 200, 256, 12, 256, 16), (2, 70, 100, 4, 128, 4),
                                   (3, 130, 68, 20, 64, 32), (16, 2048, 256, 16, 256, 16)])
def test_dt_project_softplus(dev, out_dtype, shape):
    """dt_project_softplus_kernel[grid](...) against the oracle (softplus+clamp
    pinned to torch in float64); the clamp bounds are hit on purpose."""
    import discretize_kernel as dk
    Bsz, T, H, R, BLOCK_H, BLOCK_R = shape
    g = torch.Generator().manual_seed(H + R)
    raw = (3.0 * torch.randn(Bsz, T, R, generator=g)).to(dev)
    W = (torch.randn(R, H, generator=g) / R ** 0.5).to(dev)
    bias = torch.randn(H, generator=g).to(dev)
    out = torch.full((Bsz, T, H), -1.0, device=dev, dtype=out_dtype)
    DT_MIN, DT_MAX = 1e-3, 2.5
    dk.dt_project_softplus_kernel[(Bsz, T, (H + BLOCK_H - 1) // BLOCK_H)](
        raw, W, bias, out, Bsz, T, H, R, *raw.stride(), *W.stride(), *out.stride(),
        DT_MIN=DT_MIN, DT_MAX=DT_MAX, BLOCK_H=BLOCK_H, BLOCK_R=BLOCK_R)
    torch.cuda.synchronize()
    ref = O.dt_project_softplus(raw, W, bias, DT_MIN, DT_MAX)
    assert (ref == DT_MAX).any() and (ref == DT_MIN).any()
    assert_close(out, ref, TOL[out_dtype], "dt")
    if out_dtype == torch.float32:
        rel = np.abs(np64(out) - ref) / ref
        assert rel.max() < 1e-5


def test_dt_project_partial_grid_matrix_cores(dev):
    """4-aligned operands take the matrix-core kernel: a partial grid still
    writes exactly rows (0, :3) and lanes :64."""
    import discretize_kernel as dk
    Bsz, T, H, R = 2, 100, 128, 16
    g = torch.Generator().manual_seed(3)
    raw = torch.randn(Bsz, T, R, generator=g).to(dev)
    W = torch.randn(R, H, generator=g).to(dev)
    bias = torch.randn(H, generator=g).to(dev)
    out = torch.full((Bsz, T, H), -1.0, device=dev)
    dk.dt_project_softplus_kernel[(1, 3, 1)](
        raw, W, bias, out, Bsz, T, H, R, *raw.stride(), *W.stride(), *out.stride(),
        DT_MIN=0.0, DT_MAX=100.0, BLOCK_H=64, BLOCK_R=16)
    torch.cuda.synchronize()
    ref = O.dt_project_softplus(raw[:1, :3], W[:, :64], bias[:64], 0.0, 100.0)
    assert_close(out[:1, :3, :64], ref, 1e-5, "partial dt")
    assert torch.all(out[0, :3, 64:] == -1.0) and torch.all(out[0, 3:] == -1.0)
    assert torch.all(out[1] == -1.0)


def test_dt_project_partial_grid(dev):
    import discretize_kernel as dk
    Bsz, T, H, R = 2, 5, 70, 3
    raw = torch.randn(Bsz, T, R, device=dev)
    W = torch.randn(R, H, device=dev)
    bias = torch.zeros(H, device=dev)
    out = torch.full((Bsz, T, H), -1.0, device=dev)
    dk.dt_project_softplus_kernel[(1, 3, 1)](
        raw, W, bias, out, Bsz, T, H, R, *raw.stride(), *W.stride(), *out.stride(),
        DT_MIN=0.0, DT_MAX=100.0, BLOCK_H=32, BLOCK_R=4)
    torch.cuda.synchronize()
    assert torch.all(out[0, :3, :32] >= 0) and torch.all(out[0, :3, 32:] == -1.0)
    assert torch.all(out[0, 3:] == -1.0) and torch.all(out[1] == -1.0)


# ------------------------------------------------------------------ elementwise scan
@pytest.mark.parametrize("BLK", [16, 64, 256])
def test_ssm_forward_backward(dev, BLK):
    import ssm_scan as ss
    g = torch.Generator().manual_seed(BLK)
    Bsz, L, H = 2, 300, 40
    u, B, C, dY = (torch.randn(Bsz, L, H, generator=g).to(dev) for _ in range(4))
    A = torch.empty(Bsz, L, H).uniform_(0.5, 1.0, generator=g).to(dev)
    D = torch.randn(H, generator=g).to(dev)
    y, h = ss.ssm_forward(u, A, B, C, D, BLK=BLK)
    du, dA, dB, dC = ss.ssm_backward(u, A, B, C, h, dY, BLK=BLK)
    torch.cuda.synchronize()
    y_ref, h_ref = O.ssm_forward(u, A, B, C, D)
    assert_close(h, h_ref, 1e-5, "h")
    assert_close(y, y_ref, 1e-5, "y")
    for got, ref, n in zip((du, dA, dB, dC), O.ssm_backward(u, A, B, C, h_ref, dY), "du dA dB dC".split()):
        assert_close(got, ref, 1e-5, n)


@pytest.mark.parametrize("Bsz,L,H,zeros", [(2, 5000, 256, False), (3, 129, 68, True),
                                            (1, 1, 4, False), (2, 300, 42, False),
                                            (2, 1000, 64, True)])
def test_ssm_forward_backward_shapes(dev, Bsz, L, H, zeros):
    """Single-pass path (many chunks, partial lane blocks, one step, tiles whose
    decay product is exactly zero) and the phase-kernel path (H % 4 != 0)
    against the oracle."""
    import ssm_scan as ss
    g = torch.Generator().manual_seed(L + H)
    u, B, C, dY = (torch.randn(Bsz, L, H, generator=g).to(dev) for _ in range(4))
    A = torch.empty(Bsz, L, H).uniform_(0.9, 1.0, generator=g)
    if zeros:
        A[:, ::97, ::3] = 0.0
    A = A.to(dev)
    D = torch.randn(H, generator=g).to(dev)
    y, h = ss.ssm_forward(u, A, B, C, D)
    du, dA, dB, dC = ss.ssm_backward(u, A, B, C, h, dY)
    torch.cuda.synchronize()
    y_ref, h_ref = O.ssm_forward(u, A, B, C, D)
    assert_close(h, h_ref, 1e-5, "h")
    assert_close(y, y_ref, 1e-5, "y")
    for got, ref, n in zip((du, dA, dB, dC), O.ssm_backward(u, A, B, C, h_ref, dY),
                           "du dA dB dC".split()):
        assert_close(got, ref, 1e-5, n)


def test_ssm_phase_intermediates(dev):
    import ssm_scan as ss
    g = torch.Generator().manual_seed(1)
    Bsz, L, H, BLK = 2, 100, 8, 32
    u, B = (torch.randn(Bsz, L, H, generator=g).to(dev) for _ in range(2))
    A = torch.empty(Bsz, L, H).uniform_(0.5, 1.0, generator=g).to(dev)
    nblk = ss._nxt_pow2((L + BLK - 1) // BLK)
    la, lx = torch.empty_like(A), torch.empty_like(A)
    carry = torch.empty(2 * Bsz * H * nblk, device=dev)
    ss.ssm_fwd_local_kernel[(Bsz * H, nblk)](u, A, B, la, lx, carry, Bsz, L, H, BLK, nblk)
    torch.cuda.synchronize()
    la_r, lx_r, c_r = O.ssm_fwd_local(u, A, B, BLK, nblk)
    assert_close(la, la_r, 1e-6, "loc_a")
    assert_close(lx, lx_r, 1e-6, "loc_x")
    assert_close(carry, c_r, 1e-6, "carry")
    ss.ssm_carry_scan_kernel[(Bsz * H,)](carry, Bsz * H, nblk)
    torch.cuda.synchronize()
    assert_close(carry, O.ssm_carry_scan(c_r, Bsz * H, nblk), 1e-6, "scanned carry")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("nblk", [1, 2, 32, 64, 128, 256])
def test_carry_scans(dev, dtype, nblk):
    """ssm_carry_scan_kernel and ssm_bwd_carry_scan_kernel over 37 rows with a
    grid of 30: scanned rows match the oracle, rows past the grid are untouched
    (nblk > 64 chains 64-carry segments)."""
    import ssm_scan as ss
    rows, grid_rows = 37, 30
    g = torch.Generator().manual_seed(nblk)
    a = torch.empty(rows * nblk).uniform_(0.5, 1.0, generator=g)
    x = torch.randn(rows * nblk, generator=g)
    base = torch.cat([a, x]).to(dtype)
    tol = 1e-5 if dtype == torch.float32 else TOL[dtype]
    for kern, ref in ((ss.ssm_carry_scan_kernel, O.ssm_carry_scan),
                      (ss.ssm_bwd_carry_scan_kernel, O.ssm_bwd_carry_scan)):
        carry = base.clone().to(dev)
        kern[(grid_rows,)](carry, rows, nblk)
        torch.cuda.synchronize()
        exp = ref(base, rows, nblk).reshape(2, rows, nblk)
        got = carry.view(2, rows, nblk)
        assert_close(got[:, :grid_rows], exp[:, :grid_rows], tol, f"{kern.fn_name} nblk={nblk}")
        assert torch.equal(got[:, grid_rows:].cpu(), base.view(2, rows, nblk)[:, grid_rows:])


def test_ssm_forward_bf16(dev):
    import ssm_scan as ss
    g = torch.Generator().manual_seed(2)
    Bsz, L, H = 2, 200, 16
    u, B, C = (torch.randn(Bsz, L, H, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
    A = torch.empty(Bsz, L, H).uniform_(0.5, 0.99, generator=g).to(torch.bfloat16).to(dev)
    D = torch.randn(H, generator=g).to(torch.bfloat16).to(dev)
    y, h = ss.ssm_forward(u, A, B, C, D, BLK=64)
    torch.cuda.synchronize()
    y_ref, h_ref = O.ssm_forward(u, A, B, C, D)
    assert_close(y, y_ref, 1e-2, "y bf16")


# ------------------------------------------------------------------ interpolation
def _interp_inputs(Bsz, T, F, dtype, seed, p_obs=0.7, dev=None):
    g = torch.Generator().manual_seed(seed)
    tau = torch.sort(torch.rand(Bsz, T, generator=g) * 100, dim=1).values
    M = (torch.rand(Bsz, T, F, generator=g) < p_obs).float()
    V = (torch.randn(Bsz, T, F, generator=g) * M).to(dtype)
    return V.to(dev), M.to(dev), tau.to(dev)


@pytest.mark.parametrize("dtype,name", [(torch.float32, "fused_time_aware_interp_kernel"),
                                        (torch.bfloat16, "fused_interp_bf16_kernel"),
                                        (torch.float16, "fused_interp_fp16_kernel")])
@pytest.mark.parametrize("K,FTILE,p_obs", [(10, 128, 0.7), (3, 16, 0.02), (5, 7, 0.05),
                                         (4, 48, 0.1), (2, 512, 0.3)])
def test_interp(dev, dtype, name, K, FTILE, p_obs):
    import fused_interp_kernel as fi
    Bsz, T, F = 3, 150, 100
    V, M, tau = _interp_inputs(Bsz, T, F, dtype, seed=K * FTILE, p_obs=p_obs, dev=dev)
    out = torch.full_like(V, float("nan"))
    getattr(fi, name)[(Bsz, T, (F + FTILE - 1) // FTILE)](
        V, M, tau, out, Bsz, T, F, *V.stride(), *M.stride(), *tau.stride(), *out.stride(),
        K=K, FTILE=FTILE)
    torch.cuda.synchronize()
    ref = O.time_aware_interp(V, M, tau, K, FTILE)
    assert_close(out, ref, TOL[dtype] if dtype != torch.float32 else 1e-6, name)


@pytest.mark.parametrize("F,FTILE,mdtype,p_obs,mscale", [(1000, 300, torch.float32, 0.002, 1.0),
                                                          (520, 264, torch.bfloat16, 0.004, 1.0),
                                                          (520, 264, torch.float16, 0.004, 1.0),
                                                          (96, 8, torch.float32, 0.05, 1.0),
                                                          (1000, 64, torch.bfloat16, 0.003, 1.0),
                                                          (520, 128, torch.float16, 0.004, 1.0),
                                                          (256, 128, torch.float32, 0.02, 0.3)])
def test_interp_mask_layouts(dev, F, FTILE, mdtype, p_obs, mscale):
    """Observed flags over rows of several 64-vector blocks, tiles spanning blocks,
    16-bit masks, sparse masks that leave whole tiles unobserved, and fractional
    masks (a tile counts as observed when its mask sum exceeds 0.5)."""
    import fused_interp_kernel as fi
    Bsz, T, K = 2, 90, 6
    V, M, tau = _interp_inputs(Bsz, T, F, torch.float32, seed=F + FTILE, p_obs=p_obs, dev=dev)
    M = M * mscale
    Mq = M.to(mdtype)
    out = torch.full_like(V, float("nan"))
    fi.fused_time_aware_interp_kernel[(Bsz, T, (F + FTILE - 1) // FTILE)](
        V, Mq, tau, out, Bsz, T, F, *V.stride(), *Mq.stride(), *tau.stride(), *out.stride(),
        K=K, FTILE=FTILE)
    torch.cuda.synchronize()
    assert_close(out, O.time_aware_interp(V, M, tau, K, FTILE), 1e-6, "interp mask layouts")


def test_interp_full_size(dev):
    """B=16 T=2048 F=256, K=10, FTILE=128, 30% missing (the measured interp workload)."""
    import fused_interp_kernel as fi
    from tssm import workloads
    w = workloads.interp_mamba1()
    V, M, tau = (w[k].to(dev) for k in ("V", "M", "tau"))
    Bsz, T, F = V.shape
    out = torch.empty_like(V)
    fi.fused_time_aware_interp_kernel[(Bsz, T, 2)](V, M, tau, out, Bsz, T, F, *V.stride(),
                                                  *M.stride(), *tau.stride(), *out.stride(), 10, 128)
    torch.cuda.synchronize()
    assert_close(out, O.time_aware_interp(V, M, tau, 10, 128), 1e-6, "interp full")


@pytest.mark.parametrize("Bsz,T,F,K,FT,p_obs,dtype,mdtype", [
    (4, 40, 70, 4, 32, 0.05, torch.float32, torch.float32),
    (3, 60, 300, 10, 128, 0.02, torch.bfloat16, torch.bfloat16),   # config-2 tile, K
    (2, 90, 256, 64, 256, 0.01, torch.float32, torch.float16),     # K = 64: 129 rows x 256
    (2, 50, 600, 20, 512, 0.03, torch.float32, torch.float32)])    # tiles over 256 features
@pytest.mark.parametrize("tdtype", [torch.float32, torch.bfloat16, torch.float16])
def test_interp_ssm_step(dev, Bsz, T, F, K, FT, p_obs, dtype, mdtype, tdtype):
    """fused_interp_ssm_step_kernel launched at every t against the oracle's
    step; timestamps in every dtype (the oracle sees the same rounded values)."""
    import fused_ssm_interp as fs
    V, M, tau = _interp_inputs(Bsz, T, F, dtype, seed=4 + K, p_obs=p_obs, dev=dev)
    M = M.to(mdtype)
    tau = tau.to(tdtype)
    g = torch.Generator().manual_seed(5)
    Ab = torch.rand(F, generator=g).to(dev)
    Bb = torch.randn(F, generator=g).to(dev)
    h_in = torch.randn(Bsz, F, generator=g).to(dev)
    h_out = torch.empty_like(h_in)
    Vhat = torch.zeros_like(V)
    h_ref = np64(h_in)
    for t in range(T):
        fs.fused_interp_ssm_step_kernel[(Bsz, (F + FT - 1) // FT)](
            V, M, tau, Ab, Bb, h_in, Vhat, h_out, Bsz, T, F, *V.stride(), *M.stride(),
            *tau.stride(), *Vhat.stride(), *h_in.stride(), *h_out.stride(), t, K=K, FTILE=FT)
        v_ref, h_ref = O.interp_ssm_step(V, M, tau, Ab, Bb, h_ref, t, K, FT)
        h_in, h_out = h_out, h_in
    torch.cuda.synchronize()
    assert_close(h_in, h_ref, 1e-5, "h after T steps")
    vtol = 1e-6 if dtype == torch.float32 else TOL[dtype]
    assert_close(Vhat, O.time_aware_interp(V, M, tau, K, FT), vtol, "Vhat rows")


# ------------------------------------------------------------------ streaming
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("H", [300, 301])   # 4-lane and 1-lane accesses
def test_streaming_inplace(dev, dtype, H):
    import streaming_inference_kernel as sk
    g = torch.Generator().manual_seed(6)
    Bsz, BLOCK_H, steps = 5, 128, 20
    Ab = torch.rand(H, generator=g).to(dtype).to(dev)
    Bb = torch.randn(H, generator=g).to(dtype).to(dev)
    D = torch.randn(H, generator=g).to(dtype).to(dev)
    h = torch.zeros(Bsz, H, device=dev, dtype=dtype)
    h_chain = np.zeros((Bsz, H))
    kern = sk.streaming_ssm_inplace_kernel if dtype == torch.float32 else sk.streaming_ssm_inplace_bf16_kernel
    for _ in range(steps):
        v = torch.randn(Bsz, H, generator=g).to(dtype).to(dev)
        C = torch.randn(Bsz, H, generator=g).to(dtype).to(dev)
        y = torch.empty_like(v)
        h_before = h.clone()
        kern[(Bsz, (H + BLOCK_H - 1) // BLOCK_H)](v, h, Ab, Bb, C, D, y, Bsz, H, *v.stride(),
                                                   *h.stride(), *C.stride(), BLOCK_H=BLOCK_H)
        h_step, y_ref = O.streaming_step(v, h_before, Ab, Bb, C, D)   # one step from the same state
        h_chain, _ = O.streaming_step(v, h_chain, Ab, Bb, C, D)       # full-precision chain
        torch.cuda.synchronize()
        assert_close(y, y_ref, TOL[dtype], "y")
        assert_close(h, h_step, TOL[dtype], "h (one step)")
    assert_close(h, h_chain, TOL[dtype], "h (chained)")


@pytest.mark.parametrize("H,BLOCK_H,KR", [(100, 32, 5), (1000, 64, 5), (1000, 64, 17),
                                         (300, 128, 5), (200, 64, 24), (301, 64, 5),
                                         (96, 16, 9), (1000, 256, 11), (301, 128, 5)])
def test_streaming_ring_multi_tile(dev, H, BLOCK_H, KR):
    """Ring insert + backward search + step: 16-byte lanes for BLOCK_H 16..256
    and H % 4 == 0 with the search slots in registers for KRING <= 17; other
    shapes take the per-feature kernel."""
    import streaming_inference_kernel as sk
    g = torch.Generator().manual_seed(7)
    Bsz, steps = 3, max(12, KR + 6)
    ring_V = torch.zeros(Bsz, KR, H, device=dev)
    ring_M = torch.zeros_like(ring_V)
    ring_tau = torch.zeros(Bsz, KR, device=dev)
    head = torch.zeros(Bsz, dtype=torch.int32, device=dev)
    h = torch.zeros(Bsz, H, device=dev)
    Ab, Bb, D = (torch.rand(H, generator=g).to(dev) for _ in range(3))
    st = [np64(ring_V), np64(ring_M), np64(ring_tau), np.zeros(Bsz, dtype=np.int64), np.zeros((Bsz, H))]
    for s in range(steps):
        m = (torch.rand(Bsz, H, generator=g) < (0.0 if s % 3 == 1 else 0.05)).float().to(dev)
        v = (torch.randn(Bsz, H, generator=g).to(dev)) * m
        tau = torch.full((Bsz,), float(s), device=dev)
        C = torch.randn(Bsz, H, generator=g).to(dev)
        y = torch.empty_like(v)
        sk.streaming_interp_then_ssm_kernel[(Bsz, (H + BLOCK_H - 1) // BLOCK_H)](
            ring_V, ring_M, ring_tau, head, v, m, tau, h, Ab, Bb, C, D, y, Bsz, H, KR - 1,
            *ring_V.stride(), *v.stride(), *h.stride(), *C.stride(), BLOCK_H=BLOCK_H, KRING=KR)
        rV, rM, rt, hd, h_new, y_ref = O.streaming_interp_step(*st[:4], v, m, tau, st[4], Ab, Bb,
                                                               C, D, BLOCK_H, KR)
        st = [rV, rM, rt, hd, h_new]
        torch.cuda.synchronize()
        assert_close(y, y_ref, 1e-5, f"y step {s}")
        assert np.array_equal(head.cpu().numpy(), hd)
    assert_close(h, st[4], 1e-5, "h")
    assert_close(ring_V, st[0], 0, "ring_V")
    assert_close(ring_tau, st[2], 0, "ring_tau")
