"""GPU parity of the interpolation kernels beyond the sizes their LDS and
grid used to be fixed for: search windows K far past 64 (the reference takes
any K, fused_interp_kernel.py:22,47) and more than 65535 batches (a grid
dimension), against the float64 oracle."""
import pytest
import torch

from helpers import TOL, assert_close, np64
from oracle import ssm_oracle as O

pytestmark = pytest.mark.gpu


def _inputs(Bsz, T, F, dtype, seed, p_obs, dev):
    g = torch.Generator().manual_seed(seed)
    tau = torch.sort(torch.rand(Bsz, T, generator=g) * 100, dim=1).values
    M = (torch.rand(Bsz, T, F, generator=g) < p_obs).float()
    V = (torch.randn(Bsz, T, F, generator=g) * M).to(dtype)
    return V.to(dev), M.to(dev), tau.to(dev)


@pytest.mark.parametrize("K,FTILE,T", [(100, 64, 800), (700, 16, 1500), (1500, 8, 1600)])
def test_interp_large_window(dev, K, FTILE, T):
    """Sparse masks put the nearest observed tile hundreds of steps away."""
    import fused_interp_kernel as fi
    Bsz, F = 2, 64
    V, M, tau = _inputs(Bsz, T, F, torch.float32, seed=K, p_obs=0.0004, dev=dev)
    out = torch.full_like(V, float("nan"))
    fi.fused_time_aware_interp_kernel[(Bsz, T, (F + FTILE - 1) // FTILE)](
        V, M, tau, out, Bsz, T, F, *V.stride(), *M.stride(), *tau.stride(), *out.stride(),
        K=K, FTILE=FTILE)
    torch.cuda.synchronize()
    assert_close(out, O.time_aware_interp(V, M, tau, K, FTILE), 1e-6, f"interp K={K}")


@pytest.mark.parametrize("F,FT", [(256, 256), (600, 512)])   # one thread per feature / wide tiles
def test_interp_ssm_step_large_window(dev, F, FT):
    import fused_ssm_interp as fs
    Bsz, T, K = 2, 700, 300
    V, M, tau = _inputs(Bsz, T, F, torch.float32, seed=F, p_obs=0.0005, dev=dev)
    g = torch.Generator().manual_seed(6)
    Ab = torch.rand(F, generator=g).to(dev)
    Bb = torch.randn(F, generator=g).to(dev)
    h_in = torch.randn(Bsz, F, generator=g).to(dev)
    h_out = torch.empty_like(h_in)
    Vhat = torch.zeros_like(V)
    h_ref = np64(h_in)
    for t in range(0, T, 37):   # steps spread over the sequence, each checked
        fs.fused_interp_ssm_step_kernel[(Bsz, (F + FT - 1) // FT)](
            V, M, tau, Ab, Bb, h_in, Vhat, h_out, Bsz, T, F, *V.stride(), *M.stride(),
            *tau.stride(), *Vhat.stride(), *h_in.stride(), *h_out.stride(), t, K=K, FTILE=FT)
        v_ref, h_ref = O.interp_ssm_step(V, M, tau, Ab, Bb, h_ref, t, K, FT)
        torch.cuda.synchronize()
        assert_close(Vhat[:, t], v_ref, 1e-6, f"Vhat row {t}")
        h_in, h_out = h_out, h_in
    assert_close(h_in, h_ref, 1e-5, "h")


def test_interp_corrected_large_window(dev):
    from tssm import time_aware_interp_corrected
    Bsz, T, F, K = 2, 1500, 96, 400
    V, M, tau = _inputs(Bsz, T, F, torch.float32, seed=11, p_obs=0.003, dev=dev)
    out = time_aware_interp_corrected(V, M, tau, K=K)
    torch.cuda.synchronize()
    assert_close(out, O.time_aware_interp_corrected(V, M, tau, K), 1e-6, "corrected K=400")


def test_interp_many_batches(dev):
    """70000 sequences: the offline, step and corrected kernels launch the
    batches in slices of at most 65535 grid rows."""
    import fused_interp_kernel as fi
    import fused_ssm_interp as fs
    from tssm import time_aware_interp_corrected
    Bsz, T, F, K, FT = 70000, 5, 8, 2, 8
    V, M, tau = _inputs(Bsz, T, F, torch.float32, seed=3, p_obs=0.3, dev=dev)
    out = torch.full_like(V, float("nan"))
    fi.fused_time_aware_interp_kernel[(Bsz, T, 1)](
        V, M, tau, out, Bsz, T, F, *V.stride(), *M.stride(), *tau.stride(), *out.stride(),
        K=K, FTILE=FT)
    torch.cuda.synchronize()
    assert_close(out, O.time_aware_interp(V, M, tau, K, FT), 1e-6, "interp, 70000 batches")
    g = torch.Generator().manual_seed(8)
    Ab, Bb = torch.rand(F, generator=g).to(dev), torch.randn(F, generator=g).to(dev)
    h_in = torch.randn(Bsz, F, generator=g).to(dev)
    h_out = torch.empty_like(h_in)
    Vhat = torch.zeros_like(V)
    fs.fused_interp_ssm_step_kernel[(Bsz, 1)](
        V, M, tau, Ab, Bb, h_in, Vhat, h_out, Bsz, T, F, *V.stride(), *M.stride(),
        *tau.stride(), *Vhat.stride(), *h_in.stride(), *h_out.stride(), 2, K=K, FTILE=FT)
    torch.cuda.synchronize()
    v_ref, h_ref = O.interp_ssm_step(V, M, tau, Ab, Bb, np64(h_in), 2, K, FT)
    assert_close(Vhat[:, 2], v_ref, 1e-6, "step Vhat, 70000 batches")
    assert_close(h_out, h_ref, 1e-6, "step h, 70000 batches")
    cor = time_aware_interp_corrected(V, M, tau, K=K)
    torch.cuda.synchronize()
    assert_close(cor, O.time_aware_interp_corrected(V, M, tau, K), 1e-6, "corrected, 70000")


def test_interp_window_beyond_lds_is_refused(dev):
    """A window whose flags do not fit one workgroup's LDS is refused on the
    host with a clear error (nothing launched)."""
    from tssm import time_aware_interp_corrected
    V, M, tau = _inputs(1, 8, 8, torch.float32, seed=1, p_obs=0.5, dev=dev)
    with pytest.raises(ValueError, match="449"):
        time_aware_interp_corrected(V, M, tau, K=450)
    import fused_interp_kernel as fi
    out = torch.empty_like(V)
    with pytest.raises(ValueError, match="UNSUPPORTED"):
        fi.fused_time_aware_interp_kernel[(1, 8, 1)](
            V, M, tau, out, 1, 8, 8, *V.stride(), *M.stride(), *tau.stride(), *out.stride(),
            K=40000, FTILE=8)
