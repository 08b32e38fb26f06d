"""Shared test helpers."""
import numpy as np
import torch

TOL_F32 = 1e-5   # max normwise relative error, fp32 inputs
TOL_BF16 = 1e-2  # bf16 inputs, fp32 state
TOL = {torch.float32: TOL_F32, torch.bfloat16: TOL_BF16, torch.float16: TOL_BF16}


def np64(t):
    if isinstance(t, torch.Tensor):
        return t.detach().to("cpu", torch.float64).numpy()
    return np.asarray(t, dtype=np.float64)


def relerr(got, ref):
    """max|got - ref| / max|ref| (normwise max-relative error)."""
    g, r = np64(got), np64(ref)
    assert g.shape == r.shape, (g.shape, r.shape)
    den = np.max(np.abs(r))
    return float(np.max(np.abs(g - r)) / (den if den > 0 else 1.0))


def assert_close(got, ref, tol, what=""):
    e = relerr(got, ref)
    assert e <= tol, f"{what}: normwise relative error {e:.3e} > {tol:.1e}"
    return e
