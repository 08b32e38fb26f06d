"""Model-layer drop-ins on the GPU against the float64 oracle: LayerNorm and
SwiGLU forward/backward, residual add and dropout, the mean-pool logit head
and the padding mask.  Partial grids leave the other rows untouched."""
import numpy as np
import pytest
import torch

from helpers import TOL, assert_close, np64
from oracle import ssm_oracle as O

pytestmark = pytest.mark.gpu


def _r(shape, seed, dtype=torch.float32, scale=1.0, shift=0.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale + shift).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("H,BH", [(64, 64), (100, 128), (1024, 1024), (300, 512), (99, 128),
                                  (2500, 4096)])
def test_layernorm_forward(dev, dtype, H, BH):
    import fused_ssm_interp as fs
    B, L = 3, 5
    base = _r((B, L, H + 16), seed=H, dtype=dtype, scale=2.0, shift=0.5).to(dev)
    x = base[..., 8:8 + H]                       # rows with stride H + 16
    w = _r((H,), 1, dtype).to(dev)
    b = _r((H,), 2, dtype).to(dev)
    out = torch.full_like(base, float("nan"))[..., :H]
    fs.layernorm_kernel[(B, L)](x, w, b, out, B, L, H, x.stride(0), x.stride(1), 1,
                                EPS=1e-5, BLOCK_H=BH)
    torch.cuda.synchronize()
    ref = O.layernorm(x, w, b, 1e-5, BH)
    assert_close(out, ref, TOL[dtype] if dtype != torch.float32 else 1e-5, f"LN H={H} BH={BH}")


def test_layernorm_partial_grid(dev):
    import fused_ssm_interp as fs
    B, L, H = 4, 6, 96
    x = _r((B, L, H), 7).to(dev)
    w, b = _r((H,), 8).to(dev), _r((H,), 9).to(dev)
    out = torch.full_like(x, float("nan"))
    fs.layernorm_kernel[(2, 3)](x, w, b, out, B, L, H, *x.stride(), EPS=1e-5, BLOCK_H=128)
    torch.cuda.synchronize()
    assert_close(out[:2, :3], O.layernorm(x[:2, :3], w, b, 1e-5, 128), 1e-5, "LN partial")
    assert torch.isnan(out[2:]).all() and torch.isnan(out[:2, 3:]).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,L,H,BH", [(3, 5, 100, 128), (4, 200, 256, 256), (2, 3, 1000, 1024),
                                      (3, 70, 99, 128), (2, 4, 2500, 4096), (8, 1100, 64, 64)])
def test_layernorm_backward(dev, dtype, B, L, H, BH):
    import fused_ssm_interp as fs
    x = _r((B, L, H), 10 + H, dtype, 1.5, 0.3).to(dev)
    w = _r((H,), 11, dtype).to(dev)
    dout = _r((B, L, H), 12, dtype).to(dev)
    dx = torch.full_like(x, float("nan"))
    dw0, db0 = _r((H,), 13), _r((H,), 14)          # the kernel adds into dw/db
    dw, db = dw0.to(dtype).to(dev), db0.to(dtype).to(dev)
    fs.layernorm_bwd_kernel[(B, L)](dout, x, w, dx, dw, db, B, L, H, x.stride(0), x.stride(1),
                                    EPS=1e-5, BLOCK_H=BH)
    torch.cuda.synchronize()
    rdx, rdw, rdb = O.layernorm_bwd(dout, x, w, 1e-5, BH)
    tol = TOL[dtype] if dtype != torch.float32 else 1e-5
    assert_close(dx, rdx, tol, "LN dx")
    assert_close(dw, np64(dw0.to(dtype)) + rdw, tol, "LN dw")
    assert_close(db, np64(db0.to(dtype)) + rdb, tol, "LN db")
    # deterministic: a second run gives the same dx and the same increments
    dx2 = torch.empty_like(dx)
    dw2, db2 = dw0.to(dtype).to(dev), db0.to(dtype).to(dev)
    fs.layernorm_bwd_kernel[(B, L)](dout, x, w, dx2, dw2, db2, B, L, H, x.stride(0), x.stride(1),
                                    EPS=1e-5, BLOCK_H=BH)
    torch.cuda.synchronize()
    assert torch.equal(dx, dx2) and torch.equal(dw, dw2) and torch.equal(db, db2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("H", [333, 336])   # 1-lane and 4-lane accesses
def test_swiglu_forward_backward(dev, dtype, H):
    import fused_ssm_interp as fs
    B, L = 3, 7
    gate = _r((B, L, H), 20, dtype, 3.0).to(dev)
    up = _r((B, L, H), 21, dtype).to(dev)
    dout = _r((B, L, H), 22, dtype).to(dev)
    out = torch.empty_like(gate)
    fs.swiglu_kernel[(B, L)](gate, up, out, B, L, H, gate.stride(0), gate.stride(1), BLOCK_H=512)
    dg, du = torch.empty_like(gate), torch.empty_like(gate)
    fs.swiglu_bwd_kernel[(B, L)](dout, gate, up, dg, du, B, L, H, gate.stride(0), gate.stride(1),
                                 BLOCK_H=512)
    torch.cuda.synchronize()
    tol = TOL[dtype] if dtype != torch.float32 else 1e-5
    assert_close(out, O.swiglu(gate, up), tol, "swiglu")
    rdg, rdu = O.swiglu_bwd(dout, gate, up)
    assert_close(dg, rdg, tol, "swiglu dgate")
    assert_close(du, rdu, tol, "swiglu dup")


@pytest.mark.parametrize("N,dtype", [(10_000, torch.float32), (10_001, torch.float32),
                                     (10_000, torch.bfloat16)])   # 4-element and scalar paths
def test_residual_and_dropout(dev, N, dtype):
    import multihead_ssm_kernel as mk
    BLOCK = 1024
    x, res = _r((N,), 30, dtype).to(dev), _r((N,), 31, dtype).to(dev)
    keep = (torch.rand(N, generator=torch.Generator().manual_seed(32)) < 0.8).to(torch.uint8).to(dev)
    tol = 1e-6 if dtype == torch.float32 else TOL[dtype]
    out = torch.full_like(x, float("nan"))
    mk.residual_add_kernel[(-(-N // BLOCK),)](x, res, out, N, BLOCK=BLOCK)
    torch.cuda.synchronize()
    assert_close(out, O.residual_add(x, res), tol, "residual")
    out2 = torch.full_like(x, float("nan"))
    mk.dropout_residual_kernel[(4,)](x, res, keep, out2, N, 0.8, BLOCK=BLOCK)   # first 4096 only
    torch.cuda.synchronize()
    assert_close(out2[:4096], O.dropout_residual(x[:4096], res[:4096], keep[:4096], 0.8), tol,
                 "dropout")
    assert torch.isnan(out2[4096:]).all()
    out3 = torch.empty_like(x)
    mk.dropout_residual_kernel[(10,)](x, res, keep.bool(), out3, N, 0.8, BLOCK=BLOCK)
    torch.cuda.synchronize()
    assert_close(out3, O.dropout_residual(x, res, keep, 0.8), tol, "dropout bool mask")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("H", [70, 72])
def test_mean_pool_logit(dev, dtype, H):
    import streaming_inference_kernel as sk
    B, T = 4, 300
    base = _r((B, T + 2, H), 40, dtype).to(dev)
    h = base[:, 1:T + 1]
    W = _r((H,), 41, dtype).to(dev)
    bias = torch.tensor([0.3], dtype=dtype, device=dev)
    out = torch.full((B,), float("nan"), dtype=dtype, device=dev)
    sk.mean_pool_logit_kernel[(3,)](h, W, bias, out, B, T, H, h.stride(0), h.stride(1), 1,
                                    BLOCK_H=64, BLOCK_T=16)
    torch.cuda.synchronize()
    ref = O.mean_pool_logit(h[:3], W, bias)
    got = np64(out[:3])
    # the per-batch logits are O(bias) while the pooled term is tiny: compare both parts
    assert np.abs(got - ref).max() <= (2e-2 if dtype == torch.bfloat16 else 1e-6)
    assert torch.isnan(out[3:]).all()


@pytest.mark.parametrize("mdtype", [torch.bool, torch.uint8, torch.int32, torch.float32])
@pytest.mark.parametrize("H", [37, 40])
def test_masked_fill_zero(dev, mdtype, H):
    import streaming_inference_kernel as sk
    B, T, BLOCK = 3, 50, 256
    x = _r((B, T, H), 50).to(dev)
    m = (torch.rand(B, T, generator=torch.Generator().manual_seed(51)) < 0.6).to(mdtype).to(dev)
    out = torch.full_like(x, float("nan"))
    n = B * T * H
    sk.masked_fill_zero_kernel[(-(-n // BLOCK),)](x, m, out, B, T, H, BLOCK=BLOCK)
    torch.cuda.synchronize()
    assert np.array_equal(np64(out), O.masked_fill_zero(x, m))
    # a grid covering a flat prefix that ends inside a row
    out2 = torch.full_like(x, float("nan"))
    sk.masked_fill_zero_kernel[(7,)](x, m, out2, B, T, H, BLOCK=BLOCK)
    torch.cuda.synchronize()
    k = 7 * BLOCK
    assert np.array_equal(np64(out2).reshape(-1)[:k], O.masked_fill_zero(x, m).reshape(-1)[:k])
    assert torch.isnan(out2.reshape(-1)[k:]).all()
