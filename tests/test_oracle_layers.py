"""Pins of the oracle's model-layer functions against torch float64
(independent implementations) and known answers."""
import numpy as np
import pytest
import torch
import torch.nn.functional as Fn

from oracle import ssm_oracle as O


def _r(*shape, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64) * scale


def _padded_layernorm(x, w, b, eps, BH):
    """Triton's masked block emulated literally: the row zero-padded to BH lanes,
    sums over all BH lanes, the mean divided by H (not BH)."""
    H = x.shape[-1]
    xp = Fn.pad(x, (0, BH - H))
    mu = xp.sum(-1, keepdim=True) / H
    xc = xp - mu
    var = (xc * xc).sum(-1, keepdim=True) / H
    return (xc / torch.sqrt(var + eps))[..., :H] * w + b


@pytest.mark.parametrize("H,BH", [(64, 64), (100, 128), (1, 2), (300, 512)])
def test_layernorm_forward(H, BH):
    x = _r(3, 5, H, seed=H, scale=2.0) + 0.7
    w, b = _r(H, seed=1), _r(H, seed=2)
    got = O.layernorm(x, w, b, 1e-5, BH)
    ref = _padded_layernorm(x, w, b, 1e-5, BH)
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-12, atol=1e-12)
    if BH == H:
        ln = Fn.layer_norm(x, (H,), w, b, eps=1e-5)
        np.testing.assert_allclose(got, ln.numpy(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("H,BH", [(64, 64), (100, 128), (37, 64)])
def test_layernorm_backward_is_autograd(H, BH):
    x = (_r(4, 3, H, seed=H + 1, scale=1.5) + 0.3).requires_grad_()
    w = _r(H, seed=3).requires_grad_()
    b = _r(H, seed=4).requires_grad_()
    dout = _r(4, 3, H, seed=5)
    _padded_layernorm(x, w, b, 1e-5, BH).backward(dout)
    dx, dw, db = O.layernorm_bwd(dout, x.detach(), w.detach(), 1e-5, BH)
    np.testing.assert_allclose(dx, x.grad.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dw, w.grad.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(db, b.grad.numpy(), rtol=1e-9, atol=1e-11)


def test_layernorm_padding_changes_the_result():
    """The padded-lane term is real: with a nonzero mean, BLOCK_H > H differs."""
    x = _r(2, 100, seed=9) + 3.0
    w, b = torch.ones(100, dtype=torch.float64), torch.zeros(100, dtype=torch.float64)
    assert np.abs(O.layernorm(x, w, b, 1e-5, 128) - O.layernorm(x, w, b, 1e-5, 100)).max() > 1e-2


def test_swiglu_and_backward():
    gate = _r(3, 7, 33, seed=11, scale=3.0).requires_grad_()
    up = _r(3, 7, 33, seed=12).requires_grad_()
    dout = _r(3, 7, 33, seed=13)
    out = Fn.silu(gate) * up
    np.testing.assert_allclose(O.swiglu(gate.detach(), up.detach()), out.detach().numpy(),
                               rtol=1e-12, atol=1e-12)
    out.backward(dout)
    dg, du = O.swiglu_bwd(dout, gate.detach(), up.detach())
    np.testing.assert_allclose(dg, gate.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(du, up.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_residual_dropout_known_answers():
    x = np.array([1.0, -2.0, 3.0, 4.0])
    r = np.array([0.5, 0.5, 0.5, 0.5])
    m = np.array([1, 0, 1, 0], dtype=np.uint8)
    np.testing.assert_array_equal(O.residual_add(x, r), [1.5, -1.5, 3.5, 4.5])
    np.testing.assert_allclose(O.dropout_residual(x, r, m, 0.8), [1.75, 0.5, 4.25, 0.5])
    np.testing.assert_array_equal(O.dropout_residual(x, r, np.ones(4), 1.0), x + r)


def test_mean_pool_logit():
    h = _r(3, 9, 17, seed=21)
    W = _r(17, seed=22)
    ref = (h @ W).mean(dim=1) / 17 + 0.25                 # mean over t of (h . W), / H
    np.testing.assert_allclose(O.mean_pool_logit(h, W, torch.tensor([0.25])), ref.numpy(),
                               rtol=1e-9)
    ones = O.mean_pool_logit(np.ones((2, 4, 5)), np.ones(5), np.array(0.0))
    np.testing.assert_allclose(ones, [1.0, 1.0], rtol=1e-9)


def test_masked_fill_zero():
    x = _r(2, 3, 4, seed=31)
    m = torch.tensor([[1, 0, 2], [0, 0, 1]])
    got = O.masked_fill_zero(x, m)
    ref = x.masked_fill(~(m > 0)[..., None], 0.0)
    np.testing.assert_array_equal(got, ref.numpy())
