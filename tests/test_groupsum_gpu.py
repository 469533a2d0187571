"""GroupSum kernels against the float64 oracle, on every input layout."""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl
from oracle import logic_np as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("batch,feats,k", [(1024, 12000, 10), (256, 16000, 10), (7, 25, 10),
                                           (64, 9, 3), (300, 40, 40), (5, 3, 7)])
@pytest.mark.parametrize("layout", ["transposed", "contiguous", "strided"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_group_sum_forward_backward(device, batch, feats, k, layout, dtype):
    rng = np.random.default_rng(batch + feats + k)
    xn = rng.random((batch, feats))
    base = torch.as_tensor(xn, dtype=dtype, device=device)
    if layout == "transposed":
        x = base.t().contiguous().t()                 # [batch, feats] view of [feats, batch]
    elif layout == "contiguous":
        x = base.clone()
    else:
        x = torch.zeros((batch, 2 * feats), dtype=dtype, device=device)[:, ::2]
        x.copy_(base)
    x = x.detach().requires_grad_(True)
    tau = 10.0
    out = cl.GroupSum(k, tau)(x)
    tol = dict(rtol=1e-5, atol=1e-6) if dtype == torch.float32 else dict(rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(out.detach().cpu().numpy(), O.group_sum(xn, k, tau), **tol)
    g = rng.standard_normal((batch, k))
    (gx,) = torch.autograd.grad(out, x, torch.as_tensor(g, dtype=dtype, device=device))
    ref = O.group_sum_backward(g, feats, k, tau)
    # The backward is a broadcast divide: bit-exact against torch's own division.
    assert torch.equal(gx.cpu(), (torch.as_tensor(g, dtype=dtype).repeat_interleave(-(-feats // k), 1)[:, :feats] / tau))
    np.testing.assert_allclose(gx.cpu().numpy(), ref, **tol)
    if layout == "transposed":
        assert gx.t().is_contiguous(), "gradient should keep the [features, batch] layout"


@pytest.mark.parametrize("shape,k", [((4, 3, 60), 10), ((2, 5, 7, 33), 4), ((90,), 9)])
def test_group_sum_any_leading_dims(device, shape, k):
    """[..., features] -> [..., k], as the reference's reshape-and-sum
    (compactlogic/compactlogic.py:460-465), with its gradient."""
    rng = np.random.default_rng(len(shape) + k)
    xn = rng.random(shape)
    x = torch.as_tensor(xn, device=device).requires_grad_(True)
    out = cl.GroupSum(k, 3.0)(x)
    assert out.shape == shape[:-1] + (k,)
    flat = xn.reshape(-1, shape[-1])
    np.testing.assert_allclose(out.detach().cpu().numpy().reshape(-1, k),
                               O.group_sum(flat, k, 3.0), rtol=1e-12, atol=1e-12)
    g = rng.standard_normal(out.shape)
    (gx,) = torch.autograd.grad(out, x, torch.as_tensor(g, device=device))
    ref = O.group_sum_backward(g.reshape(-1, k), shape[-1], k, 3.0).reshape(shape)
    np.testing.assert_allclose(gx.cpu().numpy(), ref, rtol=1e-12, atol=1e-12)


def test_group_sum_network_head(device):
    torch.manual_seed(0)
    model = torch.nn.Sequential(cl.LogicLayer(50, 60), cl.GroupSum(10, 2.0)).to(device)
    x = torch.rand(33, 50, device=device)
    out = model(x)
    h = model[0](x)
    np.testing.assert_allclose(out.detach().cpu().numpy(),
                               O.group_sum(h.detach().cpu().numpy(), 10, 2.0), rtol=1e-5, atol=1e-6)


def _ce_reference(xn, labels, k, tau, ignore=-100):
    """float64 numpy: scores, mean cross-entropy over counted samples, d loss / d x."""
    z = O.group_sum(xn, k, tau)
    m = z.max(1, keepdims=True)
    e = np.exp(z - m)
    lse = (m + np.log(e.sum(1, keepdims=True)))[:, 0]
    p = e / e.sum(1, keepdims=True)
    counted = labels != ignore
    cnt = counted.sum()
    safe = np.where(counted, labels, 0)
    loss = (lse - z[np.arange(len(z)), safe])[counted].sum() / cnt
    gz = p.copy()
    gz[np.arange(len(z)), safe] -= 1.0
    gz[~counted] = 0.0
    gz /= cnt
    return z, loss, O.group_sum_backward(gz, xn.shape[1], k, tau)


@pytest.mark.parametrize("batch,feats,k", [(1024, 12000, 10), (256, 16000, 10), (7, 25, 10),
                                           (300, 40, 40), (2000, 50, 5)])
@pytest.mark.parametrize("layout", ["transposed", "contiguous", "strided"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_group_sum_cross_entropy_matches_closed_form(device, batch, feats, k, layout, dtype):
    rng = np.random.default_rng(3 * batch + feats + k)
    xn = rng.random((batch, feats))
    base = torch.as_tensor(xn, dtype=dtype, device=device)
    if layout == "transposed":
        x = base.t().contiguous().t()
    elif layout == "contiguous":
        x = base.clone()
    else:
        x = torch.zeros((batch, 2 * feats), dtype=dtype, device=device)[:, ::2]
        x.copy_(base)
    x = x.detach().requires_grad_(True)
    labels = rng.integers(0, k, batch)
    labels[rng.random(batch) < 0.1] = -100                 # ignored samples
    tau = 10.0
    gs = cl.GroupSum(k, tau)
    loss, scores = gs.cross_entropy(x, torch.as_tensor(labels, device=device), return_scores=True)
    rz, rloss, rgx = _ce_reference(xn, labels, k, tau)
    tol = dict(rtol=1e-5, atol=1e-6) if dtype == torch.float32 else dict(rtol=1e-11, atol=1e-13)
    np.testing.assert_allclose(scores.cpu().numpy(), rz, **tol)
    np.testing.assert_allclose(loss.item(), rloss, **tol)
    (gx,) = torch.autograd.grad(loss * 2.5, x)              # upstream gradient 2.5
    np.testing.assert_allclose(gx.cpu().numpy(), 2.5 * rgx, **tol)
    if layout == "transposed":
        assert gx.t().is_contiguous()
    # the same function as torch's cross_entropy on GroupSum's output
    ref = torch.nn.functional.cross_entropy(gs(x.detach()), torch.as_tensor(labels, device=device))
    np.testing.assert_allclose(loss.item(), ref.item(), **tol)
    # bitwise repeatable
    loss2 = gs.cross_entropy(x.detach(), torch.as_tensor(labels, device=device))
    assert torch.equal(loss.detach(), loss2)


def test_group_sum_cross_entropy_edge_labels(device):
    x = torch.rand((64, 20), device=device, requires_grad=True)
    gs = cl.GroupSum(4, 2.0)
    all_ignored = torch.full((64,), -100, dtype=torch.int64, device=device)
    loss = gs.cross_entropy(x, all_ignored)
    assert torch.isnan(loss)                                 # mean of no samples, as torch
    (gx,) = torch.autograd.grad(loss, x)
    assert torch.equal(gx, torch.zeros_like(gx))
    bad = torch.randint(0, 4, (64,), device=device)
    bad[5] = 7                                               # outside [0, k)
    assert torch.isnan(gs.cross_entropy(x.detach(), bad))
    with pytest.raises(RuntimeError):
        gs.cross_entropy(x, bad.to(torch.int32))
    with pytest.raises(RuntimeError):
        gs.cross_entropy(x, bad[:10])
