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


def test_group_sum_network_head(device):
    torch.manual_seed(0)
    model = torch.nn.Sequential(cl.LogicLayer(50, 60), cl.GroupSum(10, 2.0)).to(device)
    x = torch.rand(33, 50, device=device)
    out = model(x)
    h = model[0](x)
    np.testing.assert_allclose(out.detach().cpu().numpy(),
                               O.group_sum(h.detach().cpu().numpy(), 10, 2.0), rtol=1e-5, atol=1e-6)
