"""The reference's default wiring (connections='random': each of a neuron's 16 slots reads its
own input pair, compactlogic/compactlogic.py:160-182) at the shape the bench times: a
12000 -> 12000 layer of the cfg2 network, batch 1024, fp32.  Every neuron is 16 runs, so the
layer trains through the multi-run kernels (cl_dense_prep + cl_dense_forward_tiled,
cl_dense_backward_tiled + cl_dense_backward_finalize).  Checked against the float64 oracle:
the forward and the input gradient on a slice of sample columns (every column is computed
independently), the logits gradient over the whole batch.  Tolerance: rtol 1e-5 / atol 1e-6,
scaled by the largest magnitude for the gradients (upstream gradients at the scale of a
mean-reduced loss)."""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl
from compactlogic_amd import configs
from oracle import logic_np as O

pytestmark = pytest.mark.gpu


def f64(t):
    return t.detach().cpu().numpy().astype(np.float64)


def check(got, ref, rtol=1e-5):
    scale = max(float(np.abs(ref).max()), 1e-30)
    np.testing.assert_allclose(got / scale, ref / scale, rtol=rtol, atol=rtol)


def test_random_wiring_layer_at_the_benched_shape(device):
    cfg = configs.CONFIGS["cfg2"]
    model = configs.dense_network(cfg, device=device, wiring="random")
    layer = model[1]                                     # 12000 -> 12000
    assert (layer.in_dim, layer.out_dim, layer.num_gates) == (12000, 12000, 16)
    plan = layer.run_plan()
    assert not plan.single_run and plan.num_runs > 15 * layer.out_dim   # the multi-run path
    batch = cfg.batch
    g = torch.Generator().manual_seed(31)
    x = (torch.rand((batch, layer.in_dim), generator=g) < 0.3).float()
    # an activation-like input: products of probabilities in [0, 1]
    x = (x * torch.rand((batch, layer.in_dim), generator=g)).to(device).requires_grad_(True)
    gy = ((torch.rand((batch, layer.out_dim), generator=g) - 0.5) / batch).to(device)
    y = layer(x)
    y.backward(gy)
    torch.cuda.synchronize()
    a, b = layer.indices[0].cpu().numpy(), layer.indices[1].cpu().numpy()
    gs = layer.gate_sequence.cpu().numpy()
    p = torch.softmax(layer.weights.detach().double(), -1).cpu().numpy()
    xr = f64(x).T                                        # [in, batch]
    gyr = f64(gy).T                                      # [out, batch]
    cols = np.r_[0:32, batch - 32:batch]                 # first and last 32 samples
    np.testing.assert_allclose(f64(y).T[:, cols], O.dense_forward(xr[:, cols], a, b, p, gs),
                               rtol=1e-5, atol=1e-6)
    check(f64(x.grad).T[:, cols], O.dense_backward_x_direct(xr[:, cols], a, b, p, gs, gyr[:, cols]))
    gp = O.dense_backward_w(xr, a, b, gs, gyr)           # whole batch
    check(f64(layer.weights.grad), p * (gp - (p * gp).sum(1, keepdims=True)))
