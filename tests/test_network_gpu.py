"""Benchmark-shaped training steps (cfg1, cfg2) checked layer by layer against the oracle.

Forward activations and input gradients are column-separable, so they are checked on a
slice of the batch; weight gradients reduce over the whole batch and are checked in full on
a subset of layers.  Tolerance as in test_dense_gpu: rtol 1e-5 / atol 1e-6 (fp32 vs float64).
"""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl
from compactlogic_amd import configs
from oracle import logic_np as O

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-5, atol=1e-6)


def np_(t):
    return t.detach().cpu().numpy().astype(np.float64)


def run_step(model, x, labels):
    acts, h = [x], x
    for layer in model[:-1]:
        h = layer(h)
        h.retain_grad()
        acts.append(h)
    out = model[-1](h)
    loss = torch.nn.functional.cross_entropy(out, labels)
    loss.backward()
    return acts, out, loss


@pytest.mark.parametrize("name,cols,wgrad_layers", [("cfg1", 128, [0, 1, 2, 3]),
                                                    ("cfg2", 48, [0, 5])])
def test_config_step_layerwise(device, name, cols, wgrad_layers):
    cfg = configs.CONFIGS[name]
    model = configs.dense_network(cfg, device=device)
    x, labels = configs.dense_inputs(cfg, device=device)
    acts, out, loss = run_step(model, x, labels)
    assert torch.isfinite(loss)
    layers = [m for m in model if isinstance(m, cl.LogicLayer)]
    sl = slice(0, cols)
    for i, layer in enumerate(layers):
        a, b = np_(layer.indices[0]).astype(np.int64), np_(layer.indices[1]).astype(np.int64)
        gs = layer.gate_sequence.cpu().numpy()
        p = np_(torch.softmax(layer.weights, -1))
        xin = np_(acts[i])[sl].T
        np.testing.assert_allclose(np_(acts[i + 1])[sl].T, O.dense_forward(xin, a, b, p, gs), **TOL)
        gy = np_(acts[i + 1].grad)
        if i > 0:
            np.testing.assert_allclose(np_(acts[i].grad)[sl].T,
                                       O.dense_backward_x_direct(xin, a, b, p, gs, gy[sl].T), **TOL)
        if i in wgrad_layers:
            gw = O.dense_backward_w(np_(acts[i]).T, a, b, gs, gy.T)
            glog = p * (gw - (p * gw).sum(1, keepdims=True))      # softmax backward
            np.testing.assert_allclose(np_(layer.weights.grad), glog, **TOL)
    head = np_(out)
    np.testing.assert_allclose(head, O.group_sum(np_(acts[-1]), cfg.k, cfg.tau), **TOL)


def test_cfg2_step_is_deterministic(device):
    cfg = configs.CONFIGS["cfg2"]
    model = configs.dense_network(cfg, device=device)
    x, labels = configs.dense_inputs(cfg, device=device)
    grads = []
    for _ in range(2):
        model.zero_grad(set_to_none=True)
        _, out, loss = run_step(model, x, labels)
        grads.append([m.weights.grad.clone() for m in model if isinstance(m, cl.LogicLayer)] + [out.detach()])
    for g1, g2 in zip(*grads):
        assert torch.equal(g1, g2)
