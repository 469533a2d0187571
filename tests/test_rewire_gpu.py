"""Rewiring and freezing during training, on the HIP kernels, against the float64 oracle.

- resample_connections (compactlogic/compactlogic.py:282-348) with weak rows (re-drawn in full)
  and strong rows (winner kept, other slots re-drawn), then a training step: every layer's
  output, logits gradient and input gradient must match the oracle evaluated on the layer's
  current (rewired) indices, opcodes and logits.  Covers per-slot wiring (several runs per
  neuron: the chunked backward) and one pair per neuron (single runs: the row backward), and
  a second rewiring after an optimizer step (the derived plans are rebuilt again).
- SequentialEntropyFreezer (:873-981) freezing the first layer: in training mode the frozen
  layer runs its discrete forward under no_grad and emits {0, 1} (:78-80, :120-130), the
  layers after it train on those values.
Tolerance: fp32 within rtol 1e-5 / atol 1e-6 of the float64 oracle; discrete outputs exact.
"""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl
from oracle import logic_np as O

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-5, atol=1e-6)


def f64(t):
    return t.detach().cpu().numpy().astype(np.float64)


def probs_of(layer):
    return f64(torch.softmax(layer.weights.detach().double(), -1))


def check_layer(layer, xin, yout):
    """Output, logits gradient and input gradient of a soft layer against the oracle;
    xin / yout are the layer's [batch, features] input and output tensors with .grad."""
    a = layer.indices[0].cpu().numpy()
    b = layer.indices[1].cpu().numpy()
    gs = layer.gate_sequence.cpu().numpy()
    p = probs_of(layer)
    x = f64(xin).T
    np.testing.assert_allclose(f64(yout).T, O.dense_forward(x, a, b, p, gs), **TOL)
    gy = f64(yout.grad).T
    gw = O.dense_backward_w(x, a, b, gs, gy)
    ref = p * (gw - (p * gw).sum(1, keepdims=True))
    scale = max(float(np.abs(ref).max()), 1e-30)
    np.testing.assert_allclose(f64(layer.weights.grad) / scale, ref / scale, **TOL)
    if xin.grad is not None:
        np.testing.assert_allclose(f64(xin.grad).T, O.dense_backward_x_direct(x, a, b, p, gs, gy),
                                   **TOL)


def train_step(model, x, y):
    """Forward through the logic layers keeping every activation, the fused loss, backward."""
    acts = [x.detach().requires_grad_(True)]
    h = acts[0]
    for m in model[:-1]:
        h = m(h)
        if h.requires_grad:
            h.retain_grad()
        acts.append(h)
    loss = model[-1].cross_entropy(h, y)
    loss.backward()
    return acts


def make_model(device, connections, seed=0):
    torch.manual_seed(seed)
    return torch.nn.Sequential(
        cl.LogicLayer(64, 128, connections=connections), cl.LogicLayer(128, 96, connections=connections),
        cl.LogicLayer(96, 80, connections=connections), cl.GroupSum(10, 2.0)).to(device)


def mark_rows(layer):
    """Rows 0..7 uniform (weak), rows 8..15 peaked on slot 3 (strong)."""
    with torch.no_grad():
        layer.weights[:8] = 0.0
        layer.weights[8:16] = -4.0
        layer.weights[8:16, 3] = 20.0
    return torch.arange(16, device=layer.weights.device)


@pytest.mark.parametrize("connections", ["random", "original"])
def test_resample_then_train_step_matches_oracle(device, connections):
    model = make_model(device, connections)
    g = torch.Generator().manual_seed(1)
    x = (torch.rand((64, 64), generator=g) < 0.4).float().to(device)
    y = torch.randint(0, 10, (64,), generator=g).to(device)
    # one step before rewiring builds and caches every derived plan
    train_step(model, x, y)
    opt = cl.FusedAdam(model.parameters(), lr=0.05)
    opt.step()
    for rnd in range(2):
        before = [l.indices.clone() for l in model[1:3]]
        for layer in model[1:3]:
            weak, strong = layer.resample_connections(mark_rows(layer), threshold_high=0.95,
                                                      threshold_low=0.5)
            assert int(weak.sum()) == 8 and int(strong.sum()) == 8
            assert bool((layer.weights[8:16].argmax(-1) == 3).all())
            # the reference's inverse index follows the new wiring
            start, yidx, code = O.backward_index(layer.indices.cpu().numpy(), layer.in_dim)
            assert np.array_equal(layer.given_x_indices_of_y_start.cpu().numpy(), start)
        assert any(not torch.equal(b, l.indices) for b, l in zip(before, model[1:3]))
        model.zero_grad(set_to_none=True)
        acts = train_step(model, x, y)
        for i, layer in enumerate(model[:3]):
            check_layer(layer, acts[i], acts[i + 1])
        opt.step()


@pytest.mark.parametrize("connections", ["random", "original"])
def test_small_rewiring_keeps_order_and_matches_oracle(device, connections):
    """Rewiring a few neurons in place keeps the inputs' processing order of the previous
    plan (only the runs and the inverse index are rebuilt): the step still matches the
    oracle on the new wiring."""
    model = make_model(device, connections, seed=4)
    g = torch.Generator().manual_seed(5)
    x = (torch.rand((64, 64), generator=g) < 0.4).float().to(device)
    y = torch.randint(0, 10, (64,), generator=g).to(device)
    train_step(model, x, y)
    layer = model[1]
    order = layer.run_plan().row_order.clone()
    with torch.no_grad():
        layer.indices[:, 3:7] = torch.randint(0, layer.in_dim, (2, 4, layer.num_gates),
                                              device=device)
    plan = layer.run_plan()
    assert plan.stale == 4 and torch.equal(plan.row_order, order)
    model.zero_grad(set_to_none=True)
    acts = train_step(model, x, y)
    for i, l in enumerate(model[:3]):
        check_layer(l, acts[i], acts[i + 1])


def test_freezer_on_partly_frozen_network(device):
    model = make_model(device, "original", seed=2)
    g = torch.Generator().manual_seed(3)
    x = (torch.rand((48, 64), generator=g) < 0.5).float().to(device)
    y = torch.randint(0, 10, (48,), generator=g).to(device)
    freezer = cl.SequentialEntropyFreezer(model, eps=1.0, patience=1)
    freezer.step(0)          # seeds the first layer's running entropy
    assert not model[0].is_frozen
    freezer.step(1)          # |h - EMA| < eps: the first layer freezes
    assert model[0].is_frozen and not model[1].is_frozen
    assert not model[0].weights.requires_grad
    model.train()
    model.zero_grad(set_to_none=True)
    acts = train_step(model, x, y)
    # the frozen layer: its argmax slot's discrete gate on {0,1} inputs, exactly, no graph
    l0 = model[0]
    ref0 = O.dense_eval(f64(x).T, l0.indices[0].cpu().numpy(), l0.indices[1].cpu().numpy(),
                        l0.w.cpu().numpy(), l0.gate_sequence.cpu().numpy())
    out0 = f64(acts[1]).T
    assert np.array_equal(out0, ref0) and set(np.unique(out0)) <= {0.0, 1.0}
    assert not acts[1].requires_grad and l0.weights.grad is None
    # the trainable layers after it, on the frozen layer's {0,1} outputs
    for i in (1, 2):
        check_layer(model[i], acts[i], acts[i + 1])
    # the next step examines the second layer only
    freezer.step(2)
    freezer.step(3)
    assert model[1].is_frozen and not model[2].is_frozen
