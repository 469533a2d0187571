"""The whole cfg3 training step at its real shapes, batch 256: ConvLayer (9,32,32) -> 256 x 16 x 16,
ConvLayer -> 512 x 7 x 7, Flatten, LogicLayer 25088 -> 16000 -> 16000, GroupSum(10, tau 30) with
the fused mean cross-entropy (GroupSum.cross_entropy), backward into every logits tensor
(compactlogic/compactlogic.py:83-118, 450-468, 598-626).

Each module is checked against the float64 oracle (oracle/logic_np.py) on the input the GPU
handed it, which isolates every module's error from the others':
  - outputs and input gradients: in full, or on a slice of samples where the oracle's
    per-position loops are slow (outputs and input gradients are per-sample, so a slice is
    exact for the samples it holds);
  - logits gradients: in full for conv1, conv2, the 25088 -> 16000 and the 16000 -> 16000
    layers (they sum over the whole batch);
  - the loss and the gradient GroupSum hands the last layer: against the closed form
    softmax(scores) - onehot(label), scores = group sums / tau.
Tolerance: fp32 within rtol 1e-5 / atol 1e-6 of the float64 oracle.  Logits gradients are
compared after dividing both by the oracle's largest magnitude (their scale is set by the
mean-reduced loss and shrinks layer by layer).
"""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl
from compactlogic_amd import configs
from oracle import logic_np as O

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-5, atol=1e-6)


def f64(t):
    return t.detach().cpu().numpy().astype(np.float64)


def softmax_np(logits):
    p = np.exp(logits - logits.max(1, keepdims=True))
    return p / p.sum(1, keepdims=True)


def logits_grad(p, gw_prob):
    return p * (gw_prob - (p * gw_prob).sum(1, keepdims=True))


def assert_scaled(got, ref):
    scale = float(np.abs(ref).max())
    assert scale > 0
    np.testing.assert_allclose(got / scale, ref / scale, **TOL)


@pytest.fixture(scope="module")
def cfg3_step(device):
    cfg = configs.CONV_CONFIGS["cfg3"]
    model = configs.conv_network(cfg, device=device)
    x, labels = configs.conv_inputs(cfg, device=device)
    assert x.shape == (256, 9, 32, 32)
    conv1, conv2, flat, d1, d2, head = list(model)
    assert isinstance(flat, torch.nn.Flatten) and isinstance(head, cl.GroupSum)
    assert (d1.in_dim, d1.out_dim, d2.out_dim) == (25088, 16000, 16000)
    outs = {}
    h = x
    for name, m in (("c1", conv1), ("c2", conv2), ("f", flat), ("d1", d1), ("d2", d2)):
        h = m(h)
        h.retain_grad()
        outs[name] = h
    loss = head.cross_entropy(h, labels)
    loss.backward()
    torch.cuda.synchronize()
    return dict(model=model, x=x, labels=labels, outs=outs, loss=loss, cfg=cfg)


def test_cfg3_loss_and_head_gradient(cfg3_step):
    s = cfg3_step
    y2 = f64(s["outs"]["d2"])                                   # [256, 16000]
    lab = s["labels"].cpu().numpy()
    scores = O.group_sum(y2, 10, 30.0)
    lse = np.log(np.exp(scores - scores.max(1, keepdims=True)).sum(1)) + scores.max(1)
    ref_loss = float(np.mean(lse - scores[np.arange(256), lab]))
    np.testing.assert_allclose(float(s["loss"].detach()), ref_loss, rtol=1e-5)
    g = softmax_np(scores)
    g[np.arange(256), lab] -= 1.0
    ref_gy = O.group_sum_backward(g / 256, 16000, 10, 30.0)
    np.testing.assert_allclose(f64(s["outs"]["d2"].grad), ref_gy, **TOL)


@pytest.mark.parametrize("which", ["d1", "d2"])
def test_cfg3_dense_layers(cfg3_step, which):
    s = cfg3_step
    layer = s["model"][3] if which == "d1" else s["model"][4]
    xin = f64(s["outs"]["f"] if which == "d1" else s["outs"]["d1"]).T      # [in, 256]
    a = layer.indices[0].cpu().numpy()
    b = layer.indices[1].cpu().numpy()
    gs = layer.gate_sequence.cpu().numpy()
    p = softmax_np(f64(layer.weights))
    # forward, full
    np.testing.assert_allclose(f64(s["outs"][which]).T, O.dense_forward(xin, a, b, p, gs), **TOL)
    gy = f64(s["outs"][which].grad).T                                      # [out, 256]
    # logits gradient, full (a sum over all 256 samples)
    assert_scaled(f64(layer.weights.grad), logits_grad(p, O.dense_backward_w(xin, a, b, gs, gy)))
    # input gradient on a slice of samples
    cols = np.arange(0, 256, 16)
    gin = s["outs"]["f"].grad if which == "d1" else s["outs"]["d1"].grad
    ref = O.dense_backward_x_direct(xin[:, cols], a, b, p, gs, gy[:, cols])
    np.testing.assert_allclose(f64(gin).T[:, cols], ref, **TOL)


def _conv_args(layer):
    return (layer.offsets_ch.cpu().numpy(), layer.offsets_h.cpu().numpy(),
            layer.offsets_w.cpu().numpy())


def test_cfg3_conv2(cfg3_step):
    s = cfg3_step
    layer = s["model"][1]
    xin = f64(s["outs"]["c1"])                                             # [256, 256, 16, 16]
    args = _conv_args(layer)
    gs = layer.gate_sequence.cpu().numpy()
    p = softmax_np(f64(layer.weights))
    np.testing.assert_allclose(
        f64(s["outs"]["c2"]),
        O.conv_forward(xin, *args, p, gs, layer.stride, layer.padding, layer.ks), **TOL)
    gy = f64(s["outs"]["c2"].grad)
    assert_scaled(f64(layer.weights.grad),
                  logits_grad(p, O.conv_backward_w(xin, *args, gs, gy, layer.stride)))
    sl = slice(0, 8)
    rgx, _ = O.conv_backward(xin[sl], *args, p, gs, gy[sl], layer.stride, layer.padding)
    np.testing.assert_allclose(f64(s["outs"]["c1"].grad)[sl], rgx, **TOL)


def test_cfg3_conv1(cfg3_step):
    s = cfg3_step
    layer = s["model"][0]
    xin = f64(s["x"])                                                      # [256, 9, 32, 32]
    args = _conv_args(layer)
    gs = layer.gate_sequence.cpu().numpy()
    p = softmax_np(f64(layer.weights))
    sl = slice(0, 32)
    np.testing.assert_allclose(
        f64(s["outs"]["c1"])[sl],
        O.conv_forward(xin[sl], *args, p, gs, layer.stride, layer.padding, layer.ks), **TOL)
    gy = f64(s["outs"]["c1"].grad)
    assert_scaled(f64(layer.weights.grad),
                  logits_grad(p, O.conv_backward_w(xin, *args, gs, gy, layer.stride)))
