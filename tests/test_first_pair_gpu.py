"""The first-layer pair (LogicLayerFirstPairFunction): the second dense layer's row backward
finishing the first layer's logits gradient.  Its gradients must be bitwise those of the two
layers' own autograd steps (cl_dense_backward_rows, then cl_dense_weight_grad on the stored
input gradient), which the oracle tests of test_network_gpu pin."""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl
from compactlogic_amd import configs, timing
from compactlogic_amd import layers as L

pytestmark = pytest.mark.gpu


def net(device, dims, k, dtype, seed):
    torch.manual_seed(seed)
    mods = [cl.LogicLayer(i, o, connections="original") for i, o in dims]
    model = torch.nn.Sequential(*mods, cl.GroupSum(k, 2.0)).to(device)
    if dtype == torch.float64:
        model = model.double()
    return model


def grads(model, x, labels, pair: bool):
    old = L.LogicLayer.first_pair
    L.LogicLayer.first_pair = pair
    try:
        model.zero_grad(set_to_none=True)
        with timing.record() as rec:
            loss = model[-1].cross_entropy(model[:-1](x), labels)
            loss.backward()
        calls = set(rec.summary())
    finally:
        L.LogicLayer.first_pair = old
    return loss.detach().clone(), [p.grad.clone() for p in model.parameters()], calls


@pytest.mark.parametrize("dims,k,batch,dtype", [
    ([(64, 256), (256, 640)], 10, 1024, torch.float32),
    ([(64, 256), (256, 320), (320, 300)], 10, 256, torch.float32),
    ([(100, 400), (400, 800)], 8, 64, torch.float64),
    ([(30, 90), (90, 200), (200, 120)], 4, 2048, torch.float32),
])
def test_pair_gradients_are_bitwise_the_unpaired_ones(device, dims, k, batch, dtype):
    model = net(device, dims, k, dtype, seed=batch)
    g = torch.Generator().manual_seed(batch)
    x = (torch.rand((batch, dims[0][0]), generator=g) < 0.4).to(dtype).to(device)
    labels = torch.randint(0, k, (batch,), generator=g).to(device)
    l0, g0, c0 = grads(model, x, labels, pair=False)
    l1, g1, c1 = grads(model, x, labels, pair=True)
    assert any(n.startswith("cl_dense_backward_rows_first") for n in c1)
    assert not any(n.startswith("cl_dense_weight_grad") for n in c1)
    assert any(n.startswith("cl_dense_weight_grad") for n in c0)
    assert torch.equal(l0, l1)
    for a, b in zip(g0, g1):
        assert torch.equal(a, b)


def test_pair_stays_off_where_waves_share_a_row(device):
    """A second layer with many entries per input row (here 16) takes several waves per row in
    its row backward, a different summation order than the first-layer mode's one wave: the
    pair stays off and both runs are the unpaired steps."""
    dims = [(64, 128), (128, 1024)]
    model = net(device, dims, 8, torch.float32, seed=5)
    g = torch.Generator().manual_seed(5)
    x = (torch.rand((512, 64), generator=g) < 0.4).float().to(device)
    labels = torch.randint(0, 8, (512,), generator=g).to(device)
    l0, g0, _ = grads(model, x, labels, pair=False)
    l1, g1, c1 = grads(model, x, labels, pair=True)
    assert not any(n.startswith("cl_dense_backward_rows_first") for n in c1)
    assert any(n.startswith("cl_dense_backward_rows[") for n in c1)
    assert torch.equal(l0, l1)
    for a, b in zip(g0, g1):
        assert torch.equal(a, b)


def test_pair_cfg2_step(device):
    cfg = configs.CONFIGS["cfg2"]
    model = configs.dense_network(cfg, device=device)
    x, labels = configs.dense_inputs(cfg, device=device)
    l0, g0, _ = grads(model, x, labels, pair=False)
    l1, g1, c1 = grads(model, x, labels, pair=True)
    assert "cl_dense_backward_rows_first[12000->12000]" in c1
    assert torch.equal(l0, l1) and all(torch.equal(a, b) for a, b in zip(g0, g1))


def test_pair_keeps_other_uses_of_the_first_output(device):
    """y1 feeding the second layer and also the loss directly: the first layer's own node
    adds the other path's gradient; retained or hooked activations keep the unpaired path."""
    model = net(device, [(64, 256), (256, 640)], 8, torch.float32, seed=3)
    g = torch.Generator().manual_seed(3)
    x = (torch.rand((512, 64), generator=g) < 0.5).float().to(device)
    labels = torch.randint(0, 8, (512,), generator=g).to(device)

    def run(pair):
        old = L.LogicLayer.first_pair
        L.LogicLayer.first_pair = pair
        try:
            model.zero_grad(set_to_none=True)
            y1 = model[0](x)
            loss = model[2].cross_entropy(model[1](y1), labels) + y1.square().mean()
            loss.backward()
        finally:
            L.LogicLayer.first_pair = old
        return [p.grad.clone() for p in model.parameters()]

    a, b = run(False), run(True)
    for u, v in zip(a, b):
        torch.testing.assert_close(u, v, rtol=1e-5, atol=1e-7)
    # a retained activation still gets its gradient
    model.zero_grad(set_to_none=True)
    y1 = model[0](x)
    y1.retain_grad()
    model[2].cross_entropy(model[1](y1), labels).backward()
    assert y1.grad is not None and torch.isfinite(y1.grad).all()


def test_pair_under_graph_capture(device):
    """The captured step with the pair replays to the eager gradients."""
    model = net(device, [(64, 256), (256, 640)], 10, torch.float32, seed=5)
    g = torch.Generator().manual_seed(5)
    x = (torch.rand((1024, 64), generator=g) < 0.5).float().to(device)
    labels = torch.randint(0, 10, (1024,), generator=g).to(device)
    l0, g0, calls = grads(model, x, labels, pair=True)
    assert any(n.startswith("cl_dense_backward_rows_first") for n in calls)

    def step():
        loss = model[-1].cross_entropy(model[:-1](x), labels)
        loss.backward()
        return loss

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        model.zero_grad(set_to_none=True)
        step()
    torch.cuda.current_stream().wait_stream(side)
    model.zero_grad(set_to_none=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static, l0)
        assert all(torch.equal(p.grad, r) for p, r in zip(model.parameters(), g0))
        torch.ones(8, device=device).sum().item()      # eager work between replays
