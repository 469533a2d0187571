"""A training step captured as a HIP graph replays to the eager result every time, with
eager work and synchronisation between replays."""
import pytest
import torch

import compactlogic_amd as cl

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fused_loss", [False, True])
def test_graph_replays_match_eager(device, fused_loss):
    torch.manual_seed(0)
    model = torch.nn.Sequential(cl.LogicLayer(100, 200, connections="original"),
                                cl.LogicLayer(200, 200), cl.GroupSum(10, 5.0)).to(device)
    x = (torch.rand(256, 100, device=device) < 0.3).float()
    labels = torch.randint(0, 10, (256,), device=device)

    def step():
        if fused_loss:
            loss = model[-1].cross_entropy(model[:-1](x), labels)
        else:
            loss = torch.nn.functional.cross_entropy(model(x), labels)
        loss.backward()
        return loss

    model.zero_grad(set_to_none=True)
    eager_loss = step().detach().clone()
    eager_grads = [p.grad.clone() for p in model.parameters()]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            model.zero_grad(set_to_none=True)
            step()
    torch.cuda.current_stream().wait_stream(side)
    model.zero_grad(set_to_none=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_loss = step()
    for i in range(4):
        junk = torch.randn(1000, device=device).sum()       # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_loss, eager_loss), f"replay {i}: loss differs"
        for p, ref in zip(model.parameters(), eager_grads):
            assert torch.equal(p.grad, ref), f"replay {i}: gradient differs"
        del junk


def test_tree_network_graph_replays_match_eager(device):
    """A logic-tree network (two complete blocks, the staged block backward with the node
    coefficients handed from the forward, dense layers, fused loss) captured as one graph
    replays bitwise to the eager step."""
    from compactlogic_amd import configs
    cfg = configs.TreeConfig("small_tree", (3, 16, 16), [(32, 3, 2, 1), (48, 3, 2, 1)],
                             [400, 400], 64)
    model = configs.tree_network(cfg, device=device)
    x, labels = configs.conv_inputs(cfg, device=device)

    def step():
        loss = model[-1].cross_entropy(model[:-1](x), labels)
        loss.backward()
        return loss

    model.zero_grad(set_to_none=True)
    eager_loss = step().detach().clone()
    eager_grads = [p.grad.clone() for p in model.parameters()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            model.zero_grad(set_to_none=True)
            step()
    torch.cuda.current_stream().wait_stream(side)
    model.zero_grad(set_to_none=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_loss = step()
    for i in range(3):
        junk = torch.randn(1000, device=device).sum()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_loss, eager_loss), f"replay {i}: loss differs"
        for p, ref in zip(model.parameters(), eager_grads):
            assert torch.equal(p.grad, ref), f"replay {i}: gradient differs"
        del junk
