"""The fused optimizer step (compactlogic_amd.FusedAdam, cl_adam_clip_step) against the
reference's optimizer half of a training step (experiments/experiment_script.py:280-293):
torch.nn.utils.clip_grad_norm_(params, max_norm) then torch.optim.Adam.step(), run in float64
on the CPU from the same gradients.  Tolerance: rtol 1e-6 (fp32 optimizer arithmetic against
float64).  A whole training step (forward, fused loss, backward, clip, Adam) captured in a HIP
graph must replay bitwise like eager steps, with the device step count advancing."""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl

pytestmark = pytest.mark.gpu


def make_model(device, seed=0):
    torch.manual_seed(seed)
    return torch.nn.Sequential(cl.LogicLayer(64, 96), cl.LogicLayer(96, 80),
                               cl.GroupSum(10, 2.0)).to(device)


def batch(device, seed=1):
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand((48, 64), generator=g) < 0.4).float().to(device)
    y = torch.randint(0, 10, (48,), generator=g).to(device)
    return x, y


def loss_of(model, x, y):
    return model[-1].cross_entropy(model[:-1](x), y)


@pytest.mark.parametrize("max_norm", [10.0, 1e-3, None])
def test_fused_adam_matches_torch_adam_with_clipping(device, max_norm):
    model = make_model(device)
    x, y = batch(device)
    ref = [p.detach().cpu().double().clone().requires_grad_(True) for p in model.parameters()]
    opt = cl.FusedAdam(model.parameters(), lr=0.01, max_norm=max_norm)
    ropt = torch.optim.Adam(ref, lr=0.01)
    for step in range(3):
        model.zero_grad(set_to_none=True)
        loss_of(model, x, y).backward()
        grads = [p.grad.detach().cpu().double() for p in model.parameters()]
        for r, g in zip(ref, grads):
            r.grad = g.clone()
        if max_norm is not None:
            norm = torch.nn.utils.clip_grad_norm_(ref, max_norm=max_norm)
            if max_norm < 1:
                assert float(norm) > max_norm     # the clipping is active in this case
        ropt.step()
        opt.step()
        torch.cuda.synchronize()
        for p, r in zip(model.parameters(), ref):
            np.testing.assert_allclose(p.detach().cpu().double().numpy(), r.detach().numpy(),
                                       rtol=1e-6, atol=1e-7)
            np.testing.assert_allclose(p.grad.cpu().double().numpy(), r.grad.numpy(),
                                       rtol=1e-6, atol=1e-12)
        assert float(opt.state[next(iter(model.parameters()))]["step"]) == step + 1


def test_fused_adam_is_reproducible_and_skips_missing_grads(device):
    outs = []
    for _ in range(2):
        model = make_model(device)
        x, y = batch(device)
        opt = cl.FusedAdam(model.parameters(), lr=0.05, max_norm=1.0)
        for _ in range(2):
            model.zero_grad(set_to_none=True)
            loss_of(model, x, y).backward()
            opt.step()
        outs.append([p.detach().clone() for p in model.parameters()])
    assert all(torch.equal(a, b) for a, b in zip(*outs))
    # a parameter without a gradient is left unchanged
    model = make_model(device)
    opt = cl.FusedAdam(model.parameters(), lr=0.05)
    before = model[0].weights.detach().clone()
    model[1].weights.grad = torch.ones_like(model[1].weights)
    opt.step()
    assert torch.equal(model[0].weights, before)
    assert not torch.equal(model[1].weights, make_model(device)[1].weights)


def test_whole_training_step_in_a_graph_replays_like_eager(device):
    x, y = batch(device)
    eager, graphed = make_model(device), make_model(device)
    opt_e = cl.FusedAdam(eager.parameters(), lr=0.01, max_norm=10.0)
    opt_g = cl.FusedAdam(graphed.parameters(), lr=0.01, max_norm=10.0)

    def step(model, opt):
        loss = loss_of(model, x, y)
        loss.backward()
        opt.step()
        return loss

    # warm-up (optimizer state exists before capture), identical on both
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for model, opt in ((eager, opt_e), (graphed, opt_g)):
            for _ in range(2):
                model.zero_grad(set_to_none=True)
                step(model, opt)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graphed.zero_grad(set_to_none=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_loss = step(graphed, opt_g)
    # the capture itself did not run the step: graphed is still at the warm-up state
    for k in range(3):
        eager.zero_grad(set_to_none=True)
        le = step(eager, opt_e)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_loss, le.detach())
        for pe, pg in zip(eager.parameters(), graphed.parameters()):
            assert torch.equal(pe, pg)
        assert float(opt_g.state[next(iter(graphed.parameters()))]["step"]) == 3 + k


def test_eval_after_fused_adam_uses_the_updated_winners(device):
    """FusedAdam writes the logits through raw pointers (no version bump): an eval after a
    training step must evaluate the winners of the updated logits, not the first eval's."""
    model = make_model(device, seed=4)
    x, y = batch(device, seed=4)
    opt = cl.FusedAdam(model.parameters(), lr=0.5, max_norm=None)
    model.eval()
    with torch.no_grad():
        model[:-1](x)                                     # the first eval caches its winners
    model.train()
    changed = False
    for _ in range(4):
        before = [m.weights.argmax(-1).clone() for m in model[:-1]]
        model.zero_grad(set_to_none=True)
        loss_of(model, x, y).backward()
        opt.step()
        changed |= any(not torch.equal(b, m.weights.argmax(-1)) for b, m in zip(before, model[:-1]))
    assert changed, "the steps moved no winner; the check would be vacuous"
    model.eval()
    for m in model[:-1]:
        assert torch.equal(m._argmax_slots().long(), m.weights.argmax(-1))
    with torch.no_grad():
        got = model[:-1](x)
        h = x
        for m in model[:-1]:
            w = m.weights.argmax(-1).to(torch.uint8)
            h = cl.difflogic_hip.eval(h.t().contiguous(), m.indices[0], m.indices[1], w,
                                      m.gate_sequence).t()
    assert torch.equal(got, h)


def test_fused_adam_resumes_from_a_checkpoint(device, tmp_path):
    """Two steps, save, two more; against: two steps, save, resume into a fresh model and a
    fresh FusedAdam (the reference's loader sequence), two more.  Bitwise equal, including the
    bias corrections (the restored step count)."""
    from compactlogic_amd import checkpoint as ck
    x, y = batch(device, seed=6)

    def run(resume_at=None):
        model = make_model(device, seed=6)
        opt = cl.FusedAdam(model.parameters(), lr=0.01, max_norm=10.0)
        for i in range(4):
            if i == resume_at:
                path = tmp_path / f"ckpt_{resume_at}.pt"
                ck.save_checkpoint(path, i, model, opt)
                model = make_model(device, seed=99)       # different initial weights
                opt = cl.FusedAdam(model.parameters(), lr=0.01, max_norm=10.0)
                step, _ = ck.resume_checkpoint(path, model, opt)
                assert step == i
            model.zero_grad(set_to_none=True)
            loss_of(model, x, y).backward()
            opt.step()
        torch.cuda.synchronize()
        return [p.detach().clone() for p in model.parameters()], opt

    ref, ropt = run()
    got, gopt = run(resume_at=2)
    assert all(torch.equal(a, b) for a, b in zip(ref, got))
    assert float(gopt._step_t) == 4.0
    # the saved optimizer state is torch.optim.Adam's layout: it loads into Adam as well
    sd = gopt.state_dict()
    assert all(v["step"].device.type == "cpu" and v["step"].dtype == torch.float32
               for v in sd["state"].values())
    params = [p.detach().clone().requires_grad_(True) for p in ref]
    adam = torch.optim.Adam(params, lr=0.01)
    adam.load_state_dict(sd)
    assert all(float(adam.state[p]["step"]) == 4.0 for p in params)
