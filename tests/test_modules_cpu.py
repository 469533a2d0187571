"""Module API, buffers and derived plans on the CPU (no kernel calls)."""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl
from compactlogic_amd import configs
from oracle import logic_np as O

REF_KEYS = {"weights", "gate_sequence", "indices", "given_x_indices_of_y_start",
            "given_x_indices_of_y", "given_x_indices_of_gate"}


def test_logic_layer_buffers_and_state_dict():
    torch.manual_seed(0)
    layer = cl.LogicLayer(20, 30, num_gates=16)
    sd = layer.state_dict()
    assert set(sd) == REF_KEYS
    assert sd["weights"].shape == (30, 16) and sd["weights"].dtype == torch.float32
    assert sd["gate_sequence"].dtype == torch.uint8
    assert torch.equal(sd["gate_sequence"][0], torch.arange(16, dtype=torch.uint8))
    assert sd["indices"].shape == (2, 30, 16) and sd["indices"].dtype == torch.int64
    assert sd["given_x_indices_of_y"].numel() == 2 * 30 * 16
    assert sd["given_x_indices_of_gate"].dtype == torch.int8
    assert layer.indices.min() >= 0 and layer.indices.max() < 20
    # strict loading of a reference-shaped state dict, and freeze() adds `w`
    other = cl.LogicLayer(20, 30)
    other.load_state_dict(sd, strict=True)
    layer.freeze()
    assert layer.is_frozen and layer.w.dtype == torch.uint8
    assert torch.equal(layer.w, layer.weights.argmax(-1).to(torch.uint8))


def test_backward_index_matches_oracle_rows():
    torch.manual_seed(1)
    layer = cl.LogicLayer(13, 17, num_gates=4)
    start, yidx, code = O.backward_index(layer.indices.numpy(), 13)
    assert np.array_equal(layer.given_x_indices_of_y_start.numpy(), start)
    for i in range(13):
        s0, s1 = start[i], start[i + 1]
        got = sorted(zip(layer.given_x_indices_of_y[s0:s1].tolist(),
                         layer.given_x_indices_of_gate[s0:s1].tolist()))
        assert got == sorted(zip(yidx[s0:s1].tolist(), code[s0:s1].tolist()))


def test_connection_assertion_and_schemes():
    with pytest.raises(AssertionError):
        cl.LogicLayer(100, 10)
    with pytest.raises(NotImplementedError):
        cl.LogicLayer(4, 4, connections="bogus")
    torch.manual_seed(2)
    orig = cl.LogicLayer(10, 12, connections="original")
    assert bool((orig.indices == orig.indices[..., :1]).all())
    assert orig.run_plan().num_runs == 12


def test_residual_init():
    layer = cl.LogicLayer(8, 8, residual_init=True)
    assert bool((layer.weights.argmax(-1) == 3).all())
    assert float(layer.weights[0, 3]) == pytest.approx(np.log(9 * 15), rel=1e-6)


def _plan_reference(ind):
    """Runs by brute force: maximal equal-pair slot ranges per neuron."""
    runs = []
    _, out, g = ind.shape
    for o in range(out):
        g0 = 0
        for s in range(1, g + 1):
            if s == g or (ind[0, o, s], ind[1, o, s]) != (ind[0, o, g0], ind[1, o, g0]):
                runs.append((o, g0, s - g0, int(ind[0, o, g0]), int(ind[1, o, g0])))
                g0 = s
    return runs


@pytest.mark.parametrize("seed", range(4))
def test_run_plan_against_brute_force(seed):
    rng = np.random.default_rng(seed)
    in_dim, out, g = 7, 9, 6
    ind = rng.integers(0, 3, (2, out, g))          # few distinct inputs -> long runs
    plan = cl.build_run_plan(torch.as_tensor(ind), in_dim)
    runs = _plan_reference(ind)
    assert plan.num_runs == len(runs)
    got = [(int(plan.run_y[r]), int(plan.run_gl[r]) & 255, int(plan.run_gl[r]) >> 8,
            int(plan.run_ab[r, 0]), int(plan.run_ab[r, 1])) for r in range(plan.num_runs)]
    assert got == runs
    ptr = plan.run_ptr.numpy()
    assert ptr[0] == 0 and ptr[-1] == len(runs)
    for o in range(out):
        assert all(runs[r][0] == o for r in range(ptr[o], ptr[o + 1]))
    inv = plan.inv_ptr.numpy()
    uses = set()
    for i in range(in_dim):
        for e in plan.inv_entry[inv[i]:inv[i + 1]].tolist():
            r, side = e >> 1, e & 1
            assert runs[r][3 + side] == i
            uses.add(e)
    assert uses == set(range(2 * len(runs)))


def test_run_plan_rejects_out_of_range_indices():
    with pytest.raises(IndexError):
        cl.build_run_plan(torch.tensor([[[0, 5]], [[1, 1]]]), 5)


def test_plan_rebuilds_after_in_place_rewiring():
    torch.manual_seed(3)
    layer = cl.LogicLayer(6, 8, connections="original")
    p1 = layer.run_plan()
    assert layer.run_plan() is p1
    with torch.no_grad():
        layer.indices[0, 0, 5] = (layer.indices[0, 0, 5] + 1) % 6
    p2 = layer.run_plan()
    assert p2 is not p1 and p2.num_runs == p1.num_runs + 2


def test_resample_connections_updates_index():
    torch.manual_seed(4)
    layer = cl.LogicLayer(10, 16)
    with torch.no_grad():
        layer.weights[:4] = 0.0               # uniform rows are weak
        layer.weights[4:8, 2] = 20.0          # peaked rows are strong
    weak, strong = layer.resample_connections(torch.arange(8), threshold_high=0.95,
                                              threshold_low=0.5)
    assert int(weak.sum()) == 4 and int(strong.sum()) == 4
    start, yidx, code = O.backward_index(layer.indices.numpy(), 10)
    assert np.array_equal(layer.given_x_indices_of_y_start.numpy(), start)
    assert bool((layer.weights[4:8].argmax(-1) == 2).all())


def test_weights_entropy_and_connected_neurons():
    torch.manual_seed(5)
    layer = cl.LogicLayer(8, 8, num_gates=16)
    with torch.no_grad():
        layer.weights.zero_()
    assert torch.allclose(layer.weights_entropy(), torch.ones(8), atol=1e-6)
    with torch.no_grad():
        layer.weights.fill_(-30.0)
        layer.weights[:, 6] = 30.0            # XOR everywhere: both inputs used
    x_flag, y_flag = layer.connected_neurons(torch.ones(8, dtype=torch.bool))
    expect = torch.zeros(8, dtype=torch.bool)
    expect[layer.indices[0, :, 6]] = True
    expect[layer.indices[1, :, 6]] = True
    assert torch.equal(x_flag, expect) and bool(y_flag.all())


def test_forward_rejects_host_tensors():
    layer = cl.LogicLayer(4, 4)
    with pytest.raises(RuntimeError):
        layer(torch.zeros(2, 4))
    with pytest.raises(RuntimeError):
        cl.GroupSum(2)(torch.zeros(2, 4))


def test_config_network_is_deterministic():
    cfg = configs.CONFIGS["cfg1"]
    m1 = configs.dense_network(cfg, device="cpu")
    m2 = configs.dense_network(cfg, device="cpu")
    for l1, l2 in zip(m1, m2):
        if isinstance(l1, cl.LogicLayer):
            assert torch.equal(l1.weights, l2.weights) and torch.equal(l1.indices, l2.indices)
            assert l1.run_plan().num_runs == l1.out_dim
