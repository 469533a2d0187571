"""Freezing and resampling schedules (compactlogic/compactlogic.py:873-1190) on CPU layers:
only torch ops on the parameters and buffers run, no kernels."""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl


def small_model(seed=0):
    torch.manual_seed(seed)
    return torch.nn.Sequential(cl.LogicLayer(12, 16), cl.LogicLayer(16, 16), cl.LogicLayer(16, 10),
                               cl.GroupSum(2, 1.0))


def test_sequential_freezer_freezes_in_order_after_patience():
    model = small_model()
    fr = cl.SequentialEntropyFreezer(model, ema_decay=0.9, eps=1e-3, patience=3)
    assert [i for i, _ in fr.logic_layers] == [0, 1]          # all logic layers but the last
    frozen_at = {}
    for it in range(20):
        fr.step(it)
        for i, layer in fr.logic_layers:
            if layer.is_frozen and i not in frozen_at:
                frozen_at[i] = it
    # constant weights: step 0 seeds layer 0, steps 1..3 count to patience -> frozen at 3;
    # step 4 seeds layer 1, steps 5..7 -> frozen at 7
    assert frozen_at == {0: 3, 1: 7}
    assert not model[2].is_frozen
    assert str(fr).startswith("ema_decay=0.9")


def test_sequential_freezer_resets_on_entropy_change():
    model = small_model(1)
    # ema_decay = 0: the EMA is the previous step's entropy
    fr = cl.SequentialEntropyFreezer(model, ema_decay=0.0, eps=1e-6, patience=2, l=1)
    fr.step(0)
    fr.step(1)
    with torch.no_grad():
        model[0].weights.mul_(3.0)                            # entropy jumps
    fr.step(2)
    assert fr.counter[0] == 0 and not model[0].is_frozen
    fr.step(3)
    fr.step(4)
    assert model[0].is_frozen


def test_fixed_freezer_schedule():
    model = small_model()
    with pytest.raises(ValueError):
        cl.FixedSequentialEntropyFreezer(model, N=0)
    fr = cl.FixedSequentialEntropyFreezer(model, N=5, min_iters=2)
    states = []
    for it in range(14):
        fr.step(it)
        states.append(tuple(m.is_frozen for m in model[:2]))
    assert states[6] == (False, False) and states[7] == (True, False)
    assert states[11] == (True, False) and states[12] == (True, True)


def test_row_resampler_resamples_converged_rows_and_clears_adam_state():
    model = small_model(2)
    layer = model[1]
    opt = torch.optim.Adam(model.parameters(), lr=1e-3)
    layer.weights.grad = torch.ones_like(layer.weights)
    opt.step()                                                 # creates exp_avg / exp_avg_sq
    st = opt.state[layer.weights]
    assert bool((st["exp_avg"] != 0).all())
    # every row converges (constant weights); threshold_low=1 makes every row weak
    rs = cl.EntropyRowResampler(model, patience=2, threshold_high=2.0, threshold_low=1.0)
    before = layer.indices.clone()
    for it in range(3):
        rs.step(it, opt)
    # step 0 seeds, steps 1 and 2 count; at step 2 all rows hit patience and are resampled
    assert not torch.equal(before, layer.indices)
    assert bool((st["exp_avg"] == 0).all()) and bool((st["exp_avg_sq"] == 0).all())
    assert int(rs.counter[1].max()) == 0
    # the derived inverse index follows the new wiring
    start = layer.given_x_indices_of_y_start
    assert int(start[-1]) == 2 * layer.out_dim * layer.num_gates
    assert "patience=2" in str(rs)


def test_row_resampler_window_and_frozen_layers():
    model = small_model(3)
    model[0].freeze()
    rs = cl.EntropyRowResampler(model, patience=1, min_iters=5, max_iters=6)
    opt = torch.optim.SGD(model.parameters(), lr=0.1)
    for it in range(5):
        rs.step(it, opt)
    assert rs.ema == {}                                       # before min_iters
    rs.step(5, opt)
    assert 0 not in rs.ema and 1 in rs.ema                    # frozen layer skipped
    rs.step(7, opt)
    assert rs.iter == 7
