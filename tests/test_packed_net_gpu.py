"""Whole-network packed inference (PackedNetwork): bit-exact against the C oracle and the
layer-by-layer packed path."""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl
from compactlogic_amd import configs
from oracle import packed as P

pytestmark = pytest.mark.gpu


def np_(t):
    return t.detach().cpu().numpy()


def frozen_net(dims, k, g_n, seed, device):
    torch.manual_seed(seed)
    layers = [cl.LogicLayer(i, o, num_gates=g_n) for i, o in dims]
    g = torch.Generator().manual_seed(seed)
    for m in layers:
        with torch.no_grad():
            m.gate_sequence.copy_(torch.randint(0, 16, m.gate_sequence.shape, generator=g).to(torch.uint8))
        m.freeze()
    model = torch.nn.Sequential(*layers, cl.GroupSum(k, 1.0)).to(device)
    model.eval()
    return model


def oracle_counts(model, words_np, n):
    layers = [P.resolve_slots(np_(m.indices), np_(m.gate_sequence), np_(m.w))
              for m in model if isinstance(m, cl.LogicLayer)]
    pad = words_np.shape[1] * 64 - n
    return P.network_counts(words_np, layers, model[-1].k, pad)


@pytest.mark.parametrize("dims,k,g_n,n", [
    ([(40, 64), (64, 60)], 6, 4, 64),
    ([(100, 300), (300, 300), (300, 200)], 10, 16, 1000),
    ([(17, 33), (33, 40)], 5, 2, 96),
    ([(64, 2000), (2000, 1000)], 8, 16, 4096),
    ([(12, 20)] + [(20, 20)] * 14 + [(20, 30)], 3, 8, 130),
    ([(64, 17000), (17000, 8500)], 10, 4, 200),     # wider than the register-table variant
    ([(3000, 5000), (5000, 2600)], 4, 16, 700),     # > 1024 input rows: 4 per thread
    ([(64, 15000), (15000, 16000)], 2, 4, 300),     # 16 gates per thread, 8000-row classes
    ([(50, 400), (400, 340)], 20, 8, 150),          # more classes than waves
])
def test_packed_network_matches_oracle_and_layerwise(device, dims, k, g_n, n):
    model = frozen_net(dims, k, g_n, sum(d[1] for d in dims), device)
    rng = np.random.default_rng(n)
    bits = rng.integers(0, 2, (n, dims[0][0])).astype(bool)
    x = cl.PackBitsTensor(torch.as_tensor(bits, device=device), 64)
    net = cl.PackedNetwork(model)
    counts = net(x)
    assert counts.shape == (n, k) and counts.dtype == torch.int32
    ref = oracle_counts(model, np_(x.t).view(np.uint64), n)
    assert np.array_equal(np_(counts), ref)
    layerwise = model(cl.PackBitsTensor.from_packed(x.t.clone(), x.pad_len))
    assert torch.equal(counts, layerwise)


def conv_oracle_counts(model, words_np, n):
    """The C oracle through a network of ConvLayers, Flatten and LogicLayers."""
    layers = []
    for m in model:
        if isinstance(m, cl.ConvLayer):
            layers.append(P.resolve_conv_slots(np_(m.offsets_ch), np_(m.offsets_h),
                                               np_(m.offsets_w), np_(m.gate_sequence), np_(m.w),
                                               m.in_shape, m.stride, m.out_shape[1:]))
        elif isinstance(m, cl.LogicLayer):
            layers.append(P.resolve_slots(np_(m.indices), np_(m.gate_sequence), np_(m.w)))
    pad = words_np.shape[1] * 64 - n
    return P.network_counts(words_np, layers, model[-1].k, pad)


def test_packed_network_cfg5_runs_layer_by_layer(device):
    """cfg5's first dense layer reads 25088 rows, more than the fused kernel stages in LDS: no
    tail is fused and every module runs on the packed kernels, then the group popcount."""
    cfg = configs.CONV_CONFIGS["cfg5"]
    model = configs.conv_network(cfg, device=device)
    configs.freeze_argmax(model)
    feats = int(np.prod(cfg.in_shape))
    xw = configs.packed_input_words(feats, 64, device=device)            # 2^12 samples
    net = cl.PackedNetwork(model)
    assert net.rows is None and len(net.prefix) == len(model) - 1
    x = cl.PackBitsTensor.from_packed(xw)
    counts = net(x)
    assert x.t is xw                                                     # input untouched
    ref = conv_oracle_counts(model, np_(xw).view(np.uint64), 1 << 12)
    assert np.array_equal(np_(counts), ref)
    assert torch.equal(counts, model(cl.PackBitsTensor.from_packed(xw.clone())))


def test_packed_network_cfg3_tree_fuses_the_dense_tail(device):
    """cfg3_tree: two ConvLogicLayer blocks layer by layer, then 2048 -> 16000 -> 16000 and
    the class counts in one launch; equal to the whole network layer by layer."""
    cfg = configs.TREE_CONFIGS["cfg3_tree"]
    model = configs.tree_network(cfg, device=device)
    configs.freeze_argmax(model)
    feats = int(np.prod(cfg.in_shape))
    xw = configs.packed_input_words(feats, 64, device=device)            # 2^12 samples
    net = cl.PackedNetwork(model)
    assert len(net.prefix) == 3 and net.rows == [2048, 16000, 16000]
    counts = net(cl.PackBitsTensor.from_packed(xw))
    layerwise = model(cl.PackBitsTensor.from_packed(xw.clone()))
    assert torch.equal(counts, layerwise)
    # the fused tail alone against the C oracle, on the blocks' packed output
    with torch.no_grad():
        h = cl.PackBitsTensor.from_packed(xw.clone())
        for m in net.prefix:
            h = m(h)
    dense = torch.nn.Sequential(*list(model)[3:])
    hw = np_(h.t).view(np.uint64)
    ref = oracle_counts(dense, hw, 1 << 12)
    assert np.array_equal(np_(counts), ref)


def test_packed_network_cfg4_slice(device):
    cfg = configs.CONFIGS["cfg2"]
    model = configs.dense_network(cfg, device=device)
    configs.freeze_uniform_gates(model)
    xw = configs.packed_input_words(cfg.in_dim, 1024, device=device)      # 2^16 samples
    counts = cl.PackedNetwork(model)(cl.PackBitsTensor.from_packed(xw))
    ref = oracle_counts(model, np_(xw).view(np.uint64), 1 << 16)
    assert np.array_equal(np_(counts), ref)


def test_packed_network_word_widths_and_errors(device):
    model = frozen_net([(30, 40), (40, 20)], 4, 4, 1, device)
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2, (200, 30)).astype(bool)
    ref = None
    for bc in (32, 64):
        x = cl.PackBitsTensor(torch.as_tensor(bits, device=device), bc)
        c = cl.PackedNetwork(model)(x)
        ref = c if ref is None else ref
        assert torch.equal(c, ref)
    bad = torch.nn.Sequential(*list(model)[:-1], cl.GroupSum(3, 1.0))
    with pytest.raises(ValueError):
        cl.PackedNetwork(bad)                                           # 20 % 3 != 0
    wide = frozen_net([(30, 30000)], 10, 2, 2, device)
    net = cl.PackedNetwork(wide)                                        # too wide for LDS
    assert net.rows is None
    x = cl.PackBitsTensor(torch.as_tensor(bits, device=device), 64)
    assert torch.equal(net(x), wide(cl.PackBitsTensor.from_packed(x.t.clone(), x.pad_len)))
    with pytest.raises(RuntimeError):
        cl.PackedNetwork(model)(torch.zeros((31, 4), dtype=torch.int64, device=device))


def test_bank_aware_layout_gives_the_same_counts(device):
    """The LDS layout of the hidden layers changes where rows live, never the counts."""
    dims = [(300, 2000), (2000, 3000), (3000, 1500)]
    model = frozen_net(dims, 10, 16, 5, device)
    n = 2048
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 2, (n, 300)).astype(bool)
    x = cl.PackBitsTensor(torch.as_tensor(bits, device=device), 64)
    a = cl.PackedNetwork(model)(x)
    b = cl.PackedNetwork(model, bank_aware=False)(x)
    assert torch.equal(a, b)
    assert np.array_equal(np_(a), oracle_counts(model, np_(x.t).view(np.uint64), n))
