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


def test_packed_network_cfg5_fuses_the_wide_tail(device):
    """cfg5: conv1 and conv2 composed into one launch that writes conv2's rows column-major
    (conv1's rows computed where conv2 reads them), then 25088 -> 16000 -> 16000 and the class
    counts in one launch (two first-layer slots held over the input column); equal to the C
    oracle and to the whole network layer by layer."""
    cfg = configs.CONV_CONFIGS["cfg5"]
    model = configs.conv_network(cfg, device=device)
    configs.freeze_argmax(model)
    feats = int(np.prod(cfg.in_shape))
    xw = configs.packed_input_words(feats, 64, device=device)            # 2^12 samples
    net = cl.PackedNetwork(model)
    assert net.producer == (model[0], model[1]) and net.prefix == []
    assert net.rows == [25088, 16000, 16000] and net.layout["split"] == 14336
    x = cl.PackBitsTensor.from_packed(xw)
    counts = net(x)
    assert x.t is xw                                                     # input untouched
    ref = conv_oracle_counts(model, np_(xw).view(np.uint64), 1 << 12)
    assert np.array_equal(np_(counts), ref)
    assert torch.equal(counts, model(cl.PackBitsTensor.from_packed(xw.clone())))


def small_conv_net(device, in_shape, c_out, widths, k, seed, convs=1, stride=1):
    torch.manual_seed(seed)
    conv, shape = [], in_shape
    for i in range(convs):
        conv.append(cl.ConvLayer(shape, padding=1, c_out=c_out, ks=3, stride=stride,
                                 num_chn=1, num_gates=4))
        shape = conv[-1].out_shape
    g = torch.Generator().manual_seed(seed)
    dims = [int(np.prod(shape))] + list(widths)
    dense = [cl.LogicLayer(i, o, num_gates=4) for i, o in zip(dims[:-1], dims[1:])]
    for m in conv + dense:
        with torch.no_grad():
            m.weights.copy_(torch.randn(m.weights.shape, generator=g))
            m.gate_sequence.copy_(torch.randint(0, 16, m.gate_sequence.shape,
                                                generator=g).to(torch.uint8))
    model = torch.nn.Sequential(*conv, torch.nn.Flatten(), *dense,
                                cl.GroupSum(k, 1.0)).to(device)
    configs.freeze_argmax(model)
    return model


@pytest.mark.parametrize("in_shape,c_out,widths,k,n,bits", [
    ((4, 16, 16), 32, [4200, 2100], 10, 1000, 64),     # 8 slots, second layer over the input
    ((2, 12, 12), 40, [12000, 10000], 10, 333, 64),    # 16 slots, nothing held
    ((5, 15, 15), 40, [12000, 10000], 20, 100, 32),    # 9000 rows: held slots; odd words
    ((3, 16, 16), 24, [5000, 4000, 2100], 3, 4096, 64),  # three layers
])
def test_packed_network_wide_tail_matches_oracle(device, in_shape, c_out, widths, k, n, bits):
    model = small_conv_net(device, in_shape, c_out, widths, k, seed=n)
    rng = np.random.default_rng(n)
    feats = int(np.prod(in_shape))
    x = cl.PackBitsTensor(torch.as_tensor(rng.integers(0, 2, (n, feats)).astype(bool),
                                          device=device), bits)
    net = cl.PackedNetwork(model)
    assert net.producer == (model[0],) and net.layout is not None
    counts = net(x)
    assert counts.shape == (n, k)
    words = np_(x.t)
    if words.dtype != np.int64:                  # 32-bit words: pad to whole 64-bit words
        words = np.concatenate([words, np.zeros((words.shape[0], words.shape[1] % 2),
                                                words.dtype)], 1)
    ref = conv_oracle_counts(model, np.ascontiguousarray(words).view(np.uint64), n)
    assert np.array_equal(np_(counts), ref)
    layerwise = model(cl.PackBitsTensor.from_packed(x.t.clone(), x.pad_len))
    assert torch.equal(counts, layerwise)


def test_packed_network_wide_tail_after_a_dense_producer(device):
    """A dense LogicLayer feeds the tail through a Flatten: it writes the columns."""
    model = frozen_net([(64, 6000), (6000, 3000), (3000, 2000)], 10, 8, 11, device)
    model = torch.nn.Sequential(model[0], torch.nn.Flatten(), model[1], model[2], model[3])
    net = cl.PackedNetwork(model)
    assert net.producer == (model[0],) and net.prefix == [] and net.rows == [6000, 3000, 2000]
    rng = np.random.default_rng(3)
    x = cl.PackBitsTensor(torch.as_tensor(rng.integers(0, 2, (777, 64)).astype(bool),
                                          device=device), 64)
    counts = net(x)
    ref = oracle_counts(model, np_(x.t).view(np.uint64), 777)
    assert np.array_equal(np_(counts), ref)


@pytest.mark.parametrize("in_shape,c_out,convs,stride,widths,k,n", [
    ((3, 16, 16), 32, 2, 1, [4200, 2100], 10, 1000),   # conv, conv composed, 8192 rows
    ((4, 16, 16), 24, 3, 1, [3100, 1550], 5, 333),     # conv layer by layer, then a pair
])
def test_packed_network_composes_two_convs(device, in_shape, c_out, convs, stride, widths, k,
                                           n):
    model = small_conv_net(device, in_shape, c_out, widths, k, seed=n, convs=convs,
                           stride=stride)
    net = cl.PackedNetwork(model)
    assert net.producer == (model[convs - 2], model[convs - 1])
    assert net.prefix == list(model)[:convs - 2]
    rng = np.random.default_rng(n)
    feats = int(np.prod(in_shape))
    x = cl.PackBitsTensor(torch.as_tensor(rng.integers(0, 2, (n, feats)).astype(bool),
                                          device=device), 64)
    counts = net(x)
    ref = conv_oracle_counts(model, np_(x.t).view(np.uint64), n)
    assert np.array_equal(np_(counts), ref)
    assert torch.equal(counts, model(cl.PackBitsTensor.from_packed(x.t.clone(), x.pad_len)))


@pytest.mark.parametrize("mid,out_dim,out_words,words", [
    (500, 1000, 1024, 130), (300, 64, 64, 64), (40, 70, 128, 3)])
def test_eval_packed_indexed_pair_columns_is_two_layers(device, mid, out_dim, out_words, words):
    """The composed pair equals layer 1 by cl_eval_packed_indexed, then layer 2 written
    column-major; negative and out-of-range indices in both layers."""
    from compactlogic_amd import _capi
    from compactlogic_amd import difflogic_hip as _dl
    rng = np.random.default_rng(mid + out_dim)
    in_dim = 200
    xw = torch.as_tensor(rng.integers(-2**31, 2**31, (in_dim, words)), dtype=torch.int32,
                         device=device)

    def tables(n_in, n_out):
        ia = rng.integers(-1, n_in, n_out).astype(np.int32)
        ib = rng.integers(-1, n_in, n_out).astype(np.int32)
        ib[::13] = n_in                                   # out of range: a zero row
        g = rng.integers(0, 16, n_out).astype(np.uint8)
        return [torch.as_tensor(t, device=device) for t in (ia, ib, g)]

    t1, t2 = tables(in_dim, mid), tables(mid, out_dim)
    row_bytes = words * 4
    s = _dl.stream_of(xw)
    h = torch.empty((mid, words), dtype=torch.int32, device=device)
    _capi.call("cl_eval_packed_indexed", xw.data_ptr(), *[t.data_ptr() for t in t1], None,
               h.data_ptr(), in_dim, mid, row_bytes, s)
    ref = torch.full((words, out_words), 5, dtype=torch.int32, device=device)
    order = torch.as_tensor(rng.permutation(out_dim).astype(np.int32), device=device)
    _capi.call("cl_eval_packed_indexed_columns", h.data_ptr(), *[t.data_ptr() for t in t2],
               order.data_ptr(), ref.data_ptr(), mid, out_dim, row_bytes, out_words, s)
    out = torch.full((words, out_words), 7, dtype=torch.int32, device=device)
    _capi.call("cl_eval_packed_indexed_pair_columns", xw.data_ptr(),
               *[t.data_ptr() for t in t1 + t2], order.data_ptr(), out.data_ptr(), in_dim, mid,
               out_dim, row_bytes, out_words, s)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert int(out[:, out_dim:].abs().sum()) == 0


@pytest.mark.parametrize("out_dim,out_words,words,bits", [
    (1000, 1024, 130, 32), (4096, 4096, 256, 32), (70, 128, 3, 32), (25, 64, 2, 64)])
def test_eval_packed_indexed_columns_is_the_transposed_layer(device, out_dim, out_words, words,
                                                             bits):
    """cl_eval_packed_indexed_columns equals cl_eval_packed_indexed transposed to 32-bit words,
    with zero rows past out_dim; negative and out-of-range indices as there."""
    from compactlogic_amd import _capi
    from compactlogic_amd import difflogic_hip as _dl
    rng = np.random.default_rng(out_dim)
    in_dim = 300
    xw = torch.as_tensor(rng.integers(-2**31, 2**31, (in_dim, words * bits // 32)),
                         dtype=torch.int32, device=device)
    ia = rng.integers(-1, in_dim, out_dim).astype(np.int32)
    ib = rng.integers(-1, in_dim, out_dim).astype(np.int32)
    ia[::17] = in_dim                                   # out of range: a zero row
    ia_t, ib_t = torch.as_tensor(ia, device=device), torch.as_tensor(ib, device=device)
    gate = torch.as_tensor(rng.integers(0, 16, out_dim).astype(np.uint8), device=device)
    row_bytes = xw.shape[1] * 4
    ref = torch.empty((out_dim, xw.shape[1]), dtype=torch.int32, device=device)
    _capi.call("cl_eval_packed_indexed", xw.data_ptr(), ia_t.data_ptr(), ib_t.data_ptr(),
               gate.data_ptr(), None, ref.data_ptr(), in_dim, out_dim, row_bytes,
               _dl.stream_of(xw))
    out = torch.full((xw.shape[1], out_words), 7, dtype=torch.int32, device=device)
    _capi.call("cl_eval_packed_indexed_columns", xw.data_ptr(), ia_t.data_ptr(),
               ib_t.data_ptr(), gate.data_ptr(), None, out.data_ptr(), in_dim, out_dim,
               row_bytes, out_words, _dl.stream_of(xw))
    torch.cuda.synchronize()
    assert torch.equal(out[:, :out_dim], ref.T)
    assert int(out[:, out_dim:].abs().sum()) == 0
    # with a row order: position p holds row order[p]
    order = torch.as_tensor(rng.permutation(out_dim).astype(np.int32), device=device)
    _capi.call("cl_eval_packed_indexed_columns", xw.data_ptr(), ia_t.data_ptr(),
               ib_t.data_ptr(), gate.data_ptr(), order.data_ptr(), out.data_ptr(), in_dim,
               out_dim, row_bytes, out_words, _dl.stream_of(xw))
    torch.cuda.synchronize()
    assert torch.equal(out[:, :out_dim], ref.T[:, order.long()])
    assert int(out[:, out_dim:].abs().sum()) == 0


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
