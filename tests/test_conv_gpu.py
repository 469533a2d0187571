"""ConvLayer kernels against the float64 CPU oracle (oracle/logic_np.py conv_*), the module
and autograd bridge, and the packed conv path bit-exact against the C oracle.

Tolerance (north star): fp32 within rtol 1e-5 / atol 1e-6 of the float64 oracle, upstream
gradients at the scale of a mean-reduced loss; fp64 within rtol 1e-10 / atol 1e-12; discrete
and packed outputs exact.
"""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl
from compactlogic_amd import configs
from compactlogic_amd import convlogic_hip as cv
from oracle import logic_np as O
from oracle import packed as P

pytestmark = pytest.mark.gpu

TOL = {torch.float32: dict(rtol=1e-5, atol=1e-6), torch.float64: dict(rtol=1e-10, atol=1e-12)}


def np_(t):
    return t.detach().cpu().numpy()


def make_conv(seed, n, c_in, h, wd, c_out, g_n, ks, stride, pad, binary_x=False):
    rng = np.random.default_rng(seed)
    och = rng.integers(0, c_in, (2, c_out, g_n)).astype(np.int32)
    oh = (rng.integers(0, ks, (2, c_out, g_n)) - pad).astype(np.int8)
    ow = (rng.integers(0, ks, (2, c_out, g_n)) - pad).astype(np.int8)
    gs = rng.integers(0, 16, (c_out, g_n)).astype(np.uint8)
    logits = rng.standard_normal((c_out, g_n))
    w = np.exp(logits) / np.exp(logits).sum(1, keepdims=True)
    x = (rng.integers(0, 2, (n, c_in, h, wd)).astype(np.float64) if binary_x
         else rng.random((n, c_in, h, wd)))
    h_out, w_out = O.conv_out_hw(h, wd, pad, ks, stride)
    gy = rng.uniform(-1, 1, (n, c_out, h_out, w_out)) / max(n, 1)
    return dict(x=x, och=och, oh=oh, ow=ow, gs=gs, w=w, logits=logits, gy=gy,
                slot=rng.integers(0, g_n, c_out).astype(np.uint8), stride=stride, pad=pad, ks=ks)


def dev(C, device, dtype):
    t = lambda v, dt: torch.as_tensor(v).to(device=device, dtype=dt).contiguous()
    return dict(x=t(C["x"], dtype), och=t(C["och"], torch.int32), oh=t(C["oh"], torch.int8),
                ow=t(C["ow"], torch.int8), gs=t(C["gs"], torch.uint8), w=t(C["w"], dtype),
                gy=t(C["gy"], dtype), slot=t(C["slot"], torch.uint8))


SHAPES = [
    # n, c_in, h, w, c_out, G, ks, stride, pad
    (2, 3, 7, 7, 5, 4, 3, 1, 1),
    (3, 4, 9, 6, 6, 16, 3, 2, 1),
    (1, 2, 5, 5, 3, 1, 1, 1, 0),
    (4, 9, 32, 32, 8, 16, 3, 2, 1),     # cfg3 conv1 geometry, fewer channels
    (2, 16, 16, 16, 12, 16, 3, 2, 0),   # cfg3 conv2 geometry, fewer channels
    (5, 3, 11, 13, 7, 8, 4, 3, 2),      # stride 3, non-square, wide padding
    (64, 3, 8, 8, 4, 16, 3, 2, 1),      # many samples: several weight-gradient blocks
    (2, 5, 6, 6, 3, 128, 2, 1, 0),      # the largest slot count
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_conv_forward_backward_vs_oracle(device, shape, dtype):
    n, c_in, h, wd, c_out, g_n, ks, stride, pad = shape
    C = make_conv(sum(shape), n, c_in, h, wd, c_out, g_n, ks, stride, pad)
    D = dev(C, device, dtype)
    y = cv.forward(D["x"], D["och"], D["oh"], D["ow"], D["w"], D["gs"], stride, pad, ks)
    ref = O.conv_forward(C["x"], C["och"], C["oh"], C["ow"], C["w"], C["gs"], stride, pad, ks)
    assert y.shape == ref.shape and y.dtype == dtype
    np.testing.assert_allclose(np_(y), ref, **TOL[dtype])
    gx = cv.backward_x(D["x"], D["och"], D["oh"], D["ow"], D["w"], D["gs"], D["gy"], stride, pad)
    gw = cv.backward_w(D["x"], D["och"], D["oh"], D["ow"], D["gs"], D["gy"], stride)
    rgx, rgw = O.conv_backward(C["x"], C["och"], C["oh"], C["ow"], C["w"], C["gs"], C["gy"],
                               stride, pad)
    np.testing.assert_allclose(np_(gx), rgx, **TOL[dtype])
    np.testing.assert_allclose(np_(gw), rgw, **TOL[dtype])
    if g_n <= 64:
        # the fused softmax backward gives the gradient of the logits
        gl = cv.backward_w(D["x"], D["och"], D["oh"], D["ow"], D["gs"], D["gy"], stride, D["w"])
        p = C["w"]
        rgl = p * (rgw - (p * rgw).sum(1, keepdims=True))
        np.testing.assert_allclose(np_(gl), rgl, **TOL[dtype])


@pytest.mark.parametrize("shape", SHAPES[:6], ids=lambda s: "x".join(map(str, s)))
def test_conv_eval_vs_oracle(device, shape):
    n, c_in, h, wd, c_out, g_n, ks, stride, pad = shape
    C = make_conv(sum(shape) + 1, n, c_in, h, wd, c_out, g_n, ks, stride, pad, binary_x=True)
    D = dev(C, device, torch.float32)
    y = cv.eval(D["x"], D["och"], D["oh"], D["ow"], D["slot"], D["gs"], stride, pad, ks)
    ref = O.conv_eval(C["x"], C["och"], C["oh"], C["ow"], C["slot"], C["gs"], stride, pad, ks)
    np.testing.assert_array_equal(np_(y), ref)


def test_conv_known_answer(device):
    """One output channel, one slot per opcode: every AB in {0,1}^2 through the 16 gates gives
    the truth table (the reference's known-answer pattern, with taps instead of features)."""
    table = O.TRUTH                                      # [16, 4] over AB = 00, 01, 10, 11
    x = torch.tensor([0., 0., 1., 1., 0., 1., 0., 1.], device=device).view(1, 2, 1, 4)
    och = torch.tensor([0, 1], dtype=torch.int32, device=device).view(2, 1, 1).repeat(1, 16, 1)
    och = och.view(2, 16, 1).contiguous()
    oh = torch.zeros((2, 16, 1), dtype=torch.int8, device=device)
    ow = torch.zeros((2, 16, 1), dtype=torch.int8, device=device)
    gs = torch.arange(16, dtype=torch.uint8, device=device).view(16, 1)
    w = torch.ones((16, 1), device=device)
    y = cv.forward(x, och, oh, ow, w, gs, 1, 0, 1)     # [1, 16, 1, 4]
    np.testing.assert_array_equal(np_(y)[0, :, 0, :], table)
    ye = cv.eval(x, och, oh, ow, torch.zeros(16, dtype=torch.uint8, device=device), gs, 1, 0, 1)
    np.testing.assert_array_equal(np_(ye)[0, :, 0, :], table)


def test_conv_backward_deterministic(device):
    C = make_conv(7, 16, 8, 16, 16, 32, 16, 3, 2, 1)
    D = dev(C, device, torch.float32)
    args = (D["x"], D["och"], D["oh"], D["ow"], D["w"], D["gs"], D["gy"], 2, 1)
    a = cv.backward_x(*args)
    b = cv.backward_x(*args)
    assert torch.equal(a, b)
    wa = cv.backward_w(D["x"], D["och"], D["oh"], D["ow"], D["gs"], D["gy"], 2)
    wb = cv.backward_w(D["x"], D["och"], D["oh"], D["ow"], D["gs"], D["gy"], 2)
    assert torch.equal(wa, wb)


def test_conv_errors(device):
    C = make_conv(3, 2, 3, 7, 7, 5, 4, 3, 1, 1)
    D = dev(C, device, torch.float32)
    with pytest.raises(RuntimeError):
        cv.forward(D["x"], D["och"], D["oh"], D["ow"], D["w"], D["gs"], 1, 0, 9)   # ks > plane
    with pytest.raises(RuntimeError):
        cv.forward(D["x"], D["och"].to(torch.int64), D["oh"], D["ow"], D["w"], D["gs"], 1, 1, 3)
    with pytest.raises(RuntimeError):
        cv.forward(D["x"].cpu(), D["och"], D["oh"], D["ow"], D["w"], D["gs"], 1, 1, 3)


def test_conv_empty_batch(device):
    C = make_conv(4, 0, 3, 7, 7, 5, 4, 3, 1, 1)
    D = dev(C, device, torch.float32)
    y = cv.forward(D["x"], D["och"], D["oh"], D["ow"], D["w"], D["gs"], 1, 1, 3)
    assert y.shape == (0, 5, 7, 7)
    gw = cv.backward_w(D["x"], D["och"], D["oh"], D["ow"], D["gs"], D["gy"], 1)
    assert torch.equal(gw, torch.zeros_like(gw))


# ------------------------------------------------------------------------------ module

@pytest.mark.parametrize("num_chn", [0, 1, 3])
def test_conv_layer_module_autograd(device, num_chn):
    torch.manual_seed(num_chn)
    layer = cl.ConvLayer((9, 10, 10), padding=1, c_out=12, ks=3, stride=2, num_chn=num_chn,
                         num_gates=16).to(device)
    x = (torch.rand((6, 9, 10, 10), device=device) < 0.5).float().requires_grad_(True)
    y = layer(x)
    assert y.shape == (6,) + layer.out_shape
    gy = torch.randn_like(y) / 6
    y.backward(gy)
    och, oh, ow = (np_(layer.offsets_ch), np_(layer.offsets_h), np_(layer.offsets_w))
    logits = np_(layer.weights).astype(np.float64)
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    xs = np_(x).astype(np.float64)
    gs = np_(layer.gate_sequence)
    ref = O.conv_forward(xs, och, oh, ow, p, gs, 2, 1, 3)
    np.testing.assert_allclose(np_(y), ref, **TOL[torch.float32])
    rgx, rgw = O.conv_backward(xs, och, oh, ow, p, gs, np_(gy).astype(np.float64), 2, 1)
    rgl = p * (rgw - (p * rgw).sum(1, keepdims=True))
    np.testing.assert_allclose(np_(x.grad), rgx, **TOL[torch.float32])
    np.testing.assert_allclose(np_(layer.weights.grad), rgl, rtol=1e-5, atol=1e-6)
    # the reference's bridge (probabilities in, gradient of the probabilities out) agrees
    w = torch.softmax(layer.weights.detach(), -1).requires_grad_(True)
    x2 = x.detach().requires_grad_(True)
    y2 = cl.ConvLayerCudaFunction.apply(x2, layer.offsets_ch, layer.offsets_h, layer.offsets_w, w,
                                        layer.gate_sequence, 2, 1, 3)
    y2.backward(gy)
    np.testing.assert_allclose(np_(w.grad), rgw, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(np_(x2.grad), rgx, **TOL[torch.float32])


def test_conv_layer_gradcheck_fp64(device):
    torch.manual_seed(5)
    layer = cl.ConvLayer((3, 5, 5), padding=1, c_out=4, ks=3, stride=2, num_chn=0,
                         num_gates=4).to(device).double()
    x = torch.rand((2, 3, 5, 5), device=device, dtype=torch.float64, requires_grad=True)
    w = torch.softmax(torch.randn((4, 4), device=device, dtype=torch.float64), -1).requires_grad_(True)
    f = lambda x_, w_: cl.ConvLayerCudaFunction.apply(x_, layer.offsets_ch, layer.offsets_h,
                                                      layer.offsets_w, w_, layer.gate_sequence,
                                                      2, 1, 3)
    assert torch.autograd.gradcheck(f, (x, w), eps=1e-6, atol=1e-8)


def test_conv_layer_eval_and_rewiring(device):
    torch.manual_seed(11)
    layer = cl.ConvLayer((4, 8, 8), padding=1, c_out=6, ks=3, stride=1, num_chn=0,
                         num_gates=8).to(device)
    x = (torch.rand((3, 4, 8, 8), device=device) < 0.5).float()
    layer.eval()
    y = layer(x)
    slot = np_(layer.weights.argmax(-1))
    ref = O.conv_eval(np_(x).astype(np.float64), np_(layer.offsets_ch), np_(layer.offsets_h),
                      np_(layer.offsets_w), slot, np_(layer.gate_sequence), 1, 1, 3)
    np.testing.assert_array_equal(np_(y), ref)
    # rewiring changes the offsets in place; the cached inverse index must follow
    layer.train()
    layer.resample_connections(torch.arange(6, device=device), threshold_high=2.0, threshold_low=1.0)
    xg = x.clone().requires_grad_(True)
    out = layer(xg)
    gy = torch.randn_like(out) / 3
    out.backward(gy)
    p = torch.softmax(layer.weights.detach().double(), -1).cpu().numpy()
    rgx, _ = O.conv_backward(np_(x).astype(np.float64), np_(layer.offsets_ch), np_(layer.offsets_h),
                             np_(layer.offsets_w), p, np_(layer.gate_sequence),
                             np_(gy).astype(np.float64), 1, 1)
    np.testing.assert_allclose(np_(xg.grad), rgx, **TOL[torch.float32])


def test_conv_connected_neurons_matches_loop(device):
    torch.manual_seed(2)
    layer = cl.ConvLayer((3, 6, 6), padding=1, c_out=8, ks=3, stride=2, num_chn=0,
                         num_gates=4).to(device)
    layer.freeze()
    rng = np.random.default_rng(0)
    y_flag = torch.as_tensor(rng.random(layer.out_shape) < 0.6, device=device)
    y_ref = np_(y_flag).copy()
    x_flag, y_out = layer.connected_neurons(y_flag.clone())
    # the reference's per-coordinate loop (compactlogic/compactlogic.py:813-833)
    w = np_(layer.w).astype(np.int64)
    g = np_(layer.gate_sequence)[np.arange(8), w]
    och = np_(layer.offsets_ch)[:, np.arange(8), w]
    oh = np_(layer.offsets_h)[:, np.arange(8), w]
    ow = np_(layer.offsets_w)[:, np.arange(8), w]
    xr = np.zeros(layer.in_shape, dtype=bool)
    const = np.isin(g, [0, 15])
    y_ref[const] = False
    for c in np.nonzero(~const)[0]:
        ua, ub = g[c] not in (5, 10), g[c] not in (3, 12)
        for oy, ox in zip(*np.nonzero(y_ref[c])):
            for side, use in ((0, ua), (1, ub)):
                hh, ww = oy * 2 + oh[side, c], ox * 2 + ow[side, c]
                if use and 0 <= hh < 6 and 0 <= ww < 6:
                    xr[och[side, c], hh, ww] = True
    y_ref[np.isin(g, [3, 5, 10, 12])] = False
    np.testing.assert_array_equal(np_(x_flag), xr)
    np.testing.assert_array_equal(np_(y_out), y_ref)


# ------------------------------------------------------------------------------ packed conv

@pytest.mark.parametrize("n", [64, 200, 1024])
def test_conv_packed_vs_float_and_oracle(device, n):
    torch.manual_seed(n)
    layer = cl.ConvLayer((3, 9, 7), padding=1, c_out=10, ks=3, stride=2, num_chn=0,
                         num_gates=4).to(device)
    layer.freeze()
    x = (torch.rand((n, 3, 9, 7), device=device) < 0.5)
    yf = layer(x.float())                                   # float discrete path
    pbt = cl.PackBitsTensor(x.reshape(n, -1).contiguous(), 64)     # [samples, features]
    out = layer(pbt)
    assert out is pbt and out.t.shape[0] == layer.out_dim
    bits = np.unpackbits(np_(out.t).view(np.uint8), axis=1, bitorder="little")[:, :n]
    np.testing.assert_array_equal(bits.T.reshape(yf.shape), np_(yf).astype(np.uint8))
    ia, ib, g = P.resolve_conv_slots(np_(layer.offsets_ch), np_(layer.offsets_h),
                                     np_(layer.offsets_w), np_(layer.gate_sequence), np_(layer.w),
                                     layer.in_shape, layer.stride, layer.out_shape[1:])
    xin, _ = P.pack_bits(np_(x.reshape(n, -1).t()), 64)
    ref = P.eval_layer(xin.view(np.uint64), ia, ib, g)
    assert np.array_equal(np_(out.t).view(np.uint64), ref)


@pytest.mark.parametrize("nbytes", [1, 3, 8, 24, 4096])
def test_eval_packed_indexed_widths(device, nbytes):
    rng = np.random.default_rng(nbytes)
    in_dim, out_dim = 23, 77
    xb = rng.integers(0, 256, (in_dim, nbytes), dtype=np.uint8)
    ia = rng.integers(-1, in_dim, out_dim).astype(np.int32)
    ib = rng.integers(-1, in_dim, out_dim).astype(np.int32)
    g = rng.integers(0, 16, out_dim).astype(np.uint8)
    y = cv.eval_packed_indexed(torch.as_tensor(xb, device=device), torch.as_tensor(ia, device=device),
                               torch.as_tensor(ib, device=device), torch.as_tensor(g, device=device))
    pad = (-nbytes) % 8
    xw = np.concatenate([xb, np.zeros((in_dim, pad), np.uint8)], 1).view(np.uint64)
    ref = P.eval_layer(xw, ia, ib, g).view(np.uint8)[:, :nbytes]
    np.testing.assert_array_equal(np_(y), ref)
    # any processing order gives the same rows
    order = torch.as_tensor(rng.permutation(out_dim).astype(np.int32), device=device)
    y2 = cv.eval_packed_indexed(torch.as_tensor(xb, device=device), torch.as_tensor(ia, device=device),
                                torch.as_tensor(ib, device=device), torch.as_tensor(g, device=device),
                                order)
    assert torch.equal(y, y2)


def test_cfg5_network_slice_bit_exact(device):
    """The cfg5 network (conv, conv, flatten, dense, dense, popcount GroupSum) on 2^12
    packed samples against the C oracle, and against the float discrete network."""
    cfg = configs.CONV_CONFIGS["cfg5"]
    model = configs.conv_network(cfg, device=device)
    configs.freeze_argmax(model)
    words = 64
    xw = configs.packed_input_words(9 * 32 * 32, words, device=device)
    counts = model(cl.PackBitsTensor.from_packed(xw.clone()))
    layers = []
    for m in model:
        if isinstance(m, cl.ConvLayer):
            layers.append(P.resolve_conv_slots(np_(m.offsets_ch), np_(m.offsets_h),
                                               np_(m.offsets_w), np_(m.gate_sequence), np_(m.w),
                                               m.in_shape, m.stride, m.out_shape[1:]))
        elif isinstance(m, cl.LogicLayer):
            layers.append(P.resolve_slots(np_(m.indices), np_(m.gate_sequence), np_(m.w)))
    ref = P.network_counts(np_(xw).view(np.uint64), layers, cfg.k)
    assert np.array_equal(np_(counts), ref)
    # float discrete network on the first 256 samples: counts = logits * tau
    bits = np.unpackbits(np_(xw[:, :4]).view(np.uint8), axis=1, bitorder="little")
    xf = torch.as_tensor(bits.T.reshape(256, 9, 32, 32), dtype=torch.float32, device=device)
    with torch.no_grad():
        logits = model(xf)
    np.testing.assert_array_equal(np.rint(np_(logits) * cfg.tau).astype(np.int64), ref[:256])


def test_cfg3_layers_vs_oracle(device):
    """cfg3's two conv layers at their real channel counts on a small batch, fwd + bwd."""
    cfg = configs.CONV_CONFIGS["cfg3"]
    model = configs.conv_network(cfg, device=device)
    x, _ = configs.conv_inputs(cfg, device=device, batch=2)
    h = x
    for layer in (model[0], model[1]):
        hin = h.detach().requires_grad_(True)
        y = layer(hin)
        gy = torch.randn_like(y) / 2
        y.backward(gy)
        logits = np_(layer.weights).astype(np.float64)
        p = np.exp(logits - logits.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        args = (np_(layer.offsets_ch), np_(layer.offsets_h), np_(layer.offsets_w))
        xs = np_(hin).astype(np.float64)
        ref = O.conv_forward(xs, *args, p, np_(layer.gate_sequence), layer.stride, layer.padding,
                             layer.ks)
        np.testing.assert_allclose(np_(y), ref, **TOL[torch.float32])
        rgx, rgw = O.conv_backward(xs, *args, p, np_(layer.gate_sequence),
                                   np_(gy).astype(np.float64), layer.stride, layer.padding)
        np.testing.assert_allclose(np_(hin.grad), rgx, **TOL[torch.float32])
        rgl = p * (rgw - (p * rgw).sum(1, keepdims=True))
        np.testing.assert_allclose(np_(layer.weights.grad), rgl, rtol=1e-5, atol=1e-6)
        h = y.detach()


# ------------------------------------------------------------------------------ window path

def _layer_vs_oracle(layer, x, gy, dtype):
    """Run layer fwd + bwd on x with upstream gy; compare y, grad_x and the logits gradient
    with the float64 oracle."""
    xg = x.detach().clone().requires_grad_(True)
    y = layer(xg)
    y.backward(gy)
    logits = np_(layer.weights).astype(np.float64)
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    args = (np_(layer.offsets_ch), np_(layer.offsets_h), np_(layer.offsets_w))
    xs = np_(x).astype(np.float64)
    gs = np_(layer.gate_sequence)
    ref = O.conv_forward(xs, *args, p, gs, layer.stride, layer.padding, layer.ks)
    np.testing.assert_allclose(np_(y), ref, **TOL[dtype])
    rgx, rgw = O.conv_backward(xs, *args, p, gs, np_(gy).astype(np.float64), layer.stride,
                               layer.padding)
    np.testing.assert_allclose(np_(xg.grad), rgx, **TOL[dtype])
    rgl = p * (rgw - (p * rgw).sum(1, keepdims=True))
    np.testing.assert_allclose(np_(layer.weights.grad), rgl, **TOL[dtype])
    layer.weights.grad = None


WINDOW_SHAPES = [
    # c_in, h, w, c_out, G, ks, stride, pad, n
    (9, 32, 32, 20, 16, 3, 2, 1, 5),     # cfg3 conv1 geometry
    (16, 16, 16, 32, 16, 3, 2, 0, 4),    # cfg3 conv2 geometry
    (3, 9, 7, 7, 4, 2, 1, 0, 3),         # 2 x 2 windows, non-square
    (4, 11, 13, 9, 64, 3, 3, 1, 2),      # stride 3, 64 slots
    (5, 6, 6, 5, 1, 3, 1, 2, 70),        # one slot, wide padding, several sample chunks
    (2, 40, 24, 3, 8, 3, 1, 1, 2),       # 960 output positions in one block
    # at least 8 output channels per input channel: the tiled moments kernel
    (9, 32, 32, 256, 16, 3, 2, 1, 6),    # cfg3 conv1 itself (28-29 channels per input channel)
    (3, 12, 12, 100, 8, 2, 1, 0, 9),     # 2 x 2 windows, 33-34 channels: two channel tiles
    (2, 9, 7, 40, 4, 2, 2, 1, 3),        # 2 x 2 windows, stride 2, 20 channels per input
    (4, 10, 10, 40, 16, 3, 1, 1, 70),    # element chunks not multiples of the staged slab
]


@pytest.mark.parametrize("shape", WINDOW_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_window_path_matches_oracle(device, shape, dtype):
    c_in, h, wd, c_out, g_n, ks, stride, pad, n = shape
    torch.manual_seed(sum(shape))
    layer = cl.ConvLayer((c_in, h, wd), padding=pad, c_out=c_out, ks=ks, stride=stride,
                         num_chn=1, num_gates=g_n).to(device).to(dtype)
    x = torch.rand((n, c_in, h, wd), device=device, dtype=dtype)
    plan = layer.window_plan(x)
    assert plan is not None and plan.kw == ks
    y_shape = (n,) + layer.out_shape
    gy = torch.empty(y_shape, device=device, dtype=dtype).uniform_(-1, 1) / n
    _layer_vs_oracle(layer, x, gy, dtype)


# The input-gradient plane sits in LDS split by the stride's phases with its row pitch padded
# so that the lanes of a half-wave add to distinct banks, split unpadded when the padding does
# not fit in 64 KiB, or in plain rows when neither split fits; each layout against the oracle.
LAYOUT_CASES = [
    # (c_in, h, w, c_out, G, ks, stride, pad, n), dtype
    ((3, 16, 20, 6, 8, 3, 4, 1, 3), torch.float32),    # stride 4, window origin -1: padded
    ((4, 16, 16, 8, 16, 3, 4, 1, 3), torch.float64),   # stride 4, whole rows per store pass
    ((2, 127, 126, 3, 8, 3, 4, 0, 2), torch.float32),  # padded split too large: unpadded
    ((2, 63, 130, 3, 8, 3, 4, 0, 2), torch.float32),   # padded split
    ((2, 63, 130, 3, 8, 3, 4, 0, 2), torch.float64),   # neither split fits: plain rows
    ((2, 125, 64, 3, 8, 3, 3, 0, 2), torch.float64),   # plain rows, whole rows per store pass
]


@pytest.mark.parametrize("shape,dtype", LAYOUT_CASES,
                         ids=lambda s: "x".join(map(str, s)) if isinstance(s, tuple) else str(s))
def test_window_input_gradient_layouts(device, shape, dtype):
    c_in, h, wd, c_out, g_n, ks, stride, pad, n = shape
    torch.manual_seed(sum(shape))
    layer = cl.ConvLayer((c_in, h, wd), padding=pad, c_out=c_out, ks=ks, stride=stride,
                         num_chn=1, num_gates=g_n).to(device).to(dtype)
    x = torch.rand((n, c_in, h, wd), device=device, dtype=dtype)
    assert layer.window_plan(x) is not None
    gy = torch.empty((n,) + layer.out_shape, device=device, dtype=dtype).uniform_(-1, 1) / n
    _layer_vs_oracle(layer, x, gy, dtype)


@pytest.mark.parametrize("c_out", [20, 256])
def test_window_path_empty_batch(device, c_out):
    """A batch of 0 samples: empty outputs and input gradient, zero logits gradient, no read of
    the (empty) inputs, on the chunked moments kernel (20 channels over 9 inputs) and on the
    tiled one (28-29 channels per input channel)."""
    torch.manual_seed(2)
    layer = cl.ConvLayer((9, 32, 32), padding=1, c_out=c_out, ks=3, stride=2, num_chn=1,
                         num_gates=16).to(device)
    x = torch.rand((0, 9, 32, 32), device=device, requires_grad=True)
    assert layer.window_plan(x) is not None
    y = layer(x)
    assert y.shape == (0, c_out, 16, 16)
    y.sum().backward()
    torch.cuda.synchronize()
    assert x.grad.shape == x.shape
    assert torch.equal(layer.weights.grad, torch.zeros_like(layer.weights))


def test_window_path_self_pairs_and_rewiring(device):
    """Slots whose two operands are the same tap (reachable through rewiring, which does not
    re-resolve conflicts) give square terms; in-place offset changes rebuild the plan."""
    torch.manual_seed(8)
    layer = cl.ConvLayer((4, 10, 10), padding=1, c_out=8, ks=3, stride=2, num_chn=1,
                         num_gates=16).to(device)
    x = torch.rand((6, 4, 10, 10), device=device)
    first = layer.window_plan(x)
    with torch.no_grad():
        layer.offsets_h[1, :, ::3] = layer.offsets_h[0, :, ::3]
        layer.offsets_w[1, :, ::3] = layer.offsets_w[0, :, ::3]
    second = layer.window_plan(x)
    assert second is not None and second is not first
    gy = torch.randn((6,) + layer.out_shape, device=device) / 6
    _layer_vs_oracle(layer, x, gy, torch.float32)
    layer.resample_connections(torch.arange(8, device=device), threshold_high=2.0, threshold_low=1.0)
    assert layer.window_plan(x) is not second
    _layer_vs_oracle(layer, x, gy, torch.float32)


def test_window_path_not_taken_for_mixed_channels(device):
    torch.manual_seed(1)
    layer = cl.ConvLayer((4, 8, 8), padding=1, c_out=6, ks=3, stride=1, num_chn=0,
                         num_gates=8).to(device)
    assert layer.window_plan(torch.rand(1, 4, 8, 8, device=device)) is None


def test_window_path_deterministic_and_input_only(device):
    torch.manual_seed(3)
    layer = cl.ConvLayer((8, 16, 16), padding=1, c_out=24, ks=3, stride=2, num_chn=1,
                         num_gates=16).to(device)
    x = torch.rand((40, 8, 16, 16), device=device, requires_grad=True)
    grads = []
    for _ in range(2):
        x.grad = None
        layer.weights.grad = None
        layer(x).square().sum().backward()
        grads.append((x.grad.clone(), layer.weights.grad.clone()))
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])
    # logits frozen: only the input gradient is produced
    layer.weights.requires_grad_(False)
    x.grad = None
    layer(x).square().sum().backward()
    assert torch.equal(x.grad, grads[0][0])
    layer.weights.requires_grad_(True)
