"""Logic-tree conv block (ConvLogicLayer / TreeLogicLayer / PoolLogicLayer) on the HIP kernels
against the float64 CPU oracle (oracle/tree_np.py) and the reference's own module tests
(third_party/convlogic_source_code/tests/convlogic/test_full_convlogic_forward.py,
test_full_convlogic_autograd.py, test_treelogic_forward.py)."""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl
from compactlogic_amd import treelogic as TL
from oracle import tree_np as T

pytestmark = pytest.mark.gpu


def np_(t):
    return t.detach().cpu().numpy()


def make(seed, n, c_in, h, w, c_out, kernel=3, nodes=7, dtype=torch.float32, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    x = torch.rand((n, c_in, h, w), generator=g, dtype=torch.float64)
    w_prob = torch.softmax(torch.randn((c_out, nodes, 16), generator=g, dtype=torch.float64), -1)
    ch = torch.randint(0, c_in, (c_out, 8), generator=g)
    r = torch.randint(0, kernel, (c_out, 8), generator=g)
    cc = torch.randint(0, kernel, (c_out, 8), generator=g)
    sel = ((ch << 16) | (r << 8) | cc).to(torch.int32)
    return x.to(device, dtype), w_prob.to(device, dtype), sel.to(device)


def tol(dtype):
    return dict(rtol=1e-5, atol=1e-6) if dtype == torch.float32 else dict(rtol=1e-10, atol=1e-12)


SHAPES = [  # stride, pad, kernel, (n, c_in, h, w, c_out)
    ((1, 1), (1, 1), (3, 3), (2, 3, 8, 8, 4)),
    ((2, 2), (2, 2), (3, 3), (3, 3, 10, 10, 5)),
    ((2, 2), (1, 1), (3, 3), (4, 9, 32, 32, 16)),     # conv1 of the tree reading of cfg3
    ((2, 2), (1, 1), (3, 3), (3, 16, 8, 8, 32)),      # conv2 of the tree reading
    ((1, 1), (0, 0), (2, 2), (2, 2, 5, 5, 3)),
    ((2, 2), (1, 1), (3, 3), (128, 9, 16, 16, 41)),   # channel groups of 2, the last one short
    ((1, 1), (1, 1), (3, 3), (2, 5, 64, 64, 3)),      # 80 KiB (fp32) / 160 KiB (fp64) planes
    # LDS-staged forward (at least two items per staged input element):
    ((2, 2), (1, 1), (3, 3), (2, 9, 32, 32, 160)),    # conv1 geometry, a channel per wave
    ((2, 2), (1, 1), (3, 3), (2, 3, 8, 8, 64)),       # 16 items per channel: 4 channels a wave
    ((1, 1), (1, 1), (3, 3), (2, 2, 10, 10, 24)),     # stride 1, 5 windows a row, 100 items
    ((2, 2), (1, 1), (3, 3), (2, 9, 32, 32, 600)),    # staged backward in three channel groups
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("stride,pad,kernel,shape", SHAPES)
def test_complete_block_forward_matches_oracle(dtype, stride, pad, kernel, shape):
    n, c_in, h, w, c_out = shape
    x, w_prob, sel = make(1, n, c_in, h, w, c_out, kernel[0], dtype=dtype)
    y, x2, x3, idx = TL.full_convlogic_forward(x, w_prob, sel, *stride, *pad, *kernel)
    ry, rx2, rx3, ridx = T.block_forward(np_(x), np_(w_prob), np_(sel), stride, pad, kernel)
    np.testing.assert_allclose(np_(y), ry, **tol(dtype))
    np.testing.assert_allclose(np_(x2), rx2, **tol(dtype))
    np.testing.assert_allclose(np_(x3), rx3, **tol(dtype))
    # winners equal the oracle's except where two positions tie within rounding
    eps = float(np.finfo(np.float32 if dtype == torch.float32 else np.float64).eps)
    free = _near_ties(_window_scores(np_(x).astype(np.float64), np_(w_prob).astype(np.float64),
                                     np_(sel), stride, pad, kernel), eps)
    assert free.mean() < 0.02, free.mean()
    assert np.array_equal(np_(idx)[~free], ridx[~free])
    y2, a, b, idx2 = TL.full_convlogic_forward(x, w_prob, sel, *stride, *pad, *kernel,
                                               intermediate=False)
    assert a is None and b is None
    assert torch.equal(y2, y) and torch.equal(idx2, idx)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("stride,pad,kernel,shape", SHAPES)
def test_conv_gates_forward_matches_oracle(dtype, stride, pad, kernel, shape):
    n, c_in, h, w, c_out = shape
    x, w_prob, sel = make(2, n, c_in, h, w, c_out, kernel[0], nodes=4, dtype=dtype)
    y = TL.convlogic_forward(x, w_prob, sel, *stride, *pad, *kernel)
    ref = T.block_forward(np_(x), np_(w_prob), np_(sel), stride, pad, kernel, complete=False)
    np.testing.assert_allclose(np_(y), ref, **tol(dtype))


@pytest.mark.parametrize("complete", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("stride,pad,kernel,shape", SHAPES)
def test_block_backward_matches_oracle_and_is_reproducible(complete, dtype, stride, pad, kernel,
                                                           shape):
    n, c_in, h, w, c_out = shape
    nodes = 7 if complete else 4
    x, w_prob, sel = make(3, n, c_in, h, w, c_out, kernel[0], nodes=nodes, dtype=dtype)
    idx = None
    if complete:
        y, _, _, idx = TL.full_convlogic_forward(x, w_prob, sel, *stride, *pad, *kernel,
                                                 intermediate=False)
    else:
        y = TL.convlogic_forward(x, w_prob, sel, *stride, *pad, *kernel)
    g = torch.Generator().manual_seed(4)
    gy = torch.randn(y.shape, generator=g, dtype=torch.float64).to(y.device, dtype)
    gx, gw = TL.tree_conv_backward(gy, x, w_prob, sel, idx, *stride, *pad, *kernel, complete)
    oidx = None
    if complete:
        # the oracle's own winners, except where rounding may pick either of two positions
        xs, ws, ss = np_(x).astype(np.float64), np_(w_prob).astype(np.float64), np_(sel)
        ridx = T.block_forward(xs, ws, ss, stride, pad, kernel)[3]
        eps = float(np.finfo(np.float32 if dtype == torch.float32 else np.float64).eps)
        free = _near_ties(_window_scores(xs, ws, ss, stride, pad, kernel), eps)
        assert np.array_equal(np_(idx)[~free], ridx[~free])
        oidx = np.where(free, np_(idx), ridx)
    rgx, rgw = T.block_backward(np_(x), np_(w_prob), np_(sel), stride, pad, kernel, np_(gy),
                                complete, idx=oidx)
    scale = max(1.0, float(np.abs(rgw).max()))
    np.testing.assert_allclose(np_(gx), rgx, **tol(dtype))
    np.testing.assert_allclose(np_(gw) / scale, rgw / scale, **tol(dtype))
    gx2, gw2 = TL.tree_conv_backward(gy, x, w_prob, sel, idx, *stride, *pad, *kernel, complete)
    assert torch.equal(gx, gx2) and torch.equal(gw, gw2)
    gx3, gw3 = TL.tree_conv_backward(gy, x, w_prob, sel, idx, *stride, *pad, *kernel, complete,
                                     need_x=False)
    assert gx3 is None and torch.equal(gw3, gw)


# global gather, conv1 / conv2 of the tree reading, and the two LDS-staged shapes
SOFTMAX_SHAPES = [SHAPES[0], SHAPES[2], SHAPES[3], SHAPES[7], SHAPES[8]]


@pytest.mark.parametrize("complete", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("stride,pad,kernel,shape", SOFTMAX_SHAPES)
def test_logit_entry_points_match_oracle_on_the_softmax(complete, dtype, stride, pad, kernel,
                                                        shape):
    """cl_tree_conv_forward_softmax / _backward_softmax take node logits: the outputs equal the
    oracle's on softmax(logits) (float64), the weight gradient equals the oracle's probability
    gradient through the softmax Jacobian p (g - sum p g), the input gradient the oracle's; the
    winners are compared away from near ties, as for the probability entry points."""
    n, c_in, h, w, c_out = shape
    nodes = 7 if complete else 4
    x, _, sel = make(11, n, c_in, h, w, c_out, kernel[0], nodes=nodes, dtype=dtype)
    g = torch.Generator().manual_seed(12)
    logits64 = 3.0 * torch.randn((c_out, nodes, 16), generator=g, dtype=torch.float64)
    p64 = np_(torch.softmax(logits64, -1))
    logits = logits64.to(x.device, dtype)
    xs, ss = np_(x).astype(np.float64), np_(sel)
    idx = oidx = None
    if complete:
        y, _, _, idx = TL.full_convlogic_forward(x, logits, sel, *stride, *pad, *kernel,
                                                 intermediate=False, softmax=True)
        ry, _, _, ridx = T.block_forward(xs, p64, ss, stride, pad, kernel)
        eps = float(np.finfo(np.float32 if dtype == torch.float32 else np.float64).eps)
        free = _near_ties(_window_scores(xs, p64, ss, stride, pad, kernel), eps)
        assert np.array_equal(np_(idx)[~free], ridx[~free])
        oidx = np.where(free, np_(idx), ridx)
    else:
        y = TL.convlogic_forward(x, logits, sel, *stride, *pad, *kernel, softmax=True)
        ry = T.block_forward(xs, p64, ss, stride, pad, kernel, complete=False)
    np.testing.assert_allclose(np_(y), ry, **tol(dtype))
    gy = torch.randn(y.shape, generator=g, dtype=torch.float64).to(y.device, dtype)
    gx, gl = TL.tree_conv_backward(gy, x, logits, sel, idx, *stride, *pad, *kernel, complete,
                                   softmax=True)
    rgx, rgw = T.block_backward(xs, p64, ss, stride, pad, kernel, np_(gy).astype(np.float64),
                                complete, idx=oidx)
    rgl = p64 * (rgw - (rgw * p64).sum(-1, keepdims=True))
    np.testing.assert_allclose(np_(gx), rgx, **tol(dtype))
    # p (g - sum p g) loses the absolute precision of g in the difference: scale by max |g|
    scale = max(1.0, float(np.abs(rgw).max()))
    np.testing.assert_allclose(np_(gl) / scale, rgl / scale, **tol(dtype))
    gx2, gl2 = TL.tree_conv_backward(gy, x, logits, sel, idx, *stride, *pad, *kernel, complete,
                                     softmax=True)
    assert torch.equal(gx, gx2) and torch.equal(gl, gl2)


@pytest.mark.parametrize("complete", [True, False])
@pytest.mark.parametrize("dtype,hw", [(torch.float32, 136), (torch.float64, 96)])
def test_backward_of_planes_beyond_lds_in_row_bands(complete, dtype, hw):
    """Input planes above 64 KiB (fp32 136 x 136, fp64 96 x 96) are gathered in bands of
    rows; the input gradient matches the oracle and repeats bitwise."""
    stride, pad, kernel = (2, 2), (1, 1), (3, 3)
    n, c_in, c_out = 2, 2, 3
    nodes = 7 if complete else 4
    x, w_prob, sel = make(13, n, c_in, hw, hw, c_out, kernel[0], nodes=nodes, dtype=dtype)
    if complete:
        y, _, _, idx = TL.full_convlogic_forward(x, w_prob, sel, *stride, *pad, *kernel,
                                                 intermediate=False)
    else:
        y, idx = TL.convlogic_forward(x, w_prob, sel, *stride, *pad, *kernel), None
    gy = torch.randn(y.shape, generator=torch.Generator().manual_seed(14),
                     dtype=torch.float64).to(y.device, dtype)
    gx, gw = TL.tree_conv_backward(gy, x, w_prob, sel, idx, *stride, *pad, *kernel, complete)
    rgx, rgw = T.block_backward(np_(x), np_(w_prob), np_(sel), stride, pad, kernel, np_(gy),
                                complete, idx=np_(idx) if complete else None)
    scale = max(1.0, float(np.abs(rgw).max()))
    np.testing.assert_allclose(np_(gx), rgx, **tol(dtype))
    np.testing.assert_allclose(np_(gw) / scale, rgw / scale, **tol(dtype))
    gx2, _ = TL.tree_conv_backward(gy, x, w_prob, sel, idx, *stride, *pad, *kernel, complete)
    assert torch.equal(gx, gx2)


def _window_scores(x, w_prob, sel, stride, pad, kernel):
    """Oracle block outputs at every conv position [N, C, Ho, Wo] (node 6 of the tree), from
    the oracle's own node values."""
    _, _, t, _ = T.block_forward(x, w_prob, sel, stride, pad, kernel)
    k6 = T.collapse(w_prob)[None, :, None, None, 6, :]
    return k6[..., 0] + k6[..., 1] * t[..., 0] + k6[..., 2] * t[..., 1] + k6[..., 3] * t[..., 0] * t[..., 1]


def _windows(r):
    """[N, C, Ho, Wo] -> [N, C, P, 4]: the four positions of each 2 x 2 pooling window in
    row-major window order."""
    n, c, ho, wo = r.shape
    hp, wp = ho // 2, wo // 2
    win = np.stack([r[:, :, dy::2, dx::2][:, :, :hp, :wp] for dy in range(2) for dx in range(2)], -1)
    return win.reshape(n, c, hp * wp, 4)


def _near_ties(r, eps):
    """Windows [N, C, P] whose two best positions differ by a nonzero amount within a few ulp
    of the working precision (32, for the rounding of three tree levels): there the lower
    precision may pick either.  Exact ties are not exempt: the first maximum in window order
    must win them."""
    top = np.sort(_windows(r), axis=-1)
    gap = top[..., 3] - top[..., 2]
    return (gap > 0) & (gap <= 32 * eps * np.maximum(np.abs(top[..., 3]), 1e-30))


BINARY_SHAPES = [  # stride, pad, kernel, (n, c_in, h, w, c_out)
    ((2, 2), (1, 1), (3, 3), (8, 9, 32, 32, 24)),     # conv1 of the tree reading of cfg3
    ((2, 2), (1, 1), (3, 3), (16, 16, 8, 8, 32)),     # conv2 of the tree reading
    ((1, 1), (1, 1), (3, 3), (4, 3, 12, 12, 6)),
    ((1, 1), (0, 0), (2, 2), (6, 2, 7, 9, 5)),        # many positions share all eight taps
    # LDS-staged forward:
    ((2, 2), (1, 1), (3, 3), (4, 9, 32, 32, 160)),    # conv1 geometry (staged node pass)
    ((2, 2), (1, 1), (3, 3), (4, 3, 8, 8, 64)),       # four channels a wave
    ((1, 1), (0, 0), (2, 2), (6, 2, 7, 9, 40)),       # 48 items per channel, 16 lanes idle
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("stride,pad,kernel,shape", BINARY_SHAPES)
def test_complete_block_binary_inputs_exact_winners(dtype, stride, pad, kernel, shape):
    """Bernoulli(0.5) inputs, as the thresholded images of cfg3 give: exact ties between
    window positions are common (positions with equal taps), and the first maximum in
    row-major window order must win each of them (strict '>' scan,
    full_convlogic_kernel.cu:126-139).  Every winner must equal the oracle's, except in
    windows whose two best scores differ by a nonzero amount of a few ulp (there rounding
    decides, and the reference's own fp32 kernel is no more determined); the backward is
    compared against the oracle's backward through the oracle's own winners outside those
    windows."""
    n, c_in, h, w, c_out = shape
    g = torch.Generator().manual_seed(11)
    x = (torch.rand((n, c_in, h, w), generator=g) < 0.5).to(torch.float64)
    _, w_prob, sel = make(12, n, c_in, h, w, c_out, kernel[0], dtype=torch.float64, device="cpu")
    xd, wd, seld = x.cuda().to(dtype), w_prob.cuda().to(dtype), sel.cuda()
    y, _, _, idx = TL.full_convlogic_forward(xd, wd, seld, *stride, *pad, *kernel)
    # the oracle sees exactly the probabilities the kernel got
    xs, ws, ss = np_(x), np_(wd).astype(np.float64), np_(sel)
    ry, _, _, ridx = T.block_forward(xs, ws, ss, stride, pad, kernel)
    r = _window_scores(xs, ws, ss, stride, pad, kernel)
    eps = float(np.finfo(np.float32 if dtype == torch.float32 else np.float64).eps)
    free = _near_ties(r, eps)
    wins = _windows(r)
    exact_ties = (wins == wins.max(-1, keepdims=True)).sum(-1) > 1
    # the inputs exercise the tie-break rule; windows left to rounding stay a small minority
    assert exact_ties.mean() > 0.01, exact_ties.mean()
    assert free.mean() < 0.02, free.mean()
    got = np_(idx)
    assert np.array_equal(got[~free], ridx[~free])
    np.testing.assert_allclose(np_(y), ry, **tol(dtype))
    # backward: the oracle routes through its own winners wherever they are determined
    gy = torch.randn(y.shape, generator=g, dtype=torch.float64)
    gx, gw = TL.tree_conv_backward(gy.cuda().to(dtype), xd, wd, seld, idx, *stride, *pad,
                                   *kernel, True)
    rgx, rgw = T.block_backward(xs, ws, ss, stride, pad, kernel, np_(gy.to(dtype)), True,
                                idx=np.where(free, got, ridx))
    scale = max(1.0, float(np.abs(rgw).max()))
    np.testing.assert_allclose(np_(gx), rgx, **tol(dtype))
    np.testing.assert_allclose(np_(gw) / scale, rgw / scale, **tol(dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_tree_level_matches_oracle(dtype):
    g = torch.Generator().manual_seed(5)
    for xin in (2, 4, 8):
        x = torch.rand((3, 5, 4, 6, xin), generator=g, dtype=torch.float64).cuda().to(dtype)
        w_prob = torch.softmax(torch.randn((5, xin // 2, 16), generator=g, dtype=torch.float64),
                               -1).cuda().to(dtype)
        y = TL.treelogic_forward(x, w_prob)
        np.testing.assert_allclose(np_(y), T.level_forward(np_(x), np_(w_prob)), **tol(dtype))
        gy = torch.randn(y.shape, generator=g, dtype=torch.float64).cuda().to(dtype)
        gx, gw = TL.treelogic_backward(gy, x, w_prob)
        rgx, rgw = T.level_backward(np_(x), np_(w_prob), np_(gy))
        np.testing.assert_allclose(np_(gx), rgx, **tol(dtype))
        np.testing.assert_allclose(np_(gw), rgw, **tol(dtype))


@pytest.mark.parametrize("complete", [True, False])
@pytest.mark.parametrize("c_in,h,w,stride,pad,kernel,words", [
    (9, 32, 32, (2, 2), (1, 1), (3, 3), 5),     # conv1 of the tree reading, partial chunk
    (9, 32, 32, (2, 2), (1, 1), (3, 3), 200),   # staged patches over seven chunks
    (3, 12, 12, (2, 2), (1, 1), (3, 3), 33),    # 3 x 3 windows, two chunks
    (2, 10, 10, (1, 1), (1, 1), (3, 3), 17),    # stride 1
    (16, 8, 8, (2, 2), (1, 1), (3, 3), 40),     # conv2 of the tree reading
])
def test_packed_block_matches_bit_oracle(complete, c_in, h, w, stride, pad, kernel, words):
    rng = np.random.default_rng(6)
    c_out = 12
    nodes = 7 if complete else 4
    xw = rng.integers(0, 2**63, (c_in * h * w, words), dtype=np.int64).view(np.uint64)
    gates = rng.integers(0, 16, (c_out, nodes)).astype(np.uint8)
    _, _, sel = make(7, 1, c_in, h, w, c_out, nodes=nodes)
    out = TL.tree_conv_eval_packed(torch.as_tensor(xw.view(np.int64)).cuda(),
                                   torch.as_tensor(gates).cuda(), sel, (c_in, h, w), stride, pad,
                                   kernel, complete)
    ref = T.block_bits(xw, gates, np_(sel), (c_in, h, w), stride, pad, kernel, complete)
    assert np.array_equal(np_(out).view(np.uint64), ref)


@pytest.mark.parametrize("c_in,h,w,words", [(4, 12, 12, 40), (16, 8, 8, 40)])
def test_packed_block_taps_outside_the_window_and_out_of_range_channels(c_in, h, w, words):
    """Staged (4 input channels) and global-gather (16) packed blocks: a channel with a tap
    outside the kernel window matches the bit oracle, one reading an input channel >= C
    gives all-ones rows."""
    rng = np.random.default_rng(8)
    c_out, stride, pad, kernel = 12, (2, 2), (1, 1), (3, 3)
    xw = rng.integers(0, 2**63, (c_in * h * w, words), dtype=np.int64).view(np.uint64)
    gates = rng.integers(0, 16, (c_out, 7)).astype(np.uint8)
    _, _, sel = make(9, 1, c_in, h, w, c_out, nodes=7)
    sel = sel.clone()
    sel[1, 2] = (sel[1, 2] & ~0xFF00) | (4 << 8)
    sel[3, 5] = (sel[3, 5] & ~0xFF) | 3
    ok = sel.clone()
    sel[4, 0] = (sel[4, 0] & 0xFFFF) | (c_in << 16)
    ok[4, 0] = ok[4, 0] & 0xFFFF
    out = np_(TL.tree_conv_eval_packed(torch.as_tensor(xw.view(np.int64)).cuda(),
                                       torch.as_tensor(gates).cuda(), sel, (c_in, h, w), stride,
                                       pad, kernel, True)).view(np.uint64)
    ref = T.block_bits(xw, gates, np_(ok), (c_in, h, w), stride, pad, kernel, True)
    P = out.shape[0] // c_out
    rows = np.arange(out.shape[0]) // P
    assert np.array_equal(out[rows != 4], ref[rows != 4])
    assert (out[rows == 4] == np.uint64(2**64 - 1)).all()


def test_module_packed_path_widens_power_of_two_rows():
    """Rows of 16 KiB are widened to an odd number of 256-byte blocks before the block reads
    them: the sample words are those of the unwidened evaluation, num_samples is unchanged."""
    torch.manual_seed(9)
    layer = cl.ConvLogicLayer(3, 4, stride=2, padding=1, kernel=3, complete=True).cuda().eval()
    words = 2048                                                   # 16 KiB rows
    xw = torch.randint(-2**62, 2**62, (3 * 8 * 8, words), dtype=torch.int64, device="cuda")
    gates = layer.weights.argmax(-1).to(torch.uint8).contiguous()
    direct = TL.tree_conv_eval_packed(xw, gates, layer.selection.to(torch.int32).contiguous(),
                                      (3, 8, 8), layer.stride, layer.padding, layer.kernel, True)
    xp = cl.PackBitsTensor.from_packed(xw.clone(), 5)
    n = xp.num_samples
    out = layer(xp)
    assert out.t.shape == (direct.shape[0], TL.tree_row_bytes(words * 8) // 8)
    assert out.num_samples == n
    assert torch.equal(out.t[:, :words], direct)


def test_module_packed_path_matches_float_eval():
    torch.manual_seed(8)
    layer = cl.ConvLogicLayer(3, 6, stride=2, padding=1, kernel=3, complete=True).cuda().eval()
    n = 128
    bits = (torch.rand((n, 3, 12, 12), device="cuda") < 0.5)
    y_float = layer(bits.float())
    xp = cl.PackBitsTensor(bits.reshape(n, -1), 64)
    out = layer(xp)
    got = torch.stack([((out.t >> j) & 1) for j in range(64)], 0)  # [64, rows, words]
    got = got.permute(2, 0, 1).reshape(-1, out.t.shape[0])[:n]
    assert torch.equal(got.float(), y_float.reshape(n, -1))


# ---- module tests in the pattern of the reference's own
@pytest.mark.parametrize("stride,pad", [(1, 1), (2, 2)])
def test_output_shape(stride, pad):
    h_in = w_in = 11 + pad
    layer = cl.ConvLogicLayer(3, 2, stride=stride, padding=pad, kernel=3, complete=True).cuda().eval()
    y = layer(torch.randn(2, 3, h_in, w_in, device="cuda"))
    h_out = (h_in + 2 * pad - 3) // stride + 1
    assert y.shape == (2, 2, h_out // 2, h_out // 2)


def test_range_determinism_and_irregular_channels():
    torch.manual_seed(0)
    layer = cl.ConvLogicLayer(1, 1, complete=True).cuda().eval()
    x = torch.rand(3, 1, 6, 6, device="cuda")
    y1, y2 = layer(x), layer(x)
    assert torch.equal(y1, y2) and bool(((y1 >= 0) & (y1 <= 1)).all())
    assert not torch.isnan(cl.ConvLogicLayer(2, 2, complete=True).cuda().eval()(
        torch.randn(4, 2, 6, 6, device="cuda"))).any()
    y = cl.ConvLogicLayer(1, 5, complete=True).cuda().eval()(torch.randn(1, 1, 6, 6, device="cuda"))
    assert y.shape[1] == 5 and y.shape[-1] == 3
    y = cl.ConvLogicLayer(1, 1, kernel=2, padding=0, complete=True).cuda().eval()(
        torch.randn(1, 1, 3, 3, device="cuda"))
    assert y.shape == (1, 1, 1, 1)


@pytest.mark.parametrize("dtype,shape", [
    (torch.float32, (3, 4, 12, 12, 64)),      # LDS-staged forward, flagged channels fixed up
    (torch.float64, (3, 4, 12, 12, 64)),
    (torch.float64, (1, 5, 64, 64, 6)),       # global gather throughout
])
@pytest.mark.parametrize("complete", [True, False])
def test_forward_taps_outside_the_window_and_out_of_range_channels(dtype, shape, complete):
    """A channel with a tap outside the kernel window (still inside the padded image) matches
    the oracle; a channel reading an input channel >= C yields NaN; the others are unchanged."""
    n, c_in, h, w, c_out = shape
    stride, pad, kernel = (2, 2), (1, 1), (3, 3)
    x, w_prob, sel = make(7, n, c_in, h, w, c_out, 3, nodes=7 if complete else 4, dtype=dtype)
    sel = sel.clone()
    sel[1, 2] = (sel[1, 2] & ~0xFF00) | (4 << 8)          # row 4 of a 3x3 window
    sel[3, 5] = (sel[3, 5] & ~0xFF) | 3                   # column 3
    ok = sel.clone()
    sel[4, 0] = (sel[4, 0] & 0xFFFF) | (c_in << 16)       # input channel C
    ok[4, 0] = ok[4, 0] & 0xFFFF
    live = [c for c in range(c_out) if c != 4]
    if complete:
        y, x2, x3, idx = TL.full_convlogic_forward(x, w_prob, sel, *stride, *pad, *kernel)
        ry, rx2, rx3, ridx = T.block_forward(np_(x), np_(w_prob), np_(ok), stride, pad, kernel)
        np.testing.assert_allclose(np_(y)[:, live], ry[:, live], **tol(dtype))
        np.testing.assert_allclose(np_(x2)[:, live], rx2[:, live], **tol(dtype))
        np.testing.assert_allclose(np_(x3)[:, live], rx3[:, live], **tol(dtype))
        assert torch.isnan(y[:, 4]).all() and torch.isnan(x2[:, 4]).all()
        # backward with the out-of-window taps only (the staged node pass leaves those
        # channels to its fix-up kernel), through the oracle's winners
        _, _, _, idx_ok = TL.full_convlogic_forward(x, w_prob, ok, *stride, *pad, *kernel)
        gy = torch.randn(ry.shape, generator=torch.Generator().manual_seed(3),
                         dtype=torch.float64)
        gx, gw = TL.tree_conv_backward(gy.to(x.device, x.dtype), x, w_prob, ok, idx_ok, *stride,
                                       *pad, *kernel, True)
        rgx, rgw = T.block_backward(np_(x), np_(w_prob), np_(ok), stride, pad, kernel,
                                    np_(gy.to(x.dtype)), True, idx=np_(idx_ok))
        scale = max(1.0, float(np.abs(rgw).max()))
        np.testing.assert_allclose(np_(gx), rgx, **tol(dtype))
        np.testing.assert_allclose(np_(gw) / scale, rgw / scale, **tol(dtype))
    else:
        y = TL.convlogic_forward(x, w_prob, sel, *stride, *pad, *kernel)
        ref = T.block_forward(np_(x), np_(w_prob), np_(ok), stride, pad, kernel, complete=False)
        np.testing.assert_allclose(np_(y)[:, live], ref[:, live], **tol(dtype))
        assert torch.isnan(y[:, 4]).all()


@pytest.mark.parametrize("complete", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_regular_taps_guarantee_skips_the_fix_up_and_poisons_a_broken_one(complete, dtype):
    """cl_tree_conv_forward_softmax with regular_taps = 1: on a sampled (regular) selection the
    outputs are bitwise those of the call without the guarantee; a channel that breaks it on
    the LDS-staged path (a tap outside the window, another channel reading input C) gets NaN
    outputs and winner -1, and every other channel is unchanged."""
    n, c_in, h, w, c_out = 3, 4, 12, 12, 64   # LDS-staged
    stride, pad, kernel = (2, 2), (1, 1), (3, 3)
    nodes = 7 if complete else 4
    x, _, sel = make(21, n, c_in, h, w, c_out, 3, nodes=nodes, dtype=dtype)
    logits = torch.randn((c_out, nodes, 16), generator=torch.Generator().manual_seed(22),
                         dtype=torch.float64).to(x.device, dtype)

    def fwd(s, regular):
        if complete:
            y, x2, x3, idx = TL.full_convlogic_forward(x, logits, s, *stride, *pad, *kernel,
                                                       softmax=True, regular=regular)
            return y, x2, x3, idx
        return (TL.convlogic_forward(x, logits, s, *stride, *pad, *kernel, softmax=True,
                                     regular=regular),)

    for a, b in zip(fwd(sel, False), fwd(sel, True)):
        assert torch.equal(a, b)
    bad = sel.clone()
    bad[1, 2] = (bad[1, 2] & ~0xFF00) | (4 << 8)        # row 4 of a 3x3 window
    bad[4, 0] = (bad[4, 0] & 0xFFFF) | (c_in << 16)     # input channel C
    ref, got = fwd(bad, False), fwd(bad, True)
    live = [c for c in range(c_out) if c not in (1, 4)]
    for a, b in zip(ref, got):
        assert torch.equal(a[:, live], b[:, live])
    assert torch.isnan(got[0][:, [1, 4]]).all()
    if complete:
        assert torch.isnan(got[1][:, [1, 4]]).all() and torch.isnan(got[2][:, [1, 4]]).all()
        assert (got[3][:, [1, 4]] == -1).all()


def test_module_regular_taps_cache_follows_the_selection():
    """ConvLogicLayer passes the guarantee only for a selection whose taps it has checked on
    the host; an in-place change of the selection is seen through its version."""
    torch.manual_seed(5)
    layer = cl.ConvLogicLayer(4, 8, stride=2, padding=1, kernel=3, complete=True).cuda()
    assert layer._regular_taps()
    with torch.no_grad():
        layer.selection[0, 0] = (layer.selection[0, 0] & ~0xFF00) | (3 << 8)
    assert not layer._regular_taps()
    x = torch.rand(2, 4, 12, 12, device="cuda")
    y = layer(x)   # the fix-up kernel computes the out-of-window channel
    ref = T.block_forward(np_(x).astype(np.float64),
                          np_(torch.softmax(layer.weights.detach().double(), -1)),
                          np_(layer.selection), (2, 2), (1, 1), (3, 3))[0]
    np.testing.assert_allclose(np_(y), ref, rtol=1e-5, atol=1e-6)


def test_module_with_warm_caches_pickles():
    """torch.save of a whole trained layer: the channel-use and regular-taps caches (weak
    references) are left out and rebuilt, and the loaded layer computes the same output."""
    import io
    torch.manual_seed(6)
    layer = cl.ConvLogicLayer(4, 8, stride=2, padding=1, kernel=3, complete=True).cuda()
    x = torch.rand(2, 4, 12, 12, device="cuda", requires_grad=True)
    layer(x).sum().backward()
    assert layer._uses is not None and layer._regular is not None
    buf = io.BytesIO()
    torch.save(layer, buf)
    buf.seek(0)
    other = torch.load(buf, weights_only=False)  # written by this test
    assert other._uses is None and other._regular is None
    with torch.no_grad():
        assert torch.equal(other(x), layer(x))
    other.eval()
    layer.eval()
    with torch.no_grad():
        assert torch.equal(other(x), layer(x))


def test_identity_init():
    layer = cl.ConvLogicLayer(2, 2, residual_init=True, complete=True).cuda().eval()
    assert bool((layer.weights.argmax(-1) == 3).all())
    x = (torch.rand(2, 2, 6, 6, device="cuda") < 0.5).float()
    # every node passes its first input: the block is the max over the window of tap 0
    y = layer(x)
    ch, r, c = TL.unpack_selection(layer.selection[:, 0].long())
    xp = torch.nn.functional.pad(x, (1, 1, 1, 1))
    for o in range(2):
        tap = xp[:, ch[o], r[o]:r[o] + 6, c[o]:c[o] + 6]
        assert torch.equal(y[:, o], torch.nn.functional.max_pool2d(tap, 2, 2))


@pytest.mark.parametrize("stride,pad", [(1, 1), (2, 2)])
def test_split_layers_vs_complete(stride, pad):
    torch.manual_seed(0)
    full = cl.ConvLogicLayer(3, 2, stride=stride, padding=pad, kernel=3, complete=True,
                             return_indices=True, return_intermediate=True).cuda()
    conv = cl.ConvLogicLayer(3, 2, stride=stride, padding=pad, kernel=3, complete=False).cuda()
    tree1 = cl.TreeLogicLayer(2, 4).cuda()
    tree2 = cl.TreeLogicLayer(2, 2).cuda()
    pool = cl.PoolLogicLayer(return_indices=True)
    conv.selection = full.selection
    with torch.no_grad():
        conv.weights.copy_(full.weights[:, 0:4])
        tree1.weights.copy_(full.weights[:, 4:6])
        tree2.weights.copy_(full.weights[:, 6:7])
    x = torch.randn(4, 3, 10, 10, device="cuda")
    with torch.no_grad():
        y_full, x1_full, x2_full, idx_full = full(x)
        x1 = conv(x)
        x2 = tree1(x1)
        y, idx = pool(tree2(x2))
    assert torch.equal(idx.flatten(start_dim=2).to(torch.int32), idx_full)
    torch.testing.assert_close(x1, x1_full, atol=1e-6, rtol=0)
    torch.testing.assert_close(x2, x2_full, atol=1e-6, rtol=0)
    torch.testing.assert_close(y, y_full, atol=1e-6, rtol=0)


def test_module_gradients_match_oracle():
    """Training mode through the module: the block's kernels on the logits (softmax and its
    backward in the kernels), and the gradients of the logits and the input against the oracle
    chained with the softmax Jacobian."""
    torch.manual_seed(9)
    layer = cl.ConvLogicLayer(4, 6, stride=2, padding=1, kernel=3, complete=True).cuda().double()
    x = torch.rand(3, 4, 12, 12, device="cuda", dtype=torch.float64, requires_grad=True)
    y = layer(x)
    gy = torch.randn_like(y)
    y.backward(gy)
    w_prob = torch.softmax(layer.weights.detach(), -1)
    rgx, rgw = T.block_backward(np_(x), np_(w_prob), np_(layer.selection), (2, 2), (1, 1), (3, 3),
                                np_(gy))
    np.testing.assert_allclose(np_(x.grad), rgx, rtol=1e-10, atol=1e-12)
    p = np_(w_prob)
    rgl = p * (rgw - (rgw * p).sum(-1, keepdims=True))
    np.testing.assert_allclose(np_(layer.weights.grad), rgl, rtol=1e-10, atol=1e-12)


def test_tree_layer_module_and_errors():
    layer = cl.TreeLogicLayer(3, 4).cuda()
    x = torch.rand(2, 3, 4, 4, 4, device="cuda", requires_grad=True)
    y = layer(x)
    assert y.shape == (2, 3, 4, 4, 2)
    y.sum().backward()
    assert x.grad is not None and layer.weights.grad.shape == (3, 2, 16)
    with pytest.raises(AssertionError):
        layer(torch.rand(2, 3, 4, 4, 6, device="cuda"))
    with pytest.raises(RuntimeError):
        TL.full_convlogic_forward(torch.rand(1, 1, 5, 5, device="cuda"),
                                  torch.rand(1, 7, 16, device="cuda"),
                                  torch.zeros(1, 8, dtype=torch.int32, device="cuda"),
                                  1, 1, 1, 1, 3, 3)            # H_out = 5 is odd
    with pytest.raises(ValueError):
        TL.channel_uses(torch.tensor([[5 << 16] * 8], dtype=torch.int32, device="cuda"), 3)
    with pytest.raises(ValueError):
        cl.ConvLogicLayer(2, 2, implementation="python")


def test_packed_tree_network_counts_match_float_eval():
    """A frozen tree network (two complete blocks, flatten, dense, GroupSum) evaluated on packed
    bits gives the class counts that the float eval gives as logits * tau (the
    counts == round(logits * tau) check of simulation/consistency.py:241)."""
    torch.manual_seed(11)
    blocks = [cl.ConvLogicLayer(3, 8, stride=2, padding=1, kernel=3, complete=True),
              cl.ConvLogicLayer(8, 16, stride=1, padding=1, kernel=3, complete=True)]
    model = torch.nn.Sequential(*blocks, torch.nn.Flatten(), cl.LogicLayer(64, 120),
                                cl.LogicLayer(120, 100), cl.GroupSum(5, 3.0)).cuda()
    for m in model:
        if isinstance(m, cl.LogicLayer):
            m.freeze()
    model.eval()
    n = 300
    bits = torch.rand((n, 3, 16, 16), device="cuda") < 0.5
    logits = model(bits.float())
    counts = model(cl.PackBitsTensor(bits.reshape(n, -1), 64))
    assert counts.dtype == torch.int32 and counts.shape == (n, 5)
    assert torch.equal(counts, torch.round(logits * 3.0).to(torch.int32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_feature_major_output_and_gradient_equal_the_nchw_ones(dtype):
    """cl_tree_conv_forward_softmax / _backward_softmax with y_rows: y is the [N, C, Hp, Wp] view
    of a [C*Hp*Wp, N] buffer holding bitwise the NCHW values, and a gradient in that layout
    gives bitwise the NCHW call's gradients (LDS-staged and global-gather shapes)."""
    for (n, c_in, h, w, c_out) in [(3, 4, 12, 12, 64), (5, 16, 8, 8, 24)]:
        stride, pad, kernel = (2, 2), (1, 1), (3, 3)
        x, _, sel = make(31, n, c_in, h, w, c_out, 3, dtype=dtype)
        logits = torch.randn((c_out, 7, 16), generator=torch.Generator().manual_seed(32),
                             dtype=torch.float64).to(x.device, dtype)
        y0, _, _, i0 = TL.full_convlogic_forward(x, logits, sel, *stride, *pad, *kernel,
                                                 intermediate=False, softmax=True)
        y1, _, _, i1 = TL.full_convlogic_forward(x, logits, sel, *stride, *pad, *kernel,
                                                 intermediate=False, softmax=True, y_rows=True)
        assert not y1.is_contiguous() and y1.permute(1, 2, 3, 0).is_contiguous()
        assert torch.equal(y0, y1) and torch.equal(i0, i1)
        gy = torch.randn(y0.shape, generator=torch.Generator().manual_seed(33),
                         dtype=torch.float64).to(x.device, dtype)
        gy_rows = gy.permute(1, 2, 3, 0).contiguous().permute(3, 0, 1, 2)
        g0 = TL.tree_conv_backward(gy, x, logits, sel, i0, *stride, *pad, *kernel, True,
                                   softmax=True)
        g1 = TL.tree_conv_backward(gy_rows, x, logits, sel, i1, *stride, *pad, *kernel, True,
                                   softmax=True)
        assert torch.equal(g0[0], g1[0]) and torch.equal(g0[1], g1[1])


def test_tree_network_with_feature_major_block_output_trains_identically():
    """The cfg3_tree-shaped network (blocks, Flatten, dense layers, GroupSum) with its last
    block's output feature-major gives bitwise the loss and gradients of the NCHW network: the
    flattened output reaches the dense layer as its rows, and the dense layer's input gradient
    reaches the block without a transpose."""
    from compactlogic_amd import configs
    cfg = configs.TreeConfig("small_tree", (3, 16, 16), [(32, 3, 2, 1), (48, 3, 2, 1)],
                             [400, 400], 64)
    net = configs.tree_network(cfg, device="cuda")
    assert net[1].rows_output
    x, labels = configs.conv_inputs(cfg, device="cuda")
    losses, grads = [], []
    for rows in (True, False):
        net[1].rows_output = rows
        net.zero_grad(set_to_none=True)
        loss = net[-1].cross_entropy(net[:-1](x), labels)
        loss.backward()
        losses.append(loss.detach())
        grads.append([p.grad.clone() for p in net.parameters()])
    assert torch.equal(losses[0], losses[1])
    assert all(torch.equal(a, b) for a, b in zip(*grads))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("stride,pad,kernel,shape,rows", [
    ((2, 2), (1, 1), (3, 3), (3, 16, 8, 8, 32), True),      # conv2 geometry, staged forward
    ((2, 2), (1, 1), (3, 3), (4, 9, 32, 32, 160), False),   # conv1 geometry, staged forward
    ((1, 1), (1, 1), (3, 3), (2, 5, 64, 64, 3), False),     # global-gather forward, big planes
])
def test_coefficient_handover_matches_the_separate_calls(dtype, stride, pad, kernel, shape, rows):
    """cl_tree_conv_forward_softmax_coefs writes each node's collapsed coefficients (checked
    against the oracle's collapse of softmax(logits)) and leaves the forward's outputs bitwise
    unchanged; cl_tree_conv_backward_softmax_coefs on them gives bitwise the gradients of the
    backward that forms them itself."""
    n, c_in, h, w, c_out = shape
    x, _, sel = make(21, n, c_in, h, w, c_out, kernel[0], dtype=dtype)
    g = torch.Generator().manual_seed(22)
    logits64 = 2.0 * torch.randn((c_out, 7, 16), generator=g, dtype=torch.float64)
    logits = logits64.to(x.device, dtype)
    y0, _, _, idx0 = TL.full_convlogic_forward(x, logits, sel, *stride, *pad, *kernel,
                                               intermediate=False, softmax=True, y_rows=rows)
    coefs = torch.full((c_out, 7, 4), float("nan"), dtype=dtype, device=x.device)
    y1, _, _, idx1 = TL.full_convlogic_forward(x, logits, sel, *stride, *pad, *kernel,
                                               intermediate=False, softmax=True, y_rows=rows,
                                               coefs=coefs)
    assert torch.equal(y0, y1) and torch.equal(idx0, idx1)
    want = T.collapse(np_(torch.softmax(logits64, -1)))
    np.testing.assert_allclose(np_(coefs), want, **tol(dtype))
    gy = torch.randn(y0.shape, generator=g, dtype=torch.float64).to(x.device, dtype)
    if rows:  # the feature-major gradient a flattened dense layer hands back
        gy = gy.permute(1, 2, 3, 0).contiguous().permute(3, 0, 1, 2)
    gx0, gw0 = TL.tree_conv_backward(gy, x, logits, sel, idx0, *stride, *pad, *kernel, True,
                                     softmax=True)
    gx1, gw1 = TL.tree_conv_backward(gy, x, logits, sel, idx0, *stride, *pad, *kernel, True,
                                     softmax=True, coefs=coefs)
    assert torch.equal(gx0, gx1) and torch.equal(gw0, gw1)
    with pytest.raises(ValueError):
        TL.tree_conv_backward(gy, x, logits, sel, idx0, *stride, *pad, *kernel, True,
                              softmax=False, coefs=coefs)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("shape", [(3, 16, 8, 8, 32), (2, 9, 32, 32, 24)])
def test_staged_backward_poisons_a_channel_reading_past_the_input(dtype, shape):
    """Weight gradient only (the network's first block): a channel with a tap on input channel
    C gets NaN logit gradients from the staged backward, as from the node pass; every other
    channel matches the oracle."""
    n, c_in, h, w, c_out = shape
    stride, pad, kernel = (2, 2), (1, 1), (3, 3)
    x, _, ok = make(41, n, c_in, h, w, c_out, 3, dtype=dtype)
    sel = ok.clone()
    sel[4, 3] = (sel[4, 3] & 0xFFFF) | (c_in << 16)
    logits64 = torch.randn((c_out, 7, 16), generator=torch.Generator().manual_seed(42),
                           dtype=torch.float64)
    logits = logits64.to(x.device, dtype)
    y, _, _, idx = TL.full_convlogic_forward(x, logits, sel, *stride, *pad, *kernel,
                                             intermediate=False, softmax=True)
    assert bool(torch.isnan(y[:, 4]).all())
    gy = torch.randn(y.shape, generator=torch.Generator().manual_seed(43),
                     dtype=torch.float64).to(x.device, dtype)
    gx, gl = TL.tree_conv_backward(gy, x, logits, sel, idx, *stride, *pad, *kernel, True,
                                   need_x=False, softmax=True)
    assert gx is None and bool(torch.isnan(gl[4]).all())
    live = [c for c in range(c_out) if c != 4]
    assert not bool(torch.isnan(gl[live]).any())
    p64 = np_(torch.softmax(logits64, -1))
    _, rgw = T.block_backward(np_(x).astype(np.float64), p64, np_(ok), stride, pad, kernel,
                              np_(gy).astype(np.float64), True, idx=np_(idx))
    rgl = p64 * (rgw - (rgw * p64).sum(-1, keepdims=True))
    scale = max(1.0, float(np.abs(rgw).max()))
    np.testing.assert_allclose(np_(gl)[live] / scale, rgl[live] / scale, **tol(dtype))


def test_cfg3_tree_blocks_at_full_size_match_oracle():
    """The cfg3_tree network's own blocks (logits, sampled taps) on Bernoulli inputs: conv2 at
    the benched batch of 256 through the staged backward with the input gradient, conv1 (the
    network's input: logits gradient only) on 32 of its samples, forward outputs and both
    gradients against the float64 oracle (winners compared away from near ties)."""
    from compactlogic_amd import configs
    cfg = configs.TREE_CONFIGS["cfg3_tree"]
    net = configs.tree_network(cfg, device="cuda")
    x, _ = configs.conv_inputs(cfg, device="cuda")
    stride, pad, kernel = (2, 2), (1, 1), (3, 3)
    with torch.no_grad():
        h1, _, _, _ = TL.full_convlogic_forward(x, net[0].weights, net[0].selection.int(),
                                                *stride, *pad, *kernel, intermediate=False,
                                                softmax=True)
    for blk, xin in ((net[0], x[:32].contiguous()), (net[2 if isinstance(net[1], torch.nn.Flatten) else 1], h1)):
        sel = blk.selection.int().contiguous()
        logits = blk.weights.detach().contiguous()
        first = blk is net[0]
        y, _, _, idx = TL.full_convlogic_forward(xin, logits, sel, *stride, *pad, *kernel,
                                                 intermediate=False, softmax=True)
        xs = np_(xin).astype(np.float64)
        p64 = np_(torch.softmax(logits.double(), -1))
        ss = np_(sel)
        ry, _, _, ridx = T.block_forward(xs, p64, ss, stride, pad, kernel)
        eps = float(np.finfo(np.float32).eps)
        free = _near_ties(_window_scores(xs, p64, ss, stride, pad, kernel), eps)
        assert np.array_equal(np_(idx)[~free], ridx[~free])
        np.testing.assert_allclose(np_(y), ry, rtol=1e-5, atol=1e-6)
        oidx = np.where(free, np_(idx), ridx)
        gy = torch.randn(y.shape, generator=torch.Generator().manual_seed(51),
                         dtype=torch.float64).to(xin.device, torch.float32)
        gx, gl = TL.tree_conv_backward(gy, xin, logits, sel, idx, *stride, *pad, *kernel, True,
                                       need_x=not first, softmax=True)
        rgx, rgw = T.block_backward(xs, p64, ss, stride, pad, kernel,
                                    np_(gy).astype(np.float64), True, idx=oidx)
        rgl = p64 * (rgw - (rgw * p64).sum(-1, keepdims=True))
        scale = max(1.0, float(np.abs(rgw).max()))
        np.testing.assert_allclose(np_(gl) / scale, rgl / scale, rtol=1e-5, atol=1e-6)
        if not first:
            np.testing.assert_allclose(np_(gx), rgx, rtol=1e-5, atol=1e-6)
