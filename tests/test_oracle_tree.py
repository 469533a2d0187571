"""Pins the CPU oracle of the logic-tree conv block (oracle/tree_np.py) against independent
formulations: the reference's 16 explicit gate polynomials with explicit tap loops
(third_party/convlogic_source_code/src/convlogic/convlogic_layer.py:236-321, the
forward_python_full pattern), torch's max_pool2d and torch autograd, and finite differences."""
import numpy as np
import pytest
import torch

from oracle import tree_np as T


def bin_op_s(a, b, p):
    """sum_i p[..., i] * op_i(a, b) with the difflogic gate polynomials, written out."""
    ab = a * b
    ops = [torch.zeros_like(a), ab, a - ab, a, b - ab, b, a + b - 2 * ab, a + b - ab,
           1 - (a + b - ab), 1 - (a + b - 2 * ab), 1 - b, 1 - b + ab, 1 - a, 1 - a + ab, 1 - ab,
           torch.ones_like(a)]
    return sum(p[..., i] * ops[i] for i in range(16))


def torch_block(x, w_prob, sel, stride, pad, kernel, complete=True):
    """Explicit-loop restatement in torch (differentiable): taps, gates, tree, max_pool2d."""
    n, c_in, h, w = x.shape
    c_out = sel.shape[0]
    ho, wo = T.out_hw(h, w, stride, pad, kernel)
    ch, ry, rx = (np.asarray(v) for v in T.unpack(sel))
    a = torch.zeros((n, c_out, ho, wo, 4), dtype=x.dtype)
    b = torch.zeros((n, c_out, ho, wo, 4), dtype=x.dtype)
    cols_a, cols_b = [], []
    for c in range(c_out):
        for p in range(4):
            for side, store in ((0, cols_a), (1, cols_b)):
                k = 2 * p + side
                plane = []
                for oy in range(ho):
                    row = []
                    for ox in range(wo):
                        iy = oy * stride[0] + ry[c, k] - pad[0]
                        ix = ox * stride[1] + rx[c, k] - pad[1]
                        if 0 <= iy < h and 0 <= ix < w:
                            row.append(x[:, ch[c, k], iy, ix])
                        else:
                            row.append(torch.zeros(n, dtype=x.dtype))
                    plane.append(torch.stack(row, -1))
                store.append(torch.stack(plane, -2))       # [N, Ho, Wo]
    a = torch.stack(cols_a, 1).view(n, c_out, 4, ho, wo).permute(0, 1, 3, 4, 2)
    b = torch.stack(cols_b, 1).view(n, c_out, 4, ho, wo).permute(0, 1, 3, 4, 2)
    wp = w_prob.view(1, c_out, 1, 1, -1, 16)
    x1 = bin_op_s(a, b, wp[..., 0:4, :])
    if not complete:
        return x1
    x2 = bin_op_s(x1[..., 0::2], x1[..., 1::2], wp[..., 4:6, :])
    x3 = bin_op_s(x2[..., 0::2], x2[..., 1::2], wp[..., 6:7, :])[..., 0]
    y, idx = torch.nn.functional.max_pool2d(x3, 2, 2, return_indices=True)
    return y, x1, x2, idx.flatten(start_dim=2)


def make(seed, n, c_in, h, w, c_out, kernel=3, complete=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.rand((n, c_in, h, w), generator=g, dtype=torch.float64)
    nodes = 7 if complete else 4
    w_prob = torch.softmax(torch.randn((c_out, nodes, 16), generator=g, dtype=torch.float64), -1)
    ch = torch.randint(0, c_in, (c_out, 8), generator=g)
    r = torch.randint(0, kernel, (c_out, 8), generator=g)
    cc = torch.randint(0, kernel, (c_out, 8), generator=g)
    sel = ((ch << 16) | (r << 8) | cc).to(torch.int32)
    return x, w_prob, sel


CASES = [((1, 1), (1, 1), (3, 3), (2, 3, 6, 6, 2)),
         ((2, 2), (2, 2), (3, 3), (2, 3, 10, 10, 3)),
         ((1, 1), (0, 0), (2, 2), (1, 2, 5, 5, 2)),
         ((2, 1), (1, 0), (3, 2), (2, 2, 11, 5, 2))]


@pytest.mark.parametrize("stride,pad,kernel,shape", CASES)
def test_block_forward_matches_explicit_polynomials_and_max_pool(stride, pad, kernel, shape):
    n, c_in, h, w, c_out = shape
    x, w_prob, sel = make(1, n, c_in, h, w, c_out, kernel[0])
    sel = sel.clone()
    if kernel[1] != kernel[0]:  # column offsets within the kernel width
        sel = (sel & ~0xFF) | (sel & 0xFF) % kernel[1]
    ho, wo = T.out_hw(h, w, stride, pad, kernel)
    if ho % 2 or wo % 2:
        pytest.skip("pooling needs even conv output sizes")
    y, x2, x3, idx = T.block_forward(x.numpy(), w_prob.numpy(), sel.numpy(), stride, pad, kernel)
    ry, rx2, rx3, ridx = torch_block(x, w_prob, sel, stride, pad, kernel)
    np.testing.assert_allclose(x2, rx2.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(x3, rx3.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(y, ry.numpy(), rtol=1e-12, atol=1e-12)
    assert np.array_equal(idx, ridx.numpy())
    g = T.block_forward(x.numpy(), w_prob[:, :4].numpy(), sel.numpy(), stride, pad, kernel, False)
    np.testing.assert_allclose(g, torch_block(x, w_prob[:, :4], sel, stride, pad, kernel,
                                              False).numpy(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("complete", [True, False])
@pytest.mark.parametrize("stride,pad,kernel,shape", CASES[:2])
def test_block_backward_matches_autograd(stride, pad, kernel, shape, complete):
    n, c_in, h, w, c_out = shape
    x, w_prob, sel = make(2, n, c_in, h, w, c_out, kernel[0], complete)
    xx = x.clone().requires_grad_(True)
    ww = w_prob.clone().requires_grad_(True)
    out = torch_block(xx, ww, sel, stride, pad, kernel, complete)
    y = out[0] if complete else out
    gy = torch.randn(y.shape, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    y.backward(gy)
    gx, gw = T.block_backward(x.numpy(), w_prob.numpy(), sel.numpy(), stride, pad, kernel,
                              gy.numpy(), complete)
    np.testing.assert_allclose(gx, xx.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(gw, ww.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_block_backward_finite_differences():
    stride, pad, kernel = (1, 1), (1, 1), (3, 3)
    x, w_prob, sel = make(4, 1, 2, 4, 4, 2)
    gy = np.random.default_rng(5).standard_normal((1, 2, 2, 2))
    gx, _ = T.block_backward(x.numpy(), w_prob.numpy(), sel.numpy(), stride, pad, kernel, gy)
    f = lambda xv: float((T.block_forward(xv, w_prob.numpy(), sel.numpy(), stride, pad,
                                          kernel)[0] * gy).sum())
    xv = x.numpy().copy()
    eps = 1e-6
    for i in range(xv.size):
        d = np.zeros(xv.size)
        d[i] = eps
        num = (f(xv + d.reshape(xv.shape)) - f(xv - d.reshape(xv.shape))) / (2 * eps)
        assert abs(num - gx.reshape(-1)[i]) < 1e-6


def test_level_matches_autograd():
    g = torch.Generator().manual_seed(6)
    x = torch.rand((2, 3, 4, 5, 4), generator=g, dtype=torch.float64, requires_grad=True)
    w_prob = torch.softmax(torch.randn((3, 2, 16), generator=g, dtype=torch.float64), -1)
    w_prob.requires_grad_(True)
    y = bin_op_s(x[..., 0::2], x[..., 1::2], w_prob.view(1, 3, 1, 1, 2, 16))
    np.testing.assert_allclose(T.level_forward(x.detach().numpy(), w_prob.detach().numpy()),
                               y.detach().numpy(), rtol=1e-12, atol=1e-12)
    gy = torch.randn(y.shape, generator=g, dtype=torch.float64)
    y.backward(gy)
    gx, gw = T.level_backward(x.detach().numpy(), w_prob.detach().numpy(), gy.numpy())
    np.testing.assert_allclose(gx, x.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(gw, w_prob.grad.numpy(), rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("complete", [True, False])
def test_block_bits_matches_float_block_on_one_hot(complete):
    rng = np.random.default_rng(7)
    n, c_in, h, w, c_out = 64, 3, 6, 6, 3
    stride, pad, kernel = (1, 1), (1, 1), (3, 3)
    nodes = 7 if complete else 4
    bits = rng.integers(0, 2, (n, c_in, h, w)).astype(np.float64)
    gates = rng.integers(0, 16, (c_out, nodes))
    w_prob = np.eye(16)[gates]
    _, _, sel = make(8, 1, c_in, h, w, c_out)
    ref = T.block_forward(bits, w_prob, sel.numpy(), stride, pad, kernel, complete)
    ref = ref[0] if complete else ref
    # pack the samples: bit j of word 0 is sample j
    words = np.zeros((c_in * h * w, 1), dtype=np.uint64)
    flat = bits.reshape(n, -1).astype(np.uint64)
    for j in range(n):
        words[:, 0] |= flat[j] << np.uint64(j)
    out = T.block_bits(words, gates, sel.numpy(), (c_in, h, w), stride, pad, kernel, complete)
    got = np.stack([(out[:, 0] >> np.uint64(j)) & np.uint64(1) for j in range(n)])
    assert np.array_equal(got.astype(np.float64), ref.reshape(n, -1))


def test_cpu_baseline_tree_block_matches_oracle():
    """The torch CPU block timed as the CPU baseline (oracle/torch_cpu.py) is the oracle's
    function: values and input gradient."""
    from oracle import torch_cpu as TC
    stride, pad, kernel = (2, 2), (1, 1), (3, 3)
    x, w_prob, sel = make(11, 2, 3, 10, 10, 4)
    logits = torch.log(w_prob)                       # softmax(log p) = p
    xx = x.clone().requires_grad_(True)
    y = TC.tree_block_forward(xx, logits, sel, stride, pad, kernel)
    ry = T.block_forward(x.numpy(), w_prob.numpy(), sel.numpy(), stride, pad, kernel)[0]
    np.testing.assert_allclose(y.detach().numpy(), ry, rtol=1e-12, atol=1e-12)
    gy = np.random.default_rng(12).standard_normal(ry.shape)
    y.backward(torch.as_tensor(gy))
    gx, _ = T.block_backward(x.numpy(), w_prob.numpy(), sel.numpy(), stride, pad, kernel, gy)
    np.testing.assert_allclose(xx.grad.numpy(), gx, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("shape,stride,pad,kernel", [((9, 16, 16), (2, 2), (1, 1), (3, 3)),
                                                     ((3, 6, 6), (1, 1), (1, 1), (3, 3)),
                                                     ((4, 8, 8), (2, 2), (0, 0), (2, 2))])
def test_c_tree_block_matches_numpy_bits(shape, stride, pad, kernel):
    """The C restatement (oracle/packed_ref.c, timed as the packed CPU baseline) equals the
    numpy bit evaluator, which is pinned against the float block above."""
    from oracle import packed as P
    rng = np.random.default_rng(13)
    c_in, h, w = shape
    c_out = 5
    xw = rng.integers(0, 2**63, (c_in * h * w, 3), dtype=np.int64).view(np.uint64)
    gates = rng.integers(0, 16, (c_out, 7)).astype(np.uint8)
    _, _, sel = make(14, 1, c_in, h, w, c_out, kernel[0])
    sel = sel.numpy()
    if kernel[1] != kernel[0]:
        sel = (sel & ~0xFF) | (sel & 0xFF) % kernel[1]
    ref = T.block_bits(xw, gates, sel, shape, stride, pad, kernel, True)
    assert np.array_equal(P.tree_block_bits(xw, gates, sel, shape, stride, pad, kernel), ref)
