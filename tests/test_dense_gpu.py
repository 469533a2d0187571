"""Dense LogicLayer kernels against the float64 CPU oracle.

Tolerance (north star): fp32 results within rtol 1e-5 / atol 1e-6 of the float64 oracle; the
upstream gradients are drawn at the scale of a mean-reduced loss (|gy| <= 1/batch) so batch
reductions stay O(1).  fp64 results within rtol 1e-10 / atol 1e-12.
"""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl
from compactlogic_amd import difflogic_hip as dl
from oracle import logic_np as O

pytestmark = pytest.mark.gpu

TOL = {torch.float32: dict(rtol=1e-5, atol=1e-6), torch.float64: dict(rtol=1e-10, atol=1e-12)}


def np_(t):
    return t.detach().cpu().numpy()


def make_layer(seed, in_dim, out_dim, g_n, batch, shared=False, binary_x=False):
    rng = np.random.default_rng(seed)
    if shared:
        a = np.repeat(rng.integers(0, in_dim, out_dim)[:, None], g_n, 1)
        b = np.repeat(rng.integers(0, in_dim, out_dim)[:, None], g_n, 1)
    else:
        a = rng.integers(0, in_dim, (out_dim, g_n))
        b = rng.integers(0, in_dim, (out_dim, g_n))
        # a few neurons with partially shared pairs, so runs of several lengths occur
        for o in range(0, out_dim, 5):
            a[o, : g_n // 2] = a[o, 0]
            b[o, : g_n // 2] = b[o, 0]
    gs = rng.integers(0, 16, (out_dim, g_n)).astype(np.uint8)
    logits = rng.standard_normal((out_dim, g_n))
    w = np.exp(logits) / np.exp(logits).sum(1, keepdims=True)
    x = rng.integers(0, 2, (in_dim, batch)).astype(np.float64) if binary_x else rng.random((in_dim, batch))
    gy = rng.uniform(-1, 1, (out_dim, batch)) / max(batch, 1)
    return dict(x=x, a=a, b=b, gs=gs, w=w, gy=gy)


def to_dev(L, device, dtype):
    t = lambda v, dt: torch.as_tensor(v).to(device=device, dtype=dt).contiguous()
    return dict(x=t(L["x"], dtype), a=t(L["a"], torch.int64), b=t(L["b"], torch.int64),
                gs=t(L["gs"], torch.uint8), w=t(L["w"], dtype), gy=t(L["gy"], dtype))


SHAPES = [
    # in, out, G, batch, shared
    (8, 64, 16, 1, False),
    (23, 37, 4, 3, False),
    (50, 40, 1, 64, False),
    (100, 120, 16, 130, True),
    (300, 256, 16, 1024, True),
    (64, 80, 8, 2500, False),
    (784, 500, 16, 128, True),
    (40, 30, 128, 40, False),
    (1000, 600, 16, 4096, True),
    # single-run neurons with 8- and 4-lane groups (the fused forward), a partial last chunk
    (200, 150, 16, 256, True),
    (60, 70, 5, 200, True),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("shape", SHAPES)
def test_dropin_kernels_match_oracle(device, dtype, shape):
    in_dim, out_dim, g_n, batch, shared = shape
    L = make_layer(hash(shape) % 1000, in_dim, out_dim, g_n, batch, shared)
    D = to_dev(L, device, dtype)
    y = dl.forward(D["x"], D["a"], D["b"], D["w"], D["gs"])
    np.testing.assert_allclose(np_(y), O.dense_forward(L["x"], L["a"], L["b"], L["w"], L["gs"]),
                               **TOL[dtype])
    gw = dl.backward_w(D["x"], D["a"], D["b"], D["gs"], D["gy"])
    np.testing.assert_allclose(np_(gw), O.dense_backward_w(L["x"], L["a"], L["b"], L["gs"], L["gy"]),
                               **TOL[dtype])
    start, yidx, code = O.backward_index(np.stack([L["a"], L["b"]]), in_dim)
    gx = dl.backward_x(D["x"], D["a"], D["b"], D["w"], D["gs"], D["gy"],
                       torch.as_tensor(start, device=device), torch.as_tensor(yidx, device=device),
                       torch.as_tensor(code, device=device))
    np.testing.assert_allclose(np_(gx), O.dense_backward_x_direct(L["x"], L["a"], L["b"], L["w"],
                                                                 L["gs"], L["gy"]), **TOL[dtype])
    # the index-free variant builds its own index and gathers through it
    gx2 = dl.backward_x_atomicAdd(D["x"], D["a"], D["b"], D["w"], D["gs"], D["gy"])
    np.testing.assert_allclose(np_(gx2), np_(gx), **TOL[dtype])


@pytest.mark.parametrize("shape", SHAPES)
def test_dropin_kernels_half_match_oracle(device, shape):
    """float16 storage, as the reference dispatches these kernels over half
    (difflogic_kernel.cu:222,267,315,397): the oracle runs in float64 on the half-rounded
    inputs; the kernels sum in fp32 and round once, so the results stay within a few half
    ulps (rtol 2e-3) of it."""
    in_dim, out_dim, g_n, batch, shared = shape
    L = make_layer(hash(shape) % 1000 + 7, in_dim, out_dim, g_n, batch, shared)
    half = {k: torch.as_tensor(L[k]).half() for k in ("x", "w", "gy")}
    R = dict(L, **{k: v.double().numpy() for k, v in half.items()})
    D = to_dev(L, device, torch.float16)
    for k, v in half.items():
        D[k] = v.to(device).contiguous()
    y = dl.forward(D["x"], D["a"], D["b"], D["w"], D["gs"])
    assert y.dtype == torch.float16
    np.testing.assert_allclose(np_(y).astype(np.float64),
                               O.dense_forward(R["x"], R["a"], R["b"], R["w"], R["gs"]),
                               rtol=2e-3, atol=1e-3)
    gw = dl.backward_w(D["x"], D["a"], D["b"], D["gs"], D["gy"])
    rgw = O.dense_backward_w(R["x"], R["a"], R["b"], R["gs"], R["gy"])
    np.testing.assert_allclose(np_(gw).astype(np.float64), rgw, rtol=2e-3,
                               atol=2e-3 * max(1e-3, float(np.abs(rgw).max())))
    start, yidx, code = O.backward_index(np.stack([L["a"], L["b"]]), in_dim)
    gx = dl.backward_x(D["x"], D["a"], D["b"], D["w"], D["gs"], D["gy"],
                       torch.as_tensor(start, device=device), torch.as_tensor(yidx, device=device),
                       torch.as_tensor(code, device=device))
    rgx = O.dense_backward_x_direct(R["x"], R["a"], R["b"], R["w"], R["gs"], R["gy"])
    np.testing.assert_allclose(np_(gx).astype(np.float64), rgx, rtol=2e-3,
                               atol=2e-3 * max(1e-4, float(np.abs(rgx).max())))
    # the discrete eval on {0, 1} inputs is exact in half
    xb = (D["x"] > 0.5).half()
    slot = torch.as_tensor(np.random.default_rng(1).integers(0, g_n, out_dim).astype(np.uint8),
                           device=device)
    assert torch.equal(dl.eval(xb, D["a"], D["b"], slot, D["gs"]).float(),
                       dl.eval(xb.float(), D["a"], D["b"], slot, D["gs"]))


def test_half_logic_layer_trains_through_the_reference_kernels(device):
    """A LogicLayer fed float16 (fp32 logits, as the reference's forward_cuda casts its softmax
    to the input dtype) runs the half kernels forward and backward; a float32 copy of the same
    network gives the same loss and gradients within half rounding."""
    torch.manual_seed(4)
    net = torch.nn.Sequential(cl.LogicLayer(96, 300), cl.LogicLayer(300, 200),
                              cl.GroupSum(10, 4.0)).to(device)
    x = (torch.rand((256, 96), device=device) < 0.5).float()
    y = torch.randint(0, 10, (256,), device=device)
    loss32 = torch.nn.functional.cross_entropy(net(x), y)
    loss32.backward()
    g32 = [m.weights.grad.clone() for m in net[:2]]
    net.zero_grad(set_to_none=True)
    out16 = net(x.half())
    assert out16.dtype == torch.float16
    loss16 = torch.nn.functional.cross_entropy(out16.float(), y)
    loss16.backward()
    np.testing.assert_allclose(float(loss16.detach()), float(loss32.detach()), rtol=2e-3)
    for m, ref in zip(net[:2], g32):
        scale = float(ref.abs().max())
        np.testing.assert_allclose(np_(m.weights.grad), np_(ref), rtol=2e-2, atol=2e-2 * scale)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("shape", SHAPES)
def test_run_plan_kernels_match_oracle(device, dtype, shape):
    in_dim, out_dim, g_n, batch, shared = shape
    L = make_layer(hash(shape) % 1000 + 1, in_dim, out_dim, g_n, batch, shared)
    D = to_dev(L, device, dtype)
    plan = cl.build_run_plan(torch.stack([D["a"], D["b"]]), in_dim)
    x = D["x"].clone().requires_grad_(True)
    w = D["w"].clone().requires_grad_(True)
    y = cl.LogicLayerRunsFunction.apply(x, w, D["gs"], plan)
    np.testing.assert_allclose(np_(y), O.dense_forward(L["x"], L["a"], L["b"], L["w"], L["gs"]),
                               **TOL[dtype])
    gx, gw = torch.autograd.grad(y, (x, w), D["gy"])
    np.testing.assert_allclose(np_(gw), O.dense_backward_w(L["x"], L["a"], L["b"], L["gs"], L["gy"]),
                               **TOL[dtype])
    np.testing.assert_allclose(np_(gx), O.dense_backward_x_direct(L["x"], L["a"], L["b"], L["w"],
                                                                 L["gs"], L["gy"]), **TOL[dtype])
    # weight gradient alone (input needs no grad: the unfused per-neuron kernel)
    w2 = D["w"].clone().requires_grad_(True)
    y2 = cl.LogicLayerRunsFunction.apply(D["x"], w2, D["gs"], plan)
    (gw2,) = torch.autograd.grad(y2, (w2,), D["gy"])
    np.testing.assert_allclose(np_(gw2), np_(gw), **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("shape", SHAPES)
def test_run_plan_softmax_path_matches_oracle(device, dtype, shape):
    """Logits in, softmax inside the kernels: forward and the gradient of the logits."""
    in_dim, out_dim, g_n, batch, shared = shape
    L = make_layer(hash(shape) % 1000 + 2, in_dim, out_dim, g_n, batch, shared)
    D = to_dev(L, device, dtype)
    logits = np.log(L["w"]) + np.random.default_rng(3).standard_normal((out_dim, 1))
    lt = torch.as_tensor(logits, dtype=dtype, device=device).requires_grad_(True)
    plan = cl.build_run_plan(torch.stack([D["a"], D["b"]]), in_dim)
    x = D["x"].clone().requires_grad_(True)
    y = cl.LogicLayerRunsFunction.apply(x, lt, D["gs"], plan, True)
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    np.testing.assert_allclose(np_(y), O.dense_forward(L["x"], L["a"], L["b"], p, L["gs"]), **TOL[dtype])
    gx, gl = torch.autograd.grad(y, (x, lt), D["gy"])
    gp = O.dense_backward_w(L["x"], L["a"], L["b"], L["gs"], L["gy"])
    np.testing.assert_allclose(np_(gl), p * (gp - (p * gp).sum(1, keepdims=True)), **TOL[dtype])
    np.testing.assert_allclose(np_(gx), O.dense_backward_x_direct(L["x"], L["a"], L["b"], p,
                                                                 L["gs"], L["gy"]), **TOL[dtype])


def test_eval_matches_truth_table(device):
    L = make_layer(5, 40, 70, 6, 97, binary_x=True)
    D = to_dev(L, device, torch.float32)
    slot = np.random.default_rng(5).integers(0, 6, 70).astype(np.uint8)
    y = dl.eval(D["x"], D["a"], D["b"], torch.as_tensor(slot, device=device), D["gs"])
    assert np.array_equal(np_(y), O.dense_eval(L["x"], L["a"], L["b"], slot, L["gs"]))


def test_all_gates_known_answer_through_module(device):
    """third_party/convlogic_source_code/tests/difflogic/test_difflogic_forward.py:74-100 on
    the module path: one-hot logits select gate g for rows 4g..4g+3."""
    layer = cl.LogicLayer(8, 64, num_gates=16).to(device)
    pairs = torch.tensor([[0, 1], [2, 3], [4, 5], [6, 7]], device=device).repeat(16, 1)
    with torch.no_grad():
        layer.indices.copy_(pairs.t().unsqueeze(-1).expand(2, 64, 16))
        logits = torch.full((64, 16), float("-inf"), device=device)
        for g in range(16):
            logits[4 * g: 4 * g + 4, g] = 0.0
        layer.weights.copy_(logits)
    flat = [0.0, 0.0, 0.0, 1.0, 1.0, 0.0, 1.0, 1.0]
    y = layer(torch.tensor([flat], device=device))
    expected = [O.TRUTH[g, 2 * int(flat[p]) + int(flat[p + 1])] for g in range(16) for p in (0, 2, 4, 6)]
    assert torch.equal(y.cpu(), torch.tensor([expected], dtype=torch.float32))
    layer.eval()
    assert torch.equal(layer(torch.tensor([flat], device=device)).cpu(),
                       torch.tensor([expected], dtype=torch.float32))


def test_module_paths_agree_and_are_deterministic(device):
    torch.manual_seed(7)
    layer = cl.LogicLayer(200, 300, num_gates=16).to(device)
    x = torch.rand(96, 200, device=device, requires_grad=True)
    gy = torch.randn(96, 300, device=device) / 96

    def run_module():
        layer.weights.grad = None
        xx = x.detach().clone().requires_grad_(True)
        y = layer(xx)
        y.backward(gy)
        return y.detach(), xx.grad, layer.weights.grad.clone()

    def run_reference_function():
        layer.weights.grad = None
        xx = x.detach().clone().requires_grad_(True)
        w = torch.softmax(layer.weights, -1)
        y = cl.LogicLayerCudaFunction.apply(
            xx.t().contiguous(), layer.indices[0], layer.indices[1], w, layer.gate_sequence,
            layer.given_x_indices_of_y_start, layer.given_x_indices_of_y,
            layer.given_x_indices_of_gate).t()
        y.backward(gy)
        return y.detach(), xx.grad, layer.weights.grad.clone()

    r1, r2, r3 = run_module(), run_module(), run_reference_function()
    for u, v in zip(r1, r2):
        assert torch.equal(u, v), "module path is not bitwise deterministic"
    for u, v in zip(r1, r3):
        torch.testing.assert_close(u, v, rtol=1e-5, atol=1e-6)


def test_gradcheck_fp64(device):
    L = make_layer(11, 9, 7, 4, 5)
    D = to_dev(L, device, torch.float64)
    plan = cl.build_run_plan(torch.stack([D["a"], D["b"]]), 9)
    x = D["x"].clone().requires_grad_(True)
    w = D["w"].clone().requires_grad_(True)
    assert torch.autograd.gradcheck(lambda xx, ww: cl.LogicLayerRunsFunction.apply(xx, ww, D["gs"], plan),
                                    (x, w), eps=1e-6, atol=1e-8)
    start, yidx, code = (torch.as_tensor(v, device=device)
                         for v in O.backward_index(np.stack([L["a"], L["b"]]), 9))
    assert torch.autograd.gradcheck(
        lambda xx, ww: cl.LogicLayerCudaFunction.apply(xx, D["a"], D["b"], ww, D["gs"], start, yidx, code),
        (x, w), eps=1e-6, atol=1e-8)


def test_invalid_indices_poison_instead_of_faulting(device):
    L = make_layer(12, 10, 8, 4, 16)
    D = to_dev(L, device, torch.float32)
    a = D["a"].clone()
    a[3, 1] = 10_000
    y = dl.forward(D["x"], a, D["b"], D["w"], D["gs"])
    assert torch.isnan(y[3]).all() and not torch.isnan(y[torch.arange(8) != 3]).any()


def test_empty_batch_and_zero_width(device):
    L = make_layer(13, 10, 6, 4, 0)
    D = to_dev(L, device, torch.float32)
    assert dl.forward(D["x"], D["a"], D["b"], D["w"], D["gs"]).shape == (6, 0)
    gw = dl.backward_w(D["x"], D["a"], D["b"], D["gs"], D["gy"])
    assert torch.equal(gw, torch.zeros_like(gw))


def test_rewiring_keeps_training_path_consistent(device):
    torch.manual_seed(8)
    layer = cl.LogicLayer(30, 40).to(device)
    with torch.no_grad():
        layer.weights[:10] = 0.0
    layer.resample_connections(torch.arange(10, device=device), threshold_low=0.5)
    x = torch.rand(16, 30, device=device)
    y = layer(x)
    ref = O.dense_forward(np_(x).T, np_(layer.indices[0]), np_(layer.indices[1]),
                          np_(torch.softmax(layer.weights, -1)), np_(layer.gate_sequence))
    np.testing.assert_allclose(np_(y).T, ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("batch", [1, 37, 200, 256, 1024])
def test_fused_forward_matches_separate_prep(device, batch):
    """cl_dense_forward_fused (softmax + collapse inside the forward) against cl_dense_prep +
    cl_dense_forward_tiled: the same outputs, probabilities, inverse-index coefficients and
    gradients, to rounding."""
    torch.manual_seed(21)
    layer = cl.LogicLayer(300, 260, num_gates=16, connections="original").to(device)
    plan = layer.run_plan()
    assert plan.single_run
    x = torch.rand(batch, 300, device=device)
    gy = torch.randn(batch, 260, device=device) / batch
    outs = []
    for fused in (True, False):
        cl.LogicLayerRunsFunction.fused_forward = fused
        try:
            layer.weights.grad = None
            xx = x.clone().requires_grad_(True)
            y = layer(xx)
            y.backward(gy)
            outs.append((y.detach(), xx.grad, layer.weights.grad.clone()))
        finally:
            cl.LogicLayerRunsFunction.fused_forward = True
    for u, v in zip(*outs):
        torch.testing.assert_close(u, v, rtol=1e-6, atol=1e-7)
    ref = O.dense_forward(np_(x).T.astype(np.float64), np_(layer.indices[0]), np_(layer.indices[1]),
                          np_(torch.softmax(layer.weights.double(), -1)), np_(layer.gate_sequence))
    np.testing.assert_allclose(np_(outs[0][0]).T, ref, rtol=1e-5, atol=1e-6)


def test_fused_forward_entry_point_checks(device):
    import ctypes
    from compactlogic_amd import _capi
    L = make_layer(31, 20, 12, 16, 64, shared=True)
    D = to_dev(L, device, torch.float32)
    plan = cl.build_run_plan(torch.stack([D["a"], D["b"]]), 20)
    probs = torch.empty_like(D["w"])
    inv = torch.empty((2 * plan.num_runs, 2), device=device)
    y = torch.empty((12, 64), device=device)
    stream = torch.cuda.current_stream().cuda_stream
    lib = _capi.load()

    def call(batch, gates):
        return lib.cl_dense_forward_fused(0, D["x"].data_ptr(), D["w"].data_ptr(), 0,
                                          D["gs"].data_ptr(), plan.nab.data_ptr(),
                                          plan.inv_pos.data_ptr(), probs.data_ptr(),
                                          inv.data_ptr(), y.data_ptr(), 20, 12, plan.num_runs,
                                          batch, gates, stream)

    assert call(64, 17) != 0 and b"16 slots" in lib.cl_last_error()
    assert call(0, 16) != 0
    assert call(64, 16) == 0
    torch.cuda.synchronize()
    np.testing.assert_allclose(np_(y), O.dense_forward(L["x"], L["a"], L["b"], L["w"], L["gs"]),
                               rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(np_(probs), L["w"].astype(np.float32))
    # a neuron whose plan record claims two runs is poisoned, never mis-computed
    nab = plan.nab.clone()
    nab[3, 3] += 1
    plan.nab, saved = nab, plan.nab
    try:
        assert call(64, 16) == 0
    finally:
        plan.nab = saved
    torch.cuda.synchronize()
    assert torch.isnan(y[3]).all() and not torch.isnan(y[torch.arange(12) != 3]).any()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("shape", [(1, 1), (3, 70), (130, 65), (64, 64), (1024, 784), (256, 25088)])
def test_transpose_kernel_is_exact(device, dtype, shape):
    x = torch.randn(shape, dtype=dtype, device=device)
    t = cl.layers.TransposeFunction.apply(x)
    assert t.is_contiguous() and torch.equal(t, x.t())
    xg = x.clone().requires_grad_(True)
    g = torch.randn(shape[1], shape[0], dtype=dtype, device=device)
    cl.layers.TransposeFunction.apply(xg).backward(g)
    assert torch.equal(xg.grad, g.t())


def test_layer_input_layout_change_keeps_gradients(device):
    """A LogicLayer fed a contiguous [batch, in] tensor (transposed by the HIP kernel) and one
    fed the transpose of a contiguous [in, batch] tensor (a view, no kernel) agree bitwise."""
    torch.manual_seed(23)
    layer = cl.LogicLayer(130, 90, connections="original").to(device)
    x = torch.rand(70, 130, device=device)
    gy = torch.randn(70, 90, device=device)
    grads = []
    for xin in (x.clone(), x.t().contiguous().t()):
        xin.requires_grad_(True)
        layer.weights.grad = None
        layer(xin).backward(gy)
        grads.append((xin.grad.clone(), layer.weights.grad.clone()))
    for u, v in zip(*grads):
        assert torch.equal(u, v)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("shape", [(3000, 1600, 16, 1024), (20, 300, 4, 256), (500, 400, 8, 96),
                                   (1200, 1000, 1, 37), (64, 64, 16, 2048)])
def test_partitioned_backward_matches_untiled(device, dtype, shape):
    """cl_dense_backward_part (internal runs through LDS) against cl_dense_backward_tiled:
    the same input gradient and logits gradient to rounding, both against the oracle, and
    bitwise reproducible.  Shapes cover full tiles (more internal runs than LDS slots),
    self-pairs, multi-slot runs, 4- to 16-lane groups and a partial last chunk."""
    in_dim, out_dim, g_n, batch = shape
    g = torch.Generator().manual_seed(sum(shape))
    idx = torch.randint(0, in_dim, (2, out_dim, g_n), generator=g)
    idx[:, ::3] = idx[:, ::3, :1]
    idx[1, ::7] = idx[0, ::7]
    idx = idx.to(device)
    plan = cl.build_run_plan(idx.contiguous(), in_dim)
    assert int(plan.tile_ptr[-1]) > 0
    logits = torch.randn(out_dim, g_n, generator=g).to(device=device, dtype=dtype)
    gs = torch.randint(0, 16, (out_dim, g_n), generator=g).to(device=device, dtype=torch.uint8)
    x0 = torch.rand(in_dim, batch, generator=g).to(device=device, dtype=dtype)
    gy = (torch.rand(out_dim, batch, generator=g) - 0.5).to(device=device, dtype=dtype) / batch
    outs = []
    default = cl.LogicLayerRunsFunction.partitioned_backward
    for part in (True, True, False):
        cl.LogicLayerRunsFunction.partitioned_backward = part
        try:
            x = x0.clone().requires_grad_(True)
            w = logits.clone().requires_grad_(True)
            y = cl.LogicLayerRunsFunction.apply(x, w, gs, plan, True)
            outs.append(torch.autograd.grad(y, (x, w), gy))
        finally:
            cl.LogicLayerRunsFunction.partitioned_backward = default
    for u, v in zip(outs[0], outs[1]):
        assert torch.equal(u, v), "partitioned backward is not bitwise deterministic"
    tol = dict(rtol=1e-6, atol=1e-7) if dtype == torch.float32 else dict(rtol=1e-12, atol=1e-14)
    for u, v in zip(outs[0], outs[2]):
        torch.testing.assert_close(u, v, **tol)
    a, b = idx[0].cpu().numpy(), idx[1].cpu().numpy()
    p = torch.softmax(logits.double(), -1).cpu().numpy()
    gyn = gy.double().cpu().numpy()
    xn = x0.double().cpu().numpy()
    gp = O.dense_backward_w(xn, a, b, gs.cpu().numpy(), gyn)
    np.testing.assert_allclose(np_(outs[0][1]), p * (gp - (p * gp).sum(1, keepdims=True)),
                               **TOL[dtype])
    np.testing.assert_allclose(np_(outs[0][0]), O.dense_backward_x_direct(xn, a, b, p, gs.cpu().numpy(), gyn),
                               **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("batch,g_n,softmax,in_dim,out_dim", [
    (4, 16, True, 700, 900), (256, 16, True, 700, 900), (1024, 16, True, 700, 900),
    (2048, 5, False, 700, 900), (100, 40, True, 700, 900), (1024, 1, False, 700, 900),
    # many entries per input row: two (about 8 per row) or four (about 27) waves share a row
    (256, 16, True, 500, 2000), (1000, 16, True, 300, 4000), (4, 5, False, 300, 4000),
    (1024, 1, False, 37, 3000)])
def test_row_backward_matches_chunked(device, dtype, batch, g_n, softmax, in_dim, out_dim):
    """cl_dense_backward_rows (one wave per input row, or several sharing a row with many
    entries; finalize inside) against the chunked backward + finalize: the same input and
    logits gradients to rounding, both against the oracle, bitwise reproducible.  Batches above
    the row kernel's limit fall back."""
    g = torch.Generator().manual_seed(batch + g_n)
    pair = torch.randint(0, in_dim, (2, out_dim, 1), generator=g)
    pair[1, ::9] = pair[0, ::9]                       # self-pairs
    idx = pair.expand(2, out_dim, g_n).contiguous().to(device)
    plan = cl.build_run_plan(idx, in_dim)
    assert plan.single_run
    w0 = torch.randn(out_dim, g_n, generator=g).to(device=device, dtype=dtype)
    if not softmax:
        w0 = torch.softmax(w0, -1)
    gs = torch.randint(0, 16, (out_dim, g_n), generator=g).to(device=device, dtype=torch.uint8)
    x0 = torch.rand(in_dim, batch, generator=g).to(device=device, dtype=dtype)
    gy = (torch.rand(out_dim, batch, generator=g) - 0.5).to(device=device, dtype=dtype) / batch
    outs = []
    default = cl.LogicLayerRunsFunction.row_backward
    for rows in (True, True, False):
        cl.LogicLayerRunsFunction.row_backward = rows
        try:
            x = x0.clone().requires_grad_(True)
            w = w0.clone().requires_grad_(True)
            y = cl.LogicLayerRunsFunction.apply(x, w, gs, plan, softmax)
            outs.append(torch.autograd.grad(y, (x, w), gy))
        finally:
            cl.LogicLayerRunsFunction.row_backward = default
    for u, v in zip(outs[0], outs[1]):
        assert torch.equal(u, v), "row backward is not bitwise deterministic"
    tol = dict(rtol=1e-6, atol=1e-7) if dtype == torch.float32 else dict(rtol=1e-12, atol=1e-14)
    for u, v in zip(outs[0], outs[2]):
        torch.testing.assert_close(u, v, **tol)
    a, b = idx[0].cpu().numpy(), idx[1].cpu().numpy()
    p = (torch.softmax(w0.double(), -1) if softmax else w0.double()).cpu().numpy()
    gyn, xn = gy.double().cpu().numpy(), x0.double().cpu().numpy()
    gp = O.dense_backward_w(xn, a, b, gs.cpu().numpy(), gyn)
    want_w = p * (gp - (p * gp).sum(1, keepdims=True)) if softmax else gp
    np.testing.assert_allclose(np_(outs[0][1]), want_w, **TOL[dtype])
    np.testing.assert_allclose(np_(outs[0][0]),
                               O.dense_backward_x_direct(xn, a, b, p, gs.cpu().numpy(), gyn),
                               **TOL[dtype])


def test_row_backward_entry_point_checks(device):
    """Limits are enforced, and a neuron that is not a single run gets NaN logits gradients
    instead of a partial sum."""
    from compactlogic_amd import _capi
    lib = _capi.load()
    L = make_layer(41, 30, 20, 4, 64)                  # per-slot wiring: multi-run neurons
    D = to_dev(L, device, torch.float32)
    plan = cl.build_run_plan(torch.stack([D["a"], D["b"]]), 30)
    assert not plan.single_run
    inv = torch.zeros((2 * plan.num_runs, 2), device=device)
    gw = torch.zeros((20, 4), device=device)
    gx = torch.empty((30, 64), device=device)
    stream = torch.cuda.current_stream().cuda_stream

    def call(batch, gates=4, x=D["x"], gyv=D["gy"]):
        return lib.cl_dense_backward_rows(0, x.data_ptr(), gyv.data_ptr(), plan.slot_rec.data_ptr(),
                                          plan.inv_rec.data_ptr(), inv.data_ptr(),
                                          D["gs"].data_ptr(), 0, plan.run_ptr.data_ptr(),
                                          gw.data_ptr(), gx.data_ptr(), 30, 20, plan.num_runs,
                                          batch, gates, stream)

    assert call(64, gates=65) != 0
    assert call(2052) != 0 and b"batch" in lib.cl_last_error()
    assert call(62) != 0
    assert call(64) == 0
    torch.cuda.synchronize()
    multi = (plan.run_ptr[1:] - plan.run_ptr[:-1]) != 1
    assert bool(multi.any())
    assert torch.isnan(gw[multi]).all() and not torch.isnan(gw[~multi]).any()
