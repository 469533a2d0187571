"""Pins the CPU oracle (oracle/) against the reference's own table and known-answer test and
against formulations that do not share its code: truth-table interpolation with torch
autograd, explicit loops, numpy's own bit packing, and the published SplitMix64 sequence.
CPU only."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import logic_np as O
from oracle import packed as P
from oracle import torch_cpu as TC

GOLDEN = json.loads((Path(__file__).parent / "golden" / "truth_table.json").read_text())
TABLE = np.array([row[2] for row in GOLDEN["gates"]], dtype=np.int64)  # [16, 4]: AB=00,01,10,11


def interp(g, a, b):
    """Bilinear interpolation of the reference truth table (independent of the oracle)."""
    t = torch.as_tensor(TABLE, dtype=torch.float64)[g]
    return ((1 - a) * (1 - b) * t[..., 0] + (1 - a) * b * t[..., 1]
            + a * (1 - b) * t[..., 2] + a * b * t[..., 3])


# ------------------------------------------------------------------------------ gate algebra

def test_truth_table_matches_reference_table():
    assert np.array_equal(O.TRUTH, TABLE)


def test_coefficients_match_difflogic_polynomials():
    rng = np.random.default_rng(0)
    a = torch.as_tensor(rng.random(257))
    b = torch.as_tensor(rng.random(257))
    for g in range(16):
        poly = TC._GATES[g](a, b).numpy()
        np.testing.assert_allclose(O.relaxed(g, a.numpy(), b.numpy()), poly, rtol=0, atol=1e-15)


def test_relaxed_is_truth_table_interpolation():
    rng = np.random.default_rng(1)
    a, b = rng.random(100), rng.random(100)
    for g in range(16):
        ref = interp(g, torch.as_tensor(a), torch.as_tensor(b)).numpy()
        np.testing.assert_allclose(O.relaxed(g, a, b), ref, atol=1e-15)
        for A in (0, 1):
            for B in (0, 1):
                assert O.relaxed(g, float(A), float(B)) == TABLE[g, 2 * A + B]


def test_all_gates_known_answer():
    kat = GOLDEN["all_gates_kat"]
    x = np.array(kat["x"])[:, None]                       # [in=8, batch=1]
    pairs = np.array(kat["pairs"])
    out = 16 * len(pairs)
    a = np.repeat(np.tile(pairs[:, 0], 16)[:, None], 16, axis=1)
    b = np.repeat(np.tile(pairs[:, 1], 16)[:, None], 16, axis=1)
    gs = np.tile(np.arange(16), (out, 1))
    w = np.zeros((out, 16))
    w[np.arange(out), np.arange(out) // len(pairs)] = 1.0   # one-hot on gate g for rows 4g..4g+3
    y = O.dense_forward(x, a, b, w, gs)[:, 0]
    expected = [TABLE[g, 2 * int(kat["x"][p0]) + int(kat["x"][p1])]
                for g in range(16) for p0, p1 in pairs]
    assert np.array_equal(y, np.array(expected, dtype=np.float64))


# ------------------------------------------------------------------------------ dense layer

def _random_layer(rng, in_dim, out_dim, g_n, batch, shared=False):
    if shared:
        pa = rng.integers(0, in_dim, out_dim)
        pb = rng.integers(0, in_dim, out_dim)
        a = np.repeat(pa[:, None], g_n, 1)
        b = np.repeat(pb[:, None], g_n, 1)
    else:
        a = rng.integers(0, in_dim, (out_dim, g_n))
        b = rng.integers(0, in_dim, (out_dim, g_n))
    gs = rng.integers(0, 16, (out_dim, g_n)).astype(np.uint8)
    logits = rng.standard_normal((out_dim, g_n))
    w = np.exp(logits) / np.exp(logits).sum(1, keepdims=True)
    x = rng.random((in_dim, batch))
    gy = rng.uniform(-1, 1, (out_dim, batch)) / batch
    return x, a, b, gs, w, gy


def _torch_layer(x, a, b, gs, w):
    """y[o, n] = sum_g w * interp(gs, x[a], x[b]) in torch (autograd-capable)."""
    xa = x[torch.as_tensor(a)]            # [out, G, batch]
    xb = x[torch.as_tensor(b)]
    op = interp(torch.as_tensor(gs.astype(np.int64))[..., None], xa, xb)
    return (w[..., None] * op).sum(1)


@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("g_n", [1, 4, 16])
def test_dense_oracle_against_autograd(shared, g_n):
    rng = np.random.default_rng(10 + g_n + 100 * shared)
    in_dim, out_dim, batch = 23, 37, 19
    x, a, b, gs, w, gy = _random_layer(rng, in_dim, out_dim, g_n, batch, shared)
    xt = torch.tensor(x, requires_grad=True)
    wt = torch.tensor(w, requires_grad=True)
    y = _torch_layer(xt, a, b, gs, wt)
    np.testing.assert_allclose(O.dense_forward(x, a, b, w, gs), y.detach().numpy(), atol=1e-13)
    gx, gw = torch.autograd.grad(y, (xt, wt), torch.tensor(gy))
    np.testing.assert_allclose(O.dense_backward_w(x, a, b, gs, gy), gw.numpy(), atol=1e-13)
    ind = np.stack([a, b])
    start, yidx, code = O.backward_index(ind, in_dim)
    np.testing.assert_allclose(O.dense_backward_x_csr(x, a, b, w, gs, gy, start, yidx, code),
                               gx.numpy(), atol=1e-13)
    np.testing.assert_allclose(O.dense_backward_x_direct(x, a, b, w, gs, gy), gx.numpy(), atol=1e-13)


def test_torch_formulation_gradcheck():
    rng = np.random.default_rng(3)
    x, a, b, gs, w, _ = _random_layer(rng, 6, 5, 4, 3)
    xt = torch.tensor(x, requires_grad=True)
    wt = torch.tensor(w, requires_grad=True)
    assert torch.autograd.gradcheck(lambda xx, ww: _torch_layer(xx, a, b, gs, ww), (xt, wt),
                                    eps=1e-6, atol=1e-8)


def test_backward_index_invariants():
    rng = np.random.default_rng(4)
    in_dim, out_dim, g_n = 11, 9, 5
    ind = rng.integers(0, in_dim, (2, out_dim, g_n))
    start, yidx, code = O.backward_index(ind, in_dim)
    assert start[0] == 0 and start[-1] == 2 * out_dim * g_n and np.all(np.diff(start) >= 0)
    seen = set()
    for i in range(in_dim):
        for e in range(start[i], start[i + 1]):
            side, g = (0, code[e]) if code[e] >= 0 else (1, -int(code[e]) - 1)
            assert ind[side, yidx[e], g] == i
            seen.add((side, int(yidx[e]), int(g)))
    assert len(seen) == 2 * out_dim * g_n


def test_dense_eval_truth_table():
    rng = np.random.default_rng(5)
    in_dim, out_dim, g_n, batch = 10, 40, 6, 33
    x = rng.integers(0, 2, (in_dim, batch)).astype(np.float64)
    a = rng.integers(0, in_dim, (out_dim, g_n))
    b = rng.integers(0, in_dim, (out_dim, g_n))
    gs = rng.integers(0, 16, (out_dim, g_n))
    slot = rng.integers(0, g_n, out_dim)
    y = O.dense_eval(x, a, b, slot, gs)
    for o in range(out_dim):
        s = slot[o]
        for n in range(batch):
            assert y[o, n] == TABLE[gs[o, s], 2 * int(x[a[o, s], n]) + int(x[b[o, s], n])]


@pytest.mark.parametrize("feats,k", [(40, 10), (25, 10), (7, 3), (12000, 10), (5, 7)])
def test_group_sum_loops_and_gradient(feats, k):
    rng = np.random.default_rng(feats)
    batch, tau = 4, 3.0
    x = rng.standard_normal((batch, feats))
    gsz = -(-feats // k)
    ref = np.zeros((batch, k))
    for n in range(batch):
        for c in range(k):
            for j in range(c * gsz, min((c + 1) * gsz, feats)):
                ref[n, c] += x[n, j]
    np.testing.assert_allclose(O.group_sum(x, k, tau), ref / tau, atol=1e-12)
    xt = torch.tensor(x, requires_grad=True)
    g = rng.standard_normal((batch, k))
    out = TC.group_sum(xt, k, tau)
    (gx,) = torch.autograd.grad(out, xt, torch.tensor(g))
    np.testing.assert_allclose(O.group_sum_backward(g, feats, k, tau), gx.numpy(), atol=1e-14)


# ------------------------------------------------------------------------------ conv

def _conv_loops(x, och, oh, ow, w, gs, stride, pad, ks):
    """Direct restatement with scalar loops (torch, autograd-capable)."""
    n_, _, h_in, w_in = x.shape
    c_out, g_n = w.shape
    h_out = (h_in + 2 * pad - ks) // stride + 1
    w_out = (w_in + 2 * pad - ks) // stride + 1
    rows = []
    for n in range(n_):
        for c in range(c_out):
            for oy in range(h_out):
                for ox in range(w_out):
                    acc = torch.zeros((), dtype=torch.float64)
                    for g in range(g_n):
                        vals = []
                        for side in (0, 1):
                            yy = oy * stride + int(oh[side, c, g])
                            xx = ox * stride + int(ow[side, c, g])
                            ok = 0 <= yy < h_in and 0 <= xx < w_in
                            vals.append(x[n, int(och[side, c, g]), yy, xx] if ok
                                        else torch.zeros((), dtype=torch.float64))
                        acc = acc + w[c, g] * interp(int(gs[c, g]), vals[0], vals[1])
                    rows.append(acc)
    return torch.stack(rows).view(n_, c_out, h_out, w_out)


@pytest.mark.parametrize("stride,pad,ks", [(2, 1, 3), (1, 0, 3), (2, 0, 3), (1, 1, 2)])
def test_conv_oracle_against_loops(stride, pad, ks):
    rng = np.random.default_rng(stride * 10 + pad + ks)
    n_, c_in, h, wd, c_out, g_n = 2, 3, 6, 5, 4, 3
    x = rng.random((n_, c_in, h, wd))
    och = rng.integers(0, c_in, (2, c_out, g_n)).astype(np.int32)
    oh = (rng.integers(0, ks, (2, c_out, g_n)) - pad).astype(np.int8)
    ow = (rng.integers(0, ks, (2, c_out, g_n)) - pad).astype(np.int8)
    gs = rng.integers(0, 16, (c_out, g_n)).astype(np.uint8)
    logits = rng.standard_normal((c_out, g_n))
    w = np.exp(logits) / np.exp(logits).sum(1, keepdims=True)
    xt = torch.tensor(x, requires_grad=True)
    wt = torch.tensor(w, requires_grad=True)
    y = _conv_loops(xt, och, oh, ow, wt, gs, stride, pad, ks)
    np.testing.assert_allclose(O.conv_forward(x, och, oh, ow, w, gs, stride, pad, ks),
                               y.detach().numpy(), atol=1e-13)
    gy = rng.standard_normal(y.shape)
    gx, gw = torch.autograd.grad(y, (xt, wt), torch.tensor(gy))
    ogx, ogw = O.conv_backward(x, och, oh, ow, w, gs, gy, stride, pad)
    np.testing.assert_allclose(ogx, gx.numpy(), atol=1e-12)
    np.testing.assert_allclose(ogw, gw.numpy(), atol=1e-12)
    # the weight-gradient-only restatement against the same scalar-loop autograd
    np.testing.assert_allclose(O.conv_backward_w(x, och, oh, ow, gs, gy, stride), gw.numpy(),
                               atol=1e-12)
    slot = rng.integers(0, g_n, c_out)
    xb = (x > 0.5).astype(np.float64)
    onehot = np.zeros_like(w)
    onehot[np.arange(c_out), slot] = 1.0
    np.testing.assert_allclose(O.conv_eval(xb, och, oh, ow, slot, gs, stride, pad, ks),
                               O.conv_forward(xb, och, oh, ow, onehot, gs, stride, pad, ks),
                               atol=0)


@pytest.mark.parametrize("stride,pad,ks", [(2, 1, 3), (2, 0, 3), (1, 1, 3)])
def test_conv_slot_tables_match_float_discrete_conv(stride, pad, ks):
    """The packed conv tables, evaluated bitwise on 64 samples per word, give the same bits
    as the float discrete conv (itself pinned against scalar loops above)."""
    rng = np.random.default_rng(40 + stride * 10 + pad)
    n_, c_in, h, wd, c_out, g_n = 130, 3, 7, 6, 5, 4
    och = rng.integers(0, c_in, (2, c_out, g_n)).astype(np.int32)
    oh = (rng.integers(0, ks, (2, c_out, g_n)) - pad).astype(np.int8)
    ow = (rng.integers(0, ks, (2, c_out, g_n)) - pad).astype(np.int8)
    gs = rng.integers(0, 16, (c_out, g_n)).astype(np.uint8)
    slot = rng.integers(0, g_n, c_out)
    xb = rng.integers(0, 2, (n_, c_in, h, wd)).astype(np.float64)
    y = O.conv_eval(xb, och, oh, ow, slot, gs, stride, pad, ks)
    h_out, w_out = y.shape[2:]
    ia, ib, g = P.resolve_conv_slots(och, oh, ow, gs, slot, (c_in, h, wd), stride, (h_out, w_out))
    assert ia.min() >= -1 and ia.max() < c_in * h * wd
    feats = xb.reshape(n_, -1).T.astype(bool)            # [features, samples]
    packed, pad_len = P.pack_bits(feats, 64)
    out = P.eval_layer(packed.view(np.uint64), ia, ib, g)
    bits = np.unpackbits(out.view(np.uint8), axis=1, bitorder="little")[:, :n_]
    np.testing.assert_array_equal(bits.T.reshape(y.shape), y.astype(np.uint8))


# ------------------------------------------------------------------------------ packed

def test_splitmix64_published_sequence():
    # SplitMix64 (Vigna) seeded with 1234567: the generator's first five outputs.
    seq = [P.splitmix64(1234567 + i * 0x9E3779B97F4A7C15) for i in range(5)]
    assert seq == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                   4593380528125082431, 16408922859458223821]
    assert P.splitmix64(0) == 0xE220A8397B1DCDAF
    filled = P.fill_splitmix64(4, 1234567)
    assert [int(v) for v in filled] == [P.splitmix64(1234567 + i) for i in range(4)]


@pytest.mark.parametrize("bits", [8, 16, 32, 64])
@pytest.mark.parametrize("n", [1, 63, 64, 65, 200])
def test_pack_bits_matches_numpy(bits, n):
    rng = np.random.default_rng(bits + n)
    t = rng.integers(0, 2, (3, n)).astype(bool)
    packed, pad = P.pack_bits(t, bits)
    words = -(-n // bits)
    assert pad == (bits - n % bits) % bits
    ref = np.packbits(np.pad(t, ((0, 0), (0, words * bits - n))), axis=1, bitorder="little")
    assert np.array_equal(packed, ref)


def test_packed_layer_matches_boolean_truth_table():
    rng = np.random.default_rng(7)
    in_dim, out_dim, n = 9, 32, 128
    bits = rng.integers(0, 2, (in_dim, n)).astype(bool)
    xw, _ = P.pack_bits(bits, 64)
    ia = rng.integers(-1, in_dim, out_dim)
    ib = rng.integers(-1, in_dim, out_dim)
    g = np.arange(out_dim) % 16
    y = P.eval_layer(xw.view(np.uint64), ia, ib, g)
    ybits = np.unpackbits(y.view(np.uint8), axis=1, bitorder="little")[:, :n]
    zero = np.zeros(n, dtype=bool)
    for o in range(out_dim):
        va = bits[ia[o]] if ia[o] >= 0 else zero
        vb = bits[ib[o]] if ib[o] >= 0 else zero
        assert np.array_equal(ybits[o], TABLE[g[o], 2 * va.astype(int) + vb.astype(int)])


@pytest.mark.parametrize("rows,k,n,bits", [(20, 10, 130, 64), (12, 3, 64, 32), (8, 8, 17, 8)])
def test_group_bit_sum_matches_unpacked(rows, k, n, bits):
    rng = np.random.default_rng(rows + k + n)
    t = rng.integers(0, 2, (rows, n)).astype(bool)
    packed, pad = P.pack_bits(t, bits)
    counts = P.group_bit_sum(packed, pad, k)
    ref = t.T.reshape(n, k, rows // k).sum(-1)
    assert counts.shape == (n, k) and np.array_equal(counts, ref)
    with pytest.raises(ValueError):
        P.group_bit_sum(packed[: rows - 1], pad, k)


def test_packed_network_agrees_with_float_discrete_path():
    """counts == round(logits * tau) (simulation/consistency.py:241) between the packed and
    float discrete evaluators of one network."""
    rng = np.random.default_rng(8)
    dims = [(12, 30), (30, 30), (30, 20)]
    n, k, tau = 192, 5, 4.0
    bits = rng.integers(0, 2, (dims[0][0], n)).astype(bool)
    layers, h = [], bits.astype(np.float64)
    for i, o in dims:
        ind = rng.integers(0, i, (2, o, 4))
        gs = rng.integers(0, 16, (o, 4))
        slot = rng.integers(0, 4, o)
        h = O.dense_eval(h, ind[0], ind[1], slot, gs)
        layers.append(P.resolve_slots(ind, gs, slot))
    logits = O.group_sum(h.T, k, tau)
    xw, pad = P.pack_bits(bits, 64)
    counts = P.network_counts(xw.view(np.uint64), layers, k, pad)
    assert np.array_equal(counts, np.round(logits * tau).astype(np.int32))


def test_torch_cpu_step_matches_oracle():
    rng = np.random.default_rng(9)
    dims = [(16, 24), (24, 24)]
    batch = 8
    layers = []
    for i, o in dims:
        pair = rng.integers(0, i, (2, o, 1)).repeat(16, axis=2)
        layers.append((torch.as_tensor(pair), torch.arange(16, dtype=torch.uint8).repeat(o, 1),
                       torch.randn(o, 16, dtype=torch.float64)))
    net = TC.CpuDenseNet(layers, k=4, tau=2.0, dtype=torch.float64)
    x = torch.as_tensor(rng.random((batch, 16)))
    out = net.forward(x).detach().numpy()
    h = x.numpy().T
    for ind, gs, lg in layers:
        p = torch.softmax(lg, -1).numpy()
        h = O.dense_forward(h, ind[0].numpy(), ind[1].numpy(), p, gs.numpy())
    np.testing.assert_allclose(out, O.group_sum(h.T, 4, 2.0), atol=1e-12)


@pytest.mark.parametrize("stride,pad", [(2, 1), (1, 0), (2, 0)])
def test_torch_cpu_conv_matches_oracle(stride, pad):
    """The CPU baseline's conv layer (gather formulation, autograd backward) against the
    loop-pinned float64 conv oracle, forward and both gradients."""
    rng = np.random.default_rng(20 + stride + pad)
    n_, c_in, h, wd, c_out, g_n, ks = 3, 4, 7, 8, 5, 6, 3
    och = torch.as_tensor(rng.integers(0, c_in, (2, c_out, g_n)).astype(np.int32))
    oh = torch.as_tensor((rng.integers(0, ks, (2, c_out, g_n)) - pad).astype(np.int8))
    ow = torch.as_tensor((rng.integers(0, ks, (2, c_out, g_n)) - pad).astype(np.int8))
    gs = torch.as_tensor(rng.integers(0, 16, (c_out, g_n)).astype(np.uint8))
    logits = torch.randn(c_out, g_n, dtype=torch.float64, requires_grad=True)
    x = torch.as_tensor(rng.random((n_, c_in, h, wd)), dtype=torch.float64).requires_grad_(True)
    hw = O.conv_out_hw(h, wd, pad, ks, stride)
    y = TC.conv_forward(x, och, oh, ow, gs, logits, stride, hw)
    p = torch.softmax(logits, -1).detach().numpy()
    args = (och.numpy(), oh.numpy(), ow.numpy())
    np.testing.assert_allclose(y.detach().numpy(),
                               O.conv_forward(x.detach().numpy(), *args, p, gs.numpy(), stride, pad, ks),
                               atol=1e-12)
    gy = rng.standard_normal(y.shape)
    y.backward(torch.as_tensor(gy))
    rgx, rgw = O.conv_backward(x.detach().numpy(), *args, p, gs.numpy(), gy, stride, pad)
    np.testing.assert_allclose(x.grad.numpy(), rgx, atol=1e-12)
    np.testing.assert_allclose(logits.grad.numpy(), p * (rgw - (p * rgw).sum(1, keepdims=True)),
                               atol=1e-12)
