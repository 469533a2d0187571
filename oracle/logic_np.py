"""float64 numpy restatement of the soft and float-discrete hot path -- TEST INFRASTRUCTURE.

Follows (paths relative to the eth-sri/CompactLogic tree):
  gate algebra      compactlogic/cuda/utils.cuh:122-243 (truth table, C0..C3, GRAD_*)
  dense forward     compactlogic/cuda/difflogic_kernel.cu:38-78
  dense backward_w  compactlogic/cuda/difflogic_kernel.cu:81-137
  dense backward_x  compactlogic/cuda/difflogic_kernel.cu:140-194 (CSR walk)
  inverse index     compactlogic/compactlogic.py:184-241 (full rebuild)
  dense eval        compactlogic/cuda/difflogic_kernel.cu:341-369, compactlogic.py:120-130
  GroupSum          compactlogic/compactlogic.py:450-468
  conv forward      compactlogic/cuda/convlogic_kernel.cu:87-138
  conv backward     compactlogic/cuda/convlogic_kernel.cu:190-246 (x), :295-382 (w)
  conv eval         compactlogic/cuda/convlogic_kernel.cu:433-476

Pinned by tests/test_oracle.py (none of these checks restates the function it checks):
  gate_coefficients  the reference truth table (tests/golden/truth_table.json), the 16
                     explicit difflogic polynomials, the reference's all-gates KAT
  dense_*            torch autograd + finite differences of an independent bilinear-
                     interpolation formulation; backward_x_csr against the scatter form
  backward_index     structural invariants (each use exactly once, starts = cumsum)
  group_sum          explicit per-class loops; gradient by autograd
  conv_*             explicit 7-deep loops at tiny sizes; gradients by autograd
  *_eval             truth-table lookup on {0,1} inputs
"""
from __future__ import annotations

import numpy as np

# Truth table: TRUTH[g, 2A+B] = (g >> (3 - (2A+B))) & 1  (utils.cuh:122-139 column order).
TRUTH = np.array([[(g >> (3 - k)) & 1 for k in range(4)] for g in range(16)], dtype=np.int64)


def gate_coefficients() -> np.ndarray:
    """[16, 4] float64 (c0, c1, c2, c3): op_g(a, b) = c0 + c1 a + c2 b + c3 a b, the
    multilinear interpolation of the truth table (utils.cuh:180-207)."""
    f00, f01, f10, f11 = (TRUTH[:, k].astype(np.float64) for k in range(4))
    return np.stack([f00, f10 - f00, f01 - f00, f11 - f10 - f01 + f00], axis=1)


_C = gate_coefficients()


def relaxed(g, a, b):
    """Relaxed value of opcode(s) g at real inputs a, b (broadcasting)."""
    c = _C[np.asarray(g)]
    return c[..., 0] + c[..., 1] * a + c[..., 2] * b + c[..., 3] * a * b


def _f64(t):
    return np.asarray(t, dtype=np.float64)


# ---------------------------------------------------------------------------------------- dense

def dense_forward(x, a, b, w, gs):
    """y[o, n] = sum_g w[o, g] * op_{gs[o,g]}(x[a[o,g], n], x[b[o,g], n]); x: [in, batch]."""
    x, w = _f64(x), _f64(w)
    a, b, gs = np.asarray(a), np.asarray(b), np.asarray(gs).astype(np.int64)
    out, g_n = w.shape
    y = np.zeros((out, x.shape[1]))
    for g in range(g_n):
        c = _C[gs[:, g]]
        xa, xb = x[a[:, g]], x[b[:, g]]
        y += w[:, g:g + 1] * (c[:, 0:1] + c[:, 1:2] * xa + c[:, 2:3] * xb + c[:, 3:4] * xa * xb)
    return y


def dense_backward_w(x, a, b, gs, gy):
    """grad_w[o, g] = sum_n gy[o, n] * op_{gs[o,g]}(x[a[o,g], n], x[b[o,g], n])."""
    x, gy = _f64(x), _f64(gy)
    a, b, gs = np.asarray(a), np.asarray(b), np.asarray(gs).astype(np.int64)
    out, g_n = a.shape
    gw = np.zeros((out, g_n))
    for g in range(g_n):
        c = _C[gs[:, g]]
        xa, xb = x[a[:, g]], x[b[:, g]]
        op = c[:, 0:1] + c[:, 1:2] * xa + c[:, 2:3] * xb + c[:, 3:4] * xa * xb
        gw[:, g] = (gy * op).sum(axis=1)
    return gw


def backward_index(indices, in_dim):
    """(start [in+1], y [2*out*G], code [2*out*G]) as refresh_backward_index builds them:
    operand-a uses carry code g, operand-b uses -(g+1); entries grouped by input (stable)."""
    ind = np.asarray(indices)
    _, out, g_n = ind.shape
    rows = np.repeat(np.arange(out), g_n)
    slots = np.tile(np.arange(g_n), out)
    inputs = np.concatenate([ind[0].reshape(-1), ind[1].reshape(-1)])
    ys = np.concatenate([rows, rows])
    codes = np.concatenate([slots, -(slots + 1)]).astype(np.int8)
    order = np.argsort(inputs, kind="stable")
    counts = np.bincount(inputs, minlength=in_dim)
    start = np.zeros(in_dim + 1, dtype=np.int64)
    start[1:] = np.cumsum(counts)
    return start, ys[order].astype(np.int64), codes[order]


def dense_backward_x_csr(x, a, b, w, gs, gy, start, yidx, gcode):
    """grad_x[i, n] = sum over entries e of row i of
    w[y,g] * (dop/d(own operand))(x[other, n]) * gy[y, n]."""
    x, w, gy = _f64(x), _f64(w), _f64(gy)
    a, b, gs = np.asarray(a), np.asarray(b), np.asarray(gs).astype(np.int64)
    start, yidx = np.asarray(start), np.asarray(yidx)
    gcode = np.asarray(gcode).astype(np.int64)
    in_dim = x.shape[0]
    gx = np.zeros_like(x)
    rows = np.repeat(np.arange(in_dim), np.diff(start))
    side_a = gcode >= 0
    g = np.where(side_a, gcode, -gcode - 1)
    c = _C[gs[yidx, g]]
    other = np.where(side_a, b[yidx, g], a[yidx, g])
    kself = np.where(side_a, c[:, 1], c[:, 2])
    chunk = 4096
    for e0 in range(0, len(yidx), chunk):
        sl = slice(e0, e0 + chunk)
        dydx = w[yidx[sl], g[sl]][:, None] * (kself[sl][:, None] + c[sl, 3][:, None] * x[other[sl]])
        np.add.at(gx, rows[sl], dydx * gy[yidx[sl]])
    return gx


def dense_backward_x_direct(x, a, b, w, gs, gy):
    """Scatter form of the input gradient (no inverse index)."""
    x, w, gy = _f64(x), _f64(w), _f64(gy)
    a, b, gs = np.asarray(a), np.asarray(b), np.asarray(gs).astype(np.int64)
    gx = np.zeros_like(x)
    for g in range(w.shape[1]):
        c = _C[gs[:, g]]
        xa, xb = x[a[:, g]], x[b[:, g]]
        np.add.at(gx, a[:, g], w[:, g:g + 1] * (c[:, 1:2] + c[:, 3:4] * xb) * gy)
        np.add.at(gx, b[:, g], w[:, g:g + 1] * (c[:, 2:3] + c[:, 3:4] * xa) * gy)
    return gx


def dense_eval(x, a, b, w_slot, gs):
    """Discrete forward: slot s = w_slot[o], y = op_{gs[o,s]}(x[a[o,s]], x[b[o,s]])."""
    x = _f64(x)
    a, b, gs = np.asarray(a), np.asarray(b), np.asarray(gs).astype(np.int64)
    s = np.asarray(w_slot).astype(np.int64)
    o = np.arange(a.shape[0])
    return relaxed(gs[o, s][:, None], x[a[o, s]], x[b[o, s]])


# ---------------------------------------------------------------------------------------- GroupSum

def group_sum(x, k, tau):
    """[batch, F] -> [batch, k]: zero-pad F to a multiple of k, sum k equal groups, / tau."""
    x = _f64(x)
    if x.shape[-1] % k:
        x = np.concatenate([x, np.zeros((x.shape[0], k - x.shape[-1] % k))], axis=1)
    return x.reshape(x.shape[0], k, x.shape[1] // k).sum(-1) / tau


def group_sum_backward(g, features, k, tau):
    """grad of group_sum: grad_x[n, j] = g[n, j // gs] / tau."""
    g = _f64(g)
    gs = -(-features // k)
    return np.repeat(g, gs, axis=1)[:, :features] / tau


# ---------------------------------------------------------------------------------------- conv

def _conv_taps(x, och, oh, ow, stride, h_out, w_out, side, c, g):
    """Values of operand `side` of slot g of output channel c at every output position:
    x[n, ch, oy*s + dh, ox*s + dw], 0 outside the input.  Returns [N, h_out, w_out] and the
    validity mask / coordinates."""
    n_, _, h_in, w_in = x.shape
    ch, dh, dw = int(och[side, c, g]), int(oh[side, c, g]), int(ow[side, c, g])
    ys = np.arange(h_out) * stride + dh
    xs = np.arange(w_out) * stride + dw
    vy = (ys >= 0) & (ys < h_in)
    vx = (xs >= 0) & (xs < w_in)
    vals = np.zeros((n_, h_out, w_out))
    iy, ix = np.nonzero(vy)[0], np.nonzero(vx)[0]
    vals[:, iy[:, None], ix[None, :]] = x[:, ch][:, ys[iy][:, None], xs[ix][None, :]]
    return vals, ch, ys, xs, vy, vx


def conv_out_hw(h_in, w_in, pad, ks, stride):
    return (h_in + 2 * pad - ks) // stride + 1, (w_in + 2 * pad - ks) // stride + 1


def conv_forward(x, och, oh, ow, w, gs, stride, pad, ks):
    """y[n, c, oy, ox] = sum_g w[c,g] op_{gs[c,g]}(tap_a, tap_b); offsets already hold -pad."""
    x, w = _f64(x), _f64(w)
    gs = np.asarray(gs).astype(np.int64)
    n_, _, h_in, w_in = x.shape
    c_out, g_n = w.shape
    h_out, w_out = conv_out_hw(h_in, w_in, pad, ks, stride)
    y = np.zeros((n_, c_out, h_out, w_out))
    for c in range(c_out):
        for g in range(g_n):
            va = _conv_taps(x, och, oh, ow, stride, h_out, w_out, 0, c, g)[0]
            vb = _conv_taps(x, och, oh, ow, stride, h_out, w_out, 1, c, g)[0]
            y[:, c] += w[c, g] * relaxed(gs[c, g], va, vb)
    return y


def conv_backward(x, och, oh, ow, w, gs, gy, stride, pad):
    """(grad_x, grad_w) of conv_forward for upstream gradient gy."""
    x, w, gy = _f64(x), _f64(w), _f64(gy)
    gs = np.asarray(gs).astype(np.int64)
    n_, _, h_in, w_in = x.shape
    c_out, g_n = w.shape
    h_out, w_out = gy.shape[2], gy.shape[3]
    gx = np.zeros_like(x)
    gw = np.zeros((c_out, g_n))
    for c in range(c_out):
        for g in range(g_n):
            cf = _C[gs[c, g]]
            va, cha, ya, xa_, vya, vxa = _conv_taps(x, och, oh, ow, stride, h_out, w_out, 0, c, g)
            vb, chb, yb, xb_, vyb, vxb = _conv_taps(x, och, oh, ow, stride, h_out, w_out, 1, c, g)
            gyc = gy[:, c]
            gw[c, g] = (gyc * relaxed(gs[c, g], va, vb)).sum()
            da = w[c, g] * (cf[1] + cf[3] * vb) * gyc
            db = w[c, g] * (cf[2] + cf[3] * va) * gyc
            for oy in range(h_out):
                for ox in range(w_out):
                    if vya[oy] and vxa[ox]:
                        gx[:, cha, ya[oy], xa_[ox]] += da[:, oy, ox]
                    if vyb[oy] and vxb[ox]:
                        gx[:, chb, yb[oy], xb_[ox]] += db[:, oy, ox]
    return gx, gw


def conv_backward_w(x, och, oh, ow, gs, gy, stride):
    """grad_w of conv_forward alone (no input gradient):
    grad_w[c, g] = sum over n, oy, ox of gy[n, c, oy, ox] * op_{gs[c,g]}(tap_a, tap_b), following
    compactlogic/cuda/convlogic_kernel.cu:295-430; the same sum as conv_backward's second
    result, without its per-position input-gradient scatter."""
    x, gy = _f64(x), _f64(gy)
    gs = np.asarray(gs).astype(np.int64)
    c_out, g_n = gs.shape
    h_out, w_out = gy.shape[2], gy.shape[3]
    gw = np.zeros((c_out, g_n))
    for c in range(c_out):
        for g in range(g_n):
            va = _conv_taps(x, och, oh, ow, stride, h_out, w_out, 0, c, g)[0]
            vb = _conv_taps(x, och, oh, ow, stride, h_out, w_out, 1, c, g)[0]
            gw[c, g] = (gy[:, c] * relaxed(gs[c, g], va, vb)).sum()
    return gw


def conv_eval(x, och, oh, ow, w_slot, gs, stride, pad, ks):
    """Discrete conv: output channel c uses its argmax slot s = w_slot[c] only."""
    x = _f64(x)
    gs = np.asarray(gs).astype(np.int64)
    n_, _, h_in, w_in = x.shape
    c_out = gs.shape[0]
    h_out, w_out = conv_out_hw(h_in, w_in, pad, ks, stride)
    y = np.zeros((n_, c_out, h_out, w_out))
    for c in range(c_out):
        s = int(w_slot[c])
        va = _conv_taps(x, och, oh, ow, stride, h_out, w_out, 0, c, s)[0]
        vb = _conv_taps(x, och, oh, ow, stride, h_out, w_out, 1, c, s)[0]
        y[:, c] = relaxed(gs[c, s], va, vb)
    return y
