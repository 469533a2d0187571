"""float64 numpy restatement of the logic-tree conv block -- TEST INFRASTRUCTURE ONLY.

Follows (paths relative to the eth-sri/CompactLogic tree, under
third_party/convlogic_source_code/src/convlogic/):
  taps / conv gates   convlogic_layer.py:188-234 (forward_python), :236-321 (forward_python_full)
                      and cuda/full_convlogic_kernel.cu:10-63: tap k of channel c reads
                      x[n, ch, oy*sh + row - ph, ox*sw + col - pw], zero outside the image
  tree levels         convlogic_layer.py:283-318; treelogic_layer.py:106-124
  pool                convlogic_layer.py:473-500 (torch max_pool2d) and
                      cuda/full_convlogic_kernel.cu:126-139: the first maximum in row-major
                      window order wins (strict >); indices oy * Wo + ox
  backward            cuda/full_convlogic_kernel.cu:233-330 (through the window winners only),
                      :470-578 (node moments), :690-700 (moments -> per-gate gradient)
  packed block        the discrete reading: argmax gates, pool = OR (third_party/convlogic/
                      extract.py:177-214, evaluate.py:117-122)

Pinned by tests/test_oracle_tree.py (none of the checks restates the function it checks):
  block_forward        an explicit-loop evaluation with the reference's 16-term gate
                       polynomials (full_convlogic_kernel.cu:50-58), and torch's max_pool2d
                       (values and indices) for the pool
  block_backward       torch autograd of a torch restatement (max_pool2d's own backward), and
                       central finite differences
  level_*              torch autograd
  block_bits           block_forward with one-hot probabilities on {0, 1} inputs
"""
from __future__ import annotations

import numpy as np

from .logic_np import TRUTH, gate_coefficients

_C = gate_coefficients()


def unpack(sel):
    sel = np.asarray(sel, dtype=np.int64)
    return (sel >> 16) & 0xFFFF, (sel >> 8) & 0xFF, sel & 0xFF


def out_hw(h, w, stride, pad, kernel):
    (sh, sw), (ph, pw), (kh, kw) = stride, pad, kernel
    return (h + 2 * ph - kh) // sh + 1, (w + 2 * pw - kw) // sw + 1


def collapse(w_prob):
    """[..., 16] probabilities -> [..., 4] coefficients (c0, c1, c2, c3) of the mixture."""
    return np.asarray(w_prob, dtype=np.float64) @ _C


def _node(k, a, b):
    return k[..., 0] + k[..., 1] * a + k[..., 2] * b + k[..., 3] * a * b


def taps(x, sel, stride, pad, kernel):
    """v [N, C, Ho, Wo, 8]: the tap values at every conv position."""
    x = np.asarray(x, dtype=np.float64)
    n, c_in, h, w = x.shape
    ho, wo = out_hw(h, w, stride, pad, kernel)
    ch, ry, rx = unpack(sel)
    c_out = ch.shape[0]
    v = np.zeros((n, c_out, ho, wo, 8))
    oy = np.arange(ho)[:, None]
    ox = np.arange(wo)[None, :]
    for c in range(c_out):
        for k in range(8):
            iy = oy * stride[0] + ry[c, k] - pad[0]
            ix = ox * stride[1] + rx[c, k] - pad[1]
            ok = (iy >= 0) & (iy < h) & (ix >= 0) & (ix < w)
            vals = x[:, ch[c, k], np.clip(iy, 0, h - 1), np.clip(ix, 0, w - 1)]
            v[:, c, :, :, k] = np.where(ok[None], vals, 0.0)
    return v


def block_forward(x, w_prob, sel, stride, pad, kernel, complete=True):
    """complete: (y [N, C, Ho/2, Wo/2], x2 [N, C, Ho, Wo, 4], x3 [.., 2], idx [N, C, P]);
    else y [N, C, Ho, Wo, 4]."""
    k = collapse(w_prob)                                   # [C, nodes, 4]
    v = taps(x, sel, stride, pad, kernel)
    kc = k[None, :, None, None]                            # broadcast over N, Ho, Wo
    g = np.stack([_node(kc[..., q, :], v[..., 2 * q], v[..., 2 * q + 1]) for q in range(4)], -1)
    if not complete:
        return g
    t = np.stack([_node(kc[..., 4 + j, :], g[..., 2 * j], g[..., 2 * j + 1]) for j in range(2)], -1)
    r = _node(kc[..., 6, :], t[..., 0], t[..., 1])        # [N, C, Ho, Wo]
    n, c_out, ho, wo = r.shape
    hp, wp = ho // 2, wo // 2
    y = np.full((n, c_out, hp, wp), -np.inf)
    idx = np.full((n, c_out, hp * wp), -1, dtype=np.int64)
    for dy in range(2):
        for dx in range(2):
            cand = r[:, :, dy::2, dx::2][:, :, :hp, :wp]
            better = cand > y
            y = np.where(better, cand, y)
            pos = (2 * np.arange(hp)[:, None] + dy) * wo + (2 * np.arange(wp)[None, :] + dx)
            idx = np.where(better.reshape(n, c_out, -1), pos.reshape(-1)[None, None], idx)
    return y, g, t, idx


def block_backward(x, w_prob, sel, stride, pad, kernel, grad_y, complete=True, idx=None):
    """(grad_x [N, C_in, H, W], grad_w_prob [C, nodes, 16]) through the window winners (those
    of block_forward, or `idx` [N, C, P] when given)."""
    x = np.asarray(x, dtype=np.float64)
    grad_y = np.asarray(grad_y, dtype=np.float64)
    n, c_in, h, w = x.shape
    k = collapse(w_prob)
    v = taps(x, sel, stride, pad, kernel)                  # [N, C, Ho, Wo, 8]
    c_out, ho, wo = v.shape[1], v.shape[2], v.shape[3]
    kc = k[None, :, None, None]
    g = np.stack([_node(kc[..., q, :], v[..., 2 * q], v[..., 2 * q + 1]) for q in range(4)], -1)
    nodes = 7 if complete else 4
    up = np.zeros((n, c_out, ho, wo, nodes))               # upstream gradient of each node
    if complete:
        _, _, t, fidx = block_forward(x, w_prob, sel, stride, pad, kernel, True)
        idx = fidx if idx is None else np.asarray(idx, dtype=np.int64)
        gy_full = np.zeros((n, c_out, ho * wo))
        np.put_along_axis(gy_full, idx, grad_y.reshape(n, c_out, -1), axis=2)
        up[..., 6] = gy_full.reshape(n, c_out, ho, wo)
        k6 = kc[..., 6, :]
        up[..., 4] = up[..., 6] * (k6[..., 1] + k6[..., 3] * t[..., 1])
        up[..., 5] = up[..., 6] * (k6[..., 2] + k6[..., 3] * t[..., 0])
        for j in range(2):
            kj = kc[..., 4 + j, :]
            up[..., 2 * j] = up[..., 4 + j] * (kj[..., 1] + kj[..., 3] * g[..., 2 * j + 1])
            up[..., 2 * j + 1] = up[..., 4 + j] * (kj[..., 2] + kj[..., 3] * g[..., 2 * j])
        node_in = [(v[..., 2 * q], v[..., 2 * q + 1]) for q in range(4)]
        node_in += [(g[..., 0], g[..., 1]), (g[..., 2], g[..., 3]), (t[..., 0], t[..., 1])]
    else:
        up[...] = grad_y
        node_in = [(v[..., 2 * q], v[..., 2 * q + 1]) for q in range(4)]
    grad_w = np.zeros((c_out, nodes, 16))
    for q in range(nodes):
        a, b = node_in[q]
        for gate in range(16):
            val = _C[gate, 0] + _C[gate, 1] * a + _C[gate, 2] * b + _C[gate, 3] * a * b
            grad_w[:, q, gate] = (up[..., q] * val).sum(axis=(0, 2, 3))
    # input gradient: scatter of the taps' derivatives
    grad_x = np.zeros_like(x)
    ch, ry, rx = unpack(sel)
    oy = np.arange(ho)[:, None]
    ox = np.arange(wo)[None, :]
    for c in range(c_out):
        for tap in range(8):
            q = tap // 2
            kq = k[c, q]
            other = v[:, c, :, :, tap ^ 1]
            der = (kq[1] + kq[3] * other) if tap % 2 == 0 else (kq[2] + kq[3] * other)
            contrib = up[:, c, :, :, q] * der              # [N, Ho, Wo]
            iy = oy * stride[0] + ry[c, tap] - pad[0]
            ix = ox * stride[1] + rx[c, tap] - pad[1]
            ok = (iy >= 0) & (iy < h) & (ix >= 0) & (ix < w)
            iyb, ixb = np.broadcast_to(iy, ok.shape)[ok], np.broadcast_to(ix, ok.shape)[ok]
            np.add.at(grad_x, (slice(None), ch[c, tap], iyb, ixb), contrib[:, ok])
    return grad_x, grad_w


def level_forward(x, w_prob):
    """One tree level: x [..., C?] with channels on axis 1: y[..., j] = node_j(x[..., 2j], x[..., 2j+1])."""
    x = np.asarray(x, dtype=np.float64)
    k = collapse(w_prob)                                   # [C, xo, 4]
    kc = k[None, :, None, None]
    return np.stack([_node(kc[..., j, :], x[..., 2 * j], x[..., 2 * j + 1])
                     for j in range(k.shape[1])], -1)


def level_backward(x, w_prob, grad_y):
    x = np.asarray(x, dtype=np.float64)
    grad_y = np.asarray(grad_y, dtype=np.float64)
    k = collapse(w_prob)
    kc = k[None, :, None, None]
    gx = np.zeros_like(x)
    gw = np.zeros((k.shape[0], k.shape[1], 16))
    for j in range(k.shape[1]):
        a, b, gy = x[..., 2 * j], x[..., 2 * j + 1], grad_y[..., j]
        gx[..., 2 * j] = gy * (kc[..., j, 1] + kc[..., j, 3] * b)
        gx[..., 2 * j + 1] = gy * (kc[..., j, 2] + kc[..., j, 3] * a)
        for gate in range(16):
            val = _C[gate, 0] + _C[gate, 1] * a + _C[gate, 2] * b + _C[gate, 3] * a * b
            gw[:, j, gate] = (gy * val).sum(axis=(0, 2, 3))
    return gx, gw


def _bit_op(g, a, b):
    """Bitwise opcode g on uint64 arrays (truth table TRUTH[g, 2A + B])."""
    a = np.asarray(a, dtype=np.uint64)
    b = np.asarray(b, dtype=np.uint64)
    out = np.zeros(np.broadcast(a, b).shape, dtype=np.uint64)
    na, nb = ~a, ~b
    for A, B, ma, mb in ((0, 0, na, nb), (0, 1, na, b), (1, 0, a, nb), (1, 1, a, b)):
        out |= np.where(np.asarray(TRUTH[g, 2 * A + B], dtype=bool), ma & mb, np.uint64(0))
    return out


def block_bits(x_words, gates, sel, in_shape, stride, pad, kernel, complete=True):
    """Packed discrete block on uint64 rows (row (ch*H + y)*W + x): gates [C, nodes] opcodes ->
    rows (c*Hp + py)*Wp + px (complete, pool = OR) or ((c*Ho + oy)*Wo + ox)*4 + q."""
    xw = np.asarray(x_words, dtype=np.uint64)
    c_in, h, w = in_shape
    words = xw.shape[1]
    ho, wo = out_hw(h, w, stride, pad, kernel)
    ch, ry, rx = unpack(sel)
    c_out = ch.shape[0]
    zero = np.zeros(words, dtype=np.uint64)

    def tap(c, k, oy, ox):
        iy = oy * stride[0] + ry[c, k] - pad[0]
        ix = ox * stride[1] + rx[c, k] - pad[1]
        if iy < 0 or iy >= h or ix < 0 or ix >= w:
            return zero
        return xw[(ch[c, k] * h + iy) * w + ix]

    def gates_at(c, oy, ox):
        return [_bit_op(int(gates[c, q]), tap(c, 2 * q, oy, ox), tap(c, 2 * q + 1, oy, ox))
                for q in range(4)]

    if not complete:
        out = np.zeros((c_out * ho * wo * 4, words), dtype=np.uint64)
        for c in range(c_out):
            for oy in range(ho):
                for ox in range(wo):
                    g = gates_at(c, oy, ox)
                    for q in range(4):
                        out[((c * ho + oy) * wo + ox) * 4 + q] = g[q]
        return out
    hp, wp = ho // 2, wo // 2
    out = np.zeros((c_out * hp * wp, words), dtype=np.uint64)
    for c in range(c_out):
        for py in range(hp):
            for px in range(wp):
                acc = zero.copy()
                for dy in range(2):
                    for dx in range(2):
                        g = gates_at(c, 2 * py + dy, 2 * px + dx)
                        t0 = _bit_op(int(gates[c, 4]), g[0], g[1])
                        t1 = _bit_op(int(gates[c, 5]), g[2], g[3])
                        acc |= _bit_op(int(gates[c, 6]), t0, t1)
                out[(c * hp + py) * wp + px] = acc
    return out
