"""Pure-PyTorch CPU training step -- TEST INFRASTRUCTURE / CPU BASELINE ONLY.

The reference's CPU formulation of a logic layer is the difflogic `bin_op_s` relaxation
(third_party/convlogic_source_code/src/difflogic/functional.py:27-71, used by
difflogic.py:112-123): gather the operand columns, evaluate the 16 relaxed gates and mix
them with the softmax probabilities; autograd provides the backward.  Here it is applied
with compactlogic's slot semantics (compactlogic/compactlogic.py:83-118): slot g of neuron o
reads its own pair (a[o,g], b[o,g]) and opcode gate_sequence[o,g].  When every neuron has a
single pair and gate_sequence = arange(16) (the benchmark configs) this is exactly
`bin_op_s(x[:, a], x[:, b], softmax(weights))`.

Used to time the CPU baseline (bench.py) and, at small sizes, as a float32 cross-check of
the float64 oracle in tests.
"""
from __future__ import annotations

import torch

# The 16 relaxed gates, in opcode order, as polynomials in (a, b).
_GATES = (
    lambda a, b: torch.zeros_like(a),
    lambda a, b: a * b,
    lambda a, b: a - a * b,
    lambda a, b: a,
    lambda a, b: b - a * b,
    lambda a, b: b,
    lambda a, b: a + b - 2 * a * b,
    lambda a, b: a + b - a * b,
    lambda a, b: 1 - (a + b - a * b),
    lambda a, b: 1 - (a + b - 2 * a * b),
    lambda a, b: 1 - b,
    lambda a, b: 1 - b + a * b,
    lambda a, b: 1 - a,
    lambda a, b: 1 - a + a * b,
    lambda a, b: 1 - a * b,
    lambda a, b: torch.ones_like(a),
)


def bin_op_s(a: torch.Tensor, b: torch.Tensor, probs: torch.Tensor) -> torch.Tensor:
    """sum_i probs[..., i] * gate_i(a, b) over the 16 gates."""
    r = torch.zeros_like(a)
    for i, gate in enumerate(_GATES):
        r = r + probs[..., i] * gate(a, b)
    return r


def layer_forward(x: torch.Tensor, indices: torch.Tensor, gate_sequence: torch.Tensor,
                  logits: torch.Tensor) -> torch.Tensor:
    """x [batch, in] -> [batch, out] for one soft layer (float CPU tensors)."""
    probs = torch.softmax(logits, dim=-1)
    g_n = logits.shape[1]
    shared = bool((indices == indices[..., :1]).all())
    arange_gates = g_n == 16 and bool((gate_sequence.long() == torch.arange(16)).all())
    if shared and arange_gates:
        return bin_op_s(x[:, indices[0, :, 0]], x[:, indices[1, :, 0]], probs)
    y = torch.zeros((x.shape[0], indices.shape[1]), dtype=x.dtype)
    gs = gate_sequence.long()
    for g in range(g_n):
        a, b = x[:, indices[0, :, g]], x[:, indices[1, :, g]]
        op = torch.stack([gate(a, b) for gate in _GATES], dim=-1)     # [batch, out, 16]
        sel = torch.gather(op, 2, gs[:, g].view(1, -1, 1).expand(x.shape[0], -1, 1)).squeeze(-1)
        y = y + probs[:, g] * sel
    return y


def conv_forward(x: torch.Tensor, och: torch.Tensor, oh: torch.Tensor, ow: torch.Tensor,
                 gate_sequence: torch.Tensor, logits: torch.Tensor, stride: int,
                 out_hw: tuple[int, int]) -> torch.Tensor:
    """x [N, C, H, W] -> [N, Cout, Ho, Wo] for one soft ConvLayer: slot (c, g) reads the taps
    x[n, ch, oy*stride + dh, ox*stride + dw] (0 outside the plane) of both operands, as in
    compactlogic/cuda/convlogic_kernel.cu:98-137, and the slots are mixed with softmax(logits).
    Each opcode's relaxed gate is applied through its four polynomial coefficients, read off
    _GATES at the corners of the unit square."""
    probs = torch.softmax(logits, dim=-1)
    n, _, h, w = x.shape
    ho, wo = out_hw
    lo = max(0, -int(min(oh.min(), ow.min())))
    hi_h = max(0, (ho - 1) * stride + int(oh.max()) - (h - 1))
    hi_w = max(0, (wo - 1) * stride + int(ow.max()) - (w - 1))
    xp = torch.nn.functional.pad(x, (lo, hi_w, lo, hi_h))
    oy = (torch.arange(ho) * stride).view(1, 1, ho, 1)
    ox = (torch.arange(wo) * stride).view(1, 1, 1, wo)
    taps = []
    for side in (0, 1):
        ch = och[side].long().unsqueeze(-1).unsqueeze(-1)                 # [Cout, G, 1, 1]
        iy = oy + oh[side].long().unsqueeze(-1).unsqueeze(-1) + lo
        ix = ox + ow[side].long().unsqueeze(-1).unsqueeze(-1) + lo
        taps.append(xp[:, ch, iy, ix])                                     # [N, Cout, G, Ho, Wo]
    a, b = taps
    one, zero = torch.ones(()), torch.zeros(())
    corners = torch.tensor([[float(gate(zero, zero)), float(gate(one, zero)),
                             float(gate(zero, one)), float(gate(one, one))] for gate in _GATES],
                           dtype=x.dtype)                                  # f00, f10, f01, f11
    coef = torch.stack((corners[:, 0], corners[:, 1] - corners[:, 0], corners[:, 2] - corners[:, 0],
                        corners[:, 3] - corners[:, 1] - corners[:, 2] + corners[:, 0]), dim=1)
    c = coef[gate_sequence.long()]                                         # [Cout, G, 4]
    c = [c[..., i].unsqueeze(-1).unsqueeze(-1) for i in range(4)]
    op = c[0] + c[1] * a + c[2] * b + c[3] * (a * b)
    return (op * probs.unsqueeze(-1).unsqueeze(-1)).sum(2)


def _gate_coefficients(dtype) -> torch.Tensor:
    """[16, 4]: gate g(a, b) = c0 + c1 a + c2 b + c3 a b, read off _GATES at the corners."""
    one, zero = torch.ones(()), torch.zeros(())
    f = torch.tensor([[float(gate(zero, zero)), float(gate(one, zero)), float(gate(zero, one)),
                       float(gate(one, one))] for gate in _GATES], dtype=dtype)
    return torch.stack((f[:, 0], f[:, 1] - f[:, 0], f[:, 2] - f[:, 0],
                        f[:, 3] - f[:, 1] - f[:, 2] + f[:, 0]), dim=1)


def tree_block_forward(x: torch.Tensor, logits: torch.Tensor, selection: torch.Tensor,
                       stride, padding, kernel) -> torch.Tensor:
    """Complete logic-tree conv block, x [N, C, H, W] -> [N, Cout, Ho/2, Wo/2], as the
    reference's python path (third_party/convlogic_source_code/src/convlogic/
    convlogic_layer.py:236-321): 8 taps per output channel (selection = ch << 16 | row << 8 |
    col, zero outside the image), relaxed gates on the tap pairs, then on (0,1), (2,3) and the
    pair of those, mixed with softmax(logits) [Cout, 7, 16]; 2x2 max pool."""
    coef = torch.softmax(logits, dim=-1) @ _gate_coefficients(x.dtype)     # [Cout, 7, 4]
    sel = selection.long()
    ch, ry, rx = (sel >> 16) & 0xFFFF, (sel >> 8) & 0xFF, sel & 0xFF       # [Cout, 8]
    (sh, sw), (ph, pw), (kh, kw) = stride, padding, kernel
    n, _, h, w = x.shape
    ho, wo = (h + 2 * ph - kh) // sh + 1, (w + 2 * pw - kw) // sw + 1
    xp = torch.nn.functional.pad(x, (pw, pw, ph, ph))
    cout = sel.shape[0]
    iy = (torch.arange(ho) * sh).view(1, 1, ho, 1) + ry.view(cout, 8, 1, 1)
    ix = (torch.arange(wo) * sw).view(1, 1, 1, wo) + rx.view(cout, 8, 1, 1)
    taps = xp[:, ch.view(cout, 8, 1, 1), iy, ix]                           # [N, Cout, 8, Ho, Wo]

    def node(q, a, b):
        c = [coef[:, q, i].view(1, cout, 1, 1) for i in range(4)]
        return c[0] + c[1] * a + c[2] * b + c[3] * (a * b)

    g = [node(j, taps[:, :, 2 * j], taps[:, :, 2 * j + 1]) for j in range(4)]
    r = node(6, node(4, g[0], g[1]), node(5, g[2], g[3]))
    return torch.nn.functional.max_pool2d(r, 2)


def group_sum(x: torch.Tensor, k: int, tau: float) -> torch.Tensor:
    if x.shape[-1] % k:
        x = torch.cat([x, torch.zeros((x.shape[0], k - x.shape[1] % k), dtype=x.dtype)], dim=1)
    return x.reshape(x.shape[0], k, x.shape[1] // k).sum(-1) / tau


class CpuDenseNet:
    """CPU copy of a network of soft layers: ('dense', indices, gate_sequence, logits),
    ('conv', offsets_ch, offsets_h, offsets_w, gate_sequence, logits, stride, out_hw) and
    ('flatten',) stages, then GroupSum; the logits are leaves that receive gradients."""

    def __init__(self, layers, k: int, tau: float, dtype=torch.float32):
        self.layers = []
        for spec in layers:
            if len(spec) == 3:                      # (indices, gate_sequence, logits)
                spec = ("dense",) + tuple(spec)
            if spec[0] == "flatten":
                self.layers.append(spec)
                continue
            ntail = {"conv": 2, "tree": 3}.get(spec[0], 0)
            *bufs, lg = spec[1:len(spec) - ntail]
            leaf = lg.detach().cpu().to(dtype).clone().requires_grad_(True)
            tail = tuple(spec[len(spec) - ntail:])
            self.layers.append((spec[0],) + tuple(b.cpu() for b in bufs) + (leaf,) + tail)
        self.k, self.tau, self.dtype = k, tau, dtype

    @classmethod
    def from_model(cls, model, dtype=torch.float32):
        from_layers, k, tau = [], None, None
        for m in model:
            if hasattr(m, "selection") and getattr(m, "complete", False):
                from_layers.append(("tree", m.selection, m.weights, m.stride, m.padding,
                                    m.kernel))
            elif hasattr(m, "offsets_ch"):
                from_layers.append(("conv", m.offsets_ch, m.offsets_h, m.offsets_w,
                                    m.gate_sequence, m.weights, m.stride, tuple(m.out_shape[1:])))
            elif hasattr(m, "indices"):
                from_layers.append(("dense", m.indices, m.gate_sequence, m.weights))
            elif isinstance(m, torch.nn.Flatten):
                from_layers.append(("flatten",))
            elif hasattr(m, "k"):
                k, tau = m.k, m.tau
        return cls(from_layers, k, tau, dtype)

    def leaves(self):
        ntail = {"conv": 2, "tree": 3}
        return [spec[-1 - ntail.get(spec[0], 0)] for spec in self.layers if spec[0] != "flatten"]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h = x.cpu().to(self.dtype)
        for spec in self.layers:
            if spec[0] == "dense":
                h = layer_forward(h, *spec[1:])
            elif spec[0] == "conv":
                h = conv_forward(h, *spec[1:])
            elif spec[0] == "tree":
                h = tree_block_forward(h, spec[2], spec[1], *spec[3:])
            else:
                h = h.flatten(1)
        return group_sum(h, self.k, self.tau)

    def train_step(self, x: torch.Tensor, labels: torch.Tensor) -> float:
        for lg in self.leaves():
            lg.grad = None
        loss = torch.nn.functional.cross_entropy(self.forward(x), labels.cpu())
        loss.backward()
        return float(loss.detach())
