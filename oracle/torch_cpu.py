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


def group_sum(x: torch.Tensor, k: int, tau: float) -> torch.Tensor:
    if x.shape[-1] % k:
        x = torch.cat([x, torch.zeros((x.shape[0], k - x.shape[1] % k), dtype=x.dtype)], dim=1)
    return x.reshape(x.shape[0], k, x.shape[1] // k).sum(-1) / tau


class CpuDenseNet:
    """CPU copy of a dense network: per layer (indices, gate_sequence, logits leaf)."""

    def __init__(self, layers, k: int, tau: float, dtype=torch.float32):
        self.layers = [(ind.cpu(), gs.cpu(), lg.detach().cpu().to(dtype).clone().requires_grad_(True))
                       for ind, gs, lg in layers]
        self.k, self.tau, self.dtype = k, tau, dtype

    @classmethod
    def from_model(cls, model, dtype=torch.float32):
        from_layers, k, tau = [], None, None
        for m in model:
            if hasattr(m, "indices"):
                from_layers.append((m.indices, m.gate_sequence, m.weights))
            elif hasattr(m, "k"):
                k, tau = m.k, m.tau
        return cls(from_layers, k, tau, dtype)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h = x.cpu().to(self.dtype)
        for ind, gs, lg in self.layers:
            h = layer_forward(h, ind, gs, lg)
        return group_sum(h, self.k, self.tau)

    def train_step(self, x: torch.Tensor, labels: torch.Tensor) -> float:
        for _, _, lg in self.layers:
            lg.grad = None
        loss = torch.nn.functional.cross_entropy(self.forward(x), labels.cpu())
        loss.backward()
        return float(loss)
