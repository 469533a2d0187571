"""The discretised Boolean circuit of a trained network, its stage-1 pruning, and its packed
evaluation on the GPU.

A frozen (or eval-mode) network is a circuit of two-input gates: every neuron of a dense or
conv layer keeps the opcode and the two inputs of its winner slot (compiler/extract.py:47-197;
a conv tap outside the input plane is the constant 0).  Signals are numbered inputs first
(0 .. D-1), then every layer's neurons in order; GroupSum sums the last layer's signals in k
zero-padded groups (compiler/ir.py:62-91).

`naive_prune` is the compiler's stage-1 pruning (compiler/prune.py:164-291, the paper's simple
strategy): references are resolved through the circuit, an inverted reference is folded into
the truth table of the gate reading it, constants are folded, a gate reading one signal twice
collapses, and constant, identity and negation gates are replaced by (possibly inverted)
references; the gates that remain, among those reachable from the outputs, are the circuit's
BOPs.  It runs over whole layers at once (numpy), with the same result as the reference's
memoised recursion from the outputs (a gate is kept when it is reached through the original
wiring and does not simplify away).

`PackedCircuit` evaluates a pruned circuit with the packed kernels (64 samples per word):
one cl_eval_packed_indexed launch per original layer over a single signal buffer (inputs,
then the kept gates), one more that gathers the class sources (a reference, its negation or a
constant), and cl_group_bit_sum.  It replaces the reference's bool evaluator of the pruned
circuit (simulation/consistency.py:147-213).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _capi
from . import difflogic_hip as _dl
from .layers import ConvLayer, GroupSum, LogicLayer, PackBitsTensor

GATE_NAMES = ("CONST0", "AND", "A_AND_NOT_B", "A", "NOT_A_AND_B", "B", "XOR", "OR", "NOR",
              "XNOR", "NOT_B", "B_IMPLIES_A", "NOT_A", "A_IMPLIES_B", "NAND", "CONST1")

# TRUTH[g, a, b]: bit 3 - 2a - b of opcode g (the opcode order of compiler/gates.py:5-22)
TRUTH = np.array([[[(g >> (3 - 2 * a - b)) & 1 for b in (0, 1)] for a in (0, 1)]
                  for g in range(16)], dtype=np.int8)


def _gate_of(t: np.ndarray) -> int:
    return int(t[0, 0]) << 3 | int(t[0, 1]) << 2 | int(t[1, 0]) << 1 | int(t[1, 1])


# the gate that reads NOT a (NOT b) in place of a (b): rows (columns) of the table swapped
INVERT_A = np.array([_gate_of(TRUTH[g][::-1, :]) for g in range(16)], dtype=np.int64)
INVERT_B = np.array([_gate_of(TRUTH[g][:, ::-1]) for g in range(16)], dtype=np.int64)


@dataclass
class Circuit:
    """input_dim inputs, then the layers' nodes; a / b are global signal ids (-1: constant 0)."""
    input_dim: int
    gates: list            # per layer: int64 [n] opcodes
    a: list                # per layer: int64 [n]
    b: list                # per layer: int64 [n]
    k: int
    tau: float = 1.0

    @property
    def node_count(self) -> int:
        return int(sum(len(g) for g in self.gates))

    @property
    def layer_starts(self) -> list:
        starts, s = [], self.input_dim
        for g in self.gates:
            starts.append(s)
            s += len(g)
        return starts

    @property
    def out_start(self) -> int:
        return self.layer_starts[-1]

    @property
    def out_dim(self) -> int:
        return len(self.gates[-1])

    @property
    def group_size(self) -> int:
        return -(-self.out_dim // self.k)


def extract_circuit(model) -> Circuit:
    """The circuit of `model` (LogicLayer / ConvLayer modules, Flatten, a final GroupSum) at
    its winner slots: `w` for a frozen layer, else the argmax of its logits (compiler/
    extract.py:47-197)."""
    mods = [m for m in model if not isinstance(m, torch.nn.Flatten)]
    if not mods or not isinstance(mods[-1], GroupSum):
        raise ValueError("the network must end with a GroupSum")
    layers = mods[:-1]
    if not layers or not all(isinstance(m, LogicLayer) for m in layers):
        raise ValueError("the circuit takes LogicLayer / ConvLayer modules, Flatten and GroupSum")
    def features_in(m):
        # a ConvLayer's in_dim counts its padded plane; its inputs are the unpadded features
        return int(np.prod(m.in_shape)) if isinstance(m, ConvLayer) else int(m.in_dim)

    gates, aa, bb = [], [], []
    start = features_in(layers[0])
    input_dim = start
    prev_start, prev_dim = 0, start
    with torch.no_grad():
        for m in layers:
            if features_in(m) != prev_dim:
                raise ValueError(f"layer expects {features_in(m)} inputs, gets {prev_dim}")
            w = getattr(m, "w", None)
            if w is None:
                w = m._argmax_slots()
            ia, ib, gate = m.packed_tables(w)[:3]
            ia = ia.to(torch.int64).cpu().numpy()
            ib = ib.to(torch.int64).cpu().numpy()
            g = gate.to(torch.int64).cpu().numpy() & 15
            if isinstance(m, ConvLayer):
                bad = np.zeros(len(g), dtype=bool)       # taps outside the plane are -1
            else:
                bad = (ia >= m.in_dim) | (ib >= m.in_dim)
            if bad.any():
                raise ValueError("a neuron's winner slot or input is out of range")
            gates.append(g)
            aa.append(np.where(ia < 0, -1, ia + prev_start))
            bb.append(np.where(ib < 0, -1, ib + prev_start))
            prev_start, prev_dim = start, int(m.out_dim)
            start += int(m.out_dim)
    gs = mods[-1]
    return Circuit(input_dim, gates, aa, bb, int(gs.k), float(gs.tau))


_CONST, _REF, _GATE = 0, 1, 2


@dataclass
class PrunedCircuit:
    """Kept gates in node-id order (node_id, layer, gate, a, b: global signal ids of inputs or
    kept gates) and the class sources [k, group_size]: src_signal (-1 for a constant), inverted,
    const_value."""
    input_dim: int
    node_id: np.ndarray
    layer: np.ndarray
    gate: np.ndarray
    a: np.ndarray
    b: np.ndarray
    src_signal: np.ndarray
    src_inverted: np.ndarray
    src_const: np.ndarray
    tau: float = 1.0
    metadata: dict = field(default_factory=dict)

    @property
    def bop_count(self) -> int:
        return int(len(self.node_id))

    @property
    def num_classes(self) -> int:
        return int(self.src_signal.shape[0])

    def gate_histogram(self) -> dict:
        counts = np.bincount(self.gate, minlength=16)
        return {GATE_NAMES[g]: int(c) for g, c in enumerate(counts) if c}


def naive_prune(c: Circuit) -> PrunedCircuit:
    """Stage-1 pruning of `c` (compiler/prune.py:164-291), layer by layer."""
    total = c.input_dim + c.node_count
    kind = np.full(total, _REF, dtype=np.int8)
    ref = np.arange(total, dtype=np.int64)       # _REF: the referenced signal; _GATE: itself
    inv = np.zeros(total, dtype=bool)
    cval = np.zeros(total, dtype=np.int8)
    kept_gate = np.zeros(total, dtype=np.int64)
    kept_a = np.zeros(total, dtype=np.int64)
    kept_b = np.zeros(total, dtype=np.int64)

    def operand(src):
        """An input's expression, with a kept gate read as a plain reference to itself."""
        is_c = src < 0
        s = np.where(is_c, 0, src)
        k_ = np.where(is_c, _CONST, np.where(kind[s] == _CONST, _CONST, _REF))
        r = np.where(kind[s] == _GATE, s, ref[s])
        v = np.where(is_c, 0, cval[s])
        i = np.where(k_ == _REF, np.where(kind[s] == _GATE, False, inv[s]), False)
        return k_, r, i, v

    for start, g0, a_src, b_src in zip(c.layer_starts, c.gates, c.a, c.b):
        n = len(g0)
        ids = np.arange(start, start + n)
        ka, ra, ia, va = operand(a_src)
        kb, rb, ib, vb = operand(b_src)
        g = np.asarray(g0, dtype=np.int64) & 15
        g = np.where((ka == _REF) & ia, INVERT_A[g], g)
        g = np.where((kb == _REF) & ib, INVERT_B[g], g)
        k_out = np.full(n, _GATE, dtype=np.int8)
        r_out = ids.copy()
        i_out = np.zeros(n, dtype=bool)
        c_out = np.zeros(n, dtype=np.int8)

        def set_fn(mask, f0, f1, sig):
            # the function of one signal with values f0 at 0 and f1 at 1
            const = mask & (f0 == f1)
            k_out[const] = _CONST
            c_out[const] = f0[const]
            r = mask & (f0 != f1)
            k_out[r] = _REF
            r_out[r] = sig[r]
            i_out[r] = f0[r] == 1

        cc = (ka == _CONST) & (kb == _CONST)
        k_out[cc] = _CONST
        c_out[cc] = TRUTH[g, va, vb][cc]
        m = (ka == _CONST) & (kb == _REF)
        set_fn(m, TRUTH[g, va, 0], TRUTH[g, va, 1], rb)
        m = (ka == _REF) & (kb == _CONST)
        set_fn(m, TRUTH[g, 0, vb], TRUTH[g, 1, vb], ra)
        both = (ka == _REF) & (kb == _REF)
        same = both & (ra == rb)
        set_fn(same, TRUTH[g, 0, 0], TRUTH[g, 1, 1], ra)
        diff = both & (ra != rb)
        cg = diff & ((g == 0) | (g == 15))
        k_out[cg] = _CONST
        c_out[cg] = (g[cg] == 15)
        for gid, sig, neg in ((3, ra, False), (5, rb, False), (10, rb, True), (12, ra, True)):
            m = diff & (g == gid)
            k_out[m] = _REF
            r_out[m] = sig[m]
            i_out[m] = neg
        kind[ids], ref[ids], inv[ids], cval[ids] = k_out, r_out, i_out, c_out
        kept_gate[ids], kept_a[ids], kept_b[ids] = g, ra, rb

    # reached through the original wiring from the outputs (the recursion visits both inputs
    # of every gate it reaches, whatever the gate simplifies to)
    reached = np.zeros(total, dtype=bool)
    gsz = c.group_size
    outs = c.out_start + np.arange(c.out_dim)
    reached[outs] = True
    for start, a_src, b_src in reversed(list(zip(c.layer_starts, c.a, c.b))):
        n = len(a_src)
        hit = reached[start:start + n]
        for src in (a_src, b_src):
            s = src[hit]
            reached[s[s >= 0]] = True
    live = np.flatnonzero(reached & (kind == _GATE))
    live = live[live >= c.input_dim]
    layer_of = np.searchsorted(np.asarray(c.layer_starts), live, side="right") - 1
    # class sources [k, gsz]; padding entries are the constant 0
    src_sig = np.full((c.k, gsz), -1, dtype=np.int64)
    src_inv = np.zeros((c.k, gsz), dtype=bool)
    src_c = np.zeros((c.k, gsz), dtype=np.int8)
    j = np.arange(c.out_dim)
    s = outs
    ks = kind[s]
    cls, pos = j // gsz, j % gsz
    is_c = ks == _CONST
    src_c[cls[is_c], pos[is_c]] = cval[s[is_c]]
    is_r = ks == _REF
    src_sig[cls[is_r], pos[is_r]] = ref[s[is_r]]
    src_inv[cls[is_r], pos[is_r]] = inv[s[is_r]]
    is_g = ks == _GATE
    src_sig[cls[is_g], pos[is_g]] = s[is_g]
    return PrunedCircuit(c.input_dim, live, layer_of, kept_gate[live], kept_a[live],
                         kept_b[live], src_sig, src_inv, src_c, c.tau,
                         {"pruning_stage": "naive", "original_node_count": c.node_count,
                          "original_layer_count": len(c.gates)})


class PackedCircuit:
    """A pruned circuit on the device: call it with a PackBitsTensor of the inputs (or its
    [input_dim, words] tensor) for int32 class counts [samples, k]."""

    def __init__(self, pruned: PrunedCircuit, device="cuda"):
        dev = torch.device(device)
        D, n = pruned.input_dim, pruned.bop_count
        self.input_dim, self.k = D, pruned.num_classes
        self.gsz = int(pruned.src_signal.shape[1])
        # rows: inputs 0 .. D-1, kept gates D .. D+n-1 in node-id order
        ids = pruned.node_id
        lut = np.full(int(ids.max()) + 1 if n else D, -1, dtype=np.int64)
        lut[ids] = D + np.arange(n)

        def rows_of(sig):
            sig = np.asarray(sig, dtype=np.int64)
            out = np.where(sig < D, sig, 0)
            g = sig >= D
            if g.any():
                if int(sig[g].max()) >= len(lut) or (lut[sig[g]] < 0).any():
                    raise ValueError("a kept gate or class source reads a signal that is "
                                     "neither an input nor a kept gate")
                out[g] = lut[sig[g]]
            return out

        self.launches = []
        if n:
            layers = pruned.layer
            bounds = np.flatnonzero(np.diff(layers)) + 1
            for lo, hi in zip(np.r_[0, bounds], np.r_[bounds, n]):
                ia = torch.as_tensor(rows_of(pruned.a[lo:hi]).astype(np.int32), device=dev)
                ib = torch.as_tensor(rows_of(pruned.b[lo:hi]).astype(np.int32), device=dev)
                g = torch.as_tensor(pruned.gate[lo:hi].astype(np.uint8), device=dev)
                self.launches.append((D + int(lo), int(hi - lo), ia, ib, g))
        # the class-source gather: A / NOT_A of a row, CONST0 / CONST1 of no row
        sig = pruned.src_signal.reshape(-1)
        is_sig = sig >= 0
        src_rows = np.where(is_sig, rows_of(np.where(is_sig, sig, 0)), -1)
        op = np.where(is_sig, np.where(pruned.src_inverted.reshape(-1), 12, 3),
                      np.where(pruned.src_const.reshape(-1) == 1, 15, 0))
        self.out_rows = int(sig.size)
        self.gather = (torch.as_tensor(src_rows.astype(np.int32), device=dev),
                       torch.as_tensor(src_rows.astype(np.int32), device=dev),
                       torch.as_tensor(op.astype(np.uint8), device=dev))
        self.total_rows = D + n
        self.device = dev

    def __call__(self, x) -> torch.Tensor:
        if isinstance(x, PackBitsTensor):
            words, pad = x.t, x.pad_len
        else:
            words, pad = x, 0
        _dl._check(words, "x")
        if words.dim() != 2 or words.shape[0] != self.input_dim:
            raise RuntimeError(f"x must be [{self.input_dim}, words], got {tuple(words.shape)}")
        row_bytes = words.shape[1] * words.element_size()
        buf = torch.empty((self.total_rows + self.out_rows, words.shape[1]), dtype=words.dtype,
                          device=words.device)
        buf[:self.input_dim].copy_(words)
        stream = _dl.stream_of(words)
        base = buf.data_ptr()
        with torch.cuda.device(words.device):
            for start, n, ia, ib, g in self.launches:
                # reads rows < start (inputs and earlier layers' gates), writes [start, start+n)
                _capi.call("cl_eval_packed_indexed", base, ia.data_ptr(), ib.data_ptr(),
                           g.data_ptr(), None, base + start * row_bytes, start, n, row_bytes,
                           stream)
            out = base + self.total_rows * row_bytes
            ia, ib, g = self.gather
            _capi.call("cl_eval_packed_indexed", base, ia.data_ptr(), ib.data_ptr(),
                       g.data_ptr(), None, out, self.total_rows, self.out_rows, row_bytes,
                       stream)
        last = PackBitsTensor.from_packed(buf[self.total_rows:], pad)
        return last.group_sum(self.k)
