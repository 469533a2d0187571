"""CPU restatement of the reference's Boolean-circuit compiler path -- TEST INFRASTRUCTURE ONLY.

Only tests/ (and bench.py's cpu_baseline leg) may import this module; the product
(compactlogic_amd.circuit) has its own implementation and never calls it.

Restated, not imported (the reference is read as text):
  * gate truth tables            compiler/gates.py:29-63 (truth_eval_scalar)
  * circuit extraction           compiler/extract.py:47-197 (dense: winner slot per neuron;
                                 conv: one node per output (c, y, x), NCHW flattening, taps
                                 outside the input plane become constant-0 inputs)
  * GroupSum groups              compiler/ir.py:62-91 (zero-padded to a multiple of k)
  * stage-1 ("naive") pruning    compiler/prune.py:164-291 (memoised simplification from the
                                 outputs: inverted references folded into the reading gate's
                                 truth table, constants folded, same-signal gates collapsed,
                                 constant / identity / negation gates replaced by references)
  * bool evaluators              simulation/consistency.py:58-213 (unpruned and pruned class
                                 counts)

Circuit form used here (plain numpy):
  {"input_dim": D,
   "layers": [{"gate": int[n], "a": int[n], "b": int[n]}, ...]   # global signal ids, -1 = const 0
   "k": k, "out_start": s, "out_dim": F}
Node ids are consecutive after the inputs, layer by layer.

Pinning (tests/test_circuit_cpu.py): the truth table against the closed form
g(a, b) = bit (3 - 2a - b) of g and the gate names; the pruner by exhaustive evaluation of
pruned against unpruned circuits on every input of small random circuits, and by hand-worked
circuits whose pruned form is known.
"""
from __future__ import annotations

import numpy as np

# compiler/gates.py:29-63, one formula per gate id
_FORMULAS = (
    lambda a, b: 0,                    # CONST0
    lambda a, b: a & b,                # AND
    lambda a, b: a & (1 - b),          # A_AND_NOT_B
    lambda a, b: a,                    # A
    lambda a, b: (1 - a) & b,          # NOT_A_AND_B
    lambda a, b: b,                    # B
    lambda a, b: a ^ b,                # XOR
    lambda a, b: a | b,                # OR
    lambda a, b: 1 - (a | b),          # NOR
    lambda a, b: 1 - (a ^ b),          # XNOR
    lambda a, b: 1 - b,                # NOT_B
    lambda a, b: (1 - b) | a,          # B_IMPLIES_A
    lambda a, b: 1 - a,                # NOT_A
    lambda a, b: (1 - a) | b,          # A_IMPLIES_B
    lambda a, b: 1 - (a & b),          # NAND
    lambda a, b: 1,                    # CONST1
)
TRUTH = np.array([[[f(a, b) for b in (0, 1)] for a in (0, 1)] for f in _FORMULAS], dtype=np.int64)


def truth(g: int, a: int, b: int) -> int:
    return int(TRUTH[g, a, b])


def gate_of_table(t00: int, t01: int, t10: int, t11: int) -> int:
    """compiler/prune.py:93-104: the gate id with this truth table."""
    for g in range(16):
        if (truth(g, 0, 0), truth(g, 0, 1), truth(g, 1, 0), truth(g, 1, 1)) == (t00, t01, t10, t11):
            return g
    raise ValueError("no gate has this truth table")


def invert_a(g: int) -> int:
    """compiler/prune.py:107-114: the gate reading NOT a."""
    return gate_of_table(truth(g, 1, 0), truth(g, 1, 1), truth(g, 0, 0), truth(g, 0, 1))


def invert_b(g: int) -> int:
    """compiler/prune.py:117-124: the gate reading NOT b."""
    return gate_of_table(truth(g, 0, 1), truth(g, 0, 0), truth(g, 1, 1), truth(g, 1, 0))


# ---------------------------------------------------------------------------------- extraction

def extract_dense(weights, indices, gate_sequence, input_start: int):
    """compiler/extract.py:47-95: winner slot = argmax of the logits (first maximum)."""
    w = np.asarray(weights).argmax(axis=1)
    rows = np.arange(w.shape[0])
    a = np.asarray(indices)[0, rows, w].astype(np.int64) + input_start
    b = np.asarray(indices)[1, rows, w].astype(np.int64) + input_start
    g = np.asarray(gate_sequence)[rows, w].astype(np.int64)
    return {"gate": g, "a": a, "b": b}


def extract_conv(weights, gate_sequence, offsets_ch, offsets_h, offsets_w, in_shape, out_shape,
                 stride: int, input_start: int):
    """compiler/extract.py:98-197: output feature (c, y, x) in NCHW order reads input feature
    (ch * H + y * stride + dh) * W + x * stride + dw of its channel's winner slot, or the
    constant 0 when the tap falls outside the plane."""
    c_in, h_in, w_in = in_shape
    c_out, h_out, w_out = out_shape
    win = np.asarray(weights).argmax(axis=1)
    rows = np.arange(c_out)
    g = np.asarray(gate_sequence)[rows, win].astype(np.int64)
    gate, a, b = [], [], []
    for c in range(c_out):
        taps = []
        for side in (0, 1):
            ch = int(np.asarray(offsets_ch)[side, c, win[c]])
            dh = int(np.asarray(offsets_h)[side, c, win[c]])
            dw = int(np.asarray(offsets_w)[side, c, win[c]])
            taps.append((ch, dh, dw))
        for y in range(h_out):
            for x in range(w_out):
                gate.append(g[c])
                for side, dst in ((0, a), (1, b)):
                    ch, dh, dw = taps[side]
                    iy, ix = y * stride + dh, x * stride + dw
                    if 0 <= iy < h_in and 0 <= ix < w_in:
                        dst.append(input_start + (ch * h_in + iy) * w_in + ix)
                    else:
                        dst.append(-1)
    return {"gate": np.array(gate, np.int64), "a": np.array(a, np.int64),
            "b": np.array(b, np.int64)}


def groups(circuit):
    """compiler/ir.py:76-91: class c reads signals out_start + c * gsz + j, None past out_dim."""
    k, F, s = circuit["k"], circuit["out_dim"], circuit["out_start"]
    gsz = -(-F // k)
    return [[s + c * gsz + j if c * gsz + j < F else None for j in range(gsz)] for c in range(k)]


# --------------------------------------------------------------------------------- evaluation

def evaluate(circuit, bits: np.ndarray) -> np.ndarray:
    """simulation/consistency.py:58-128: class counts [n, k] of bool inputs [n, D]."""
    n = bits.shape[0]
    sig = [bits[:, j].astype(np.int64) for j in range(circuit["input_dim"])]
    zero = np.zeros(n, np.int64)
    for layer in circuit["layers"]:
        for g, a, b in zip(layer["gate"], layer["a"], layer["b"]):
            va = sig[a] if a >= 0 else zero
            vb = sig[b] if b >= 0 else zero
            sig.append(TRUTH[g][va, vb])
    out = np.zeros((n, circuit["k"]), np.int64)
    for c, grp in enumerate(groups(circuit)):
        for s in grp:
            if s is not None:
                out[:, c] += sig[s]
    return out


def evaluate_pruned(pruned, bits: np.ndarray) -> np.ndarray:
    """simulation/consistency.py:147-213: the pruned circuit's class counts."""
    n = bits.shape[0]
    sig = {j: bits[:, j].astype(np.int64) for j in range(pruned["input_dim"])}
    for node_id, g, a, b in pruned["nodes"]:
        sig[node_id] = TRUTH[g][sig[a], sig[b]]
    out = np.zeros((n, len(pruned["groups"])), np.int64)
    for c, grp in enumerate(pruned["groups"]):
        for src in grp:
            if src[0] == "const":
                out[:, c] += src[1]
            else:
                v = sig[src[1]]
                out[:, c] += (1 - v) if src[2] else v
    return out


# ------------------------------------------------------------------------------------ pruning

def naive_prune(circuit):
    """compiler/prune.py:164-291 restated.  Returns {"input_dim", "nodes": [(node_id, gate,
    a, b)] in node-id order (the reached gates that stay non-trivial), "groups": per class a
    list of ("const", v) / ("sig", signal_id, inverted)}.  Expressions: ("const", v),
    ("ref", signal, inverted), ("gate", signal)."""
    D = circuit["input_dim"]
    node = {}
    nid = D
    for layer in circuit["layers"]:
        for g, a, b in zip(layer["gate"], layer["a"], layer["b"]):
            node[nid] = (int(g), int(a), int(b))
            nid += 1
    memo = {}
    live = {}

    def expr_of_input(src):
        # compiler/prune.py:184-188 (a constant gate input is the constant 0)
        return ("const", 0) if src < 0 else simplify(src)

    def simplify(s):
        # compiler/prune.py:190-201
        if s < D:
            return ("ref", s, False)
        if s in memo:
            return memo[s]
        g, a, b = node[s]
        ea, eb = expr_of_input(a), expr_of_input(b)
        memo[s] = r = simplify_gate(s, g, ea, eb)
        return r

    def simplify_gate(s, g, ea, eb):
        # compiler/prune.py:203-265
        if ea[0] == "gate":
            ea = ("ref", ea[1], False)
        if eb[0] == "gate":
            eb = ("ref", eb[1], False)
        if ea[0] == "ref" and ea[2]:
            g, ea = invert_a(g), ("ref", ea[1], False)
        if eb[0] == "ref" and eb[2]:
            g, eb = invert_b(g), ("ref", eb[1], False)
        if ea[0] == "const" and eb[0] == "const":
            return ("const", truth(g, ea[1], eb[1]))
        if ea[0] == "const":
            return collapse(truth(g, ea[1], 0), truth(g, ea[1], 1), eb[1])
        if eb[0] == "const":
            return collapse(truth(g, 0, eb[1]), truth(g, 1, eb[1]), ea[1])
        if ea[1] == eb[1]:
            return collapse(truth(g, 0, 0), truth(g, 1, 1), ea[1])
        if g in (0, 15):
            return ("const", 0 if g == 0 else 1)
        if g == 3:
            return ("ref", ea[1], False)
        if g == 5:
            return ("ref", eb[1], False)
        if g == 10:
            return ("ref", eb[1], True)
        if g == 12:
            return ("ref", ea[1], True)
        live[s] = (s, g, ea[1], eb[1])
        return ("gate", s)

    def collapse(f0, f1, sig):
        # compiler/prune.py:127-161: the function of one signal with values f0 (at 0), f1 (at 1)
        if f0 == f1:
            return ("const", f0)
        return ("ref", sig, f0 == 1)

    out_groups = []
    for grp in groups(circuit):
        srcs = []
        for s in grp:
            if s is None:
                srcs.append(("const", 0))
                continue
            e = simplify(s)
            if e[0] == "const":
                srcs.append(("const", e[1]))
            elif e[0] == "ref":
                srcs.append(("sig", e[1], e[2]))
            else:
                srcs.append(("sig", e[1], False))
        out_groups.append(srcs)
    return {"input_dim": D, "nodes": [live[s] for s in sorted(live)], "groups": out_groups}
