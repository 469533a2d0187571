"""The circuit path on the CPU: the oracle's restatement of the reference's gate tables and
stage-1 pruning (compiler/gates.py, compiler/prune.py) pinned by closed forms, exhaustive
evaluation and hand-worked circuits; the product's vectorised pruner and extraction
(compactlogic_amd.circuit) against the oracle; checkpoints in the reference's format
(experiments/experiment_script.py:520-547) written and read back."""
import json

import numpy as np
import pytest
import torch

from compactlogic_amd import checkpoint as ck
from compactlogic_amd import circuit as C
from compactlogic_amd.layers import ConvLayer, GroupSum, LogicLayer
from oracle import circuit_ref as R


# ------------------------------------------------------------------------------ oracle pinning

def test_truth_tables_closed_form_and_names():
    # g(a, b) = bit 3 - 2a - b of the opcode: the 16 two-input functions in the order AND = 1,
    # A = 3, B = 5, XOR = 6, OR = 7, NAND = 14 (compiler/gates.py:5-22)
    for g in range(16):
        for a in (0, 1):
            for b in (0, 1):
                assert R.truth(g, a, b) == (g >> (3 - 2 * a - b)) & 1
    named = {1: lambda a, b: a & b, 3: lambda a, b: a, 5: lambda a, b: b, 6: lambda a, b: a ^ b,
             7: lambda a, b: a | b, 14: lambda a, b: 1 - (a & b), 12: lambda a, b: 1 - a}
    for g, f in named.items():
        assert all(R.truth(g, a, b) == f(a, b) for a in (0, 1) for b in (0, 1))
    assert np.array_equal(C.TRUTH.astype(np.int64), R.TRUTH)


def test_inverted_operand_tables():
    for g in range(16):
        for a in (0, 1):
            for b in (0, 1):
                assert R.truth(R.invert_a(g), a, b) == R.truth(g, 1 - a, b)
                assert R.truth(R.invert_b(g), a, b) == R.truth(g, a, 1 - b)
        assert C.INVERT_A[g] == R.invert_a(g) and C.INVERT_B[g] == R.invert_b(g)


def circ(D, layers, k):
    """Oracle circuit from [(gates, a, b)] with global signal ids."""
    out_start = D + sum(len(g) for g, _, _ in layers[:-1])
    return {"input_dim": D, "k": k, "out_start": out_start, "out_dim": len(layers[-1][0]),
            "layers": [{"gate": np.array(g), "a": np.array(a), "b": np.array(b)}
                       for g, a, b in layers]}


def test_hand_worked_pruning():
    # inputs 0, 1; layer 1: n2 = NOT_A(0), n3 = AND(0, 1), n4 = CONST1, n5 = XOR(1, 1)
    # layer 2: n6 = NOT_A(n2) = x0, n7 = A(n3) = n3, n8 = AND(n4, n3) = n3, n9 = OR(n5, 1) = x1
    c = circ(2, [([12, 1, 15, 6], [0, 0, 0, 1], [0, 1, 1, 1]),
                 ([12, 3, 1, 7], [2, 3, 4, 5], [2, 3, 3, 1])], k=2)
    p = R.naive_prune(c)
    assert p["nodes"] == [(3, 1, 0, 1)]                         # only the AND survives
    assert p["groups"] == [[("sig", 0, False), ("sig", 3, False)],
                           [("sig", 3, False), ("sig", 1, False)]]
    # an inverted reference is folded into the reading gate: AND(NOT x0, x1) = NOT_A_AND_B
    c = circ(2, [([12, 5], [0, 0], [0, 1]), ([1, 3], [2, 3], [3, 3])], k=1)
    p = R.naive_prune(c)
    assert p["nodes"] == [(4, 4, 0, 1)]
    assert p["groups"] == [[("sig", 4, False), ("sig", 1, False)]]
    # a conv padding tap (constant 0): AND(0, x) = 0, OR(0, x) = x, NOR(0, x) = NOT x
    c = circ(1, [([1, 7, 8], [-1, -1, -1], [0, 0, 0])], k=3)
    p = R.naive_prune(c)
    assert p["nodes"] == []
    assert p["groups"] == [[("const", 0)], [("sig", 0, False)], [("sig", 0, True)]]
    # zero padding of the last group (compiler/ir.py:76-91): 3 outputs, k = 2 -> 2 + (1, pad)
    c = circ(2, [([1, 7, 6], [0, 0, 0], [1, 1, 1])], k=2)
    p = R.naive_prune(c)
    assert p["groups"][1][1] == ("const", 0) and len(p["nodes"]) == 3


def test_orphan_gate_reached_through_the_original_wiring_is_kept():
    # n3 = XOR(0, 1) is reached (input of n4) but n4 = CONST0-like AND(n3, NOT n3)? Use
    # n4 = AND(n3, c0): AND with a constant-0 input folds to 0, yet the reference's recursion
    # has simplified (and kept) n3 on the way (compiler/prune.py:190-201).
    c = circ(2, [([6], [0], [1]), ([1], [2], [-1])], k=1)
    p = R.naive_prune(c)
    assert p["nodes"] == [(2, 6, 0, 1)] and p["groups"] == [[("const", 0)]]
    q = C.naive_prune(C.Circuit(2, [np.array([6]), np.array([1])], [np.array([0]), np.array([2])],
                                [np.array([1]), np.array([-1])], 1))
    assert list(q.node_id) == [2] and q.src_signal[0, 0] == -1 and q.src_const[0, 0] == 0


def random_circuit(rng, D, widths, k, p_const=0.1, p_same=0.1):
    gates, A, B = [], [], []
    prev_start, prev, s = 0, D, D
    for w in widths:
        a = rng.integers(0, prev, w) + prev_start
        b = rng.integers(0, prev, w) + prev_start
        same = rng.random(w) < p_same
        b[same] = a[same]
        a[rng.random(w) < p_const] = -1
        b[rng.random(w) < p_const] = -1
        gates.append(rng.integers(0, 16, w))
        A.append(a)
        B.append(b)
        prev_start, prev, s = s, w, s + w
    return C.Circuit(D, gates, A, B, k)


def as_oracle(c: C.Circuit):
    return {"input_dim": c.input_dim, "k": c.k, "out_start": c.out_start, "out_dim": c.out_dim,
            "layers": [{"gate": g, "a": a, "b": b} for g, a, b in zip(c.gates, c.a, c.b)]}


def test_oracle_pruning_preserves_every_input_exhaustively():
    rng = np.random.default_rng(1)
    for _ in range(150):
        D = int(rng.integers(1, 9))
        c = as_oracle(random_circuit(rng, D, [int(rng.integers(1, 10))
                                               for _ in range(int(rng.integers(1, 5)))],
                                     int(rng.integers(1, 4))))
        bits = (np.arange(2 ** D)[:, None] >> np.arange(D)[None]) & 1
        p = R.naive_prune(c)
        assert np.array_equal(R.evaluate(c, bits), R.evaluate_pruned(p, bits))
        assert len(p["nodes"]) <= sum(len(l["gate"]) for l in c["layers"])
        # a kept gate is never constant, identity or negation, and reads two signals
        for _, g, a, b in p["nodes"]:
            assert g not in (0, 3, 5, 10, 12, 15) and a != b


def test_product_pruner_equals_oracle():
    rng = np.random.default_rng(2)
    for _ in range(200):
        c = random_circuit(rng, int(rng.integers(2, 20)),
                           [int(rng.integers(2, 40)) for _ in range(int(rng.integers(1, 6)))],
                           int(rng.integers(1, 5)), p_const=float(rng.choice([0.0, 0.1, 0.3])))
        p, r = C.naive_prune(c), R.naive_prune(as_oracle(c))
        assert [(int(i), int(g), int(a), int(b)) for i, g, a, b in
                zip(p.node_id, p.gate, p.a, p.b)] == [tuple(x) for x in r["nodes"]]
        for ci, grp in enumerate(r["groups"]):
            for j, src in enumerate(grp):
                if src[0] == "const":
                    assert p.src_signal[ci, j] == -1 and p.src_const[ci, j] == src[1]
                else:
                    assert (p.src_signal[ci, j], bool(p.src_inverted[ci, j])) == src[1:]
        assert p.bop_count == len(r["nodes"])


# ----------------------------------------------------------------------------------- extraction

def test_extraction_matches_the_oracle_dense_and_conv():
    torch.manual_seed(0)
    conv = ConvLayer((3, 8, 8), padding=1, c_out=6, ks=3, stride=2, num_chn=1, num_gates=4)
    conv2 = ConvLayer(conv.out_shape, padding=0, c_out=5, ks=1, stride=1, num_chn=0, num_gates=4)
    dense = LogicLayer(conv2.out_dim, 40, num_gates=8)
    model = torch.nn.Sequential(conv, conv2, torch.nn.Flatten(), dense, GroupSum(4, 2.0, device="cpu"))
    model.eval()
    c = C.extract_circuit(model)
    sd = {k: v.numpy() for k, v in model.state_dict().items()}
    D = 3 * 8 * 8
    l0 = R.extract_conv(sd["0.weights"], sd["0.gate_sequence"], sd["0.offsets_ch"],
                        sd["0.offsets_h"], sd["0.offsets_w"], conv.in_shape, conv.out_shape,
                        conv.stride, 0)
    l1 = R.extract_conv(sd["1.weights"], sd["1.gate_sequence"], sd["1.offsets_ch"],
                        sd["1.offsets_h"], sd["1.offsets_w"], conv2.in_shape, conv2.out_shape,
                        conv2.stride, D)
    l2 = R.extract_dense(sd["3.weights"], sd["3.indices"], sd["3.gate_sequence"],
                         D + conv.out_dim)
    for got_g, got_a, got_b, ref in zip(c.gates, c.a, c.b, (l0, l1, l2)):
        assert np.array_equal(got_g, ref["gate"])
        assert np.array_equal(got_a, ref["a"]) and np.array_equal(got_b, ref["b"])
    assert (l0["a"] < 0).any()                           # the padding taps are exercised


# ----------------------------------------------------------------------------------- checkpoints

@pytest.mark.parametrize("struct", ["regular", "conv_spm"])
def test_checkpoint_round_trip_in_the_reference_format(tmp_path, struct):
    args = {"dataset": "mnist", "struct": struct, "num_gates": 16, "tau": 10.0,
            "model_scale": 400 if struct == "regular" else 4, "num_layers": 3}
    torch.manual_seed(3)
    model = ck.build_model(args)
    layers = [m for m in model if isinstance(m, LogicLayer)]
    layers[0].freeze()                                   # a frozen layer: its .w is not saved
    opt = torch.optim.Adam([p for p in model.parameters() if p.requires_grad], lr=0.01)
    path = tmp_path / "run" / "ckpt_best_100.pt"
    ck.save_checkpoint(path, 100, model, opt, freezer_info={"frozen": 1})
    ck.save_meta_data(path.parent, args)
    raw = torch.load(path, map_location="cpu", weights_only=True)
    assert set(raw) == {"step", "model_state", "optim_state", "rng_state", "freezer_info"}
    assert not any(k.endswith(".w") for k in raw["model_state"])
    assert json.loads((path.parent / "meta_data.json").read_text())["args"] == args
    loaded, got_args, step = ck.load_checkpoint(path, device="cpu")
    assert step == 100 and got_args == args and not loaded.training
    ref = ck.filtered_model_state_dict(model)
    got = loaded.state_dict()
    for k, v in ref.items():
        assert torch.equal(got[k], v), k
    assert set(raw["rng_state"]) == {"torch", "cuda"}
    # the reference's training loader sequence (experiments/experiment_script.py:543-569)
    # restores model, frozen flags, optimizer state and RNG from it
    fresh = ck.build_model(args)
    [m for m in fresh if isinstance(m, LogicLayer)][0].freeze()   # as the freezer left it
    fopt = torch.optim.Adam([p for p in fresh.parameters() if p.requires_grad], lr=0.01)
    torch.manual_seed(12345)
    step, info = ck.resume_checkpoint(path, fresh, fopt)
    assert step == 100 and info == {"frozen": 1}
    assert torch.equal(torch.get_rng_state(), raw["rng_state"]["torch"])
    assert [getattr(m, "is_frozen", False) for m in fresh] == \
        [getattr(m, "w", None) is not None for m in fresh]
    assert fopt.state_dict()["param_groups"] == opt.state_dict()["param_groups"]
    # the loaded network's circuit is the saved network's (argmax of the saved logits)
    model.eval()
    a, b = C.extract_circuit(model), C.extract_circuit(loaded)
    for x, y in zip(a.gates + a.a + a.b, b.gates + b.a + b.b):
        assert np.array_equal(x, y)
