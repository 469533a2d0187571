"""The pruned circuit on the packed kernels (compactlogic_amd.circuit.PackedCircuit): class
counts bit-exact against the unpruned network on 2^16 samples (the reference's full-test
semantic check, simulation/consistency.py:147-213, on the GPU) and against the oracle's bool
evaluator of its own pruning on a sample subset; the checkpoint -> circuit -> pruned evaluator
path end to end (experiments/experiment_script.py:527-547, compiler/extract.py:200-264)."""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl
from compactlogic_amd import checkpoint as ck
from compactlogic_amd import circuit as C
from compactlogic_amd import configs
from oracle import circuit_ref as R

pytestmark = pytest.mark.gpu

SAMPLES = 1 << 16


def unpack(words: torch.Tensor, n: int) -> np.ndarray:
    """[rows, words] int64 -> bool bits [n, rows] (sample s = bit s % 64 of word s // 64)."""
    w = words.cpu().numpy().view(np.uint64)
    bits = (w[:, :, None] >> np.arange(64, dtype=np.uint64)) & np.uint64(1)
    return bits.reshape(w.shape[0], -1)[:, :n].T.astype(np.int64)


def as_oracle(c: C.Circuit):
    return {"input_dim": c.input_dim, "k": c.k, "out_start": c.out_start, "out_dim": c.out_dim,
            "layers": [{"gate": g, "a": a, "b": b} for g, a, b in zip(c.gates, c.a, c.b)]}


def check_against_oracle(circuit, pruned, words, got, n=256):
    """The oracle prunes the same circuit and evaluates it on the first n samples."""
    bits = unpack(words, n)
    ref = R.evaluate_pruned(R.naive_prune(as_oracle(circuit)), bits)
    assert np.array_equal(got[:n].cpu().numpy(), ref)


def test_pruned_cfg4_network_counts_equal_the_unpruned(device):
    cfg = configs.CONFIGS["cfg2"]
    model = configs.dense_network(cfg, device=device)
    configs.freeze_uniform_gates(model)                     # the cfg4 network
    words = configs.packed_input_words(cfg.in_dim, SAMPLES // 64, device=device)
    x = cl.PackBitsTensor.from_packed(words)
    unpruned = cl.PackedNetwork(model)(x)
    layerwise = model(cl.PackBitsTensor.from_packed(words.clone()))
    assert torch.equal(unpruned, layerwise)
    circuit = C.extract_circuit(model)
    pruned = C.naive_prune(circuit)
    assert 0 < pruned.bop_count < circuit.node_count
    got = C.PackedCircuit(pruned, device)(x)
    assert torch.equal(got, unpruned)
    check_against_oracle(circuit, pruned, words, got)


def test_pruned_conv_network_counts_equal_the_unpruned(device):
    cfg = configs.CONV_CONFIGS["cfg5"]
    model = configs.conv_network(cfg, device=device)
    configs.freeze_argmax(model)
    feats = int(np.prod(cfg.in_shape))
    words = configs.packed_input_words(feats, SAMPLES // 64, device=device)
    unpruned = model(cl.PackBitsTensor.from_packed(words.clone()))
    circuit = C.extract_circuit(model)
    pruned = C.naive_prune(circuit)
    assert 0 < pruned.bop_count < circuit.node_count
    got = C.PackedCircuit(pruned, device)(cl.PackBitsTensor.from_packed(words))
    assert torch.equal(got, unpruned)
    check_against_oracle(circuit, pruned, words, got, n=64)


def test_checkpoint_to_pruned_packed_evaluator(device, tmp_path):
    args = {"dataset": "mnist", "struct": "regular", "num_gates": 16, "tau": 10.0,
            "model_scale": 1000, "num_layers": 3}
    torch.manual_seed(11)
    trained = ck.build_model(args)
    path = tmp_path / "exp" / "ckpt_best_7.pt"
    ck.save_checkpoint(path, 7, trained, torch.optim.Adam(trained.parameters(), lr=0.01))
    ck.save_meta_data(path.parent, args)
    model, _, step = ck.load_checkpoint(path, device=device)
    assert step == 7
    # the extraction reads the checkpoint's winners as the reference's extractor does
    state = torch.load(path, map_location="cpu", weights_only=True)["model_state"]
    circuit = C.extract_circuit(model)
    start = 0
    for i, (g, a, b) in enumerate(zip(circuit.gates, circuit.a, circuit.b)):
        p = str(i + 1)                                      # Flatten is module 0
        ref = R.extract_dense(state[p + ".weights"].numpy(), state[p + ".indices"].numpy(),
                              state[p + ".gate_sequence"].numpy(), start)
        assert np.array_equal(g, ref["gate"]) and np.array_equal(a, ref["a"])
        assert np.array_equal(b, ref["b"])
        start = circuit.layer_starts[i]
    words = configs.packed_input_words(784, SAMPLES // 64, device=device, seed=5)
    unpruned = model(cl.PackBitsTensor.from_packed(words.clone()))
    pruned = C.naive_prune(circuit)
    got = C.PackedCircuit(pruned, device)(cl.PackBitsTensor.from_packed(words))
    assert torch.equal(got, unpruned)
    assert got.shape == (SAMPLES, 10)
    check_against_oracle(circuit, pruned, words, got)
