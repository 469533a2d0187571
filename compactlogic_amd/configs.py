"""Seeded synthetic workloads of the benchmark configurations.

Networks are generated on the CPU with ``torch.Generator`` in a fixed draw order, then moved
to the device, so every run (and the CPU baseline) sees identical parameters and inputs.

  cfg1  LogicLayer 784->8000 x4, G=16, GroupSum(10, tau=10), batch 128, inputs Bernoulli(0.5)
  cfg2  LogicLayer 784->12000 then 12000->12000 x5, G=16, GroupSum(10, 10), batch 1024,
        inputs Bernoulli(0.3)
  cfg3  ConvLayer((9,32,32), pad 1, c_out 256, ks 3, stride 2) -> ConvLayer((256,16,16), pad 0,
        c_out 512, ks 3, stride 2) -> flatten 25088 -> LogicLayer 16000 x2, G=16,
        GroupSum(10, tau=30), batch 256, inputs Bernoulli(0.5)
  cfg4  the cfg2 network frozen to argmax gates (uniform opcode per neuron), 2^24 samples
        bit-packed 64 per word
  cfg5  the cfg3 network with G=4, each row's gate_sequence 4 distinct seeded opcodes, frozen
        to the argmax of N(0, 1) logits; 2^20 samples bit-packed 64 per word

Dense wiring of these configs: one input pair (a, b) per neuron, drawn uniformly and shared
by its slots; gate_sequence = arange(G) & 15 unless stated; logits ~ N(0, 1).  Conv layers
draw their taps with ConvLayer's own sampler (num_chn = 1: channel c mod c_in, offsets
uniform in [0, ks) minus the padding, coinciding operands re-drawn) under a seeded global RNG.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .layers import ConvLayer, GroupSum, LogicLayer
from .treelogic import ConvLogicLayer

NET_SEED, INPUT_SEED, LABEL_SEED = 0, 1, 2


@dataclass
class DenseConfig:
    name: str
    in_dim: int
    widths: list[int]
    batch: int
    p_one: float
    k: int = 10
    tau: float = 10.0
    num_gates: int = 16
    notes: str = ""

    @property
    def dims(self):
        return list(zip([self.in_dim] + self.widths[:-1], self.widths))


CONFIGS = {
    "cfg1": DenseConfig("cfg1", 784, [8000] * 4, 128, 0.5),
    "cfg2": DenseConfig("cfg2", 784, [12000] * 6, 1024, 0.3),
}


@dataclass
class ConvConfig:
    name: str
    in_shape: tuple
    convs: list          # (c_out, ks, stride, padding) per ConvLayer
    widths: list         # dense LogicLayers after the flatten
    batch: int
    p_one: float = 0.5
    k: int = 10
    tau: float = 30.0
    num_gates: int = 16
    gate_subset: bool = False   # per-row gate_sequence = num_gates distinct seeded opcodes


CONV_CONFIGS = {
    "cfg3": ConvConfig("cfg3", (9, 32, 32), [(256, 3, 2, 1), (512, 3, 2, 0)], [16000, 16000], 256),
    "cfg5": ConvConfig("cfg5", (9, 32, 32), [(256, 3, 2, 1), (512, 3, 2, 0)], [16000, 16000], 256,
                       num_gates=4, gate_subset=True),
}


def _seeded_layer(in_dim: int, out_dim: int, gen: torch.Generator, num_gates: int) -> LogicLayer:
    # Build without disturbing the global RNG, then overwrite the draws from `gen`.
    with torch.random.fork_rng(devices=[]):
        layer = LogicLayer(in_dim, out_dim, connections="original", num_gates=num_gates)
    a = torch.randint(0, in_dim, (out_dim,), generator=gen)
    b = torch.randint(0, in_dim, (out_dim,), generator=gen)
    logits = torch.randn((out_dim, num_gates), generator=gen)
    with torch.no_grad():
        layer.weights.copy_(logits)
        layer.indices.copy_(torch.stack((a, b)).unsqueeze(-1).expand(2, out_dim, num_gates))
        layer.gate_sequence.copy_(
            (torch.arange(num_gates, dtype=torch.int64) & 15).to(torch.uint8).expand(out_dim, num_gates))
    layer.refresh_backward_index()
    return layer


def _seeded_random_layer(in_dim: int, out_dim: int, gen: torch.Generator,
                         num_gates: int) -> LogicLayer:
    """The reference's default wiring, connections='random' (compactlogic/compactlogic.py:
    160-182): every slot its own input pair, drawn by the layer's own sampler under a seeded
    RNG; logits from `gen`; gate_sequence = arange(16)."""
    layer_seed = int(torch.randint(0, 2**31 - 1, (1,), generator=gen))
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(layer_seed)
        layer = LogicLayer(in_dim, out_dim, connections="random", num_gates=num_gates)
    logits = torch.randn((out_dim, num_gates), generator=gen)
    with torch.no_grad():
        layer.weights.copy_(logits)
        layer.gate_sequence.copy_(
            (torch.arange(num_gates, dtype=torch.int64) & 15).to(torch.uint8).expand(out_dim, num_gates))
    layer.refresh_backward_index()
    return layer


def dense_network(cfg: DenseConfig, device="cuda", seed: int = NET_SEED,
                  wiring: str = "original") -> torch.nn.Sequential:
    """cfg's network.  wiring 'original': one seeded input pair per neuron shared by its
    slots (the benched configs); 'random': the reference's default, a pair per slot."""
    gen = torch.Generator().manual_seed(seed)
    make = _seeded_random_layer if wiring == "random" else _seeded_layer
    layers = [make(i, o, gen, cfg.num_gates) for i, o in cfg.dims]
    model = torch.nn.Sequential(*layers, GroupSum(cfg.k, cfg.tau))
    return model.to(device)


def _gate_subsets(rows: int, num_gates: int, gen: torch.Generator) -> torch.Tensor:
    """rows x num_gates distinct opcodes per row: the first num_gates of a seeded permutation
    of 0..15 (the resampler's gate pool, compactlogic/compactlogic.py:315-321)."""
    return torch.argsort(torch.rand((rows, 16), generator=gen), dim=1)[:, :num_gates].to(torch.uint8)


def conv_network(cfg: ConvConfig, device="cuda", seed: int = NET_SEED) -> torch.nn.Sequential:
    gen = torch.Generator().manual_seed(seed)
    layers = []
    shape = cfg.in_shape
    for c_out, ks, stride, pad in cfg.convs:
        layer_seed = int(torch.randint(0, 2**31 - 1, (1,), generator=gen))
        with torch.random.fork_rng(devices=[]):
            torch.manual_seed(layer_seed)
            layer = ConvLayer(shape, padding=pad, c_out=c_out, ks=ks, stride=stride, num_chn=1,
                              num_gates=cfg.num_gates)
        with torch.no_grad():
            layer.weights.copy_(torch.randn((c_out, cfg.num_gates), generator=gen))
            if cfg.gate_subset:
                layer.gate_sequence.copy_(_gate_subsets(c_out, cfg.num_gates, gen))
        layers.append(layer)
        shape = layer.out_shape
    layers.append(torch.nn.Flatten())
    in_dim = int(shape[0] * shape[1] * shape[2])
    for out_dim in cfg.widths:
        layer = _seeded_layer(in_dim, out_dim, gen, cfg.num_gates)
        if cfg.gate_subset:
            with torch.no_grad():
                layer.gate_sequence.copy_(_gate_subsets(out_dim, cfg.num_gates, gen))
        layers.append(layer)
        in_dim = out_dim
    model = torch.nn.Sequential(*layers, GroupSum(cfg.k, cfg.tau))
    return model.to(device)


@dataclass
class TreeConfig:
    """The logic-tree reading of cfg3: ConvLogicLayer blocks (8 taps, 4 -> 2 -> 1 gates, 2x2 max
    pool) in place of ConvLayer, then the dense layers and GroupSum."""
    name: str
    in_shape: tuple
    blocks: list         # (c_out, ks, stride, padding) per complete ConvLogicLayer
    widths: list
    batch: int
    p_one: float = 0.5
    k: int = 10
    tau: float = 30.0
    num_gates: int = 16
    num_chn: int = 2     # the ConvLogicLayer default


TREE_CONFIGS = {
    "cfg3_tree": TreeConfig("cfg3_tree", (9, 32, 32), [(256, 3, 2, 1), (512, 3, 2, 1)],
                            [16000, 16000], 256),
}


def tree_network(cfg: TreeConfig, device="cuda", seed: int = NET_SEED) -> torch.nn.Sequential:
    """(9,32,32) -> (256,8,8) -> (512,2,2) = 2048 -> 16000 -> 16000 -> GroupSum for cfg3_tree.
    Block logits ~ N(0, 1); taps drawn by ConvLogicLayer's own sampler under a seeded RNG."""
    gen = torch.Generator().manual_seed(seed)
    layers = []
    c, h, w = cfg.in_shape
    for c_out, ks, stride, pad in cfg.blocks:
        layer_seed = int(torch.randint(0, 2**31 - 1, (1,), generator=gen))
        with torch.random.fork_rng(devices=[]):
            torch.manual_seed(layer_seed)
            layer = ConvLogicLayer(c, c_out, stride=stride, padding=pad, kernel=ks, complete=True,
                                   num_chn=cfg.num_chn)
        with torch.no_grad():
            layer.weights.copy_(torch.randn(layer.weights.shape, generator=gen))
        layers.append(layer)
        ho, wo = (h + 2 * pad - ks) // stride + 1, (w + 2 * pad - ks) // stride + 1
        c, h, w = c_out, ho // 2, wo // 2
    # the last block feeds the flattened dense layers: its training output feature-major
    layers[-1].rows_output = True
    layers.append(torch.nn.Flatten())
    in_dim = c * h * w
    for out_dim in cfg.widths:
        layers.append(_seeded_layer(in_dim, out_dim, gen, cfg.num_gates))
        in_dim = out_dim
    model = torch.nn.Sequential(*layers, GroupSum(cfg.k, cfg.tau))
    return model.to(device)


def conv_inputs(cfg: ConvConfig, device="cuda", batch: int | None = None):
    batch = cfg.batch if batch is None else batch
    gx = torch.Generator().manual_seed(INPUT_SEED)
    gl = torch.Generator().manual_seed(LABEL_SEED)
    x = (torch.rand((batch,) + tuple(cfg.in_shape), generator=gx) < cfg.p_one).float()
    labels = torch.randint(0, cfg.k, (batch,), generator=gl)
    return x.to(device), labels.to(device)


def freeze_argmax(model: torch.nn.Sequential) -> None:
    """cfg5: fix every layer to the argmax slot of its logits."""
    for layer in model:
        if isinstance(layer, LogicLayer):
            layer.freeze()
    model.eval()


def dense_inputs(cfg: DenseConfig, device="cuda", batch: int | None = None):
    batch = cfg.batch if batch is None else batch
    gx = torch.Generator().manual_seed(INPUT_SEED)
    gl = torch.Generator().manual_seed(LABEL_SEED)
    x = (torch.rand((batch, cfg.in_dim), generator=gx) < cfg.p_one).float()
    labels = torch.randint(0, cfg.k, (batch,), generator=gl)
    return x.to(device), labels.to(device)


def freeze_uniform_gates(model: torch.nn.Sequential, seed: int = NET_SEED + 100) -> None:
    """cfg4: fix every neuron to a uniformly drawn opcode (argmax slot = opcode, since
    gate_sequence = arange(16))."""
    gen = torch.Generator().manual_seed(seed)
    for layer in model:
        if isinstance(layer, LogicLayer):
            slot = torch.randint(0, 16, (layer.out_dim,), generator=gen).to(torch.uint8)
            layer.freeze()
            layer.w.copy_(slot.to(layer.w.device))
    model.eval()


def packed_input_words(in_dim: int, words: int, device="cuda", seed: int = INPUT_SEED):
    """[in_dim, words] int64 rows; word (f, w) = splitmix64(seed * 2^40 + f * words + w), i.e.
    64 Bernoulli(0.5) samples per word."""
    from . import difflogic_hip
    out = torch.empty((in_dim, words), dtype=torch.int64, device=device)
    return difflogic_hip.fill_splitmix64(out, seed << 40)
