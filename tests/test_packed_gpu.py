"""Bit-packed inference kernels: bit-exact against the C oracle and the float discrete path."""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl
from compactlogic_amd import configs
from compactlogic_amd import difflogic_hip as dl
from oracle import logic_np as O
from oracle import packed as P

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [8, 16, 32, 64])
@pytest.mark.parametrize("n", [1, 63, 64, 65, 1000, 4096])
def test_pack_bits(device, bits, n):
    rng = np.random.default_rng(bits * n)
    t = rng.integers(0, 2, (5, n)).astype(bool)
    packed, pad = dl.tensor_packbits_cuda(torch.as_tensor(t, device=device), bits)
    ref, ref_pad = P.pack_bits(t, bits)
    assert pad == ref_pad
    assert packed.dtype == {8: torch.int8, 16: torch.int16, 32: torch.int32, 64: torch.int64}[bits]
    assert np.array_equal(packed.cpu().numpy().view(np.uint8), ref)


@pytest.mark.parametrize("words,dtype", [(1, torch.int64), (3, torch.int64), (8, torch.int64),
                                         (4096, torch.int64), (5, torch.int8), (6, torch.int32),
                                         (100, torch.int16)])
def test_eval_packed_layer(device, words, dtype):
    rng = np.random.default_rng(words)
    in_dim, out_dim, g_n = 37, 130, 4
    nbytes = words * torch.tensor([], dtype=dtype).element_size()
    xb = rng.integers(0, 256, (in_dim, nbytes), dtype=np.uint8)
    ind = rng.integers(0, in_dim, (2, out_dim, g_n))
    gs = rng.integers(0, 16, (out_dim, g_n)).astype(np.uint8)
    slot = rng.integers(0, g_n, out_dim).astype(np.uint8)
    x = torch.as_tensor(xb, device=device).view(dtype)
    y = dl.eval_packed(x, torch.as_tensor(ind[0], device=device), torch.as_tensor(ind[1], device=device),
                       torch.as_tensor(slot, device=device), torch.as_tensor(gs, device=device))
    ia, ib, g = P.resolve_slots(ind, gs, slot)
    pad8 = (-nbytes) % 8
    xw = np.pad(xb, ((0, 0), (0, pad8))).view(np.uint64)
    ref = P.eval_layer(xw, ia, ib, g).view(np.uint8)[:, :nbytes]
    assert np.array_equal(y.cpu().numpy().view(np.uint8), ref)


@pytest.mark.parametrize("rows,k,n", [(20, 10, 130), (12000, 10, 64 * 300), (12, 3, 4096 + 17),
                                      (64, 1, 200), (34, 17, 640), (6, 2, 9)])
def test_group_bit_sum(device, rows, k, n):
    rng = np.random.default_rng(rows + n)
    t = rng.integers(0, 2, (rows, n)).astype(bool)
    packed, pad = P.pack_bits(t, 64)
    got = dl.groupbitsum(torch.as_tensor(packed, device=device).view(torch.int64), pad, k)
    assert got.dtype == torch.int32 and got.shape == (n, k)
    assert np.array_equal(got.cpu().numpy(), P.group_bit_sum(packed, pad, k))


def test_group_bit_sum_odd_row_bytes(device):
    rng = np.random.default_rng(1)
    t = rng.integers(0, 2, (8, 37)).astype(bool)
    packed, pad = P.pack_bits(t, 8)                      # 5 bytes per row
    got = dl.groupbitsum(torch.as_tensor(packed, device=device).view(torch.int8), pad, 4)
    assert np.array_equal(got.cpu().numpy(), P.group_bit_sum(packed, pad, 4))


def test_group_bit_sum_rejects_indivisible(device):
    x = torch.zeros((7, 2), dtype=torch.int64, device=device)
    with pytest.raises(ValueError):
        dl.groupbitsum(x, 0, 2)


def test_fill_splitmix64(device):
    out = torch.empty(1000, dtype=torch.int64, device=device)
    dl.fill_splitmix64(out, 12345)
    assert np.array_equal(out.cpu().numpy().view(np.uint64), P.fill_splitmix64(1000, 12345))


def test_packed_network_matches_float_discrete_and_oracle(device):
    """Module path: PackBitsTensor through frozen LogicLayers and GroupSum gives the class
    counts round(logits * tau) of the float discrete path, and the C oracle's counts."""
    torch.manual_seed(3)
    dims = [(40, 60), (60, 60), (60, 50)]
    model = torch.nn.Sequential(*[cl.LogicLayer(i, o, num_gates=8) for i, o in dims],
                                cl.GroupSum(5, 4.0)).to(device)
    for m in model:
        if isinstance(m, cl.LogicLayer):
            m.freeze()
    model.eval()
    n = 1000
    x = torch.rand(n, 40, device=device) > 0.5
    logits = model(x.float())
    counts = model(cl.PackBitsTensor(x, 64))
    assert counts.dtype == torch.int32 and counts.shape == (n, 5)
    assert torch.equal(counts.cpu(), torch.round(logits * 4.0).to(torch.int32).cpu())
    layers = [P.resolve_slots(m.indices.cpu().numpy(), m.gate_sequence.cpu().numpy(), m.w.cpu().numpy())
              for m in model if isinstance(m, cl.LogicLayer)]
    xw, pad = P.pack_bits(x.cpu().numpy().T, 64)
    assert np.array_equal(counts.cpu().numpy(), P.network_counts(xw.view(np.uint64), layers, 5, pad))


def test_cfg4_network_slice_bit_exact(device):
    """cfg4's 6 x 12000 frozen network on 2^16 generated samples, bit-exact against the C
    oracle (the benchmark runs the same code on 2^24 samples)."""
    cfg = configs.CONFIGS["cfg2"]
    model = configs.dense_network(cfg, device=device)
    configs.freeze_uniform_gates(model)
    words = 1024
    xw = configs.packed_input_words(cfg.in_dim, words, device=device)
    counts = model(cl.PackBitsTensor.from_packed(xw.clone()))
    layers = [P.resolve_slots(m.indices.cpu().numpy(), m.gate_sequence.cpu().numpy(), m.w.cpu().numpy())
              for m in model if isinstance(m, cl.LogicLayer)]
    ref_x = np.stack([P.fill_splitmix64(words, (1 << 40) + f * words) for f in range(cfg.in_dim)])
    assert np.array_equal(xw.cpu().numpy().view(np.uint64), ref_x)
    ref = P.network_counts(ref_x, layers, cfg.k)
    assert np.array_equal(counts.cpu().numpy(), ref)
