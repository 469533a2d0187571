"""Module API, buffers and derived plans on the CPU (no kernel calls)."""
import numpy as np
import pytest
import torch

import compactlogic_amd as cl
from compactlogic_amd import configs
from oracle import logic_np as O

REF_KEYS = {"weights", "gate_sequence", "indices", "given_x_indices_of_y_start",
            "given_x_indices_of_y", "given_x_indices_of_gate"}


def test_logic_layer_buffers_and_state_dict():
    torch.manual_seed(0)
    layer = cl.LogicLayer(20, 30, num_gates=16)
    sd = layer.state_dict()
    assert set(sd) == REF_KEYS
    assert sd["weights"].shape == (30, 16) and sd["weights"].dtype == torch.float32
    assert sd["gate_sequence"].dtype == torch.uint8
    assert torch.equal(sd["gate_sequence"][0], torch.arange(16, dtype=torch.uint8))
    assert sd["indices"].shape == (2, 30, 16) and sd["indices"].dtype == torch.int64
    assert sd["given_x_indices_of_y"].numel() == 2 * 30 * 16
    assert sd["given_x_indices_of_gate"].dtype == torch.int8
    assert layer.indices.min() >= 0 and layer.indices.max() < 20
    # strict loading of a reference-shaped state dict, and freeze() adds `w`
    other = cl.LogicLayer(20, 30)
    other.load_state_dict(sd, strict=True)
    layer.freeze()
    assert layer.is_frozen and layer.w.dtype == torch.uint8
    assert torch.equal(layer.w, layer.weights.argmax(-1).to(torch.uint8))


def test_backward_index_matches_oracle_rows():
    torch.manual_seed(1)
    layer = cl.LogicLayer(13, 17, num_gates=4)
    start, yidx, code = O.backward_index(layer.indices.numpy(), 13)
    assert np.array_equal(layer.given_x_indices_of_y_start.numpy(), start)
    for i in range(13):
        s0, s1 = start[i], start[i + 1]
        got = sorted(zip(layer.given_x_indices_of_y[s0:s1].tolist(),
                         layer.given_x_indices_of_gate[s0:s1].tolist()))
        assert got == sorted(zip(yidx[s0:s1].tolist(), code[s0:s1].tolist()))


def test_connection_assertion_and_schemes():
    with pytest.raises(AssertionError):
        cl.LogicLayer(100, 10)
    with pytest.raises(NotImplementedError):
        cl.LogicLayer(4, 4, connections="bogus")
    torch.manual_seed(2)
    orig = cl.LogicLayer(10, 12, connections="original")
    assert bool((orig.indices == orig.indices[..., :1]).all())
    assert orig.run_plan().num_runs == 12


def test_residual_init():
    layer = cl.LogicLayer(8, 8, residual_init=True)
    assert bool((layer.weights.argmax(-1) == 3).all())
    assert float(layer.weights[0, 3]) == pytest.approx(np.log(9 * 15), rel=1e-6)


def _plan_reference(ind):
    """Runs by brute force: maximal equal-pair slot ranges per neuron."""
    runs = []
    _, out, g = ind.shape
    for o in range(out):
        g0 = 0
        for s in range(1, g + 1):
            if s == g or (ind[0, o, s], ind[1, o, s]) != (ind[0, o, g0], ind[1, o, g0]):
                runs.append((o, g0, s - g0, int(ind[0, o, g0]), int(ind[1, o, g0])))
                g0 = s
    return runs


@pytest.mark.parametrize("seed", range(4))
def test_run_plan_against_brute_force(seed):
    rng = np.random.default_rng(seed)
    in_dim, out, g = 7, 9, 6
    ind = rng.integers(0, 3, (2, out, g))          # few distinct inputs -> long runs
    plan = cl.build_run_plan(torch.as_tensor(ind), in_dim)
    runs = _plan_reference(ind)
    assert plan.num_runs == len(runs)
    got = [(int(plan.run_y[r]), int(plan.run_gl[r]) & 255, int(plan.run_gl[r]) >> 8,
            int(plan.run_ab[r, 0]), int(plan.run_ab[r, 1])) for r in range(plan.num_runs)]
    assert got == runs
    ptr = plan.run_ptr.numpy()
    assert ptr[0] == 0 and ptr[-1] == len(runs)
    for o in range(out):
        assert all(runs[r][0] == o for r in range(ptr[o], ptr[o + 1]))
    inv = plan.inv_ptr.numpy()
    uses = set()
    for i in range(in_dim):
        for e in plan.inv_entry[inv[i]:inv[i + 1]].tolist():
            r, side = e >> 1, e & 1
            assert runs[r][3 + side] == i
            uses.add(e)
    assert uses == set(range(2 * len(runs)))


def test_run_plan_rejects_out_of_range_indices():
    with pytest.raises(IndexError):
        cl.build_run_plan(torch.tensor([[[0, 5]], [[1, 1]]]), 5)


def test_plan_rebuilds_after_in_place_rewiring():
    torch.manual_seed(3)
    layer = cl.LogicLayer(6, 8, connections="original")
    p1 = layer.run_plan()
    assert layer.run_plan() is p1
    with torch.no_grad():
        layer.indices[0, 0, 5] = (layer.indices[0, 0, 5] + 1) % 6
    p2 = layer.run_plan()
    assert p2 is not p1 and p2.num_runs == p1.num_runs + 2


def _plan_fields(plan):
    return {k: getattr(plan, k) for k in ("run_ptr", "run_ab", "run_gl", "run_y", "inv_ptr",
                                          "inv_entry", "inv_rec", "inv_pos", "row_order", "nab",
                                          "slot_rec", "inv_slot", "tile_ptr", "tile_run",
                                          "tile_loc")}


def test_small_rewiring_keeps_the_input_order():
    """An in-place rewiring of at most REORDER_FRACTION of the neurons (counted since the last
    full order) keeps the previous plan's input order and rebuilds everything else from the new
    wiring: the plan equals build_run_plan with that order given.  Past the fraction, or for a
    new indices tensor, the order is recomputed (locality_order of the new runs)."""
    from compactlogic_amd.plan import REORDER_FRACTION, build_run_plan, locality_order
    torch.manual_seed(11)
    layer = cl.LogicLayer(64, 100, connections="random")
    p1 = layer.run_plan()
    assert p1.stale == 0
    n1 = int(REORDER_FRACTION * 100) // 2                   # 5 neurons
    with torch.no_grad():
        layer.indices[:, :n1] = torch.randint(0, 64, (2, n1, layer.num_gates))
    p2 = layer.run_plan()
    assert p2 is not p1 and p2.stale == n1
    assert torch.equal(p2.row_order, p1.row_order)
    want = build_run_plan(layer.indices, 64, row_order=p1.row_order)
    for k, v in _plan_fields(want).items():
        assert torch.equal(getattr(p2, k), v), k
    # the runs themselves are those of a fresh build: only the input order is carried over
    fresh = build_run_plan(layer.indices, 64)
    for k in ("run_ptr", "run_ab", "run_gl", "run_y", "inv_ptr", "nab"):
        assert torch.equal(getattr(p2, k), getattr(fresh, k)), k
    # rewirings accumulate (each counts the neurons it changed) until the fraction is passed
    with torch.no_grad():
        layer.indices[:, :n1] = torch.randint(0, 64, (2, n1, layer.num_gates))
    p3 = layer.run_plan()
    assert p3.stale == 2 * n1 and torch.equal(p3.row_order, p1.row_order)
    with torch.no_grad():
        layer.indices[:, n1:n1 + 1] = torch.randint(0, 64, (2, 1, layer.num_gates))
    p4 = layer.run_plan()
    assert p4.stale == 0
    ab = p4.run_ab.long()
    assert torch.equal(p4.row_order.long(), locality_order(ab[:, 0], ab[:, 1], 64))
    # a new tensor is a full build
    layer.indices = layer.indices.clone()
    p5 = layer.run_plan()
    assert p5.stale == 0 and torch.equal(p5.row_order, p4.row_order)


def test_run_plan_rejects_a_bad_row_order():
    ind = torch.randint(0, 6, (2, 4, 3))
    with pytest.raises(ValueError):
        cl.build_run_plan(ind, 6, row_order=torch.arange(5))


def test_resample_connections_updates_index():
    torch.manual_seed(4)
    layer = cl.LogicLayer(10, 16)
    with torch.no_grad():
        layer.weights[:4] = 0.0               # uniform rows are weak
        layer.weights[4:8, 2] = 20.0          # peaked rows are strong
    weak, strong = layer.resample_connections(torch.arange(8), threshold_high=0.95,
                                              threshold_low=0.5)
    assert int(weak.sum()) == 4 and int(strong.sum()) == 4
    start, yidx, code = O.backward_index(layer.indices.numpy(), 10)
    assert np.array_equal(layer.given_x_indices_of_y_start.numpy(), start)
    assert bool((layer.weights[4:8].argmax(-1) == 2).all())


def test_weights_entropy_and_connected_neurons():
    torch.manual_seed(5)
    layer = cl.LogicLayer(8, 8, num_gates=16)
    with torch.no_grad():
        layer.weights.zero_()
    assert torch.allclose(layer.weights_entropy(), torch.ones(8), atol=1e-6)
    with torch.no_grad():
        layer.weights.fill_(-30.0)
        layer.weights[:, 6] = 30.0            # XOR everywhere: both inputs used
    x_flag, y_flag = layer.connected_neurons(torch.ones(8, dtype=torch.bool))
    expect = torch.zeros(8, dtype=torch.bool)
    expect[layer.indices[0, :, 6]] = True
    expect[layer.indices[1, :, 6]] = True
    assert torch.equal(x_flag, expect) and bool(y_flag.all())


def test_forward_rejects_host_tensors():
    layer = cl.LogicLayer(4, 4)
    with pytest.raises(RuntimeError):
        layer(torch.zeros(2, 4))
    with pytest.raises(RuntimeError):
        cl.GroupSum(2)(torch.zeros(2, 4))


def test_tree_row_bytes():
    from compactlogic_amd.treelogic import tree_row_bytes
    for nbytes in [0, 8, 4096, 16376, 16384, 16392, 16640, 131072, 131080, 1 << 21]:
        got = tree_row_bytes(nbytes)
        if nbytes < 16384:
            assert got == nbytes                  # short rows are read as they are
        else:
            assert got % 256 == 0 and (got // 256) % 2 == 1 and 0 <= got - nbytes < 512
    # 2^20 samples in 64-bit words: a 128 KiB row becomes 128 KiB + 256 B
    assert tree_row_bytes(131072) == 131328 and tree_row_bytes(131328) == 131328


def test_config_network_is_deterministic():
    cfg = configs.CONFIGS["cfg1"]
    m1 = configs.dense_network(cfg, device="cpu")
    m2 = configs.dense_network(cfg, device="cpu")
    for l1, l2 in zip(m1, m2):
        if isinstance(l1, cl.LogicLayer):
            assert torch.equal(l1.weights, l2.weights) and torch.equal(l1.indices, l2.indices)
            assert l1.run_plan().num_runs == l1.out_dim


# ------------------------------------------------------------------------------ ConvLayer

@pytest.mark.parametrize("num_chn,ks,pad", [(0, 3, 1), (1, 3, 1), (3, 3, 0), (0, 1, 0)])
def test_conv_layer_buffers_and_sampler(num_chn, ks, pad):
    torch.manual_seed(num_chn * 7 + ks)
    layer = cl.ConvLayer((9, 10, 12), padding=pad, c_out=18, ks=ks, stride=2, num_chn=num_chn,
                         num_gates=16)
    sd = layer.state_dict()
    assert set(sd) == {"weights", "gate_sequence", "offsets_ch", "offsets_h", "offsets_w"}
    assert sd["weights"].shape == (18, 16)
    assert sd["offsets_ch"].dtype == torch.int32 and sd["offsets_h"].dtype == torch.int8
    for k in ("offsets_ch", "offsets_h", "offsets_w"):
        assert sd[k].shape == (2, 18, 16) and sd[k].is_contiguous()
    h_out = (10 + 2 * pad - ks) // 2 + 1
    w_out = (12 + 2 * pad - ks) // 2 + 1
    assert layer.out_shape == (18, h_out, w_out)
    assert layer.in_dim == 9 * (10 + 2 * pad) * (12 + 2 * pad)   # padded plane, as the reference
    assert layer.out_dim == 18 * h_out * w_out
    och, oh, ow = layer.offsets_ch, layer.offsets_h, layer.offsets_w
    assert int(oh.min()) >= -pad and int(oh.max()) < ks - pad
    assert int(ow.min()) >= -pad and int(ow.max()) < ks - pad
    assert int(och.min()) >= 0 and int(och.max()) < 9
    same = (och[0] == och[1]) & (oh[0] == oh[1]) & (ow[0] == ow[1])
    assert not bool(same.any())                                    # resolve_conflicts
    if num_chn == 1:
        expect = (torch.arange(18) % 9).to(torch.int32)
        assert torch.equal(och[0][:, 0], expect) and torch.equal(och[1][:, 5], expect)
    if num_chn == 3:                                              # 3 groups of 3 channels
        group = torch.clamp(torch.arange(18) // 6, 0, 2)
        assert torch.equal(och[0] // 3, group.view(-1, 1).expand(18, 16).to(torch.int32))
    assert "num_chn={}".format(num_chn) in layer.extra_repr()


def test_conv_packed_tables_match_oracle():
    from oracle import packed as P
    torch.manual_seed(3)
    layer = cl.ConvLayer((3, 7, 9), padding=1, c_out=5, ks=3, stride=2, num_chn=0, num_gates=4)
    layer.freeze()
    ia, ib, g = layer.packed_tables(layer.w)
    ra, rb, rg = P.resolve_conv_slots(layer.offsets_ch.numpy(), layer.offsets_h.numpy(),
                                      layer.offsets_w.numpy(), layer.gate_sequence.numpy(),
                                      layer.w.numpy(), layer.in_shape, 2, layer.out_shape[1:])
    assert np.array_equal(ia.numpy(), ra) and np.array_equal(ib.numpy(), rb)
    assert np.array_equal(g.numpy(), rg)
    # cached until the winners change
    assert layer.packed_tables(layer.w)[0] is ia
    layer.w.fill_(1)
    assert layer.packed_tables(layer.w)[0] is not ia


def test_conv_packed_tables_not_hit_by_recycled_storage():
    """A new winners tensor over the same storage (same data_ptr, version 0) must rebuild the
    tables, not return those of the tensor it replaces."""
    from oracle import packed as P
    torch.manual_seed(5)
    layer = cl.ConvLayer((2, 6, 6), padding=1, c_out=4, ks=3, stride=1, num_chn=0, num_gates=4)
    store = torch.zeros(layer.c_out, dtype=torch.uint8)
    w0 = store.view(layer.c_out)
    t0 = layer.packed_tables(w0)
    del w0
    store.numpy()[:] = [1, 2, 3, 0]          # a write torch does not see: versions stay 0
    w1 = store.view(layer.c_out)
    assert w1.data_ptr() == store.data_ptr() and w1._version == 0
    ia, ib, g = layer.packed_tables(w1)
    assert ia is not t0[0]
    ra, rb, rg = P.resolve_conv_slots(layer.offsets_ch.numpy(), layer.offsets_h.numpy(),
                                      layer.offsets_w.numpy(), layer.gate_sequence.numpy(),
                                      w1.numpy(), layer.in_shape, 1, layer.out_shape[1:])
    assert np.array_equal(ia.numpy(), ra) and np.array_equal(ib.numpy(), rb)
    assert np.array_equal(g.numpy(), rg)


def test_conv_eval_winners_follow_weight_updates():
    """An unfrozen layer in eval mode takes its winners from the logits; an in-place update of
    the logits must change the cached winners."""
    torch.manual_seed(6)
    layer = cl.ConvLayer((2, 6, 6), padding=1, c_out=4, ks=3, stride=1, num_chn=0, num_gates=4)
    w0 = layer._argmax_slots()
    assert layer._argmax_slots() is w0
    with torch.no_grad():
        layer.weights.zero_()
        layer.weights[:, 2] = 1.0
    w1 = layer._argmax_slots()
    assert w1 is not w0 and torch.equal(w1, torch.full((4,), 2, dtype=torch.uint8))
    # a write that leaves the version unchanged (an optimizer's raw-pointer update, a graph
    # replay) must change the winners as well: they are recomputed on every call
    v = layer.weights._version
    layer.weights.data[:, 3] = 5.0                   # .data writes do not bump the version
    assert layer.weights._version == v
    w2 = layer._argmax_slots()
    assert torch.equal(w2, torch.full((4,), 3, dtype=torch.uint8))
    assert layer._argmax_slots() is w2               # unchanged winners: the same tensor


def test_fused_adam_state_dict_interchanges_with_torch_adam():
    """FusedAdam resumes its shared step count from a loaded torch.optim.Adam state dict and
    writes Adam's layout (float32 host step per parameter); disagreeing steps are refused."""
    torch.manual_seed(2)
    params = [torch.randn(5, 4, requires_grad=True), torch.randn(3, requires_grad=True)]
    adam = torch.optim.Adam(params, lr=0.01)
    for _ in range(3):
        for p in params:
            p.grad = torch.randn_like(p)
        adam.step()
    fused = cl.FusedAdam([p.detach().clone().requires_grad_(True) for p in params], lr=0.01)
    assert fused._loaded_step() == 0.0
    fused.load_state_dict(adam.state_dict())
    assert fused._step_t is None and fused._loaded_step() == 3.0
    sd = fused.state_dict()
    assert all(v["step"].dtype == torch.float32 and v["step"].device.type == "cpu"
               and float(v["step"]) == 3.0 for v in sd["state"].values())
    bad = adam.state_dict()
    bad["state"][1]["step"] = torch.tensor(7.0)
    fused.load_state_dict(bad)
    with pytest.raises(RuntimeError, match="several"):
        fused._loaded_step()


def test_checkpoint_needs_the_optimizer(tmp_path):
    from compactlogic_amd import checkpoint as ck
    model = torch.nn.Sequential(torch.nn.Flatten(), cl.LogicLayer(16, 20))
    with pytest.raises(TypeError):
        ck.save_checkpoint(tmp_path / "c.pt", 1, model, None)


def test_conv_layer_rewiring_keeps_ranges():
    torch.manual_seed(4)
    layer = cl.ConvLayer((4, 8, 8), padding=1, c_out=6, ks=3, stride=1, num_chn=0, num_gates=8)
    before = layer.offsets_h.clone()
    weak, strong = layer.resample_connections(torch.arange(6), threshold_high=2.0, threshold_low=1.0)
    assert bool(weak.all()) and not bool(strong.any())
    assert not torch.equal(before, layer.offsets_h)
    assert int(layer.offsets_h.min()) >= -1 and int(layer.offsets_h.max()) <= 1


def test_conv_forward_rejects_host_tensors():
    layer = cl.ConvLayer((3, 6, 6), padding=1, c_out=4, ks=3, stride=1, num_chn=0)
    with pytest.raises(RuntimeError):
        layer(torch.rand(2, 3, 6, 6))


def test_conv_config_network_shapes():
    model = configs.conv_network(configs.CONV_CONFIGS["cfg5"], device="cpu")
    assert model[0].out_shape == (256, 16, 16) and model[1].out_shape == (512, 7, 7)
    assert model[3].in_dim == 25088 and model[4].out_dim == 16000
    gs = model[0].gate_sequence
    assert gs.shape == (256, 4)
    assert all(len(set(r.tolist())) == 4 for r in gs)          # distinct opcodes per row


def test_conv_inverse_index_cache_follows_tensors():
    """The cached inverse index is reused only for the same live, unmodified offsets: a new
    tensor at a recycled address, or an in-place change, rebuilds it (CPU torch ops)."""
    import gc
    from compactlogic_amd import convlogic_hip as cv
    g = torch.Generator().manual_seed(0)
    och = torch.randint(0, 3, (2, 4, 5), generator=g, dtype=torch.int32)
    oh = torch.randint(-1, 2, (2, 4, 5), generator=g).to(torch.int8)
    ow = torch.randint(-1, 2, (2, 4, 5), generator=g).to(torch.int8)
    first = cv.inverse_index(och, oh, ow, 3, 2)
    assert cv.inverse_index(och, oh, ow, 3, 2) is first
    oh[1, 2, 3] = 1 - int(oh[1, 2, 3])
    second = cv.inverse_index(och, oh, ow, 3, 2)
    assert second is not first
    del och
    gc.collect()
    och2 = torch.zeros((2, 4, 5), dtype=torch.int32)
    third = cv.inverse_index(och2, oh, ow, 3, 2)
    assert third is not second
    # bucket contents: every tap once, in the bucket of its channel and stride phase
    inv_ptr, inv_ent = third
    assert int(inv_ptr[-1]) == 40 and sorted(inv_ent.tolist()) == list(range(40))
    for k in range(3 * 4):
        for e in inv_ent[int(inv_ptr[k]):int(inv_ptr[k + 1])].tolist():
            side, slot = e & 1, e >> 1
            c, gg = divmod(slot, 5)
            assert int(och2[side, c, gg]) * 4 + (int(oh[side, c, gg]) % 2) * 2 + int(ow[side, c, gg]) % 2 == k


def test_run_plan_processing_order():
    """row_order is the preorder of a depth-first spanning forest of the run graph with every
    input's children visited smallest subtree first, inputs of degree 0 last; slot_rec
    follows it."""
    from compactlogic_amd.plan import build_run_plan
    from plan_reference import dfs_forest
    g = torch.Generator().manual_seed(11)
    in_dim, out_dim = 3000, 1600
    pair = torch.randint(0, in_dim, (2, out_dim, 1), generator=g).expand(2, out_dim, 16)
    plan = build_run_plan(pair.contiguous(), in_dim)
    order = plan.row_order.long()
    assert sorted(order.tolist()) == list(range(in_dim))
    deg = (plan.inv_ptr[1:] - plan.inv_ptr[:-1]).long()
    d = deg[order]
    nz = int((deg > 0).sum())
    assert bool((d[nz:] == 0).all()) and bool((d[:nz] > 0).all())
    ab = plan.run_ab.long()
    roots, parent, children = dfs_forest(ab[:, 0], ab[:, 1], deg, in_dim)
    nbrs = [set() for _ in range(in_dim)]
    for x, y in ab.tolist():
        nbrs[x].add(y)
        nbrs[y].add(x)
    # a spanning forest of the inputs of nonzero degree, each edge to a neighbour
    assert sorted(v for v in range(in_dim) if parent[v] != -2) == sorted(
        v for v in range(in_dim) if deg[v] > 0)
    assert all(parent[v] in nbrs[v] for v in range(in_dim) if parent[v] >= 0)
    assert [r for r in range(in_dim) if parent[r] == -1] == sorted(roots)
    # depth-first: every run joins an input to one of its ancestors (no cross edges)
    def ancestors(v):
        out = set()
        while parent[v] >= 0:
            v = parent[v]
            out.add(v)
        return out
    anc = [ancestors(v) if parent[v] != -2 else set() for v in range(in_dim)]
    for x, y in ab.tolist():
        assert x == y or x in anc[y] or y in anc[x]
    # preorder with smallest subtrees first: the subtree of u is the block of size(u)
    # positions starting at u, and its children's blocks follow in increasing size
    pos = torch.empty(in_dim, dtype=torch.long)
    pos[order] = torch.arange(in_dim)
    size = [1] * in_dim
    for v in sorted(range(in_dim), key=lambda v: -len(anc[v])):
        if parent[v] >= 0:
            size[parent[v]] += size[v]
    for u in range(in_dim):
        if parent[u] == -2:
            continue
        nxt = int(pos[u]) + 1
        for c in sorted(children[u], key=lambda c: int(pos[c])):
            assert int(pos[c]) == nxt
            nxt += size[c]
        sizes = [size[c] for c in sorted(children[u], key=lambda c: int(pos[c]))]
        assert sizes == sorted(sizes)
    assert len(roots) < nz // 4
    rec = plan.slot_rec.long()
    assert torch.equal(rec[:, 0], order)
    assert torch.equal(rec[:, 1], plan.inv_ptr.long()[order])
    assert torch.equal(rec[:, 2], plan.inv_ptr.long()[order + 1])


@pytest.mark.parametrize("in_dim,out_dim,g_n,seed", [(3000, 1600, 16, 11), (20, 300, 4, 12),
                                                     (64, 64, 1, 13), (1000, 900, 8, 14)])
def test_run_plan_tiles(in_dim, out_dim, g_n, seed):
    """The tiles of the partitioned input gradient: every internal run has both inputs in its
    tile, at the recorded positions, with two distinct LDS slots that the entries' inv_slot
    name; at most PART_SLOTS / 2 internal runs per tile, and a run left external only when its
    tile is full; all other entries are external (-1)."""
    from compactlogic_amd.plan import PART_ROWS, PART_SLOTS, build_run_plan
    g = torch.Generator().manual_seed(seed)
    idx = torch.randint(0, in_dim, (2, out_dim, g_n), generator=g)
    idx[:, ::3] = idx[:, ::3, :1]                      # some multi-slot runs
    idx[1, ::7] = idx[0, ::7]                          # self-pairs
    plan = build_run_plan(idx.contiguous(), in_dim)
    pos = torch.empty(in_dim, dtype=torch.long)
    pos[plan.row_order.long()] = torch.arange(in_dim)
    ab = plan.run_ab.long()
    tile_of = pos // PART_ROWS
    ptr = plan.tile_ptr.long()
    assert ptr.numel() == (in_dim + PART_ROWS - 1) // PART_ROWS + 1 and int(ptr[0]) == 0
    inv_slot = plan.inv_slot.long()
    inv_pos = plan.inv_pos.long()
    internal = set()
    for t in range(ptr.numel() - 1):
        k0, k1 = int(ptr[t]), int(ptr[t + 1])
        assert 0 <= k1 - k0 <= PART_SLOTS // 2
        runs = plan.tile_run[k0:k1].long()
        locs = plan.tile_loc[k0:k1].long()
        assert runs[:, 1].tolist() == sorted(runs[:, 1].tolist())
        used = set()
        for (o, r, pa, pb), loc in zip(runs.tolist(), locs.tolist()):
            a, b = ab[r].tolist()
            assert int(plan.run_y[r]) == o and tile_of[a] == t and tile_of[b] == t
            al, bl, sa, sb = loc & 255, (loc >> 8) & 255, (loc >> 16) & 255, (loc >> 24) & 255
            assert pos[a] == t * PART_ROWS + al and pos[b] == t * PART_ROWS + bl
            assert pa == int(inv_pos[2 * r]) and pb == int(inv_pos[2 * r + 1])
            assert sa != sb and sa < PART_SLOTS and sb < PART_SLOTS and not {sa, sb} & used
            used |= {sa, sb}
            assert int(inv_slot[pa]) == sa and int(inv_slot[pb]) == sb
            internal.add(r)
        if k1 - k0 < PART_SLOTS // 2:
            same = [r for r in range(ab.shape[0]) if tile_of[ab[r, 0]] == t == tile_of[ab[r, 1]]]
            assert set(same) <= internal
    ext = [r for r in range(ab.shape[0]) if r not in internal]
    for r in ext:
        assert int(inv_slot[inv_pos[2 * r]]) == -1 and int(inv_slot[inv_pos[2 * r + 1]]) == -1


def _clashes(p, pa, pb, banks=32):
    """Extra LDS cycles of a layout: per block of 32 positions, reads beyond one per bank."""
    n = 0
    for blk in range(int(p.max()) // 32 + 1):
        m = p // 32 == blk
        for k in (pa[m] % banks, pb[m] % banks):
            n += len(k) - len(set(k.tolist()))
    return n


@pytest.mark.parametrize("rows,seed", [(12000, 0), (1000, 1), (47, 2), (32, 3)])
def test_bank_aware_positions(rows, seed):
    """The fused packed layout is a permutation of the layer's rows whose blocks of 32
    consecutive positions read their a rows and their b rows from distinct LDS banks (word %
    32, per half-wave) more often than the identity layout; when every bank is read equally
    often (a regular multigraph) the colouring is conflict-free."""
    from compactlogic_amd.packed_net import bank_aware_positions
    rng = np.random.default_rng(seed)
    pa = rng.integers(0, 5 * rows, rows)
    pb = rng.integers(0, 5 * rows, rows)
    pb[::5] = pa[::5]
    pos = bank_aware_positions(pa, pb, rows)
    assert sorted(pos.tolist()) == list(range(rows))
    assert _clashes(pos, pa, pb) <= _clashes(np.arange(rows), pa, pb)
    if rows % 32 == 0:
        ra = rng.permutation(np.arange(rows) % 32) + 32 * rng.integers(0, 100, rows)
        rb = rng.permutation(np.arange(rows) % 32) + 32 * rng.integers(0, 100, rows)
        pos = bank_aware_positions(ra, rb, rows)
        assert sorted(pos.tolist()) == list(range(rows))
        assert _clashes(pos, ra, rb) == 0


def test_bank_aware_chain_levels_the_next_layer():
    """With the next layer's fan-outs, positions inside each block level that layer's bank
    degrees, and its own layout is then nearly conflict-free."""
    from compactlogic_amd.packed_net import bank_aware_positions
    rng = np.random.default_rng(7)
    n = 12000
    a1, b1 = rng.integers(0, 784, n), rng.integers(0, 784, n)   # layer 1 reads the inputs
    a2, b2 = rng.integers(0, n, n), rng.integers(0, n, n)       # layer 2 reads layer 1
    plain = bank_aware_positions(a1, b1, n)
    level = bank_aware_positions(a1, b1, n, np.bincount(a2, minlength=n),
                                 np.bincount(b2, minlength=n))
    assert _clashes(plain, a1, b1) == _clashes(level, a1, b1)  # same blocks for layer 1
    deg = lambda p, idx: np.bincount(p[idx] % 32, minlength=32).max()
    assert deg(level, a2) < deg(plain, a2) and deg(level, b2) < deg(plain, b2)
    c_plain = _clashes(bank_aware_positions(plain[a2], plain[b2], n), plain[a2], plain[b2])
    c_level = _clashes(bank_aware_positions(level[a2], level[b2], n), level[a2], level[b2])
    assert c_level * 4 < c_plain and c_level < 0.1 * 2 * (n // 32)


@pytest.mark.parametrize("rows,k", [(12000, 10), (1500, 10), (96, 3), (100, 4)])
def test_bank_aware_positions_grouped(rows, k):
    """The last layer's layout keeps every gate inside its class range, is a permutation, and
    has fewer bank clashes than the identity layout."""
    from compactlogic_amd.packed_net import bank_aware_positions_grouped
    rng = np.random.default_rng(rows + k)
    pa = rng.integers(0, 3 * rows, rows)
    pb = rng.integers(0, 3 * rows, rows)
    pos = bank_aware_positions_grouped(pa, pb, rows, rows // k)
    assert sorted(pos.tolist()) == list(range(rows))
    gs = rows // k
    assert all(o // gs == p // gs for o, p in enumerate(pos.tolist()))

    def clashes(p):
        return _clashes(p, pa, pb)

    # a class spans few blocks, so the choice is narrower than for hidden layers
    assert clashes(pos) <= clashes(np.arange(rows))
    if gs >= 1000:
        assert clashes(np.arange(rows)) > 3 * max(1, clashes(pos))
    elif rows >= 1000:
        assert clashes(np.arange(rows)) > 1.5 * max(1, clashes(pos))


def _spans_overlap(a, b):
    return a[0] < b[1] and b[0] < a[1]


@pytest.mark.parametrize("rows", [
    [25088, 16000, 16000],       # cfg5's tail: two first-layer slots held over the input
    [8192, 3000, 2000],          # 8-slot layers, the second over the dead input
    [9000, 12000, 10000],        # held slots, the second layer at the top of LDS
    [5760, 12000, 10000],        # 16 slots, nothing held
    [30000, 8000, 6000, 4000],   # three 8-slot layers, held slots
    [32768, 100],                # one 8-slot layer after the widest input that leaves room
    [34000, 100, 100],           # wider: two slots held
])
def test_columns_layout_places_every_layer_apart_from_what_it_reads(rows):
    """The wide-input fused pass's LDS placement (a restatement of what its kernel does with
    it): every step's slot writes, junk slots included, stay inside 160 KiB and off the words
    that step and later ones still read; rows keep their LDS bank (bases are multiples of 32
    words)."""
    from compactlogic_amd.packed_net import columns_layout
    lay = columns_layout(rows)
    assert lay is not None
    J = 8 if max(rows[1:]) <= 8192 else 16
    span, split, words = J * 1024, lay["split"], 40960
    held = span - split
    assert lay["in_words"] >= rows[0] and lay["in_words"] % 64 == 0
    assert split % 1024 == 0 and 0 <= held <= 2048
    assert all(b % 32 == 0 for b in lay["base"]) and lay["hold_base"] % 32 == 0
    inp = (0, lay["in_words"])
    unheld = (lay["base"][0], lay["base"][0] + split)
    hold = (lay["hold_base"], lay["hold_base"] + held)
    assert unheld[1] <= words and not _spans_overlap(unheld, inp)      # written while read
    if held:
        assert len(rows) >= 3                                              # counts read one run
        assert hold[1] <= lay["in_words"] and not _spans_overlap(hold, unheld)
    live = [unheld, hold] if held else [unheld]
    for l in range(1, len(rows) - 1):
        out = (lay["base"][l], lay["base"][l] + span)
        assert out[1] <= words and not any(_spans_overlap(out, r) for r in live if r[1] > r[0])
        live = [out]


@pytest.mark.parametrize("rows", [
    [25088, 16385],              # a layer wider than 16 slots
    [30000, 16000],              # one wide layer: no room without holding, nothing to hold for
    [30000, 16000, 16000, 100],  # three 16-slot layers
    [41000, 100, 100],           # the input column alone exceeds LDS
    [38000, 8000, 100],          # the first layer does not fit even with two slots held
])
def test_columns_layout_rejects_what_does_not_fit(rows):
    from compactlogic_amd.packed_net import columns_layout
    assert columns_layout(rows) is None


@pytest.mark.parametrize("pair", [False, True])
def test_producer_order_groups_rows_by_input_blocks(pair):
    """The column producer's row order is a permutation along which the sorted input-block
    tuples of the rows never decrease (a reading rows from the same blocks run together), ties
    kept in row order; negative and out-of-range indices count as no input."""
    from compactlogic_amd.packed_net import producer_order
    rng = np.random.default_rng(int(pair))
    in_rows, mid, out = 1600, 900, 700
    ia1, ib1 = rng.integers(-1, in_rows + 1, mid), rng.integers(-1, in_rows + 1, mid)
    ia2, ib2 = rng.integers(-1, mid + 1, out), rng.integers(-1, mid + 1, out)
    tabs = [(ia1, ib1), (ia2, ib2)] if pair else [(ia2 % in_rows, ib1[:out])]
    order = producer_order(tabs, in_rows)
    assert sorted(order.tolist()) == list(range(out))
    blk, none = in_rows // 16, in_rows // (in_rows // 16) + 1

    def key(o):
        if not pair:
            rows = [tabs[0][0][o], tabs[0][1][o]]
        else:
            rows = []
            for p in (ia2[o], ib2[o]):
                for r1 in (ia1, ib1):
                    rows.append(r1[p] if 0 <= p < mid else -1)
        return tuple(sorted(r // blk if 0 <= r < in_rows else none for r in rows))

    keys = [key(o) for o in order.tolist()]
    assert all(keys[i] < keys[i + 1] or (keys[i] == keys[i + 1] and order[i] < order[i + 1])
               for i in range(out - 1))


def test_columns_layout_cfg5():
    """cfg5's tail: the input column takes words [0, 25088), the first layer's slots 0-13 the
    next 14336 words, its slots 14-15 are held and written over the input's first 2048 words,
    and the second layer goes after them."""
    from compactlogic_amd.packed_net import columns_layout
    assert columns_layout([25088, 16000, 16000]) == {
        "in_words": 25088, "split": 14336, "hold_base": 0, "base": [25088, 2048]}


def test_conv_packed_order_groups_channels_by_input():
    """The packed evaluation order is a permutation of the output features that visits the
    output channels in order of the input channel their winner slot reads."""
    torch.manual_seed(3)
    layer = cl.ConvLayer((6, 8, 8), padding=1, c_out=20, ks=3, stride=2, num_chn=1)
    layer.freeze()
    order = layer.packed_order(layer.w).long()
    hw = layer.h_out * layer.w_out
    assert sorted(order.tolist()) == list(range(20 * hw))
    chans = order.view(20, hw)[:, 0] // hw
    assert torch.equal(order.view(20, hw) - (chans * hw).view(-1, 1), torch.arange(hw).expand(20, hw))
    src = layer.offsets_ch[0, chans, layer.w.long()[chans]]
    assert bool((src[1:] >= src[:-1]).all())


@pytest.mark.parametrize("case", ["shared", "per_slot", "self_pairs", "sparse"])
def test_native_processing_order_equals_python_reference(case):
    """The library's host-side order (cl_plan_locality_order) is the same traversal as the
    Python statement of it in tests/plan_reference.py: identical orders."""
    import plan_reference as ref
    from compactlogic_amd.plan import locality_order
    g = torch.Generator().manual_seed(21)
    in_dim, out_dim = 2000, 1500
    if case == "shared":
        ind = torch.randint(0, in_dim, (2, out_dim, 1), generator=g).expand(2, out_dim, 4)
    elif case == "per_slot":
        ind = torch.randint(0, in_dim, (2, out_dim, 4), generator=g)
    elif case == "self_pairs":
        a = torch.randint(0, in_dim, (out_dim, 1), generator=g)
        ind = torch.stack((a, torch.where(torch.rand((out_dim, 1), generator=g) < 0.3, a,
                                          torch.randint(0, in_dim, (out_dim, 1), generator=g))))
    else:  # few runs: many rows of degree 0, many small components
        ind = torch.randint(0, in_dim, (2, 300, 1), generator=g)
    ind = ind.contiguous()
    plan = cl.build_run_plan(ind, in_dim)
    ra, rb = plan.run_ab[:, 0].long(), plan.run_ab[:, 1].long()
    deg = torch.bincount(torch.cat((ra, rb)), minlength=in_dim)
    want = ref.locality_order(ra, rb, deg, in_dim)
    assert torch.equal(locality_order(ra, rb, in_dim), want)
    assert torch.equal(plan.row_order.long(), want)


def test_native_processing_order_rejects_bad_runs():
    from compactlogic_amd.plan import locality_order
    with pytest.raises(RuntimeError, match="outside"):
        locality_order(torch.tensor([0, 5]), torch.tensor([1, 2]), 4)


def test_dense_packed_tables_and_order():
    """A frozen LogicLayer's packed tables: the winner slot's inputs and opcode per neuron, row
    in_dim (zero words) for a winner outside the slots, and an evaluation order that is a
    permutation in which most neighbours share an input row."""
    torch.manual_seed(8)
    layer = cl.LogicLayer(300, 400, connections="original")
    layer.freeze()
    w = layer.w.clone()
    w[5] = 200                                    # a slot that does not exist
    ia, ib, gate, order = layer.packed_tables(w)
    assert order is not None
    o = torch.arange(400)
    s = w.long().clamp(max=15)
    ok = w.long() < 16
    assert torch.equal(ia[ok].long(), layer.indices[0, o, s][ok])
    assert torch.equal(ib[ok].long(), layer.indices[1, o, s][ok])
    assert torch.equal(gate[ok], layer.gate_sequence[o, s][ok])
    assert int(ia[5]) == 300 and int(ib[5]) == 300
    assert sorted(order.tolist()) == list(range(400))
    a, b = ia[order.long()], ib[order.long()]
    share = ((a[1:] == a[:-1]) | (a[1:] == b[:-1]) | (b[1:] == a[:-1]) | (b[1:] == b[:-1]))
    assert share.float().mean() > 0.5
    assert layer.packed_tables(w)[0] is ia            # cached
    w2 = w.clone()
    assert layer.packed_tables(w2)[0] is not ia       # another winners tensor
    wide = cl.LogicLayer(50, 400, connections="original")   # 16 reads per input row
    wide.freeze()
    assert wide.packed_tables(wide.w)[3] is None


def test_layers_with_warm_caches_pickle_and_rebuild():
    """torch.save of a whole module pickles it: the weak-reference caches are left out and
    rebuilt on the next call, and the loaded layer's plans equal the original's."""
    import io
    torch.manual_seed(5)
    dense = cl.LogicLayer(12, 20, num_gates=16)
    plan = dense.run_plan()
    dense._argmax_slots()
    conv = cl.ConvLayer((3, 7, 9), padding=1, c_out=5, ks=3, stride=2, num_chn=0, num_gates=4)
    conv.freeze()
    ia, ib, g = conv.packed_tables(conv.w)
    buf = io.BytesIO()
    torch.save(torch.nn.Sequential(dense, conv), buf)
    buf.seek(0)
    loaded = torch.load(buf, weights_only=False)  # written by this test
    d2, c2 = loaded[0], loaded[1]
    assert d2._plan is None and d2._plan_key is None and c2._packed_key is None
    p2 = d2.run_plan()
    assert p2.num_runs == plan.num_runs
    assert torch.equal(d2._argmax_slots(), dense._argmax_slots())
    for a, b in zip(c2.packed_tables(c2.w), (ia, ib, g)):
        assert torch.equal(a, b)
    # the original keeps its caches
    assert dense.run_plan() is plan and conv.packed_tables(conv.w)[0] is ia
