"""Connection-run plan of a dense LogicLayer (derived state, rebuilt when `indices` change).

A run is a maximal range of consecutive gate slots [g0, g0 + len) of one neuron whose slots
read the same input pair (a, b).  The relaxed operators are affine in the gate weights, so a
run's slots collapse into one set of four coefficients and cost one pair of row gathers.
With the one-pair-per-neuron wiring of `connections='original'` every neuron is one run;
with per-slot random wiring most slots are runs of length one.

The plan also carries the inverse index over inputs that the input-gradient kernel walks:
row i lists the (run, operand side) uses of input i, encoded as 2 * run + side.  Entries
within a row are ordered by the distance, in the processing order below, between the row and
the run's other input (ties: side, then run), so the result is deterministic.  Each entry
also has a ready record (neuron, other input, run, side) so the kernel needs no second
lookup, `inv_pos` maps a run side to its entry (where the per-step coefficients are written),
and `row_order` is the processing order of the inputs: a depth-first preorder over the graph
whose edges are the runs (small subtrees first), so that inputs joined by runs are mostly
close together.  `nab` and
`slot_rec` hold, per neuron and per processing slot, what a kernel needs before its first
gather (first run's pair and run range; input row and entry range), so each is one load away.

The processing slots are cut into tiles of PART_ROWS inputs.  A run whose two inputs lie in
the same tile is *internal* to it: the input-gradient kernel then reads its grad_y row once,
takes both input rows from the tile's copy in LDS and leaves the two contributions in LDS
slots (`inv_slot` of the two entries) for the rows' owners to add in entry order.  With the
depth-first order about two thirds of the runs of a random wiring are internal, which saves
three of the four row reads such a run costs otherwise.  A tile holds at most PART_SLOTS / 2
internal runs (the rest stay external).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _capi


PART_ROWS = 16    # inputs per tile of the partitioned input-gradient kernel
PART_SLOTS = 32   # LDS contribution slots per tile (two per internal run)


@dataclass
class RunPlan:
    in_dim: int
    out_dim: int
    num_gates: int
    run_ptr: torch.Tensor    # int32 [out_dim + 1]
    run_ab: torch.Tensor     # int32 [R, 2]
    run_gl: torch.Tensor     # int32 [R]  g0 | len << 8
    run_y: torch.Tensor      # int32 [R]
    inv_ptr: torch.Tensor    # int32 [in_dim + 1]
    inv_entry: torch.Tensor  # int32 [2R]
    inv_rec: torch.Tensor    # int32 [2R, 4]  (neuron, other input, run, side) per entry
    inv_pos: torch.Tensor    # int32 [2R]     entry position of run side 2r + s
    row_order: torch.Tensor  # int32 [in_dim] processing order of the inputs (locality_order)
    nab: torch.Tensor        # int32 [out_dim, 4] (a, b of the first run, run_ptr[o], run_ptr[o+1])
    slot_rec: torch.Tensor   # int32 [in_dim, 4]  (input, first entry, end entry, 0) in row_order
    single_run: bool = False  # every neuron is exactly one run (all its slots share a pair)
    inv_slot: torch.Tensor = None   # int32 [2R] LDS slot of an internal entry, -1 external
    tile_ptr: torch.Tensor = None   # int32 [ntiles + 1] internal runs of tile t
    tile_run: torch.Tensor = None   # int32 [N, 4] (neuron, run, entry of a, entry of b)
    tile_loc: torch.Tensor = None   # int32 [N] a_local | b_local << 8 | slot_a << 16 | slot_b << 24
    src_indices: torch.Tensor = None  # the indices the plan was built from (a copy)
    stale: int = 0                    # neurons rewired since row_order was last computed

    @property
    def num_runs(self) -> int:
        return int(self.run_gl.numel())


def locality_order(ra: torch.Tensor, rb: torch.Tensor, in_dim: int) -> torch.Tensor:
    """Processing order of the inputs for the input-gradient pass (int64 [in_dim], on ra's
    device): the preorder of a depth-first spanning forest of the graph whose edges are the
    runs (a, b), every input's children visited in increasing order of their subtree sizes
    (equal sizes in discovery order), inputs of degree 0 last.  Searches start from the
    highest-degree unvisited input and scan an input's runs in run order (operand a, then
    operand b).

    A subtree occupies consecutive positions, so a run between a parent and its child spans
    only the subtrees of the child's smaller siblings; visiting the small subtrees first keeps
    that span short for every child, and with it the time between the two reads of the
    run's grad_y row and of the shared input rows.  Deterministic; built on the host by the
    library (cl_plan_locality_order), in linear time."""
    dev = ra.device
    a = np.ascontiguousarray(ra.detach().cpu().numpy().astype(np.int32))
    b = np.ascontiguousarray(rb.detach().cpu().numpy().astype(np.int32))
    out = np.empty(in_dim, dtype=np.int32)
    i32p = ctypes.POINTER(ctypes.c_int32)
    _capi.call("cl_plan_locality_order", a.ctypes.data_as(i32p), b.ctypes.data_as(i32p),
               a.size, in_dim, out.ctypes.data_as(i32p))
    return torch.as_tensor(out.astype(np.int64), device=dev)


def partition_tiles(row_order: torch.Tensor, ra: torch.Tensor, rb: torch.Tensor,
                    run_y: torch.Tensor, inv_pos: torch.Tensor, in_dim: int):
    """Internal runs of the tiles of PART_ROWS consecutive processing slots (see the module
    docstring): (inv_slot, tile_ptr, tile_run, tile_loc).  The internal runs of a tile are
    taken in run order, at most PART_SLOTS // 2 of them; run k of a tile owns the LDS slots
    2k (its operand-a entry) and 2k + 1 (operand b)."""
    dev = ra.device
    r = ra.numel()
    ntiles = (in_dim + PART_ROWS - 1) // PART_ROWS
    pos = torch.empty(in_dim, dtype=torch.int64, device=dev)
    pos[row_order] = torch.arange(in_dim, dtype=torch.int64, device=dev)
    ta, tb = pos[ra] // PART_ROWS, pos[rb] // PART_ROWS
    cand = (ta == tb).nonzero().squeeze(1)                      # ascending run order
    tile = ta[cand]
    order = torch.sort(tile, stable=True).indices
    cand, tile = cand[order], tile[order]
    counts = torch.bincount(tile, minlength=ntiles)
    first = torch.zeros(ntiles + 1, dtype=torch.int64, device=dev)
    first[1:] = torch.cumsum(counts, 0)
    rank = torch.arange(cand.numel(), dtype=torch.int64, device=dev) - first[tile]
    keep = rank < PART_SLOTS // 2
    cand, tile, rank = cand[keep], tile[keep], rank[keep]
    kept = torch.bincount(tile, minlength=ntiles)
    tile_ptr = torch.zeros(ntiles + 1, dtype=torch.int64, device=dev)
    tile_ptr[1:] = torch.cumsum(kept, 0)
    pa, pb = inv_pos[2 * cand], inv_pos[2 * cand + 1]
    sa, sb = 2 * rank, 2 * rank + 1
    inv_slot = torch.full((2 * r,), -1, dtype=torch.int64, device=dev)
    inv_slot[pa] = sa
    inv_slot[pb] = sb
    tile_run = torch.stack((run_y[cand], cand, pa, pb), dim=1)
    loc = (pos[ra[cand]] % PART_ROWS) | ((pos[rb[cand]] % PART_ROWS) << 8) | (sa << 16) | (sb << 24)
    i32 = torch.int32
    return (inv_slot.to(i32).contiguous(), tile_ptr.to(i32).contiguous(),
            tile_run.reshape(-1, 4).to(i32).contiguous(), loc.to(i32).contiguous())


# A rewiring that changes at most this fraction of a layer's neurons (counted since the last
# full order) keeps the previous processing order of the inputs: the order only sets memory
# locality, and recomputing it is the plan's one host round trip.
REORDER_FRACTION = 0.1


def build_run_plan(indices: torch.Tensor, in_dim: int,
                   row_order: torch.Tensor | None = None) -> RunPlan:
    """Derive the run plan from `indices` [2, out_dim, G] (int64) on its device.  With
    `row_order` (a permutation of the inputs, e.g. a previous plan's) the inputs' processing
    order is taken from it instead of being recomputed (locality_order): every result is the
    same up to the order of additions within a row."""
    if indices.dim() != 3 or indices.shape[0] != 2:
        raise ValueError(f"indices must be [2, out_dim, num_gates], got {tuple(indices.shape)}")
    _, out_dim, g = indices.shape
    if g < 1 or g > 128:
        raise ValueError(f"num_gates must be in [1, 128], got {g}")
    dev = indices.device
    if indices.numel() and (int(indices.min()) < 0 or int(indices.max()) >= in_dim):
        raise IndexError(f"connection indices must lie in [0, {in_dim})")
    if in_dim >= 2**31 or out_dim * g >= 2**30:
        raise ValueError("layer too large for the int32 run plan")
    a = indices[0].reshape(out_dim, g)
    b = indices[1].reshape(out_dim, g)
    start = torch.ones((out_dim, g), dtype=torch.bool, device=dev)
    if g > 1:
        start[:, 1:] = (a[:, 1:] != a[:, :-1]) | (b[:, 1:] != b[:, :-1])
    pos = start.reshape(-1).nonzero().squeeze(1)          # flat o*G + g0, ascending
    r = pos.numel()
    run_y = torch.div(pos, g, rounding_mode="floor")
    g0 = pos - run_y * g
    nxt = torch.empty_like(pos)
    if r:
        nxt[:-1] = pos[1:]
        nxt[-1] = out_dim * g
    length = nxt - pos                                      # slot 0 always starts a run
    counts = torch.bincount(run_y, minlength=out_dim)
    run_ptr = torch.zeros(out_dim + 1, dtype=torch.int64, device=dev)
    run_ptr[1:] = torch.cumsum(counts, 0)
    ra = a.reshape(-1)[pos]
    rb = b.reshape(-1)[pos]
    run_ab = torch.stack((ra, rb), dim=1)
    run_gl = g0 | (length << 8)
    # Inverse index: the entries of every input row, nearest partner first: ordered by the
    # distance between the row and the run's other input in the processing order (then by
    # side-0 entries of all runs before side-1 entries, in run order).  Two rows joined by a
    # run then tend to reach that run's entry at the same step, while its grad_y row and
    # their two input rows are in cache.
    inputs = torch.cat((ra, rb))
    others = torch.cat((rb, ra))
    ids = torch.arange(r, dtype=torch.int64, device=dev) * 2
    entry = torch.cat((ids, ids + 1))
    inv_counts = torch.bincount(inputs, minlength=in_dim)
    if row_order is None:
        row_order = locality_order(ra, rb, in_dim)
    else:
        row_order = row_order.to(device=dev, dtype=torch.int64)
        if row_order.shape != (in_dim,):
            raise ValueError(f"row_order must have {in_dim} entries")
    rpos = torch.empty(in_dim, dtype=torch.int64, device=dev)
    rpos[row_order] = torch.arange(in_dim, dtype=torch.int64, device=dev)
    dist = (rpos[inputs] - rpos[others]).abs()
    nent = max(2 * r, 1)
    key = (inputs * (in_dim + 1) + dist) * nent + torch.arange(2 * r, dtype=torch.int64, device=dev)
    order = torch.sort(key).indices
    inv_ptr = torch.zeros(in_dim + 1, dtype=torch.int64, device=dev)
    inv_ptr[1:] = torch.cumsum(inv_counts, 0)
    i32 = torch.int32
    inv_entry = entry[order]
    ent_run = torch.div(inv_entry, 2, rounding_mode="floor")
    ent_side = inv_entry - 2 * ent_run
    ent_other = torch.where(ent_side == 0, rb[ent_run], ra[ent_run])
    inv_rec = torch.stack((run_y[ent_run], ent_other, ent_run, ent_side), dim=1)
    inv_pos = torch.empty_like(inv_entry)
    inv_pos[inv_entry] = torch.arange(inv_entry.numel(), dtype=torch.int64, device=dev)
    first = run_ptr[:-1].clamp(max=max(r - 1, 0))
    has = run_ptr[1:] > run_ptr[:-1]
    nab = torch.stack((torch.where(has, ra[first] if r else first, 0),
                       torch.where(has, rb[first] if r else first, 0),
                       run_ptr[:-1], run_ptr[1:]), dim=1)
    slot_rec = torch.stack((row_order, inv_ptr[row_order], inv_ptr[row_order + 1],
                            torch.zeros_like(row_order)), dim=1)
    inv_slot, tile_ptr, tile_run, tile_loc = partition_tiles(row_order, ra, rb, run_y, inv_pos,
                                                             in_dim)
    return RunPlan(
        in_dim=int(in_dim), out_dim=int(out_dim), num_gates=int(g),
        run_ptr=run_ptr.to(i32).contiguous(),
        run_ab=run_ab.to(i32).contiguous(),
        run_gl=run_gl.to(i32).contiguous(),
        run_y=run_y.to(i32).contiguous(),
        inv_ptr=inv_ptr.to(i32).contiguous(),
        inv_entry=inv_entry.to(i32).contiguous(),
        inv_rec=inv_rec.to(i32).contiguous(),
        inv_pos=inv_pos.to(i32).contiguous(),
        row_order=row_order.to(i32).contiguous(),
        nab=nab.to(i32).contiguous(),
        slot_rec=slot_rec.to(i32).contiguous(),
        single_run=bool(out_dim > 0 and r == out_dim),
        inv_slot=inv_slot, tile_ptr=tile_ptr, tile_run=tile_run, tile_loc=tile_loc,
        src_indices=indices.detach().clone(),
    )
