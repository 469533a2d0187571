"""Connection-run plan of a dense LogicLayer (derived state, rebuilt when `indices` change).

A run is a maximal range of consecutive gate slots [g0, g0 + len) of one neuron whose slots
read the same input pair (a, b).  The relaxed operators are affine in the gate weights, so a
run's slots collapse into one set of four coefficients and cost one pair of row gathers.
With the one-pair-per-neuron wiring of `connections='original'` every neuron is one run;
with per-slot random wiring most slots are runs of length one.

The plan also carries the inverse index over inputs that the input-gradient kernel walks:
row i lists the (run, operand side) uses of input i, encoded as 2 * run + side.  Entries
within a row are in ascending (side, run) order, so the result is deterministic.  Each entry
also has a ready record (neuron, other input, run, side) so the kernel needs no second
lookup, `inv_pos` maps a run side to its entry (where the per-step coefficients are written),
and `row_order` is the processing order of the inputs (breadth-first over the run graph for
cache reuse, degree-sorted in blocks so that rows processed side by side have equal work).  `nab` and `slot_rec` hold, per neuron and per processing slot, what a
kernel needs before its first gather (first run's pair and run range; input row and entry
range), so each is one load away.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


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

    @property
    def num_runs(self) -> int:
        return int(self.run_gl.numel())


def locality_order(ra: torch.Tensor, rb: torch.Tensor, degree: torch.Tensor, in_dim: int,
                   block: int = 1024) -> torch.Tensor:
    """Processing order of the inputs for the input-gradient pass: breadth-first over the
    graph whose edges are the runs (a, b), then sorted by descending degree inside blocks of
    `block` consecutive inputs.  Both uses of a run (its rows a and b) and of an input (as a
    row and as the other operand of its neighbours' entries) then fall close together in
    time, so the second read of a row segment hits the L2; the block sort keeps the inputs
    processed side by side of equal work.  Inputs of degree 0 come last.  Deterministic:
    searches start from the highest-degree unvisited input (lowest index on ties)."""
    dev = ra.device
    a = ra.cpu().numpy().astype(np.int64)
    b = rb.cpu().numpy().astype(np.int64)
    deg = degree.cpu().numpy().astype(np.int64)
    src = np.concatenate((a, b))
    dst = np.concatenate((b, a))
    order = np.argsort(src, kind="stable")
    nbr = dst[order]
    ptr = np.zeros(in_dim + 1, dtype=np.int64)
    np.cumsum(np.bincount(src, minlength=in_dim), out=ptr[1:])
    seen = deg == 0
    out = []
    for start in np.argsort(-deg, kind="stable"):
        if seen[start]:
            continue
        seen[start] = True
        frontier = np.array([start], dtype=np.int64)
        while frontier.size:
            out.append(frontier)
            cnt = ptr[frontier + 1] - ptr[frontier]
            tot = int(cnt.sum())
            if tot == 0:
                break
            first = np.repeat(ptr[frontier], cnt)
            offs = np.arange(tot) - np.repeat(np.cumsum(cnt) - cnt, cnt)
            cand = nbr[first + offs]
            cand = cand[~seen[cand]]
            _, keep = np.unique(cand, return_index=True)
            frontier = cand[np.sort(keep)]
            seen[frontier] = True
    out.append(np.nonzero(deg == 0)[0])
    visit = np.concatenate(out) if out else np.zeros(0, dtype=np.int64)
    for s0 in range(0, visit.size, block):
        seg = visit[s0:s0 + block]
        visit[s0:s0 + block] = seg[np.argsort(-deg[seg], kind="stable")]
    return torch.as_tensor(visit, dtype=torch.int64, device=dev)


def build_run_plan(indices: torch.Tensor, in_dim: int) -> RunPlan:
    """Derive the run plan from `indices` [2, out_dim, G] (int64) on its device."""
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
    # Inverse index: side-0 entries of all runs, then side-1 entries; a stable sort by
    # input keeps that order inside every row.
    inputs = torch.cat((ra, rb))
    ids = torch.arange(r, dtype=torch.int64, device=dev) * 2
    entry = torch.cat((ids, ids + 1))
    order = torch.sort(inputs, stable=True).indices
    inv_counts = torch.bincount(inputs, minlength=in_dim)
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
    row_order = locality_order(ra, rb, inv_counts, in_dim)
    first = run_ptr[:-1].clamp(max=max(r - 1, 0))
    has = run_ptr[1:] > run_ptr[:-1]
    nab = torch.stack((torch.where(has, ra[first] if r else first, 0),
                       torch.where(has, rb[first] if r else first, 0),
                       run_ptr[:-1], run_ptr[1:]), dim=1)
    slot_rec = torch.stack((row_order, inv_ptr[row_order], inv_ptr[row_order + 1],
                            torch.zeros_like(row_order)), dim=1)
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
    )
