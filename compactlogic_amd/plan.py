"""Connection-run plan of a dense LogicLayer (derived state, rebuilt when `indices` change).

A run is a maximal range of consecutive gate slots [g0, g0 + len) of one neuron whose slots
read the same input pair (a, b).  The relaxed operators are affine in the gate weights, so a
run's slots collapse into one set of four coefficients and cost one pair of row gathers.
With the one-pair-per-neuron wiring of `connections='original'` every neuron is one run;
with per-slot random wiring most slots are runs of length one.

The plan also carries the inverse index over inputs that the input-gradient kernel walks:
row i lists the (run, operand side) uses of input i, encoded as 2 * run + side.  Entries
within a row are in ascending (side, run) order, so the result is deterministic.
"""
from __future__ import annotations

from dataclasses import dataclass

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

    @property
    def num_runs(self) -> int:
        return int(self.run_gl.numel())


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
    return RunPlan(
        in_dim=int(in_dim), out_dim=int(out_dim), num_gates=int(g),
        run_ptr=run_ptr.to(i32).contiguous(),
        run_ab=run_ab.to(i32).contiguous(),
        run_gl=run_gl.to(i32).contiguous(),
        run_y=run_y.to(i32).contiguous(),
        inv_ptr=inv_ptr.to(i32).contiguous(),
        inv_entry=entry[order].to(i32).contiguous(),
    )
