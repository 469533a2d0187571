"""Training-time schedules around the logic layers (compactlogic/compactlogic.py:873-1190):
entropy-driven sequential freezing, fixed-schedule freezing, and per-row resampling of
converged rows.  They act through the layers' own methods (`weights_entropy`, `freeze`,
`resample_connections`), so every connection change they make also rebuilds the layers'
derived indices (the inverse index and the kernels' run plan / window tables) before the
next kernel call.
"""
from __future__ import annotations

import numpy as np
import torch


def _logic_layers(model, cap):
    """(position, layer) of every element of `model` that has `freeze`; all but the last one
    when `cap` is None, else the first `cap`."""
    found = [(i, m) for i, m in enumerate(model) if hasattr(m, "freeze")]
    return found[:-1] if cap is None else found[:int(cap)]


class SequentialEntropyFreezer:
    """Freeze the managed layers one after another (compactlogic/compactlogic.py:873-981).

    Each step, the first unfrozen layer whose predecessors are all frozen is examined: its mean
    normalised gate entropy h is compared with the running EMA of h; when |h - EMA| < eps for
    `patience` consecutive steps the layer is frozen.  The first visit of a layer only seeds
    its EMA.  At most one layer is frozen per step; nothing happens before `min_iters`.
    """

    def __init__(self, model, ema_decay=0.99, eps=5e-4, patience=200, min_iters=0, l=None):
        self.model = model
        self.ema_decay = ema_decay
        self.eps = eps
        self.patience = patience
        self.min_iters = min_iters
        self.l = l
        self.logic_layers = _logic_layers(model, l)
        self.ema = {}
        self.counter = {}
        self.iter = 0

    def _can_consider_layer(self, idx):
        return all(layer.is_frozen for i, layer in self.logic_layers if i < idx)

    def _freeze_layer(self, layer):
        layer.freeze()

    def step(self, iter: int):
        self.iter = iter
        if iter < self.min_iters:
            return
        for idx, layer in self.logic_layers:
            if not self._can_consider_layer(idx) or layer.is_frozen:
                continue
            h = layer.weights_entropy().mean().item()
            if idx not in self.ema:
                self.ema[idx] = h
                self.counter[idx] = 0
                return
            previous = self.ema[idx]
            self.ema[idx] = self.ema_decay * previous + (1 - self.ema_decay) * h
            self.counter[idx] = self.counter[idx] + 1 if abs(h - previous) < self.eps else 0
            if self.counter[idx] >= self.patience:
                self._freeze_layer(layer)
                break

    def __str__(self):
        return (f"ema_decay={self.ema_decay}, eps={self.eps}, patience={self.patience}, "
                f"min_iters={self.min_iters}")


class FixedSequentialEntropyFreezer:
    """Freeze the k-th managed layer once the step reaches min_iters + k * N
    (compactlogic/compactlogic.py:984-1054); at most one layer per step, in order."""

    def __init__(self, model, N: int, min_iters: int = 0, l=None):
        if N <= 0:
            raise ValueError(f'N must be > 0, got {N}.')
        self.model = model
        self.N = int(N)
        self.min_iters = min_iters
        self.l = l
        self.logic_layers = _logic_layers(model, l)
        self.iter = 0

    def step(self, iter: int):
        self.iter = iter
        for k, (_, layer) in enumerate(self.logic_layers, start=1):
            if layer.is_frozen:
                continue
            if iter >= self.min_iters + k * self.N:
                layer.freeze()
            break

    def __str__(self):
        return f"N={self.N}, min_iters={self.min_iters}"


class EntropyRowResampler:
    """Per-row convergence monitor with resampling (compactlogic/compactlogic.py:1057-1190).

    Every step in [min_iters, max_iters], for each layer with `resample_connections` (frozen
    ones skipped when `only_unfrozen`): the per-row entropy h is compared with its EMA; rows
    with |h - EMA| < eps for `patience` consecutive steps are handed to
    `layer.resample_connections(rows, **kwargs)`, their Adam moments are cleared and their
    counters restart.  The first visit of a layer only seeds its EMA and counters.
    """

    def __init__(self, model, ema_decay: float = 0.99, eps: float = 5e-4, patience: int = 200,
                 min_iters: int = 0, max_iters=np.inf, only_unfrozen: bool = True, **kwargs):
        self.model = model
        self.ema_decay = ema_decay
        self.eps = eps
        self.patience = patience
        self.min_iters = min_iters
        self.max_iters = max_iters
        self.only_unfrozen = only_unfrozen
        self.resample_kwargs = kwargs
        self.layers = [(i, m) for i, m in enumerate(model) if hasattr(m, "resample_connections")]
        self.ema = {}
        self.counter = {}
        self.iter = 0

    @torch.no_grad()
    def step(self, iter: int, optimizer):
        self.iter = iter
        if iter < self.min_iters or iter > self.max_iters:
            return
        for idx, layer in self.layers:
            if self.only_unfrozen and getattr(layer, "is_frozen", False):
                continue
            h = layer.weights_entropy().detach()
            assert h.dim() == 1
            if idx not in self.ema:
                self.ema[idx] = h.clone()
                self.counter[idx] = torch.zeros_like(h, dtype=torch.int32)
                continue
            previous = self.ema[idx]
            self.ema[idx] = self.ema_decay * previous + (1.0 - self.ema_decay) * h
            steady = (h - previous).abs() < self.eps
            count = torch.where(steady, self.counter[idx] + 1, torch.zeros_like(self.counter[idx]))
            self.counter[idx] = count
            rows = (count >= self.patience).nonzero(as_tuple=False).flatten()
            if rows.numel() > 0:
                weak, strong = layer.resample_connections(rows, **self.resample_kwargs)
                touched = (weak | strong)[:, None].expand_as(layer.weights)
                self.reset_adam_state_for_mask(optimizer, layer.weights, touched)
                self.counter[idx][rows] = 0

    @torch.no_grad()
    def reset_adam_state_for_mask(self, optimizer, param, mask):
        """Zero the Adam moments (exp_avg, exp_avg_sq, max_exp_avg_sq) of the masked entries."""
        state = optimizer.state.get(param, None)
        if not state:
            return
        for key in ("exp_avg", "exp_avg_sq", "max_exp_avg_sq"):
            if key in state:
                state[key].masked_fill_(mask, 0.0)

    def __str__(self):
        return (f"ema_decay={self.ema_decay}, eps={self.eps}, patience={self.patience}, "
                f"min_iters={self.min_iters}, max_iters={self.max_iters}, "
                f"resample_kwargs={self.resample_kwargs}")
