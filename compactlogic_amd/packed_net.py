"""Whole-network packed inference: a frozen dense network (LogicLayer ... GroupSum) evaluated
in one kernel launch per batch of packed samples (csrc/packed_net.hip).

This is the cross-module fusion of the layer-by-layer packed path (LogicLayer.forward on a
PackBitsTensor, then GroupSum): the counts are identical, but no intermediate layer is written
to HBM.  It plays the role of the compiled whole-network evaluators of the reference lineage
(third_party/convlogic_source_code/src/difflogic/compiled_model.py:159-242), built from the
same argmax-slot semantics as compactlogic/compactlogic.py:120-130.
"""
from __future__ import annotations

import ctypes

import torch

from . import _capi
from . import difflogic_hip as _dl
from .layers import ConvLayer, GroupSum, LogicLayer, PackBitsTensor


def _limits():
    nl, rows = ctypes.c_int64(0), ctypes.c_int64(0)
    _capi.call("cl_packed_network_limits", ctypes.byref(nl), ctypes.byref(rows))
    return nl.value, rows.value


class PackedNetwork:
    """Fused packed evaluator of `model`: LogicLayers (frozen or in eval mode; each neuron uses
    its argmax slot `w`) followed by a GroupSum.  Call it with a PackBitsTensor of the first
    layer's input (or its [features, words] tensor) to get int32 class counts [samples, k].

    Widths are limited by LDS: every layer at most cl_packed_network_limits()'s row count.  The
    gate tables are built once here; rebuild after changing the model.
    """

    def __init__(self, model):
        mods = list(model)
        if not mods or not isinstance(mods[-1], GroupSum):
            raise ValueError("the network must end with a GroupSum")
        layers = mods[:-1]
        if not layers or not all(isinstance(m, LogicLayer) and not isinstance(m, ConvLayer)
                                 for m in layers):
            raise ValueError("the fused packed pass takes dense LogicLayers followed by GroupSum")
        max_layers, max_rows = _limits()
        if len(layers) > max_layers:
            raise ValueError(f"at most {max_layers} layers")
        self.k = int(mods[-1].k)
        self.rows = [int(layers[0].in_dim)] + [int(m.out_dim) for m in layers]
        for i, (prev, m) in enumerate(zip(self.rows[:-1], layers)):
            if m.in_dim != prev:
                raise ValueError(f"layer {i} expects {m.in_dim} inputs, gets {prev}")
        if max(self.rows) > max_rows:
            raise ValueError(f"layer widths must be at most {max_rows} for the fused pass")
        if self.rows[-1] % self.k:
            raise ValueError(f"in_dim ({self.rows[-1]}) has to be divisible by k ({self.k}) "
                             "but it is not")
        entries = []
        with torch.no_grad():
            for m in layers:
                w = getattr(m, "w", None)
                if w is None:
                    w = m.weights.argmax(-1)
                slot = w.to(torch.long).view(-1, 1)
                a = torch.gather(m.indices[0], 1, slot).view(-1).to(torch.int64)
                b = torch.gather(m.indices[1], 1, slot).view(-1).to(torch.int64)
                g = torch.gather(m.gate_sequence, 1, slot).view(-1).to(torch.int64) & 15
                if int(a.min()) < 0 or int(a.max()) >= m.in_dim or int(b.min()) < 0 or \
                        int(b.max()) >= m.in_dim:
                    raise IndexError("connection indices out of range")
                entries.append((a * 4) | ((b * 4) << 20) | (g << 40))
        self.tables = torch.cat(entries).contiguous()
        self.device = self.tables.device
        self._rows_host = (ctypes.c_int64 * len(self.rows))(*self.rows)

    def __call__(self, x) -> torch.Tensor:
        if isinstance(x, PackBitsTensor):
            words, n = x.t, x.num_samples
        else:
            words, n = x, x.shape[1] * x.element_size() * 8
        _dl._check(words, "x")
        if words.device != self.device:
            raise RuntimeError(f"x is on {words.device}, the network on {self.device}")
        if words.dim() != 2 or words.shape[0] != self.rows[0]:
            raise RuntimeError(f"x must be [{self.rows[0]}, words], got {tuple(words.shape)}")
        row_bytes = words.shape[1] * words.element_size()
        counts = torch.empty((n, self.k), dtype=torch.int32, device=words.device)
        with torch.cuda.device(words.device):
            _capi.call("cl_packed_network", words.data_ptr(), row_bytes, n,
                       self.tables.data_ptr(), self._rows_host, len(self.rows) - 1, self.k,
                       counts.data_ptr(), _dl.stream_of(words))
        return counts
