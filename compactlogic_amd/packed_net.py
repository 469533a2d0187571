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

import numpy as np
import torch

from . import _capi
from . import timing
from . import difflogic_hip as _dl
from .layers import ConvLayer, GroupSum, LogicLayer, PackBitsTensor


def _limits():
    nl, rows = ctypes.c_int64(0), ctypes.c_int64(0)
    _capi.call("cl_packed_network_limits", ctypes.byref(nl), ctypes.byref(rows))
    return nl.value, rows.value


# LDS geometry of gfx950 as the fused kernel uses it (measured with 64-lane ds_read_b32
# patterns and SQ_LDS_BANK_CONFLICT): a read instruction is served one half-wave (32 lanes) at
# a time, and the lanes of a half-wave conflict when their words share word % 32.  The lanes of
# one half-wave read the rows of 32 consecutive positions of the layer being computed.
_LDS_BANKS = 32
_HALF_WAVE = 32


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def _layout(ka, kb, fa, fb, rows: int, class_size: int) -> np.ndarray:
    P = ctypes.POINTER(ctypes.c_int32)
    ka, kb = _i32(ka), _i32(kb)
    pos = np.empty(int(rows), dtype=np.int32)
    fa_ = None if fa is None else _i32(fa)
    fb_ = None if fb is None else _i32(fb)
    _capi.call("cl_packed_bank_layout", ka.ctypes.data_as(P), kb.ctypes.data_as(P),
               None if fa_ is None else fa_.ctypes.data_as(P),
               None if fb_ is None else fb_.ctypes.data_as(P), int(rows), int(class_size),
               pos.ctypes.data_as(P))
    return pos.astype(np.int64)


def bank_aware_positions(pos_a: np.ndarray, pos_b: np.ndarray, rows: int,
                         fan_a: np.ndarray | None = None,
                         fan_b: np.ndarray | None = None) -> np.ndarray:
    """Positions (LDS words, a permutation of 0..rows-1) for the gates of one layer whose
    inputs sit at words pos_a / pos_b of the previous layer (cl_packed_bank_layout): blocks of
    32 consecutive positions (one half-wave of the kernel's row reads) that read their a rows
    from 32 distinct banks and their b rows from 32 distinct banks, from an edge colouring of
    the (bank a, bank b) multigraph with one colour per block.  Inside a block the position is
    free for this layer; with the next layer's fan-outs of these rows (fan_a: reads as operand
    a, fan_b: as operand b) it is chosen to level the next layer's bank degrees, which is what
    lets that layer's colouring avoid conflicts.  Deterministic."""
    return _layout(np.asarray(pos_a) % _LDS_BANKS, np.asarray(pos_b) % _LDS_BANKS, fan_a, fan_b,
                   rows, 0)


def bank_aware_positions_grouped(pos_a: np.ndarray, pos_b: np.ndarray, rows: int,
                                 group_size: int) -> np.ndarray:
    """bank_aware_positions for the last layer, whose rows must stay in their class: gate o
    (class o // group_size) is placed inside [class * group_size, (class + 1) * group_size).
    Deterministic."""
    return _layout(np.asarray(pos_a) % _LDS_BANKS, np.asarray(pos_b) % _LDS_BANKS, None, None,
                   rows, group_size)


# the fused kernel stages each 32-sample column of its input in LDS: at most _LDS_INPUT_ROWS
# input rows (four per thread).  Gathering one word of every input row per column from a wider
# input is bound by L2 capacity (the rows' lines of 32 columns must stay resident), and a
# kernel that did so measured 3.7-7x slower than the layer path.
_LDS_INPUT_ROWS = 4096


def _fusable(in_rows: int, outs: list, max_layers: int, max_rows: int) -> bool:
    """Whether cl_packed_network takes dense layers of widths `outs` on `in_rows` inputs."""
    return (bool(outs) and len(outs) <= max_layers and in_rows <= _LDS_INPUT_ROWS
            and max(outs) <= max_rows)


def columns_layout(rows: list) -> dict | None:
    """LDS placement of the wide-input fused pass for layer widths `rows` (input first), or
    None when it does not apply (cl_packed_network_columns_layout): in_words (LDS words per
    input column), split and hold_base (row p of the first layer is word base[0] + p below
    split, else hold_base + p - split) and base (row p of layer l >= 1 is word base[l] + p)."""
    n = len(rows) - 1
    if n < 1 or n > _limits()[0]:
        return None
    arr = (ctypes.c_int64 * len(rows))(*[int(r) for r in rows])
    applies, in_words, split, hold = (ctypes.c_int64() for _ in range(4))
    base = (ctypes.c_int64 * n)()
    _capi.call("cl_packed_network_columns_layout", arr, n, ctypes.byref(applies),
               ctypes.byref(in_words), ctypes.byref(split), ctypes.byref(hold), base)
    if not applies.value:
        return None
    return {"in_words": in_words.value, "split": split.value, "hold_base": hold.value,
            "base": list(base)}


def producer_order(tabs: list, in_rows: int) -> np.ndarray:
    """Order in which the column producer evaluates its rows (int32, a permutation): rows
    sorted by the sorted tuple of the blocks (in_rows // 16 rows each) of the input rows they
    read, ties in row order.  Rows reading the same input blocks then run together, so the
    input words of a column tile they need stay in one XCD's L2.  tabs: the (ia, ib) index
    arrays of the producer's layers (one, or two composed, the second reading the first's
    rows); a negative or out-of-range index reads nothing."""
    blk = max(1, in_rows // 16)
    none = in_rows // blk + 1

    def blocks(rows, n):
        ok = (rows >= 0) & (rows < n)
        return ok, np.where(ok, rows, 0)

    if len(tabs) == 1:
        ia, ib = tabs[0]
        cols = []
        for r in (ia, ib):
            ok, rr = blocks(r, in_rows)
            cols.append(np.where(ok, rr // blk, none))
    else:
        (ia1, ib1), (ia2, ib2) = tabs
        mid = ia1.size
        cols = []
        for r2 in (ia2, ib2):
            ok2, p = blocks(r2, mid)
            for r1 in (ia1, ib1):
                ok1, rr = blocks(r1[p], in_rows)
                cols.append(np.where(ok2 & ok1, rr // blk, none))
    key = np.sort(np.stack(cols, 1), axis=1)
    n = key.shape[0]
    return np.lexsort((np.arange(n),) + tuple(key[:, j] for j in reversed(range(key.shape[1])))
                      ).astype(np.int32)


def _table_layer_before(body: list, j: int):
    """Index of the module before body[j] (Flatten modules pass a PackBitsTensor through
    unchanged) when it is a packed layer from index tables (ConvLayer or LogicLayer); else
    None."""
    j -= 1
    while j >= 0 and type(body[j]) is torch.nn.Flatten:
        j -= 1
    if j < 0 or type(body[j]) not in (ConvLayer, LogicLayer):
        return None
    return j


class PackedNetwork:
    """Fused packed evaluator of `model` (frozen or in eval mode; each neuron uses its argmax
    slot `w`), ending in a GroupSum.  Call it with a PackBitsTensor of the network's input (or
    its [features, words] tensor) to get int32 class counts [samples, k].

    The longest tail of dense LogicLayers that the fused kernel takes (an input of at most
    4096 rows, widths within LDS) runs in one launch with every 32-sample column held in LDS;
    the modules before it (ConvLayers, ConvLogicLayers, wider dense layers, Flatten) run layer
    by layer on the packed kernels first.  A tail whose input is wider (cfg5's 25088 conv
    outputs) is fused when a ConvLayer or dense LogicLayer feeds it and its layers fit
    (columns_layout): that layer writes its output column-major
    (cl_eval_packed_indexed_columns) and the tail runs on those columns
    (cl_packed_network_columns).  When no tail qualifies every module runs layer by
    layer and the counts come from the group popcount.  The gate tables are built once here;
    rebuild after changing the model.  With `bank_aware` (default), each fused layer's rows
    are laid out in LDS by bank_aware_positions, so that the row reads of the kernel's
    half-waves hit distinct LDS banks; the counts do not depend on the layout.
    """

    def __init__(self, model, bank_aware: bool = True):
        mods = list(model)
        if not mods or not isinstance(mods[-1], GroupSum):
            raise ValueError("the network must end with a GroupSum")
        body = mods[:-1]
        if not body:
            raise ValueError("the network needs a layer before its GroupSum")
        max_layers, max_rows = _limits()
        self.k = int(mods[-1].k)
        # the fused tail: the longest run of trailing dense layers that the kernel takes
        first = len(body)
        while first > 0 and type(body[first - 1]) is LogicLayer:
            first -= 1
        start = next((j for j in range(first, len(body))
                      if _fusable(int(body[j].in_dim), [int(m.out_dim) for m in body[j:]],
                                  max_layers, max_rows)), len(body))
        # a tail whose input is too wide to stage row by row: its input comes column-major
        # from the packed layer before it (cl_eval_packed_indexed_columns)
        self.producer = None     # the layer (or pair of layers) writing the tail's columns
        self.layout = None
        if start != first and first < len(body):
            prod = _table_layer_before(body, first)
            rows = [int(body[first].in_dim)] + [int(m.out_dim) for m in body[first:]]
            layout = columns_layout(rows) if prod is not None else None
            if layout is not None:
                start, self.layout = first, layout
                # a table layer before the producer is composed into it: its rows are
                # computed where the producer reads them, never stored
                pre = _table_layer_before(body, prod)
                if pre is not None:
                    self.producer, self.prefix = (body[pre], body[prod]), body[:pre]
                else:
                    self.producer, self.prefix = (body[prod],), body[:prod]
        layers = body[start:]
        if self.producer is None:
            self.prefix = body[:start]
        if not layers:
            self.rows = None            # no fused tail: layer by layer, then the popcount
            self.device = None
            return
        self.rows = [int(layers[0].in_dim)] + [int(m.out_dim) for m in layers]
        for i, (prev, m) in enumerate(zip(self.rows[:-1], layers)):
            if m.in_dim != prev:
                raise ValueError(f"layer {i} expects {m.in_dim} inputs, gets {prev}")
        if self.rows[-1] % self.k:
            raise ValueError(f"in_dim ({self.rows[-1]}) has to be divisible by k ({self.k}) "
                             "but it is not")
        entries = []
        with torch.no_grad():
            wiring = []
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
                wiring.append((a.cpu().numpy(), b.cpu().numpy(), g.cpu().numpy(), a.device))
            prev_pos = np.arange(self.rows[0], dtype=np.int64)   # input rows stay in place
            lay = self.layout
            self.col_order = None
            if self.producer is not None:
                # the producer writes its rows in producer_order; input row r of the tail is
                # then at position inv[r] of a column
                tabs = []
                for m in self.producer:
                    w = getattr(m, "w", None)
                    if w is None:
                        w = m._argmax_slots()
                    ia, ib = m.packed_tables(w)[:2]
                    tabs.append((ia.cpu().numpy().astype(np.int64),
                                 ib.cpu().numpy().astype(np.int64)))
                m0 = self.producer[0]
                in_rows = m0.in_dim if type(m0) is LogicLayer else int(np.prod(m0.in_shape))
                order = producer_order(tabs, in_rows)
                prev_pos = np.empty(self.rows[0], dtype=np.int64)
                prev_pos[order] = np.arange(self.rows[0], dtype=np.int64)
                self.col_order = torch.as_tensor(order, device=layers[0].weights.device)
            for i, (m, (a, b, g, dev)) in enumerate(zip(layers, wiring)):
                pa, pb = prev_pos[a], prev_pos[b]
                if not bank_aware:
                    pos = np.arange(m.out_dim, dtype=np.int64)
                elif i + 1 < len(layers):
                    na, nb = wiring[i + 1][:2]
                    pos = bank_aware_positions(pa, pb, m.out_dim,
                                               np.bincount(na, minlength=m.out_dim),
                                               np.bincount(nb, minlength=m.out_dim))
                else:  # class groups stay contiguous
                    pos = bank_aware_positions_grouped(pa, pb, m.out_dim, m.out_dim // self.k)
                ent = np.empty(m.out_dim, dtype=np.int64)
                if lay is None:
                    ent[pos] = (pa * 4) | ((pb * 4) << 20) | (g << 40)   # LDS byte offsets
                    prev_pos = pos
                else:
                    ent[pos] = pa | (pb << 16) | (g << 32)               # LDS words
                    # the LDS word of each row (banks as the positions': every base is a
                    # multiple of 32 words)
                    if i == 0:
                        prev_pos = np.where(pos < lay["split"], lay["base"][0] + pos,
                                            lay["hold_base"] + pos - lay["split"])
                    else:
                        prev_pos = lay["base"][i] + pos
                entries.append(torch.as_tensor(ent, device=dev))
        self.tables = torch.cat(entries).contiguous()
        self.device = self.tables.device
        self._rows_host = (ctypes.c_int64 * len(self.rows))(*self.rows)

    def __call__(self, x) -> torch.Tensor:
        if self.producer is not None:
            return self._call_columns(x)
        if self.prefix:
            if isinstance(x, PackBitsTensor):
                h = PackBitsTensor.from_packed(x.t, x.pad_len)   # the caller's object stays
            else:
                h = PackBitsTensor.from_packed(x)
            with torch.no_grad():
                for m in self.prefix:
                    h = m(h)
            if self.rows is None:
                return h.group_sum(self.k)
            x = h
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
            timing.timed(f"cl_packed_network[{self.rows[0]}->{self.rows[-1]}]", lambda: _capi.call(
                "cl_packed_network", words.data_ptr(), row_bytes, n, self.tables.data_ptr(),
                self._rows_host, len(self.rows) - 1, self.k, counts.data_ptr(),
                _dl.stream_of(words)))
        return counts

    def _call_columns(self, x) -> torch.Tensor:
        """The wide-input path: the prefix layer by layer, the producer layer (or pair of
        layers) written column-major, then the fused tail on those columns."""
        if isinstance(x, PackBitsTensor):
            h = PackBitsTensor.from_packed(x.t, x.pad_len)   # the caller's object stays
        else:
            h = PackBitsTensor.from_packed(x)
        tabs = []
        with torch.no_grad():
            for m in self.prefix:
                h = m(h)
            for m in self.producer:
                w = getattr(m, "w", None)
                if w is None:
                    w = m._argmax_slots()
                tabs.append(m.packed_tables(w)[:3])
        words, n = h.t, h.num_samples
        _dl._check(words, "x")
        if words.device != self.device:
            raise RuntimeError(f"x is on {words.device}, the network on {self.device}")
        in_rows = words.shape[0]
        m = self.producer[0]
        expect = m.in_dim if type(m) is LogicLayer else int(np.prod(m.in_shape))
        if in_rows != expect:
            raise RuntimeError(f"the layer before the fused tail gets {in_rows} rows, "
                               f"expects {expect}")
        if tabs[-1][0].numel() != self.rows[0]:
            raise RuntimeError(f"the layer before the fused tail has {tabs[-1][0].numel()} "
                               f"outputs, the tail reads {self.rows[0]}")
        row_bytes = words.shape[1] * words.element_size()
        if row_bytes % 4:
            raise RuntimeError("packed rows must be a multiple of 4 bytes")
        cols, in_words = row_bytes // 4, self.layout["in_words"]
        colmaj = torch.empty((cols, in_words), dtype=torch.int32, device=words.device)
        counts = torch.empty((n, self.k), dtype=torch.int32, device=words.device)
        stream = _dl.stream_of(words)
        ptrs = [t.data_ptr() for tab in tabs for t in tab]
        with torch.cuda.device(words.device):
            order = self.col_order.data_ptr()
            if len(tabs) == 2:
                mid = tabs[0][0].numel()
                timing.timed(f"cl_eval_packed_indexed_pair_columns[{in_rows}->{mid}->"
                             f"{self.rows[0]}]", lambda: _capi.call(
                    "cl_eval_packed_indexed_pair_columns", words.data_ptr(), *ptrs, order,
                    colmaj.data_ptr(), in_rows, mid, self.rows[0], row_bytes, in_words, stream))
            else:
                timing.timed(f"cl_eval_packed_indexed_columns[{in_rows}->{self.rows[0]}]",
                             lambda: _capi.call(
                    "cl_eval_packed_indexed_columns", words.data_ptr(), *ptrs, order,
                    colmaj.data_ptr(), in_rows, self.rows[0], row_bytes, in_words, stream))
            timing.timed(f"cl_packed_network_columns[{self.rows[0]}->{self.rows[-1]}]",
                         lambda: _capi.call(
                "cl_packed_network_columns", colmaj.data_ptr(), cols, in_words, n,
                self.tables.data_ptr(), self._rows_host, len(self.rows) - 1, self.k,
                counts.data_ptr(), stream))
        return counts
